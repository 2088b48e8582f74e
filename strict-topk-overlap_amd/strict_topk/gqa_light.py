"""GQA saved-state repair in one launch, for steps with few misses per head.

Drop-in for the reference ``strict_topk/gqa_light.py`` (``repair_saved_light``
:63-77, ``repair_saved_auto`` :80-92).
"""
import torch

from . import _lib, gqa
from .kernels import _args


def repair_saved_light(q, k, v, selected, predicted, state):
    """Repair the strict selected set with one workgroup per query head."""
    hq, n, b, d, group, sa = gqa._shape(q, k, v, selected)
    gqa._validate_ids(q, predicted)
    sp = predicted.shape[1]
    if state.m.shape != (hq, sp) or state.l.shape != (hq, sp) or state.u.shape != (hq, sp, d):
        raise ValueError("state must contain a softmax partial for every predicted block")
    out = torch.empty((hq, d), device=q.device, dtype=torch.float32)
    _lib.call("stk_repair_light", *_args(q, k, v), _lib.ptr(selected), _lib.id_code(selected), sa,
              _lib.ptr(predicted), _lib.id_code(predicted), sp, _lib.ptr(state.m),
              _lib.ptr(state.l), _lib.ptr(state.u), _lib.ptr(out), _lib.stream(q.device))
    return out


def repair_saved_auto(q, k, v, selected, predicted, state, expected_miss_fraction):
    """Pick the one-launch or the split repair from a caller's miss estimate.

    The one-launch repair is taken when there are at least 16 query heads
    and at most two misses per head are expected (a fixed rule, so the
    choice is made on the host and a captured graph stays valid).  Either
    repair returns the exact output over the selected set, whatever the
    estimate.
    """
    if not 0 <= expected_miss_fraction <= 1:
        raise ValueError("expected_miss_fraction must be in [0, 1]")
    if (q.ndim == 2 and q.shape[0] >= 16 and selected.ndim == 2
            and selected.shape[1] * expected_miss_fraction <= 2):
        return repair_saved_light(q, k, v, selected, predicted, state)
    return gqa.repair_saved(q, k, v, selected, predicted, state)
