"""Signed repair of saved, hybrid or compact predictions, corrections in parallel.

Drop-in for the reference ``strict_topk/signed_repair.py``
(``SignedRepairResult`` :12-15, ``repair_signed`` :175-232): schedule a
per-head job queue (misses first, then wrong low blocks), compute signed
block-local states in parallel, merge with the guards in the low frame, and
recompute the selected set on flagged heads.
"""
from dataclasses import dataclass

import torch

from . import _lib
from .kernels import RepairResult, _args, _shape, prediction_args


@dataclass
class SignedRepairResult(RepairResult):
    positive_jobs: torch.Tensor | None = None
    total_jobs: torch.Tensor | None = None


def _signed(q, k, v, selected, predicted, prediction, min_remaining, cancellation_tol,
            max_extra_mass, fused, msg):
    h, n, b, d, sa = _shape(q, k, v, selected)
    _, _, _, _, sp = _shape(q, k, v, predicted)
    hybrid = prediction.mode in ("hybrid", "compact")
    if not 0 <= max_extra_mass <= 1:
        raise ValueError(msg)
    if hybrid and max_extra_mass > 0 and (prediction.mass_m is None or prediction.mass_l is None):
        raise ValueError("positive max_extra_mass requires speculate(..., keep_mass=True)")
    pa = prediction_args(prediction, q)
    mode, sc = pa[0], pa[1]
    capacity = sa + sp if hybrid else sa
    dev = q.device
    id_dtype = torch.promote_types(selected.dtype, predicted.dtype)
    queue = torch.empty((h, capacity), device=dev, dtype=id_dtype)
    positive = torch.empty((h,), device=dev, dtype=torch.int32)
    total = torch.empty_like(positive)
    out = torch.empty((h, d), device=dev, dtype=torch.float32)
    fallback = torch.empty((h,), device=dev, dtype=torch.bool)
    remaining = torch.empty((h,), device=dev, dtype=torch.float32)
    approximate = torch.empty_like(fallback) if max_extra_mass > 0 else None
    extra = torch.empty_like(remaining) if max_extra_mass > 0 else None
    ws = _lib.workspace(_lib.size("stk_signed_workspace_bytes", h, sa, sp, sc, d, mode), dev)
    _lib.call("stk_repair_signed", *_args(q, k, v), _lib.ptr(selected), _lib.id_code(selected), sa,
              _lib.ptr(predicted), _lib.id_code(predicted), sp, *pa, _lib.ptr(prediction.mass_m),
              _lib.ptr(prediction.mass_l), float(min_remaining), float(cancellation_tol),
              float(max_extra_mass), 1 if fused else 0, _lib.ptr(queue), _lib.id_code(queue),
              _lib.ptr(positive), _lib.ptr(total), _lib.ptr(out), _lib.ptr(fallback),
              _lib.ptr(remaining), _lib.ptr(approximate), _lib.ptr(extra), _lib.ptr(ws),
              ws.numel(), _lib.stream(dev))
    return SignedRepairResult(out, fallback, remaining, approximate, extra, positive, total)


def repair_signed(q, k, v, selected, predicted, prediction, min_remaining=1.e-3,
                  cancellation_tol=1.e-5, max_extra_mass=0.):
    """Signed repair in four launches (schedule, corrections, merge, fallback).

    Each head's job list holds its missed selected blocks, then its wrong
    low blocks; one kernel computes every job's state.  The merge removes
    the subtracted states in the low group's exponent frame under the
    guards, and heads that fail a guard are recomputed over the selected set
    alone.  positive_jobs / total_jobs count the list as scheduled, before
    any fallback.
    """
    return _signed(q, k, v, selected, predicted, prediction, min_remaining, cancellation_tol,
                   max_extra_mass, False, "max_extra_mass must be in [0, 1]")
