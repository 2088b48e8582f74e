"""The full speculative decode step as one call (an extension of the drop-in API).

The reference composes the step in its harness
(``benchmarks/run_benchmark.py:99-118``, ``overlap_run``):
``gqa.select_blocks`` on one stream while ``gqa.partials`` speculates on the
already-known predicted blocks on another, then the repair on the joined
stream (``gqa_light.repair_saved_auto`` / ``gqa.repair_saved``, or
``gqa.repair_union``).  ``speculative_step`` computes the same three results
(selected IDs, prediction state, repaired output) with two launches on the
current stream: one grid that scores blocks and computes the predicted
blocks' states side by side, then one workgroup per query head doing the
exact top-K and the repair.  Shapes the fused kernels do not cover (fp32,
other head dims, long rows) run the same steps through the individual entry
points, still on the GPU.
"""
from dataclasses import dataclass

import torch

from . import _lib, gqa, gqa_light
from .kernels import PartialState, _allocate_state, _args


@dataclass
class StepResult:
    selected: torch.Tensor     # int32 [Hq, topk], ascending block IDs
    state: PartialState        # prediction state over the predicted blocks
    output: torch.Tensor       # float32 [Hq, D]


def supported(q, k, lo, topk, predicted):
    hkv, n, b, d = k.shape
    return bool(_lib.lib().stk_step_supported(_lib.dtype_code(q), q.shape[0], hkv, n, b, d,
                                              int(topk), predicted.shape[1],
                                              _lib.id_code(predicted)))


def speculative_step(q, k, v, lo, hi, predicted, topk, union=False):
    """select(q, lo, hi, topk) || partials(q, k, v, predicted), then repair.

    Validation follows ``gqa.select_blocks`` and ``gqa.partials`` (same
    ValueError messages).  ``union`` selects ``repair_union`` semantics.
    """
    gqa._shape(q, k, v, predicted)
    if lo.ndim != 3 or hi.shape != lo.shape or lo.shape[0] != k.shape[0] or \
            lo.shape[1:] != (k.shape[1], k.shape[3]):
        raise ValueError("expected LO/HI[Hkv,N,D] matching K")
    if lo.dtype != torch.float32 or hi.dtype != torch.float32:
        raise ValueError("lo and hi must be FP32")
    if any(x.device != q.device or not x.is_contiguous() for x in (lo, hi)):
        raise ValueError("Q/LO/HI must be contiguous and on the same CUDA device")
    topk = int(topk)
    hq, d = q.shape
    hkv, n, b, _ = k.shape
    if topk < 1 or topk > n:
        raise RuntimeError("selected index k out of range")
    sp = predicted.shape[1]
    if supported(q, k, lo, topk, predicted):
        dev = q.device
        selected = torch.empty((hq, topk), device=dev, dtype=torch.int32)
        state = _allocate_state(hq, sp, d, dev)
        out = torch.empty((hq, d), device=dev, dtype=torch.float32)
        ws = _lib.workspace(_lib.size("stk_step_workspace_bytes", hq, hkv, n, d, topk), dev)
        _lib.call("stk_speculative_step", *_args(q, k, v), _lib.ptr(lo), _lib.ptr(hi), topk,
                  _lib.ptr(predicted), _lib.id_code(predicted), sp, 1 if union else 0,
                  _lib.ptr(selected), _lib.ptr(state.m), _lib.ptr(state.l), _lib.ptr(state.u),
                  _lib.ptr(out), _lib.ptr(ws), ws.numel(), _lib.stream(dev))
        return StepResult(selected, state, out)
    selected = gqa.select_blocks(q, lo, hi, topk)
    state = gqa.partials(q, k, v, predicted)
    if union:
        out = gqa.repair_union(q, k, v, selected, predicted, state)
    else:
        out = gqa_light.repair_saved_light(q, k, v, selected, predicted, state)
    return StepResult(selected, state, out)
