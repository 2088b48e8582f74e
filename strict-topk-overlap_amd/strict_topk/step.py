"""The full speculative decode step as one call (an extension of the drop-in API).

The reference composes the step in its harness
(``benchmarks/run_benchmark.py:99-118``, ``overlap_run``):
``gqa.select_blocks`` on one stream while ``gqa.partials`` speculates on the
already-known predicted blocks on another, then the repair on the joined
stream (``gqa_light.repair_saved_auto`` / ``gqa.repair_saved``, or
``gqa.repair_union``).  ``speculative_step`` computes the same three results
(selected IDs, prediction state, repaired output) on the current stream.
Where the library's one-launch step covers the shape (bf16/fp16, blocks of
32 tokens, D of 64 or 128, at most four query heads per KV head), that is
one grid: workgroups that score blocks, workgroups that compute the
predicted blocks' states, and one workgroup per query head that waits for
its scores, runs the exact top-K while the states still stream, then waits
for its states and repairs.  Other fused shapes take two launches (the
scoring and state workgroups, then the per-head tails).  Shapes the fused
kernels do not cover (fp32, other head dims, long rows) run the same steps
through the individual entry points, still on the GPU.

``speculative_signed_step`` does the same for the signed strategy:
``select_blocks`` || ``kernels.speculate(mode, keep_mass=True)``, then
``signed_fused.repair_signed_fused`` (strict_topk/signed_fused.py:148-193),
again in two launches (the same front, then one workgroup per query head for
the top-K, the hybrid grouping, the signed corrections, the guarded merge
and the strict fallback).
"""
from dataclasses import dataclass

import torch

from . import _lib, gqa, gqa_light
from .kernels import PartialState, _allocate_state, _args
from .selector import select_ids


@dataclass
class StepResult:
    selected: torch.Tensor     # int32 [Hq, topk], ascending block IDs
    state: PartialState        # prediction state over the predicted blocks
    output: torch.Tensor       # float32 [Hq, D]


def _check_bounds(q, k, lo, hi):
    """lo / hi [Hkv, N, D], float32 or (lossless) the element type of Q/K/V."""
    if lo.ndim != 3 or hi.shape != lo.shape or lo.shape[0] != k.shape[0] or \
            lo.shape[1:] != (k.shape[1], k.shape[3]):
        raise ValueError("expected LO/HI[Hkv,N,D] matching K")
    if hi.dtype != lo.dtype or lo.dtype not in (torch.float32, q.dtype):
        raise ValueError("lo and hi must be FP32 or the element type of Q/K/V")
    if any(x.device != q.device or not x.is_contiguous() for x in (lo, hi)):
        raise ValueError("Q/LO/HI must be contiguous and on the same CUDA device")


def select_blocks(q, lo, hi, topk):
    """``gqa.select_blocks`` that also takes bounds stored in the queries' own
    16-bit type (the same IDs, from half the bound bytes)."""
    if q.ndim != 2 or lo.ndim != 3 or hi.shape != lo.shape:
        raise ValueError("expected Q[Hq,D] and LO/HI[Hkv,N,D]")
    hkv, n, d = lo.shape
    hq, qd = q.shape
    if min(hq, hkv, n, d) <= 0 or qd != d or hq % hkv != 0:
        raise ValueError("expected nonempty shapes, matching head dimensions and Hq divisible by Hkv")
    if hi.dtype != lo.dtype or lo.dtype not in (torch.float32, q.dtype):
        raise ValueError("lo and hi must be FP32 or the element type of Q/K/V")
    if not q.is_cuda or any(x.device != q.device or not x.is_contiguous() for x in (q, lo, hi)):
        raise ValueError("Q/LO/HI must be contiguous and on the same CUDA device")
    return select_ids(q, lo, hi, topk, hq, hkv, n, d)


def serial_step(q, k, v, lo, hi, topk):
    """The same-work serial path: select_blocks, then the exact attention over
    the selected blocks (``gqa.exact``); returns (selected, output)."""
    sel = select_blocks(q, lo, hi, topk)
    return sel, gqa.exact(q, k, v, sel)


def supported(q, k, lo, topk, predicted, v=None, hi=None):
    """True when the fused kernels serve this shape: bf16/fp16, int32
    predictions, D in {64, 128, 256}, B a multiple of 16, N <= 8192, K and SP
    <= 256, SP * D <= 32768, and 16-byte aligned Q/K/V/LO/HI (V and HI are
    checked when given)."""
    hkv, n, b, d = k.shape
    if any(t.data_ptr() % 16 for t in (q, k, lo, v, hi) if t is not None):
        return False
    return bool(_lib.lib().stk_step_supported(_lib.dtype_code(q), q.shape[0], hkv, n, b, d,
                                              int(topk), predicted.shape[1],
                                              _lib.id_code(predicted)))


def speculative_step(q, k, v, lo, hi, predicted, topk, union=False):
    """select(q, lo, hi, topk) || partials(q, k, v, predicted), then repair.

    Validation follows ``gqa.select_blocks`` and ``gqa.partials`` (same
    ValueError messages).  ``union`` selects ``repair_union`` semantics.
    """
    gqa._shape(q, k, v, predicted)
    _check_bounds(q, k, lo, hi)
    topk = int(topk)
    hq, d = q.shape
    hkv, n, b, _ = k.shape
    if topk < 1 or topk > n:
        raise RuntimeError("selected index k out of range")
    sp = predicted.shape[1]
    if supported(q, k, lo, topk, predicted, v, hi):
        dev = q.device
        _lib.prepare(dev)
        selected = torch.empty((hq, topk), device=dev, dtype=torch.int32)
        state = _allocate_state(hq, sp, d, dev)
        out = torch.empty((hq, d), device=dev, dtype=torch.float32)
        ws = _lib.workspace(_lib.size("stk_step_workspace_bytes", hq, hkv, n, d, topk), dev)
        _lib.call("stk_speculative_step", *_args(q, k, v), _lib.ptr(lo), _lib.ptr(hi),
                  _lib.bounds_code(lo, q), topk,
                  _lib.ptr(predicted), _lib.id_code(predicted), sp, 1 if union else 0,
                  _lib.ptr(selected), _lib.ptr(state.m), _lib.ptr(state.l), _lib.ptr(state.u),
                  _lib.ptr(out), _lib.ptr(ws), ws.numel(), _lib.stream(dev))
        return StepResult(selected, state, out)
    selected = select_blocks(q, lo, hi, topk)
    state = gqa.partials(q, k, v, predicted)
    if union:
        out = gqa.repair_union(q, k, v, selected, predicted, state)
    else:
        out = gqa_light.repair_saved_light(q, k, v, selected, predicted, state)
    return StepResult(selected, state, out)


def check_into(into, hq, sp, topk, d, device):
    """ValueError unless ``into`` (a StepResult) holds this step's outputs:
    contiguous int32 selected [Hq, topk], float32 state m, l [Hq, SP] and
    u [Hq, SP, D] and float32 output [Hq, D], all on ``device``, u 16-byte
    aligned.  The kernels write every element of these shapes, so a
    mismatched ``into`` would be written past its ends."""
    def ok(t, shape, dtype):
        return (isinstance(t, torch.Tensor) and tuple(t.shape) == shape and t.dtype == dtype
                and t.device == device and t.is_contiguous())
    st = getattr(into, "state", None)
    if not (ok(getattr(into, "selected", None), (hq, topk), torch.int32) and st is not None
            and ok(getattr(st, "m", None), (hq, sp), torch.float32)
            and ok(getattr(st, "l", None), (hq, sp), torch.float32)
            and ok(getattr(st, "u", None), (hq, sp, d), torch.float32)
            and ok(getattr(into, "output", None), (hq, d), torch.float32)):
        raise ValueError("into must hold contiguous int32 selected[Hq,topk], float32 "
                         "state m,l[Hq,SP], u[Hq,SP,D] and output[Hq,D] on Q's device")
    if st.u.data_ptr() % 16:
        raise ValueError("into.state.u must be 16-byte aligned")


def speculative_step_noalloc(q, k, v, lo, hi, predicted, topk, union=False, into=None):
    """``speculative_step`` for callers that cannot allocate device memory
    (graph capture, serving loops): the library keeps the step's scratch in a
    fixed per-GPU array, so the call allocates nothing.  ``into``: an
    optional ``StepResult`` whose tensors receive the results (else they are
    allocated here, before the call).  Only shapes the fused kernels support
    with Hq * N <= 524288 are accepted (ValueError otherwise).  Calls that
    overlap in time on one GPU share the array and must not run
    concurrently."""
    gqa._shape(q, k, v, predicted)
    _check_bounds(q, k, lo, hi)
    topk = int(topk)
    hq, d = q.shape
    hkv, n, b, _ = k.shape
    sp = predicted.shape[1]
    if not supported(q, k, lo, topk, predicted, v, hi):
        raise ValueError("shape not supported by the fused step")
    dev = q.device
    if into is None:
        into = StepResult(torch.empty((hq, topk), device=dev, dtype=torch.int32),
                          _allocate_state(hq, sp, d, dev),
                          torch.empty((hq, d), device=dev, dtype=torch.float32))
    else:
        check_into(into, hq, sp, topk, d, dev)
    _lib.prepare(dev)
    _lib.call("stk_speculative_step_noalloc", *_args(q, k, v), _lib.ptr(lo), _lib.ptr(hi),
              _lib.bounds_code(lo, q), topk,
              _lib.ptr(predicted), _lib.id_code(predicted), sp, 1 if union else 0,
              _lib.ptr(into.selected), _lib.ptr(into.state.m), _lib.ptr(into.state.l),
              _lib.ptr(into.state.u), _lib.ptr(into.output), _lib.stream(dev))
    return into


@dataclass
class SignedStepResult:
    selected: torch.Tensor     # int32 [Hq, topk], ascending block IDs
    state: PartialState        # prediction state over the predicted blocks
    result: "SignedRepairResult"   # output and guard results of repair_signed_fused


def speculative_signed_step(q, k, v, lo, hi, predicted, topk, mode="hybrid", mass_threshold=0.1,
                            min_remaining=1.e-3, cancellation_tol=1.e-5, max_extra_mass=0.):
    """select(q, lo, hi, topk) || speculate(q, k, v, predicted, mode,
    mass_threshold, keep_mass=True), then repair_signed_fused.

    ``mode`` is "hybrid" or "saved".  The result's fields are those of
    ``signed_fused.repair_signed_fused`` on the same selection and
    prediction.  Shapes the fused kernels do not cover (and the "compact"
    mode) run the same three steps through the individual entry points.
    """
    from . import kernels, signed_fused
    from .signed_repair import SignedRepairResult
    if mode not in ("saved", "hybrid", "compact"):
        raise ValueError(mode)
    if not 0 <= mass_threshold <= 1:
        raise ValueError("mass_threshold must be in [0,1]")
    if not 0 <= max_extra_mass <= 1:
        raise ValueError("max_extra_mass must be in [0,1]")
    gqa._shape(q, k, v, predicted)
    _check_bounds(q, k, lo, hi)
    topk = int(topk)
    hq, d = q.shape
    hkv, n, b, _ = k.shape
    if topk < 1 or topk > n:
        raise RuntimeError("selected index k out of range")
    sp = predicted.shape[1]
    if mode != "compact" and supported(q, k, lo, topk, predicted, v, hi):
        dev = q.device
        selected = torch.empty((hq, topk), device=dev, dtype=torch.int32)
        state = _allocate_state(hq, sp, d, dev)
        out = torch.empty((hq, d), device=dev, dtype=torch.float32)
        fallback = torch.empty((hq,), device=dev, dtype=torch.bool)
        remaining = torch.empty((hq,), device=dev, dtype=torch.float32)
        approx = torch.empty_like(fallback) if max_extra_mass > 0 else None
        extra = torch.empty_like(remaining) if max_extra_mass > 0 else None
        positive = torch.empty((hq,), device=dev, dtype=torch.int32)
        total = torch.empty_like(positive)
        ws = _lib.workspace(_lib.size("stk_step_workspace_bytes", hq, hkv, n, d, topk), dev)
        _lib.call("stk_signed_step", *_args(q, k, v), _lib.ptr(lo), _lib.ptr(hi),
                  _lib.bounds_code(lo, q), topk,
                  _lib.ptr(predicted), _lib.id_code(predicted), sp, 1 if mode == "hybrid" else 0,
                  float(mass_threshold), float(min_remaining), float(cancellation_tol),
                  float(max_extra_mass), _lib.ptr(selected), _lib.ptr(state.m),
                  _lib.ptr(state.l), _lib.ptr(state.u), _lib.ptr(out), _lib.ptr(fallback),
                  _lib.ptr(remaining), _lib.ptr(approx), _lib.ptr(extra), _lib.ptr(positive),
                  _lib.ptr(total), _lib.ptr(ws), ws.numel(), _lib.stream(dev))
        res = SignedRepairResult(out, fallback, remaining, approx, extra, positive, total)
        return SignedStepResult(selected, state, res)
    selected = select_blocks(q, lo, hi, topk)
    pred = kernels.speculate(q, k, v, predicted, mode, mass_threshold, keep_mass=True)
    res = signed_fused.repair_signed_fused(q, k, v, selected, predicted, pred, min_remaining,
                                           cancellation_tol, max_extra_mass)
    return SignedStepResult(selected, pred.state, res)
