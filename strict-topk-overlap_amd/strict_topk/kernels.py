"""Forward-only FP32-state sparse attention on hand-written gfx950 kernels.

Drop-in for the reference ``strict_topk/kernels.py`` (dataclasses :13-39,
``block_partials`` :425-434, ``merge_partials`` :437-442,
``exact_attention`` :445-447, ``speculate`` :450-501, ``repair`` :504-550,
``touch_kv`` :553-560).  Inputs are contiguous Q[H,D], K/V[Hkv,N,B,D] and
unique valid block IDs[H,S] (int32 or int64).  As a superset of the
reference, H may be any multiple of Hkv (query head h reads KV head
h // (H // Hkv)); with H == Hkv this is the reference layout.  Every output
is FP32; IDs are not validated on the device (no synchronisation), but an
out-of-range ID never reads memory: it contributes an empty state.
"""
from dataclasses import dataclass

import torch

from . import _lib


@dataclass
class PartialState:
    m: torch.Tensor
    l: torch.Tensor
    u: torch.Tensor


@dataclass
class Prediction:
    state: PartialState
    mode: str
    high: torch.Tensor | None = None
    low: PartialState | None = None
    retained_ids: torch.Tensor | None = None
    overflow: torch.Tensor | None = None
    low_abs: torch.Tensor | None = None
    mass_m: torch.Tensor | None = None
    mass_l: torch.Tensor | None = None


@dataclass
class RepairResult:
    output: torch.Tensor
    fallback: torch.Tensor
    remaining: torch.Tensor
    approximate_heads: torch.Tensor | None = None
    extra_mass_bound: torch.Tensor | None = None


MODES = {"saved": 0, "hybrid": 1, "compact": 2}


def _shape(q, k, v, ids):
    assert q.is_cuda and k.is_cuda and v.is_cuda and ids.is_cuda
    assert q.ndim == 2 and k.ndim == 4 and v.shape == k.shape
    h, n, b, d = k.shape
    assert q.shape[1] == d and q.shape[0] % h == 0 and q.shape[0] > 0
    assert ids.ndim == 2 and ids.shape[0] == q.shape[0]
    assert ids.dtype in (torch.int32, torch.int64) and ids.shape[1] > 0
    assert all(x.is_contiguous() for x in (q, k, v, ids))
    assert q.dtype == k.dtype == v.dtype
    return q.shape[0], n, b, d, ids.shape[1]


def _args(q, k, v):
    """Common (q, k, v, dtype, hq, hkv, n, b, d) argument prefix."""
    hkv, n, b, d = k.shape
    return (_lib.ptr(q), _lib.ptr(k), _lib.ptr(v), _lib.dtype_code(q), q.shape[0], hkv, n, b, d)


def _check_mask(mask, device, name):
    """A mask is read by the kernels as one byte per entry on the device."""
    if not isinstance(mask, torch.Tensor) or not mask.is_cuda or mask.device != device:
        raise ValueError(f"{name} must be a tensor on the query's CUDA device")
    if mask.dtype not in (torch.bool, torch.uint8, torch.int8):
        raise ValueError(f"{name} must be a bool mask")


def _allocate_state(h, s, d, device):
    m = torch.empty((h, s), device=device, dtype=torch.float32)
    return PartialState(m, torch.empty_like(m), torch.empty((h, s, d), device=device, dtype=torch.float32))


def block_partials(q, k, v, ids, active=None):
    """Per listed block: m = max logit, l = sum exp(logit - m), u = sum exp(logit - m) V."""
    h, n, b, d, s = _shape(q, k, v, ids)
    state = _allocate_state(h, s, d, q.device)
    kind = 0
    if active is not None:
        _check_mask(active, q.device, "active")
        assert active.is_contiguous() and active.shape in ((h,), (h, s))
        kind = 1 if active.ndim == 1 else 2
        active = active.to(torch.bool) if active.dtype != torch.bool else active
    _lib.call("stk_block_partials", *_args(q, k, v), _lib.ptr(ids), _lib.id_code(ids), s,
              _lib.ptr(active), kind, _lib.ptr(state.m), _lib.ptr(state.l), _lib.ptr(state.u),
              _lib.stream(q.device))
    return state


def merge_partials(state, include=None):
    h, s, d = state.u.shape
    if include is not None:
        _check_mask(include, state.u.device, "include")
        if include.shape != (h, s) or not include.is_contiguous():
            raise ValueError("include must be a contiguous [H, S] mask")
        include = include.to(torch.bool) if include.dtype != torch.bool else include
    out = torch.empty((h, d), device=state.u.device, dtype=torch.float32)
    _lib.call("stk_merge_partials", _lib.ptr(state.m), _lib.ptr(state.l), _lib.ptr(state.u),
              _lib.ptr(include), h, s, d, _lib.ptr(out), _lib.stream(state.u.device))
    return out


def exact_attention(q, k, v, selected):
    """Serial baseline: attention over the selected blocks through per-block states."""
    h, n, b, d, s = _shape(q, k, v, selected)
    out = torch.empty((h, d), device=q.device, dtype=torch.float32)
    ws = _lib.workspace(_lib.size("stk_exact_workspace_bytes", h, s, d), q.device)
    _lib.call("stk_exact_attention", *_args(q, k, v), _lib.ptr(selected), _lib.id_code(selected),
              s, _lib.ptr(out), _lib.ptr(ws), ws.numel(), _lib.stream(q.device))
    return out


def compact_capacity(s, mass_threshold):
    """Retained-state capacity (reference kernels.py:485)."""
    return s if mass_threshold <= 1 / s else min(s, int(1 / mass_threshold) + 1)


def speculate(q, k, v, predicted, mode='saved', mass_threshold=0.1, *, keep_mass=False):
    """Prediction states for the predicted blocks, computed with this step's query.

    The mass threshold is relative to the mass of the predicted set itself.
    saved: per-block states of the predicted blocks.  hybrid: additionally a
    per-block high/low split at ``mass_threshold`` of the predicted-set mass
    and one low aggregate (m, l, u) with its absolute envelope.  compact: a
    K-only mass pass, capacity-bounded retained states (IDs in rank order,
    padded with -1, overflow flag) and a low aggregate accumulated per token
    in the low frame.  keep_mass: also return every predicted block's FP32
    (m, l), in the order of the predicted row.
    """
    if mode not in ('saved', 'hybrid', 'compact'):
        raise ValueError(mode)
    if not 0 <= mass_threshold <= 1:
        raise ValueError('mass_threshold must be in [0,1]')
    h, n, b, d, s = _shape(q, k, v, predicted)
    dev = q.device
    if mode == 'compact':
        c = compact_capacity(s, mass_threshold)
        pm = torch.empty((h, s), device=dev, dtype=torch.float32)
        pl = torch.empty_like(pm)
        state = _allocate_state(h, c, d, dev)
        low = _allocate_state(h, 1, d, dev)
        low_abs = torch.empty((h, d), device=dev, dtype=torch.float32)
        high = torch.empty((h, s), device=dev, dtype=torch.bool)
        retained_ids = torch.empty((h, c), device=dev, dtype=predicted.dtype)
        overflow = torch.empty((h,), device=dev, dtype=torch.bool)
        _lib.call("stk_speculate", *_args(q, k, v), _lib.ptr(predicted), _lib.id_code(predicted),
                  s, 2, float(mass_threshold), c, _lib.ptr(state.m), _lib.ptr(state.l),
                  _lib.ptr(state.u), _lib.ptr(high), _lib.ptr(low.m), _lib.ptr(low.l),
                  _lib.ptr(low.u), _lib.ptr(low_abs), _lib.ptr(retained_ids), _lib.ptr(overflow),
                  _lib.ptr(pm), _lib.ptr(pl), _lib.stream(dev))
        mass_m, mass_l = (pm, pl) if keep_mass else (None, None)
        return Prediction(state, 'compact', high, low, retained_ids, overflow, low_abs, mass_m, mass_l)
    state = _allocate_state(h, s, d, dev)
    high = low = low_abs = None
    if mode == 'hybrid':
        high = torch.empty((h, s), device=dev, dtype=torch.bool)
        low = _allocate_state(h, 1, d, dev)
        low_abs = torch.empty((h, d), device=dev, dtype=torch.float32)
    _lib.call("stk_speculate", *_args(q, k, v), _lib.ptr(predicted), _lib.id_code(predicted), s,
              MODES[mode], float(mass_threshold), s, _lib.ptr(state.m), _lib.ptr(state.l),
              _lib.ptr(state.u), _lib.ptr(high), _lib.ptr(low.m if low else None),
              _lib.ptr(low.l if low else None), _lib.ptr(low.u if low else None),
              _lib.ptr(low_abs), None, None, None, None, _lib.stream(dev))
    mass_m, mass_l = (state.m, state.l) if keep_mass else (None, None)
    if mode == 'saved':
        return Prediction(state, mode, mass_m=mass_m, mass_l=mass_l)
    return Prediction(state, mode, high, low, low_abs=low_abs, mass_m=mass_m, mass_l=mass_l)


def prediction_args(prediction, q):
    """(mode, sc, pm, pl, pu, high, low_m, low_l, low_u, low_abs, retained_ids)."""
    p = prediction.state
    hybrid = prediction.mode in ('hybrid', 'compact')
    low = prediction.low if hybrid else None
    return (MODES[prediction.mode], p.m.shape[1], _lib.ptr(p.m), _lib.ptr(p.l), _lib.ptr(p.u),
            _lib.ptr(prediction.high if hybrid else None), _lib.ptr(low.m if low else None),
            _lib.ptr(low.l if low else None), _lib.ptr(low.u if low else None),
            _lib.ptr(prediction.low_abs if hybrid else None),
            _lib.ptr(prediction.retained_ids if prediction.mode == 'compact' else None))


def repair(q, k, v, selected, predicted, prediction, min_remaining=1.e-3, cancellation_tol=1.e-5):
    """Bring a prediction back to the exact output over the selected set.

    remaining = (low denominator after removing wrong blocks) / (low
    denominator before).  A low group none of whose blocks is selected is
    dropped whole, with no subtraction.  The cancellation guard compares
    every coordinate of the remaining low numerator with the low group's
    absolute sum times cancellation_tol; it is a rounding heuristic, not an
    error bound.  Heads that fail a guard are recomputed over the selected
    blocks directly.
    """
    h, n, b, d, sa = _shape(q, k, v, selected)
    sp = predicted.shape[1]
    pa = prediction_args(prediction, q)
    mode, sc = pa[0], pa[1]
    out = torch.empty((h, d), device=q.device, dtype=torch.float32)
    fallback = torch.empty((h,), device=q.device, dtype=torch.bool)
    remaining = torch.empty((h,), device=q.device, dtype=torch.float32)
    ws = _lib.workspace(_lib.size("stk_repair_workspace_bytes", h, sa, sp, sc, d, mode), q.device)
    _lib.call("stk_repair", *_args(q, k, v), _lib.ptr(selected), _lib.id_code(selected), sa,
              _lib.ptr(predicted), _lib.id_code(predicted), sp, *pa, float(min_remaining),
              float(cancellation_tol), _lib.ptr(out), _lib.ptr(fallback), _lib.ptr(remaining),
              _lib.ptr(ws), ws.numel(), _lib.stream(q.device))
    return RepairResult(out, fallback, remaining)


def touch_kv(k, v, predicted):
    """Stream the predicted blocks' K/V once, returning per-tile checksums (a
    prefetch baseline; nothing guarantees the data stay cached)."""
    h, n, b, d = k.shape
    s = predicted.shape[1]
    nt = (b * d + 1023) // 1024
    scratch = torch.empty((h, s, nt), device=k.device, dtype=torch.float32)
    _lib.call("stk_touch_kv", _lib.ptr(k), _lib.ptr(v), _lib.dtype_code(k), h, n, b, d,
              _lib.ptr(predicted), _lib.id_code(predicted), s, _lib.ptr(scratch),
              _lib.stream(k.device))
    return scratch
