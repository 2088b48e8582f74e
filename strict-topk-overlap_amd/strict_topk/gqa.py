"""Block-sparse attention over grouped-query KV (no head expansion).

Layouts: queries [Hq, D]; keys and values [Hkv, N, B, D], query head h
reading KV head h // (Hq // Hkv).  ID rows are nonempty, hold distinct
in-range block numbers and have one row per query head; every tensor is
contiguous with finite values.

Drop-in for the reference ``strict_topk/gqa.py`` (``partials`` :128-137,
``exact`` :140-142, ``select_blocks`` :145-161, ``repair_saved`` :186-188,
``repair_union`` :191-193) with the same ValueError messages.
"""
import torch

from . import _lib
from .kernels import _allocate_state, _args
from .selector import select_ids


def _validate_ids(q, ids):
    if (ids.ndim != 2 or ids.shape[0] != q.shape[0] or ids.shape[1] == 0
            or ids.dtype not in (torch.int32, torch.int64)):
        raise ValueError("ids must be a nonempty int32/int64 matrix with one row per query head")
    if ids.device != q.device or not ids.is_contiguous():
        raise ValueError("ids must be contiguous and on the query's CUDA device")


def _shape(q, k, v, ids):
    if q.ndim != 2 or k.ndim != 4 or k.shape != v.shape:
        raise ValueError("expected Q[Hq,D] and K/V[Hkv,N,B,D]")
    hkv, n, b, d = k.shape
    hq, qd = q.shape
    if min(hq, hkv, n, b, d) <= 0 or qd != d or hq % hkv != 0:
        raise ValueError("expected nonempty shapes, matching head dimensions and Hq divisible by Hkv")
    if not q.is_cuda or any(x.device != q.device or not x.is_contiguous() for x in (q, k, v)):
        raise ValueError("Q/K/V must be contiguous and on the same CUDA device")
    if not (q.dtype == k.dtype == v.dtype):
        raise ValueError("Q/K/V must share one element dtype")
    _validate_ids(q, ids)
    return hq, n, b, d, hq // hkv, ids.shape[1]


def partials(q, k, v, ids):
    """FP32 softmax state (m, l, u) of every (query head, listed block)."""
    hq, n, b, d, group, sa = _shape(q, k, v, ids)
    state = _allocate_state(hq, sa, d, q.device)
    _lib.call("stk_block_partials", *_args(q, k, v), _lib.ptr(ids), _lib.id_code(ids), sa, None, 0,
              _lib.ptr(state.m), _lib.ptr(state.l), _lib.ptr(state.u), _lib.stream(q.device))
    return state


def exact(q, k, v, selected):
    """Attention over the selected blocks: per-block states, then one LSE merge."""
    hq, n, b, d, group, sa = _shape(q, k, v, selected)
    out = torch.empty((hq, d), device=q.device, dtype=torch.float32)
    ws = _lib.workspace(_lib.size("stk_exact_workspace_bytes", hq, sa, d), q.device)
    _lib.call("stk_exact_attention", *_args(q, k, v), _lib.ptr(selected), _lib.id_code(selected),
              sa, _lib.ptr(out), _lib.ptr(ws), ws.numel(), _lib.stream(q.device))
    return out


def select_blocks(q, lo, hi, topk):
    """Top-k blocks per query head by the bound score on FP32 LO/HI[Hkv,N,D]."""
    if q.ndim != 2 or lo.ndim != 3 or hi.shape != lo.shape:
        raise ValueError("expected Q[Hq,D] and LO/HI[Hkv,N,D]")
    hkv, n, d = lo.shape
    hq, qd = q.shape
    if min(hq, hkv, n, d) <= 0 or qd != d or hq % hkv != 0:
        raise ValueError("expected nonempty shapes, matching head dimensions and Hq divisible by Hkv")
    if lo.dtype != torch.float32 or hi.dtype != torch.float32:
        raise ValueError("lo and hi must be FP32")
    if not q.is_cuda or any(x.device != q.device or not x.is_contiguous() for x in (q, lo, hi)):
        raise ValueError("Q/LO/HI must be contiguous and on the same CUDA device")
    return select_ids(q, lo, hi, topk, hq, hkv, n, d)


def _repair(q, k, v, selected, predicted, state, union):
    hq, n, b, d, group, sa = _shape(q, k, v, selected)
    _validate_ids(q, predicted)
    sp = predicted.shape[1]
    if state.m.shape != (hq, sp) or state.l.shape != (hq, sp) or state.u.shape != (hq, sp, d):
        raise ValueError("state must contain a softmax partial for every predicted block")
    out = torch.empty((hq, d), device=q.device, dtype=torch.float32)
    ws = _lib.workspace(_lib.size("stk_gqa_repair_workspace_bytes", hq, sa, d), q.device)
    _lib.call("stk_gqa_repair", *_args(q, k, v), _lib.ptr(selected), _lib.id_code(selected), sa,
              _lib.ptr(predicted), _lib.id_code(predicted), sp, _lib.ptr(state.m),
              _lib.ptr(state.l), _lib.ptr(state.u), 1 if union else 0, _lib.ptr(out),
              _lib.ptr(ws), ws.numel(), _lib.stream(q.device))
    return out


def repair_saved(q, k, v, selected, predicted, state):
    """Strict output: predicted states of selected blocks, new states for the rest."""
    return _repair(q, k, v, selected, predicted, state, union=False)


def repair_union(q, k, v, selected, predicted, state):
    """Output over selected and predicted blocks together, each block counted once."""
    return _repair(q, k, v, selected, predicted, state, union=True)
