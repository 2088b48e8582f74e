"""Block selection by the query-sign min/max bound of every block's keys.

Drop-in for the reference ``strict_topk/selector.py`` (same names, argument
meaning and ValueError messages, :23-43).  Scores are evaluated in FP64 on the
GPU (exact products, fixed summation order) and returned as FP32; selection
is exact top-K with ties toward the lower block index, emitted in ascending
block order -- one valid instance of the reference's
``torch.topk(sorted=False)`` result, whose order is unspecified.
"""
import torch

from . import _lib


def _check(q, lo, hi):
    if lo.ndim != 3 or hi.shape != lo.shape:
        raise ValueError("lo and hi must have the same [heads, blocks, dim] shape")
    h, n, d = lo.shape
    if q.shape != (h, d) or min(h, n, d) <= 0:
        raise ValueError("q must have shape [heads, dim], with nonempty input dimensions")
    if lo.dtype != torch.float32 or hi.dtype != torch.float32:
        raise ValueError("lo and hi must be FP32")
    if not q.is_cuda or any(x.device != q.device or not x.is_contiguous() for x in (q, lo, hi)):
        raise ValueError("q, lo and hi must be contiguous on the same CUDA device")
    return h, n, d


def block_scores(q, lo, hi):
    """scores[h, n] = sum_d q[h,d] * (hi if q[h,d] >= 0 else lo)[h,n,d], as FP32."""
    h, n, d = _check(q, lo, hi)
    scores = torch.empty((h, n), device=q.device, dtype=torch.float32)
    _lib.call("stk_block_scores", _lib.ptr(q), _lib.dtype_code(q), _lib.ptr(lo), _lib.ptr(hi),
              0, h, h, n, d, _lib.ptr(scores), _lib.stream(q.device))
    return scores


def select_blocks(q, lo, hi, topk):
    """int32 [H, topk]: the blocks with the highest bound scores, per head."""
    h, n, d = _check(q, lo, hi)
    return select_ids(q, lo, hi, topk, h, h, n, d)


def select_ids(q, lo, hi, topk, hq, hkv, n, d):
    topk = int(topk)
    if topk < 0 or topk > n:
        raise RuntimeError("selected index k out of range")
    ids = torch.empty((hq, topk), device=q.device, dtype=torch.int32)
    if topk == 0:
        return ids
    nbytes = _lib.size("stk_select_workspace_bytes", hq, hkv, n, d, topk)
    ws = _lib.workspace(nbytes, q.device)
    _lib.call("stk_select_blocks", _lib.ptr(q), _lib.dtype_code(q), _lib.ptr(lo), _lib.ptr(hi),
              _lib.bounds_code(lo, q), hq, hkv, n, d, topk, None, _lib.ptr(ids), _lib.ptr(ws),
              ws.numel(), _lib.stream(q.device))
    return ids
