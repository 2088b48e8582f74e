"""Shared-selection indexer scorer (an extension of the drop-in API).

The reference evaluates the QSA indexer formula in its benchmark
(``benchmarks/selector_window.py:126-142``): ``score[n] = sum_h
relu(iq_h . ik_n) / sqrt(D)`` over indexer queries ``iq[H, D]`` and one
indexer key per block ``ik[N, D]``, then ``scores.topk(topk, sorted=False)``
shared by every query head (:76-84), the selection that
``gqa_hierarchical.repair_saved_shared`` assumes.  Scores are evaluated in
FP64 in a fixed order; the IDs come back in ascending block order with ties
toward the lower index, like ``gqa.select_blocks``.
"""
import torch

from . import _lib


def _check(iq, ik):
    if not (iq.is_cuda and ik.is_cuda) or iq.ndim != 2 or ik.ndim != 2 or \
            iq.shape[1] != ik.shape[1]:
        raise ValueError("expected CUDA IQ[H,D] and IK[N,D]")
    if iq.dtype != ik.dtype or not iq.is_contiguous() or not ik.is_contiguous():
        raise ValueError("IQ and IK must be contiguous and of one dtype")


def scores(iq, ik):
    """float32[N] indexer scores."""
    _check(iq, ik)
    h, d = iq.shape
    n = ik.shape[0]
    out = torch.empty((n,), device=ik.device, dtype=torch.float32)
    ws = _lib.workspace(_lib.size("stk_indexer_workspace_bytes", n), ik.device)
    _lib.call("stk_indexer_scores", _lib.ptr(iq), _lib.ptr(ik), _lib.dtype_code(ik), h, n, d,
              _lib.ptr(out), _lib.ptr(ws), ws.numel(), _lib.stream(ik.device))
    return out


def select_shared(iq, ik, topk, rows):
    """int32[rows, topk]: the same topk highest-scoring blocks in every row."""
    _check(iq, ik)
    h, d = iq.shape
    n = ik.shape[0]
    topk, rows = int(topk), int(rows)
    if topk < 1 or topk > n:
        raise RuntimeError("selected index k out of range")
    ids = torch.empty((rows, topk), device=ik.device, dtype=torch.int32)
    ws = _lib.workspace(_lib.size("stk_indexer_workspace_bytes", n), ik.device)
    _lib.call("stk_indexer_select", _lib.ptr(iq), _lib.ptr(ik), _lib.dtype_code(ik), h, n, d,
              topk, rows, None, _lib.ptr(ids), _lib.ptr(ws), ws.numel(), _lib.stream(ik.device))
    return ids
