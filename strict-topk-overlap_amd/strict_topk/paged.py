"""Paged, ragged KV and batched decode steps (an extension of the drop-in API).

Wire format (one pool shared by a batch of requests of different lengths):

  k_pages, v_pages  [P, B, D]      one page = one KV head's block of B tokens
  lo_pages, hi_pages [P, D]        per-dim key min / max of the page, FP32 or
                                   (exact, half the bytes) the pages' dtype
  block_table       [R, Hkv, NB]   int32 page of logical block j of (request r,
                                   KV head h), valid for j < nblocks[r]
  nblocks           [R] int32      blocks per request, on the device
  ntokens           [R] int32      tokens per request, on the device (optional):
                                   token t of block j holds data when
                                   j * B + t < ntokens[r], so the last block
                                   may be partly filled; its other tokens get
                                   no weight, whatever the page holds there

The reference reaches a paged cache only through FlashInfer's page table
(``strict_topk/flashinfer_backend.py:35-40``: page = block + kv_head * N over
``k.view(hkv * n, b, 1, d)``, one request per call).  Here the table is
explicit per (request, KV head), so requests share one pool and one launch:
``speculative_step`` and ``speculative_signed_step`` run the fused steps of
``strict_topk.step`` over the whole batch in two launches, and ``exact`` is
the serial path (top-K, then exact attention over the selected blocks) in
the same two launches with no prediction; ``append`` writes one decode token
per request into its page and widens that page's bounds.  Per request the
results are those of the dense steps on the request's own blocks, bit for
bit, except that a request with fewer blocks than ``topk`` selects all of them
(the rest of its ID row is -1).  A table entry outside [0, P) is an invalid page: its block
scores lowest and has the empty state, and nothing is read from it.
"""
from __future__ import annotations

from dataclasses import dataclass

import torch

from . import _lib
from .kernels import PartialState
from .signed_repair import SignedRepairResult
from .step import SignedStepResult, StepResult


@dataclass
class PagedKV:
    k_pages: torch.Tensor       # [P, B, D]
    v_pages: torch.Tensor       # [P, B, D]
    lo_pages: torch.Tensor      # [P, D] float32 or the pages' dtype
    hi_pages: torch.Tensor      # [P, D] float32 or the pages' dtype
    block_table: torch.Tensor   # [R, Hkv, NB] int32
    nblocks: torch.Tensor       # [R] int32
    ntokens: torch.Tensor | None = None   # [R] int32; None: every block full

    @property
    def requests(self):
        return self.block_table.shape[0]

    @property
    def hkv(self):
        return self.block_table.shape[1]

    @property
    def width(self):
        return self.block_table.shape[2]

    @property
    def pages(self):
        return self.k_pages.shape[0]

    @property
    def block(self):
        return self.k_pages.shape[1]

    @property
    def dim(self):
        return self.k_pages.shape[2]


def pack(caches, width=None, order=None, spare=0, tokens=None, bounds_dtype=torch.float32):
    """Pack dense per-request caches [(k, v), ...] (k, v: [Hkv, N_r, B, D])
    into one pool, building lo/hi pages on the device (``bounds.block_bounds``
    on the pool).  ``order``: an optional permutation of the pages (pages are
    placed in that order, to exercise the indirection); ``spare`` extra
    zeroed pages at the end of the pool; ``width``: the table's row width
    (default: the longest request); ``tokens``: each request's token count
    ((N_r - 1) * B < tokens[r] <= N_r * B; default N_r * B), the bounds of a
    partly filled last block taken over its tokens that hold data;
    ``bounds_dtype``: float32, or the caches' 16-bit dtype (exact, half the
    bytes for the scorer)."""
    from .bounds import block_bounds
    if not caches:
        raise ValueError("expected at least one request")
    k0 = caches[0][0]
    hkv, _, b, d = k0.shape
    counts = [k.shape[1] for k, _ in caches]
    for k, v in caches:
        if k.shape[0] != hkv or k.shape[2:] != (b, d) or v.shape != k.shape or k.dtype != k0.dtype:
            raise ValueError("every request needs K/V [Hkv, N_r, B, D] of one shape and dtype")
    if tokens is None:
        tokens = [n * b for n in counts]
    tokens = [int(t) for t in tokens]
    if len(tokens) != len(counts) or any(not (n - 1) * b < t <= n * b
                                         for n, t in zip(counts, tokens)):
        raise ValueError("tokens[r] must end inside request r's last block")
    width = max(counts) if width is None else int(width)
    if width < max(counts):
        raise ValueError("the table is narrower than the longest request")
    total = hkv * sum(counts)
    dev = k0.device
    slot = torch.arange(total, device=dev) if order is None else order.to(dev)
    if slot.numel() != total:
        raise ValueError("order must permute the requests' pages")
    k_pages = torch.zeros((total + spare, b, d), dtype=k0.dtype, device=dev)
    v_pages = torch.zeros_like(k_pages)
    table = torch.full((len(caches), hkv, width), -1, dtype=torch.int32)
    base = 0
    for r, (k, v) in enumerate(caches):
        n = k.shape[1]
        idx = slot[base:base + hkv * n]
        k_pages[idx] = k.reshape(hkv * n, b, d)
        v_pages[idx] = v.reshape(hkv * n, b, d)
        table[r, :, :n] = idx.view(hkv, n).to(torch.int32).cpu()
        base += hkv * n
    lo, hi = block_bounds(k_pages.unsqueeze(0), bounds_dtype)
    lo, hi = lo[0], hi[0]
    for r, (n, t) in enumerate(zip(counts, tokens)):
        part = t - (n - 1) * b
        if part < b:
            pages = table[r, :, n - 1].to(dev).long()
            lo[pages] = k_pages[pages, :part].amin(1).to(lo.dtype)
            hi[pages] = k_pages[pages, :part].amax(1).to(hi.dtype)
    return PagedKV(k_pages, v_pages, lo, hi, table.to(dev),
                   torch.tensor(counts, dtype=torch.int32, device=dev),
                   torch.tensor(tokens, dtype=torch.int32, device=dev))


def append(kv, k_new, v_new, positions):
    """Write one decode token per request in place: k_new, v_new [R, Hkv, D]
    at token position positions[r] (block pos // B, offset pos % B) of that
    block's page; the page's lo/hi are widened by the new key (offset 0 starts
    them over), nblocks[r] becomes pos // B + 1 and ntokens[r] pos + 1, in
    one launch.  positions is an int32 tensor on the device, so a captured
    graph can advance it.  A position outside [0, NB * B) writes nothing; a
    block without a valid page for some KV head writes nothing for that head
    and leaves the counts unchanged."""
    if not isinstance(kv, PagedKV):
        raise TypeError("kv must be a PagedKV")
    shape = (kv.requests, kv.hkv, kv.dim)
    if k_new.shape != shape or v_new.shape != shape:
        raise ValueError("expected K_NEW/V_NEW[R,Hkv,D] matching the pool")
    if positions.shape != (kv.requests,) or positions.dtype != torch.int32:
        raise ValueError("expected int32 positions[R]")
    if k_new.dtype != kv.k_pages.dtype or v_new.dtype != kv.k_pages.dtype:
        raise ValueError("K_NEW/V_NEW must match the pages' dtype")
    ts = [k_new, v_new, positions, kv.k_pages, kv.v_pages, kv.lo_pages, kv.hi_pages,
          kv.block_table, kv.nblocks]
    if kv.ntokens is not None:
        ts.append(kv.ntokens)
    if not kv.k_pages.is_cuda or any(t.device != kv.k_pages.device or not t.is_contiguous()
                                     for t in ts):
        raise ValueError("all tensors must be contiguous and on one CUDA device")
    if kv.ntokens is not None and (kv.ntokens.dtype != torch.int32 or
                                   kv.ntokens.shape != (kv.requests,)):
        raise ValueError("ntokens must be int32 [R]")
    _lib.call("stk_paged_append", _lib.ptr(k_new), _lib.ptr(v_new), _lib.dtype_code(k_new),
              kv.requests, kv.hkv, kv.width, kv.block, kv.dim, kv.pages, _lib.ptr(kv.k_pages),
              _lib.ptr(kv.v_pages), _lib.ptr(kv.lo_pages), _lib.ptr(kv.hi_pages),
              _lib.bounds_code(kv.lo_pages, kv.k_pages),
              _lib.ptr(kv.block_table), _lib.ptr(kv.nblocks), _lib.ptr(kv.ntokens),
              _lib.ptr(positions), _lib.stream(k_new.device))
    return kv


def _check(q, kv, predicted, topk):
    if not isinstance(kv, PagedKV):
        raise TypeError("kv must be a PagedKV")
    if q.ndim != 3 or q.shape[0] != kv.requests or q.shape[2] != kv.dim:
        raise ValueError("expected Q[R,Hq,D] matching the pool")
    r, hq, _ = q.shape
    if hq % kv.hkv:
        raise ValueError("Hq must be divisible by Hkv")
    if predicted is not None and (predicted.ndim != 3 or predicted.shape[:2] != (r, hq)):
        raise ValueError("expected P[R,Hq,SP]")
    if predicted is not None and predicted.dtype != torch.int32:
        raise ValueError("predicted IDs must be int32")
    if q.dtype != kv.k_pages.dtype:
        raise ValueError("Q and the pages must share a dtype")
    if kv.hi_pages.dtype != kv.lo_pages.dtype or \
            kv.lo_pages.dtype not in (torch.float32, kv.k_pages.dtype):
        raise ValueError("lo and hi pages must be FP32 or the pages' dtype")
    if kv.block_table.dtype != torch.int32 or kv.nblocks.dtype != torch.int32:
        raise ValueError("block_table and nblocks must be int32")
    if kv.ntokens is not None and (kv.ntokens.dtype != torch.int32 or
                                   kv.ntokens.shape != (kv.requests,)):
        raise ValueError("ntokens must be int32 [R]")
    topk = int(topk)
    if not 1 <= topk <= 256:
        raise ValueError("topk must be in [1, 256]")
    ts = [q, kv.k_pages, kv.v_pages, kv.lo_pages, kv.hi_pages, kv.block_table, kv.nblocks]
    if predicted is not None:
        ts.append(predicted)
    if kv.ntokens is not None:
        ts.append(kv.ntokens)
    if not q.is_cuda or any(t.device != q.device or not t.is_contiguous() for t in ts):
        raise ValueError("all tensors must be contiguous and on one CUDA device")
    return r, hq, topk


def _common(q, kv, predicted, topk):
    r, hq, topk = _check(q, kv, predicted, topk)
    sp = 0 if predicted is None else predicted.shape[2]
    dev = q.device
    d = kv.dim
    selected = torch.empty((r, hq, topk), device=dev, dtype=torch.int32)
    if sp:
        m = torch.empty((r, hq, sp), device=dev, dtype=torch.float32)
        state = PartialState(m, torch.empty_like(m),
                             torch.empty((r, hq, sp, d), device=dev, dtype=torch.float32))
    else:
        state = None
    out = torch.empty((r, hq, d), device=dev, dtype=torch.float32)
    ws = _lib.workspace(_lib.size("stk_paged_workspace_bytes", r, hq, kv.width), dev)
    head = (_lib.ptr(q), _lib.ptr(kv.k_pages), _lib.ptr(kv.v_pages), _lib.dtype_code(q), r, hq,
            kv.hkv, kv.width, kv.block, d, kv.pages, _lib.ptr(kv.lo_pages),
            _lib.ptr(kv.hi_pages), _lib.bounds_code(kv.lo_pages, q), _lib.ptr(kv.block_table),
            _lib.ptr(kv.nblocks),
            _lib.ptr(kv.ntokens), topk, _lib.ptr(predicted), sp)
    st = (None, None, None) if state is None else (_lib.ptr(state.m), _lib.ptr(state.l),
                                                   _lib.ptr(state.u))
    return head, selected, state, st, out, ws


def speculative_step(q, kv, predicted, topk, union=False):
    """The batched ``step.speculative_step``: per request, select(q, lo, hi,
    topk) || partials(q, k, v, predicted), then the saved (or union) repair.
    q [R, Hq, D], predicted [R, Hq, SP] int32 logical IDs; results [R, Hq, ...]."""
    head, selected, state, st, out, ws = _common(q, kv, predicted, topk)
    _lib.call("stk_paged_step", *head, 1 if union else 0, _lib.ptr(selected), *st,
              _lib.ptr(out), _lib.ptr(ws), ws.numel(), _lib.stream(q.device))
    return StepResult(selected, state, out)


def exact(q, kv, topk):
    """The serial path over the batch: the top-K of the bound scores, then the
    exact attention over the selected blocks (no prediction).  Returns
    (selected [R, Hq, topk], out [R, Hq, D])."""
    head, selected, _, st, out, ws = _common(q, kv, None, topk)
    _lib.call("stk_paged_step", *head, 0, _lib.ptr(selected), *st, _lib.ptr(out),
              _lib.ptr(ws), ws.numel(), _lib.stream(q.device))
    return selected, out


def speculative_signed_step(q, kv, predicted, topk, mode="hybrid", mass_threshold=0.1,
                            min_remaining=1.e-3, cancellation_tol=1.e-5, max_extra_mass=0.):
    """The batched ``step.speculative_signed_step`` (modes "hybrid" and
    "saved"); the result's fields are laid out [R, Hq, ...]."""
    if mode not in ("saved", "hybrid"):
        raise ValueError(mode)
    if not 0 <= mass_threshold <= 1:
        raise ValueError("mass_threshold must be in [0,1]")
    if not 0 <= max_extra_mass <= 1:
        raise ValueError("max_extra_mass must be in [0,1]")
    head, selected, state, st, out, ws = _common(q, kv, predicted, topk)
    r, hq = q.shape[:2]
    dev = q.device
    fallback = torch.empty((r, hq), device=dev, dtype=torch.bool)
    remaining = torch.empty((r, hq), device=dev, dtype=torch.float32)
    approx = torch.empty_like(fallback) if max_extra_mass > 0 else None
    extra = torch.empty_like(remaining) if max_extra_mass > 0 else None
    positive = torch.empty((r, hq), device=dev, dtype=torch.int32)
    total = torch.empty_like(positive)
    _lib.call("stk_paged_signed_step", *head, 1 if mode == "hybrid" else 0,
              float(mass_threshold), float(min_remaining), float(cancellation_tol),
              float(max_extra_mass), _lib.ptr(selected), *st, _lib.ptr(out),
              _lib.ptr(fallback), _lib.ptr(remaining), _lib.ptr(approx), _lib.ptr(extra),
              _lib.ptr(positive), _lib.ptr(total), _lib.ptr(ws), ws.numel(),
              _lib.stream(dev))
    res = SignedRepairResult(out, fallback, remaining, approx, extra, positive, total)
    return SignedStepResult(selected, state, res)
