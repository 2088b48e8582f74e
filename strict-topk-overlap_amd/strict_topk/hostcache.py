"""Host-backed KV cache (an extension of the drop-in API).

The reference describes, for SGLang's HiSparse, a decode path whose full KV
lives in a pinned host pool with a hot device buffer per request
(``docs/hisparse_integration.md:11-27``): the selector picks the logical
top-K, swap-in finds the resident hits, updates the LRU, copies the missing
blocks in and hands attention a device slot table; speculation reads only
the resident predicted blocks (P n R) and the repair recomputes the rest of
the selected set A from the slots.  Here that is one call,
``speculative_step(q, cache, predicted, topk)``, five launches on the
current stream (``stk_cache_step``; the swap-in is two of them):

  scores of every block (their bounds stay on the device) || prediction
  states of P n R;  top-K;  swap-in (LRU over each (request, KV head)'s C
  slots, host pages copied in by the GPU, bytes counted);  strict repair.

Layout (``HostCache``): host pages [HP, B, D] in pinned memory, one per
(request, KV head, logical block); ``host_table`` [R, Hkv, NB] maps a block
to its host page; device slots [R * Hkv * C, B, D], group r * Hkv + kvh
owning slots [g * C, (g + 1) * C); ``table`` [R, Hkv, NB] the device slot of
a resident block or -1 (the block table the paged kernels read);
``slot_block`` / ``slot_stamp`` the reverse map and the LRU stamps;
``clock`` the step counter; ``h2d_bytes`` the bytes copied so far.
"""
from __future__ import annotations

from dataclasses import dataclass

import torch

from . import _lib
from .kernels import PartialState
from .step import StepResult


@dataclass
class HostCache:
    host_k: torch.Tensor        # [HP, B, D] pinned host memory
    host_v: torch.Tensor        # [HP, B, D] pinned host memory
    lo_pages: torch.Tensor      # [HP, D] device, FP32 or the pages' dtype
    hi_pages: torch.Tensor      # [HP, D] device
    host_table: torch.Tensor    # [R, Hkv, NB] int32 device
    k_slots: torch.Tensor       # [R * Hkv * C, B, D] device
    v_slots: torch.Tensor       # [R * Hkv * C, B, D] device
    table: torch.Tensor         # [R, Hkv, NB] int32 device: slot or -1
    slot_block: torch.Tensor    # [R * Hkv * C] int32 device: block or -1
    slot_stamp: torch.Tensor    # [R * Hkv * C] int32 device: last step used
    clock: torch.Tensor         # [1] int32 device
    h2d_bytes: torch.Tensor     # [1] int64 device, bytes copied host -> device so far
    nblocks: torch.Tensor       # [R] int32 device
    ntokens: torch.Tensor       # [R] int32 device
    slots_per_group: int

    @property
    def requests(self):
        return self.host_table.shape[0]

    @property
    def hkv(self):
        return self.host_table.shape[1]

    @property
    def width(self):
        return self.host_table.shape[2]

    @property
    def block(self):
        return self.host_k.shape[1]

    @property
    def dim(self):
        return self.host_k.shape[2]

    def resident(self):
        """Number of resident blocks per (request, KV head), [R, Hkv]."""
        return (self.table >= 0).sum(dim=2)


def build(caches, slots_per_group, device=None, bounds_dtype=torch.float32, tokens=None):
    """A cache over dense per-request K/V [(k, v), ...] (k, v: [Hkv, N_r, B,
    D], any device): the pages go to pinned host memory, the bounds of every
    block to the device, and no block is resident yet.  ``tokens``: each
    request's token count, as in ``paged.pack``."""
    from .bounds import block_bounds
    if not caches:
        raise ValueError("expected at least one request")
    k0 = caches[0][0]
    hkv, _, b, d = k0.shape
    if k0.dtype not in (torch.float16, torch.bfloat16):
        raise ValueError("the host-backed cache takes bf16 or fp16 K/V")
    device = torch.device(device) if device is not None else torch.device("cuda")
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
    r_, nb = len(caches), max(counts)
    total = hkv * sum(counts)
    host_k = torch.empty((total, b, d), dtype=k0.dtype, pin_memory=True)
    host_v = torch.empty((total, b, d), dtype=k0.dtype, pin_memory=True)
    lo_pages = torch.empty((total, d), dtype=bounds_dtype, device=device)
    hi_pages = torch.empty_like(lo_pages)
    table = torch.full((r_, hkv, nb), -1, dtype=torch.int32)
    base = 0
    for r, ((k, v), t) in enumerate(zip(caches, tokens)):
        n = k.shape[1]
        host_k[base:base + hkv * n] = k.reshape(hkv * n, b, d).cpu()
        host_v[base:base + hkv * n] = v.reshape(hkv * n, b, d).cpu()
        kd = k.to(device)
        lo, hi = block_bounds(kd.contiguous(), bounds_dtype)
        part = t - (n - 1) * b
        if part < b:   # a partly filled last block: bounds over its live tokens
            lo[:, n - 1] = kd[:, n - 1, :part].amin(1).to(bounds_dtype)
            hi[:, n - 1] = kd[:, n - 1, :part].amax(1).to(bounds_dtype)
        lo_pages[base:base + hkv * n] = lo.reshape(hkv * n, d)
        hi_pages[base:base + hkv * n] = hi.reshape(hkv * n, d)
        table[r, :, :n] = torch.arange(base, base + hkv * n, dtype=torch.int32).view(hkv, n)
        base += hkv * n
    c = int(slots_per_group)
    slots = r_ * hkv * c
    return HostCache(
        host_k, host_v, lo_pages, hi_pages, table.to(device),
        torch.zeros((slots, b, d), dtype=k0.dtype, device=device),
        torch.zeros((slots, b, d), dtype=k0.dtype, device=device),
        torch.full((r_, hkv, nb), -1, dtype=torch.int32, device=device),
        torch.full((slots,), -1, dtype=torch.int32, device=device),
        torch.full((slots,), -1, dtype=torch.int32, device=device),
        torch.zeros((1,), dtype=torch.int32, device=device),
        torch.zeros((1,), dtype=torch.int64, device=device),
        torch.tensor(counts, dtype=torch.int32, device=device),
        torch.tensor(tokens, dtype=torch.int32, device=device), c)


def exact(q, cache, topk):
    """The serial path over the cache: select, swap-in, then the exact
    attention over the selected blocks (no prediction).  Returns (selected,
    out), laid out [R, Hq, ...]."""
    res = _step(q, cache, None, topk)
    return res.selected, res.output


def speculative_step(q, cache, predicted, topk):
    """One decode step over the batch: select(q) || partials over the resident
    predicted blocks, then swap-in of the selected blocks that are not
    resident, then the strict repair.  q [R, Hq, D], predicted [R, Hq, SP]
    int32; returns ``StepResult`` laid out [R, Hq, ...] (the prediction
    state of a non-resident predicted block is the empty state).  The output
    is the exact attention over each request's selected blocks."""
    return _step(q, cache, predicted, topk)


def _step(q, cache, predicted, topk):
    if not isinstance(cache, HostCache):
        raise TypeError("cache must be a HostCache")
    if q.ndim != 3 or q.shape[0] != cache.requests or q.shape[2] != cache.dim:
        raise ValueError("expected Q[R,Hq,D] matching the cache")
    r, hq, d = q.shape
    if hq % cache.hkv:
        raise ValueError("Hq must be divisible by Hkv")
    if predicted is not None and (predicted.ndim != 3 or predicted.shape[:2] != (r, hq) or
                                  predicted.dtype != torch.int32):
        raise ValueError("expected int32 P[R,Hq,SP]")
    if q.dtype != cache.k_slots.dtype:
        raise ValueError("Q and the cache must share a dtype")
    topk = int(topk)
    sp = 0 if predicted is None else predicted.shape[2]
    if not 1 <= topk <= 256 or not 0 <= sp <= 256:
        raise ValueError("topk must be in [1, 256] and the predicted width in [0, 256]")
    dev = q.device
    ts = [q, cache.k_slots, cache.v_slots, cache.lo_pages, cache.hi_pages,
          cache.host_table, cache.table, cache.slot_block, cache.slot_stamp, cache.clock,
          cache.h2d_bytes, cache.nblocks, cache.ntokens]
    if predicted is not None:
        ts.append(predicted)
    if not q.is_cuda or any(t.device != dev or not t.is_contiguous() for t in ts):
        raise ValueError("all device tensors must be contiguous and on Q's CUDA device")
    if not (cache.host_k.is_pinned() and cache.host_v.is_pinned()):
        raise ValueError("the host pool must be pinned memory")
    selected = torch.empty((r, hq, topk), device=dev, dtype=torch.int32)
    state = None
    if sp:
        m = torch.empty((r, hq, sp), device=dev, dtype=torch.float32)
        state = PartialState(m, torch.empty_like(m),
                             torch.empty((r, hq, sp, d), device=dev, dtype=torch.float32))
    out = torch.empty((r, hq, d), device=dev, dtype=torch.float32)
    ws = _lib.workspace(_lib.size("stk_cache_workspace_bytes", r, hq, cache.hkv, cache.width),
                        dev)
    _lib.call("stk_cache_step", _lib.ptr(q), _lib.dtype_code(q), r, hq, cache.hkv, cache.width,
              cache.block, d, _lib.ptr(cache.k_slots), _lib.ptr(cache.v_slots),
              cache.slots_per_group, _lib.ptr(cache.host_k), _lib.ptr(cache.host_v),
              cache.host_k.shape[0], _lib.ptr(cache.lo_pages), _lib.ptr(cache.hi_pages),
              _lib.bounds_code(cache.lo_pages, q), _lib.ptr(cache.host_table),
              _lib.ptr(cache.table), _lib.ptr(cache.slot_block), _lib.ptr(cache.slot_stamp),
              _lib.ptr(cache.clock), _lib.ptr(cache.nblocks), _lib.ptr(cache.ntokens), topk,
              _lib.ptr(predicted), sp, _lib.ptr(selected),
              *((None, None, None) if state is None else
                (_lib.ptr(state.m), _lib.ptr(state.l), _lib.ptr(state.u))), _lib.ptr(out), _lib.ptr(cache.h2d_bytes), _lib.ptr(ws),
              ws.numel(), _lib.stream(dev))
    return StepResult(selected, state, out)
