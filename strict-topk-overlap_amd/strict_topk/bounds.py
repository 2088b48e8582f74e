"""Block metadata of the bound scorer (an extension of the drop-in API).

The reference builds the per-block key bounds in its harness, outside the
timed step, as ``k.amin(dim=2).float()`` / ``k.amax(dim=2).float()``
(``benchmarks/critical_path.py:186``, ``benchmarks/run_benchmark.py:43``).
``block_bounds`` computes the same tensors on the GPU, and ``append`` is the
per-token update a decode loop needs when a token is written to the last
block.  NaN keys give NaN bounds, as torch does.  The bounds may also be
kept in K's own 16-bit type (``dtype=k.dtype``): the minimum and maximum of
16-bit keys are 16-bit values, so the storage is exact, the fused steps
select the same blocks, and their scorer reads half the bytes.
"""
import torch

from . import _lib


def _check_k(k):
    if not k.is_cuda or k.ndim != 4 or not k.is_contiguous():
        raise ValueError("expected contiguous CUDA K[Hkv,N,B,D]")


def block_bounds(k, dtype=torch.float32):
    """lo, hi[Hkv, N, D]: per-block minimum and maximum over tokens, as
    float32 (the reference's layout) or, with ``dtype=k.dtype``, in K's own
    16-bit type."""
    _check_k(k)
    if dtype not in (torch.float32, k.dtype):
        raise ValueError("bounds are FP32 or K's own dtype")
    hkv, n, b, d = k.shape
    lo = torch.empty((hkv, n, d), device=k.device, dtype=dtype)
    hi = torch.empty_like(lo)
    _lib.call("stk_block_bounds", _lib.ptr(k), _lib.dtype_code(k), hkv, n, b, d, _lib.ptr(lo),
              _lib.ptr(hi), _lib.bounds_code(lo, k), _lib.stream(k.device))
    return lo, hi


def append(lo, hi, k_new, block, pos):
    """Widen block ``block``'s bounds (in place) by the token k_new[Hkv, D]
    written at position ``pos`` of the block; position 0 starts them over."""
    if not k_new.is_cuda or k_new.ndim != 2 or not k_new.is_contiguous():
        raise ValueError("expected contiguous CUDA K_NEW[Hkv,D]")
    hkv, d = k_new.shape
    if lo.shape != hi.shape or lo.ndim != 3 or lo.shape[0] != hkv or lo.shape[2] != d:
        raise ValueError("expected LO/HI[Hkv,N,D] matching K_NEW")
    if hi.dtype != lo.dtype or lo.dtype not in (torch.float32, k_new.dtype):
        raise ValueError("lo and hi must be FP32 or K_NEW's dtype")
    if any(not x.is_cuda or x.device != k_new.device or not x.is_contiguous() for x in (lo, hi)):
        raise ValueError("lo and hi must be contiguous and on K_NEW's CUDA device")
    n = lo.shape[1]
    _lib.call("stk_bounds_append", _lib.ptr(k_new), _lib.dtype_code(k_new), hkv, n, d,
              int(block), int(pos), _lib.ptr(lo), _lib.ptr(hi), _lib.bounds_code(lo, k_new),
              _lib.stream(k_new.device))
    return lo, hi
