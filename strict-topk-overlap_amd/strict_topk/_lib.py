"""ctypes binding of libstrict_topk_hip.so (the C ABI declared in
include/strict_topk.h).

The library is loaded lazily on first use, after ``torch`` so that the HIP
runtime it links (SONAME libamdhip64.so.7) resolves to the copy torch already
loaded: streams and device pointers are then shared.  There is no fallback:
a missing or unloadable library raises immediately.
"""
from __future__ import annotations

import ctypes
import os
import threading
from pathlib import Path

import torch

_PATH = Path(os.environ.get("STRICT_TOPK_LIB", Path(__file__).with_name("libstrict_topk_hip.so")))
_lock = threading.Lock()
_lib = None

P = ctypes.c_void_p
I = ctypes.c_int
F = ctypes.c_float
Z = ctypes.c_size_t

# (name, restype, argtypes)
_SIGS = {
    "stk_last_error": (ctypes.c_char_p, []),
    "stk_abi_version": (I, []),
    "stk_block_scores": (I, [P, I, P, P, I, I, I, I, I, P, P]),
    "stk_select_workspace_bytes": (Z, [I, I, I, I, I]),
    "stk_select_blocks": (I, [P, I, P, P, I, I, I, I, I, I, P, P, P, Z, P]),
    "stk_block_partials": (I, [P, P, P, I, I, I, I, I, I, P, I, I, P, I, P, P, P, P]),
    "stk_merge_partials": (I, [P, P, P, P, I, I, I, P, P]),
    "stk_exact_workspace_bytes": (Z, [I, I, I]),
    "stk_exact_attention": (I, [P, P, P, I, I, I, I, I, I, P, I, I, P, P, Z, P]),
    "stk_speculate": (I, [P, P, P, I, I, I, I, I, I, P, I, I, I, F, I,
                          P, P, P, P, P, P, P, P, P, P, P, P, P]),
    "stk_touch_kv": (I, [P, P, I, I, I, I, I, P, I, I, P, P]),
    "stk_fallback": (I, [P, P, P, I, I, I, I, I, I, P, I, I, P, P, P]),
    "stk_repair_workspace_bytes": (Z, [I, I, I, I, I, I]),
    "stk_repair": (I, [P, P, P, I, I, I, I, I, I, P, I, I, P, I, I, I, I,
                       P, P, P, P, P, P, P, P, P, F, F, P, P, P, P, Z, P]),
    "stk_repair_fused": (I, [P, P, P, I, I, I, I, I, I, P, I, I, P, I, I, I, I,
                             P, P, P, P, P, P, P, P, P, P, P, F, F, F, P, P, P, P, P, P]),
    "stk_gqa_repair_workspace_bytes": (Z, [I, I, I]),
    "stk_gqa_repair": (I, [P, P, P, I, I, I, I, I, I, P, I, I, P, I, I, P, P, P, I, P, P, Z, P]),
    "stk_repair_light": (I, [P, P, P, I, I, I, I, I, I, P, I, I, P, I, I, P, P, P, P, P]),
    "stk_signed_workspace_bytes": (Z, [I, I, I, I, I, I]),
    "stk_repair_signed": (I, [P, P, P, I, I, I, I, I, I, P, I, I, P, I, I, I, I,
                              P, P, P, P, P, P, P, P, P, P, P, F, F, F, I,
                              P, I, P, P, P, P, P, P, P, P, Z, P]),
    "stk_hier_exact_workspace_bytes": (Z, [I, I, I]),
    "stk_hier_exact": (I, [P, P, P, I, I, I, I, I, I, P, I, I, P, P, Z, P]),
    "stk_hier_repair_workspace_bytes": (Z, [I, I, I, I]),
    "stk_hier_repair": (I, [P, P, P, I, I, I, I, I, I, P, I, I, P, I, I, P, P, P, I, P, P, Z, P]),
    "stk_step_workspace_bytes": (Z, [I, I, I, I, I]),
    "stk_step_supported": (I, [I, I, I, I, I, I, I, I, I]),
    "stk_speculative_step": (I, [P, P, P, I, I, I, I, I, I, P, P, I, I, P, I, I, I,
                                 P, P, P, P, P, P, Z, P]),
    "stk_step1_supported": (I, [I, I, I, I, I, I, I, I, I]),
    "stk_step_small_supported": (I, [I, I, I, I, I, I, I, I, I, I]),
    "stk_step1_timeouts": (I, []),
    "stk_step1_test_hook": (I, [ctypes.c_ulonglong, I]),
    "stk_step_noalloc_max_keys": (Z, []),
    "stk_step_prepare": (I, []),
    "stk_speculative_step_noalloc": (I, [P, P, P, I, I, I, I, I, I, P, P, I, I, P, I, I, I,
                                         P, P, P, P, P, P]),
    "stk_step_front": (I, [P, P, P, I, I, I, I, I, I, P, P, I, I, P, I, I, P, P, P, P, Z, P]),
    "stk_step_tail": (I, [P, P, P, I, I, I, I, I, I, I, P, I, I, I, P, P, P, P, P, P, Z, P]),
    "stk_indexer_workspace_bytes": (Z, [I]),
    "stk_indexer_scores": (I, [P, P, I, I, I, I, P, P, Z, P]),
    "stk_indexer_select": (I, [P, P, I, I, I, I, I, I, P, P, P, Z, P]),
    "stk_block_bounds": (I, [P, I, I, I, I, I, P, P, I, P]),
    "stk_bounds_append": (I, [P, I, I, I, I, I, I, P, P, I, P]),
    "stk_signed_step": (I, [P, P, P, I, I, I, I, I, I, P, P, I, I, P, I, I, I, F, F, F, F,
                            P, P, P, P, P, P, P, P, P, P, P, P, Z, P]),
    "stk_paged_workspace_bytes": (Z, [I, I, I]),
    "stk_paged_append": (I, [P, P, I, I, I, I, I, I, I, P, P, P, P, I, P, P, P, P, P]),
    "stk_paged_step": (I, [P, P, P, I, I, I, I, I, I, I, I, P, P, I, P, P, P, I, P, I, I,
                           P, P, P, P, P, P, Z, P]),
    "stk_paged_signed_step": (I, [P, P, P, I, I, I, I, I, I, I, I, P, P, I, P, P, P, I, P, I, I,
                                  F, F, F, F, P, P, P, P, P, P, P, P, P, P, P, P, Z, P]),
    "stk_cache_workspace_bytes": (Z, [I, I, I, I]),
    "stk_cache_step": (I, [P, I, I, I, I, I, I, I, P, P, I, P, P, I, P, P, I, P, P, P, P, P,
                           P, P, I, P, I, P, P, P, P, P, P, P, Z, P]),
}

EXPORTS = tuple(_SIGS)

DTYPE = {torch.float32: 0, torch.float16: 1, torch.bfloat16: 2}
ITYPE = {torch.int32: 0, torch.int64: 1}


def lib():
    global _lib
    if _lib is None:
        with _lock:
            if _lib is None:
                if not _PATH.exists():
                    raise RuntimeError(
                        f"strict_topk HIP library not built: {_PATH} is missing "
                        "(run `python strict-topk-overlap_amd/build_lib.py`)")
                handle = ctypes.CDLL(str(_PATH))
                for name, (res, args) in _SIGS.items():
                    fn = getattr(handle, name)
                    fn.restype = res
                    fn.argtypes = args
                _lib = handle
    return _lib


def ptr(t):
    """Device address of a tensor, or None."""
    return None if t is None else t.data_ptr()


def dtype_code(t):
    try:
        return DTYPE[t.dtype]
    except KeyError:
        raise ValueError(f"unsupported element dtype {t.dtype}; expected float16, bfloat16 or float32")


def bounds_code(bound, q):
    """bounds_dtype of the C ABI: STK_F32 for float32 lo/hi, or the code of
    the queries' 16-bit type when the bounds are stored in it (exact: the
    min / max of 16-bit keys are 16-bit values)."""
    if bound.dtype == torch.float32:
        return 0
    if bound.dtype == q.dtype and q.dtype in (torch.float16, torch.bfloat16):
        return DTYPE[q.dtype]
    raise ValueError("lo and hi must be FP32 or the element type of Q/K/V")


def id_code(t):
    return ITYPE[t.dtype]


def stream(device):
    return torch.cuda.current_stream(device).cuda_stream


def workspace(nbytes, device):
    return torch.empty(max(int(nbytes), 1), dtype=torch.uint8, device=device)


def call(name, *args):
    fn = getattr(lib(), name)
    rc = fn(*args)
    if rc != 0:
        msg = lib().stk_last_error().decode(errors="replace")
        if rc == -1:
            raise ValueError(msg)
        raise RuntimeError(msg)
    return rc


def size(name, *args):
    return int(getattr(lib(), name)(*args))


_prepared = set()


def prepare(device):
    """Look up the fused step's device memory (the allocation-free step's
    scratch, the one-launch step's flag slots) on ``device`` once, outside
    any stream capture: the C entry points refuse a device's first lookup
    under capture."""
    idx = device.index if device.index is not None else torch.cuda.current_device()
    if idx in _prepared or torch.cuda.is_current_stream_capturing():
        return
    with torch.cuda.device(idx):
        call("stk_step_prepare")
    _prepared.add(idx)
