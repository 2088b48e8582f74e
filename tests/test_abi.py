"""The C ABI: every function declared in include/strict_topk.h is exported by
the built library and bound by strict_topk/_lib.py with the same arity.
No GPU is needed (only symbol lookup and host-only queries are called)."""
import ctypes
import re
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parents[1]
HEADER = ROOT / "include" / "strict_topk.h"


def _declarations():
    text = HEADER.read_text()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    decls = {}
    for m in re.finditer(r"\b(?:const\s+)?[a-z_0-9]+\s*\*?\s*(stk_[a-z0-9_]+)\s*\(([^)]*)\)\s*;", text):
        args = m.group(2).strip()
        decls[m.group(1)] = 0 if args in ("", "void") else len(args.split(","))
    return decls


@pytest.fixture(scope="module")
def lib():
    from strict_topk import _lib
    if not _lib._PATH.exists():
        import build_lib
        build_lib.build()
    return _lib


def test_header_declares_the_abi():
    decls = _declarations()
    assert len(decls) >= 25
    assert "stk_speculative_step" in decls and "stk_select_blocks" in decls


def test_every_declared_symbol_is_exported(lib):
    handle = ctypes.CDLL(str(lib._PATH))
    missing = [name for name in _declarations() if not hasattr(handle, name)]
    assert not missing, missing


def test_binding_matches_header(lib):
    decls = _declarations()
    assert set(lib._SIGS) == set(decls)
    for name, nargs in decls.items():
        assert len(lib._SIGS[name][1]) == nargs, name


def test_host_only_queries(lib):
    L = lib.lib()
    assert L.stk_abi_version() == 1
    assert L.stk_step_supported(2, 32, 8, 2048, 32, 128, 64, 64, 0) == 1
    assert L.stk_step_supported(0, 32, 8, 2048, 32, 128, 64, 64, 0) == 0   # fp32
    assert L.stk_step_supported(2, 32, 8, 2048, 32, 96, 64, 64, 0) == 0    # D = 96
    assert lib.size("stk_select_workspace_bytes", 32, 8, 2048, 128, 64) >= 32 * 2048 * 8
    # argument errors are reported without touching a device
    rc = L.stk_block_scores(None, 2, None, None, 0, 4, 3, 10, 8, None, None)
    assert rc == -1 and b"divisible" in L.stk_last_error()


def test_one_launch_support_matches_the_flag_slot(lib):
    """stk_step1_supported reports one launch exactly when the flags,
    Hq * (ceil(N / 64) + SP) words, fit a slot of 16384 words beside its
    time-out counter: 16383 words fit, 16384 do not."""
    L = lib.lib()
    # 127 heads * (65 chunks + 64 slots) = 16383
    assert L.stk_step1_supported(2, 127, 127, 4160, 32, 64, 64, 64, 0) == 1
    # 128 heads * (64 chunks + 64 slots) = 16384
    assert L.stk_step1_supported(2, 128, 32, 4096, 32, 64, 64, 64, 0) == 0
    assert L.stk_step_supported(2, 128, 32, 4096, 32, 64, 64, 64, 0) == 1


def test_small_step_support_bounds(lib):
    """stk_step_small_supported covers N <= 128, K and SP in [1, 16], B = 32,
    D in {64, 128}, bf16 / fp16 K/V with FP32 or same-type bounds, int32
    predictions, and nothing the fused step itself rejects."""
    L = lib.lib()
    ok = (2, 8, 2, 64, 32, 128, 8, 8, 0, 0)            # bf16, FP32 bounds
    assert L.stk_step_small_supported(*ok) == 1
    assert L.stk_step_small_supported(1, 4, 4, 1, 32, 64, 1, 1, 0, 1) == 1   # fp16, fp16 bounds
    assert L.stk_step_small_supported(2, 8, 2, 128, 32, 128, 16, 16, 0, 0) == 1   # the largest
    for i, bad in ((3, 129), (6, 17), (6, 0), (7, 17), (7, 0), (4, 64), (5, 256), (8, 1)):
        args = list(ok)
        args[i] = bad
        assert L.stk_step_small_supported(*args) == 0, (i, bad)
    assert L.stk_step_small_supported(2, 8, 2, 8, 32, 128, 9, 8, 0, 0) == 0    # K > N
    assert L.stk_step_small_supported(2, 8, 3, 64, 32, 128, 8, 8, 0, 0) == 0   # Hq % Hkv
    assert L.stk_step_small_supported(0, 8, 2, 64, 32, 128, 8, 8, 0, 0) == 0   # fp32 K/V


def test_noalloc_step_rejects_oversized_key_rows(lib):
    """The allocation-free step refuses Hq * N above its fixed scratch before
    touching a device."""
    L = lib.lib()
    assert L.stk_step_noalloc_max_keys() == 1 << 19
    fake = ctypes.c_void_p(256)
    rc = L.stk_speculative_step_noalloc(fake, fake, fake, 2, 128, 8, 8192, 32, 128, fake, fake,
                                        0, 64, fake, 0, 64, 0, fake, fake, fake, fake, fake, None)
    assert rc == -1 and b"524288" in L.stk_last_error()


def _doc_bindings():
    """(name, kind, count) for every `<lib>.stk_*.argtypes = [...]` assignment
    and every `<lib>.stk_*(...)` call in INTEGRATION.md's Python blocks."""
    import ast
    text = (ROOT / "INTEGRATION.md").read_text()
    found = []
    for block in re.findall(r"```python\n(.*?)```", text, flags=re.S):
        for node in ast.walk(ast.parse(block)):
            if isinstance(node, ast.Assign) and isinstance(node.value, ast.List):
                for tgt in node.targets:
                    if (isinstance(tgt, ast.Attribute) and tgt.attr == "argtypes" and
                            isinstance(tgt.value, ast.Attribute) and
                            tgt.value.attr.startswith("stk_")):
                        found.append((tgt.value.attr, "argtypes", len(node.value.elts)))
            elif (isinstance(node, ast.Call) and isinstance(node.func, ast.Attribute) and
                  node.func.attr.startswith("stk_")):
                found.append((node.func.attr, "call", len(node.args)))
    return found


def test_documented_binding_matches_header():
    """The reference-side ctypes binding shown in INTEGRATION.md declares and
    passes exactly the parameters the header declares."""
    decls = _declarations()
    found = _doc_bindings()
    names = {name for name, _, _ in found}
    assert {"stk_select_blocks", "stk_select_workspace_bytes"} <= names
    assert any(kind == "argtypes" for _, kind, _ in found)
    assert any(kind == "call" for _, kind, _ in found)
    wrong = [(name, kind, n, decls.get(name)) for name, kind, n in found if decls.get(name) != n]
    assert not wrong, wrong
