"""The allocation-free step (stk_speculative_step_noalloc) against
stk_speculative_step, through the C ABI: two calls in a row, the second on a
smaller input, then a captured graph replayed while the query changes in
place.  Both entry points run the same kernels on the same inputs, so every
result must be bit-identical; the oracle checks the IDs and the output too."""
import pytest
import torch

from oracle import stk_oracle as O
from tests import cases as C

pytestmark = pytest.mark.gpu

DEV = "cuda"


@pytest.fixture(scope="module", autouse=True)
def _gpu():
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    from strict_topk import _lib
    _lib.lib()


def _inputs(hq, hkv, n, b, d, topk, dtype, seed, overlap):
    from stk_harness.configs import make_qkv, perturb
    q, k, v, lo, hi = make_qkv(hq, hkv, d, b, n, dtype, True, seed)
    ids = O.select_blocks(C.f64(q), lo.numpy(), hi.numpy(), topk)
    p = perturb(torch.from_numpy(ids), n, topk, overlap, seed)
    return [t.to(DEV) for t in (q, k, v, lo, hi, p)], (q, k, v, ids)


def _noalloc(q, k, v, lo, hi, p, topk, union):
    """stk_speculative_step_noalloc through the C ABI into fresh outputs."""
    from strict_topk import _lib
    from strict_topk.kernels import _allocate_state, _args
    hq, d = q.shape
    sp = p.shape[1]
    sel = torch.full((hq, topk), -7, device=DEV, dtype=torch.int32)
    st = _allocate_state(hq, sp, d, q.device)
    out = torch.full((hq, d), float("nan"), device=DEV)
    _lib.call("stk_speculative_step_noalloc", *_args(q, k, v), _lib.ptr(lo), _lib.ptr(hi),
              _lib.bounds_code(lo, q), topk,
              _lib.ptr(p), _lib.id_code(p), sp, 1 if union else 0, _lib.ptr(sel),
              _lib.ptr(st.m), _lib.ptr(st.l), _lib.ptr(st.u), _lib.ptr(out),
              _lib.stream(q.device))
    return sel, st, out


def _same(ref, sel, st, out):
    assert torch.equal(ref.selected, sel)
    assert torch.equal(ref.state.m, st.m) and torch.equal(ref.state.l, st.l)
    assert torch.equal(ref.state.u, st.u)
    assert torch.equal(ref.output, out)


@pytest.mark.parametrize("union", [False, True])
def test_noalloc_matches_workspace_step(union):
    from strict_topk import step
    shapes = [(32, 8, 2048, 32, 128, 64, torch.bfloat16, 0.9),   # c3
              (8, 2, 300, 16, 64, 20, torch.float16, 0.75),     # smaller, second
              (4, 4, 100, 32, 64, 12, torch.float16, 0.75)]     # one workgroup per head
    for i, (hq, hkv, n, b, d, topk, dt, ov) in enumerate(shapes):
        print(f"noalloc call {i}: hq={hq} n={n} d={d} union={union}", flush=True)
        (q, k, v, lo, hi, p), (qh, kh, vh, ids) = _inputs(hq, hkv, n, b, d, topk, dt,
                                                          20261103 + i, ov)
        ref = step.speculative_step(q, k, v, lo, hi, p, topk, union=union)
        sel, st, out = _noalloc(q, k, v, lo, hi, p, topk, union)
        torch.cuda.synchronize()
        _same(ref, sel, st, out)
        assert sel.cpu().numpy().tolist() == ids.tolist()
        if not union:
            m = C.error_metrics(C.f64(out), O.attention(C.f64(qh), C.f64(kh), C.f64(vh), ids))
            assert m["passed"], m


def test_noalloc_in_a_captured_graph():
    from strict_topk import step
    (q, k, v, lo, hi, p), _ = _inputs(16, 8, 512, 32, 128, 64, torch.bfloat16, 5, 0.9)
    res = step.speculative_step_noalloc(q, k, v, lo, hi, p, 64)   # eager, outside capture
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        step.speculative_step_noalloc(q, k, v, lo, hi, p, 64, into=res)
    q0 = q.clone()
    for scale in (1.0, -1.0, 0.25):
        q.copy_(q0 * scale)
        g.replay()
        torch.cuda.synchronize()
        ref = step.speculative_step(q, k, v, lo, hi, p, 64)
        torch.cuda.synchronize()
        _same(ref, res.selected, res.state, res.output)


def test_noalloc_rejects_too_many_keys():
    from strict_topk import step
    q = torch.zeros((128, 128), device=DEV, dtype=torch.bfloat16)
    k = torch.zeros((8, 8192, 16, 128), device=DEV, dtype=torch.bfloat16)
    lo = torch.zeros((8, 8192, 128), device=DEV)
    p = torch.zeros((128, 8), device=DEV, dtype=torch.int32)
    assert step.supported(q, k, lo, 8, p)
    with pytest.raises(ValueError, match="524288"):
        step.speculative_step_noalloc(q, k, k, lo, lo, p, 8)


_FIRST_UNDER_CAPTURE = r"""
import sys
sys.path[:0] = [{pkg!r}, {root!r}]
import torch
from strict_topk import _lib, step
from stk_harness.configs import make_qkv
q, k, v, lo, hi = (t.cuda() for t in make_qkv(8, 2, 128, 32, 256, torch.bfloat16, True, 11))
lo, hi = lo.to(torch.bfloat16), hi.to(torch.bfloat16)
gen = torch.Generator().manual_seed(3)
p = torch.stack([torch.randperm(256, generator=gen)[:32] for _ in range(8)]).int().cuda()
if {prepare}:
    _lib.prepare(q.device)
g = torch.cuda.CUDAGraph()
try:
    with torch.cuda.graph(g):
        res = step.speculative_step_noalloc(q, k, v, lo, hi, p, 16)
except Exception as e:
    print("REFUSED", "stk_step_prepare" in str(e), flush=True)
    sys.exit(0)
g.replay()
torch.cuda.synchronize()
ref = step.speculative_step(q, k, v, lo, hi, p, 16)
same = torch.equal(ref.selected, res.selected) and torch.equal(ref.output, res.output)
print("CAPTURED", same, flush=True)
"""


@pytest.mark.parametrize("prepare,expected", [(False, "REFUSED True"), (True, "CAPTURED True")])
def test_noalloc_first_call_under_capture(prepare, expected):
    """In a fresh process whose first step call is under graph capture: the
    library refuses to look up its device memory there (a clear error naming
    stk_step_prepare), and after stk_step_prepare the captured call works and
    matches the eager step."""
    import subprocess
    import sys
    from pathlib import Path
    root = Path(__file__).resolve().parents[1]
    code = _FIRST_UNDER_CAPTURE.format(pkg=str(root / "strict-topk-overlap_amd"), root=str(root),
                                       prepare=prepare)
    r = subprocess.run([sys.executable, "-c", code], capture_output=True, text=True, timeout=300)
    assert r.returncode == 0, r.stderr[-2000:]
    assert expected in r.stdout, (r.stdout, r.stderr[-2000:])
