"""GPU parity of the small-shape step (one workgroup per query head).

stk_speculative_step runs shapes with at most 128 blocks per KV head and at
most sixteen selected and sixteen predicted rows per head in one workgroup per
query head (k_step_small).  Bars, as for the other fused paths: selected IDs
bit-exact against the FP64 oracle (ties toward the lower index, ascending);
the prediction's block states and the output within the reference tolerance
|err| <= 3e-4 + 3e-4 |ref| (tests/check_correctness.py:22).  The saved output
is exact attention over the selection (kernels.py:120-247); the union output
merges every predicted state with the misses (gqa.py:62-104, 384-413).
"""
import numpy as np
import pytest
import torch

from oracle import stk_oracle as O
from tests import cases as C

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module", autouse=True)
def _gpu():
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    from strict_topk import _lib
    _lib.lib()


def _small(q, k, topk, sp, lo):
    from strict_topk import _lib
    hkv, n, b, d = k.shape
    return _lib.lib().stk_step_small_supported(_lib.dtype_code(q), q.shape[0], hkv, n, b, d,
                                               topk, sp, 0, _lib.bounds_code(lo, q)) == 1


def _check(res, host, p_host, topk, union, what):
    q, k, v, lo, hi = host
    qn, kn, vn = (C.f64(t) for t in (q, k, v))
    n = k.shape[1]
    ids = O.select_blocks(qn, lo.double().numpy(), hi.double().numpy(), topk)
    assert res.selected.cpu().numpy().tolist() == ids.tolist(), what
    pv = p_host.numpy().astype(np.int64)
    pv = np.where((pv >= 0) & (pv < n), pv, -1)
    ref = O.block_states(qn, kn, vn, pv)
    m, l, u = (x.cpu().double().numpy() for x in (res.state.m, res.state.l, res.state.u))
    np.testing.assert_allclose(m, ref.m, rtol=1e-5, atol=1e-5, err_msg=str(what))
    np.testing.assert_allclose(l, ref.l, rtol=1e-4, atol=1e-6, err_msg=str(what))
    np.testing.assert_allclose(u, ref.u, rtol=1e-4, atol=1e-4, err_msg=str(what))
    if union:
        expected = O.gqa_repair(qn, kn, vn, ids, pv, ref, union=True)
    else:
        expected = O.attention(qn, kn, vn, ids)
    met = C.error_metrics(C.f64(res.output), expected)
    assert met["passed"], (what, met)


@pytest.mark.parametrize("hq,hkv,n,d,topk,overlap,dtype,bounds,union", [
    (4, 4, 64, 64, 8, 0.75, torch.float16, "fp32", False),   # c1 as the benchmark runs it
    (4, 4, 64, 64, 8, 0.75, torch.float16, "k", False),      # c1, 16-bit bounds
    (4, 4, 64, 64, 8, 0.75, torch.float16, "fp32", True),    # c1, repair_union
    (4, 4, 64, 64, 8, 1.0, torch.float16, "k", False),       # every selected block predicted
    (4, 4, 64, 64, 8, 0.0, torch.float16, "k", False),       # no hit: eight misses per head
    (8, 2, 50, 128, 8, 0.5, torch.bfloat16, "k", False),     # G = 4, D = 128, N not 64
    (8, 2, 50, 128, 8, 0.5, torch.bfloat16, "fp32", True),
    (6, 3, 17, 64, 3, 0.6, torch.bfloat16, "k", False),      # small K
    (4, 2, 1, 128, 1, 1.0, torch.bfloat16, "k", False),      # one block
    (4, 4, 8, 64, 8, 1.0, torch.float16, "k", False),        # K = N
    (4, 4, 128, 64, 8, 0.75, torch.float16, "fp32", False),  # two blocks per lane of the rank
    (8, 2, 100, 128, 8, 0.5, torch.bfloat16, "k", True),     # N between 64 and 128, union
    (6, 3, 65, 128, 5, 0.0, torch.bfloat16, "fp32", False),  # one block past 64, every block missed
    (4, 4, 128, 64, 16, 0.75, torch.float16, "fp32", False), # sixteen rows: two slots per wave
    (8, 2, 100, 128, 12, 0.5, torch.bfloat16, "k", True),    # twelve rows, union
    (4, 4, 64, 64, 16, 0.0, torch.float16, "k", False),      # sixteen misses: two rounds of halves
    (4, 2, 40, 128, 9, 0.6, torch.bfloat16, "fp32", False),  # nine rows
])
def test_small_step(hq, hkv, n, d, topk, overlap, dtype, bounds, union):
    from stk_harness.configs import make_qkv, perturb
    from strict_topk import step
    q, k, v, lo, hi = make_qkv(hq, hkv, d, 32, n, dtype, True, 20261300 + n + hq + topk)
    ids = O.select_blocks(C.f64(q), lo.numpy(), hi.numpy(), topk)
    p = perturb(torch.from_numpy(ids), n, topk, overlap, n + topk)
    if bounds == "k":
        lo, hi = lo.to(dtype), hi.to(dtype)
    qd, kd, vd, lod, hid, pd = (t.cuda() for t in (q, k, v, lo, hi, p))
    assert _small(qd, kd, topk, p.shape[1], lod)
    res = step.speculative_step(qd, kd, vd, lod, hid, pd, topk, union=union)
    torch.cuda.synchronize()
    _check(res, (q, k, v, lo, hi), p, topk, union, (hq, n, d, topk, overlap, bounds, union))


def test_small_step_predictions_with_invalid_and_repeated_ids():
    """Predicted rows holding -1, an ID past N and a repeated block: a
    repeat's state is computed for every slot holding it; saved repair merges
    the highest slot's state once; union merges every slot."""
    from stk_harness.configs import make_qkv
    from strict_topk import step
    hq, hkv, n, d, topk = 4, 2, 40, 128, 6
    q, k, v, lo, hi = make_qkv(hq, hkv, d, 32, n, torch.bfloat16, True, 77)
    ids = O.select_blocks(C.f64(q), lo.numpy(), hi.numpy(), topk)
    p = torch.from_numpy(ids[:, :5].copy()).to(torch.int32)
    p = torch.cat([p[:, :1], torch.full((hq, 1), -1, dtype=torch.int32),
                   torch.full((hq, 1), n + 3, dtype=torch.int32), p[:, 1:3], p[:, :1]], 1)
    lo16, hi16 = lo.to(torch.bfloat16), hi.to(torch.bfloat16)
    qd, kd, vd, lod, hid, pd = (t.cuda() for t in (q, k, v, lo16, hi16, p))
    assert _small(qd, kd, topk, p.shape[1], lod)
    for union in (False, True):
        res = step.speculative_step(qd, kd, vd, lod, hid, pd, topk, union=union)
        torch.cuda.synchronize()
        _check(res, (q, k, v, lo16, hi16), p, topk, union, ("repeats", union))


def test_small_step_not_covered():
    """Past 128 blocks, 16 selected or 16 predicted rows, other block sizes and
    head dims, the step takes the other paths."""
    from strict_topk import _lib
    L = _lib.lib()
    assert L.stk_step_small_supported(1, 4, 4, 64, 32, 64, 8, 8, 0, 0) == 1
    assert L.stk_step_small_supported(1, 4, 4, 128, 32, 64, 8, 8, 0, 0) == 1
    assert L.stk_step_small_supported(1, 4, 4, 129, 32, 64, 8, 8, 0, 0) == 0  # N
    assert L.stk_step_small_supported(1, 4, 4, 64, 32, 64, 16, 16, 0, 0) == 1
    assert L.stk_step_small_supported(1, 4, 4, 64, 32, 64, 17, 8, 0, 0) == 0  # TOPK
    assert L.stk_step_small_supported(1, 4, 4, 64, 32, 64, 8, 17, 0, 0) == 0  # SP
    assert L.stk_step_small_supported(1, 4, 4, 64, 16, 64, 8, 8, 0, 0) == 0   # B
    assert L.stk_step_small_supported(2, 4, 4, 64, 32, 256, 8, 8, 0, 2) == 0  # D
    assert L.stk_step_small_supported(0, 4, 4, 64, 32, 64, 8, 8, 0, 0) == 0   # fp32 K/V
    assert L.stk_step_small_supported(1, 4, 4, 64, 32, 64, 8, 8, 1, 0) == 0   # int64 IDs


@pytest.mark.parametrize("n,topk", [(64, 8), (120, 16)])   # eight rows; two keys per lane, sixteen rows
def test_small_step_in_a_graph(n, topk):
    """Captured in a graph and replayed while the query changes in place:
    every replay equals the eager step on the same inputs."""
    from stk_harness.configs import make_qkv, perturb
    from strict_topk import step
    q, k, v, lo, hi = make_qkv(4, 4, 64, 32, n, torch.float16, True, 5)
    ids = O.select_blocks(C.f64(q), lo.numpy(), hi.numpy(), topk)
    p = perturb(torch.from_numpy(ids), n, topk, 0.75, 5)
    qd, kd, vd, lod, hid, pd = (t.cuda() for t in (q, k, v, lo, hi, p))
    assert _small(qd, kd, topk, topk, lod)
    step.speculative_step(qd, kd, vd, lod, hid, pd, topk)
    g = torch.cuda.CUDAGraph()
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        with torch.cuda.graph(g, stream=s):
            out = step.speculative_step(qd, kd, vd, lod, hid, pd, topk)
    torch.cuda.current_stream().wait_stream(s)
    gen = torch.Generator().manual_seed(3)
    for _ in range(3):
        qd.copy_(torch.randn((4, 64), generator=gen).to(torch.float16))
        g.replay()
        torch.cuda.synchronize()
        eager = step.speculative_step(qd, kd, vd, lod, hid, pd, topk)
        torch.cuda.synchronize()
        assert torch.equal(out.selected, eager.selected)
        assert torch.equal(out.output, eager.output)
        assert torch.equal(out.state.u, eager.state.u)


@pytest.mark.parametrize("n", [40, 100, 130])   # one workgroup per head (up to 128 blocks); the flag grid
def test_step_nonfinite_bounds(n):
    """-inf / +inf bounds and NaN scores through the fused step (its own FP64
    scores and top-K): the selected IDs equal the oracle's, NaN ranking below
    -inf and ties toward the lower index."""
    from stk_harness.configs import make_qkv
    from strict_topk import step
    hq, hkv, d, topk = 4, 2, 64, 8
    q, k, v, lo, hi = make_qkv(hq, hkv, d, 32, n, torch.float16, True, 4242 + n)
    lo, hi = lo.clone(), hi.clone()
    lo[0, 3] = float("-inf")
    hi[1, 5] = float("inf")
    lo[1, 7, 0] = float("nan")
    hi[1, 7, 0] = float("nan")
    lo[0, 9:12] = lo[0, 12]          # exact ties
    hi[0, 9:12] = hi[0, 12]
    ref = O.select_blocks(C.f64(q), lo.double().numpy(), hi.double().numpy(), topk)
    p = torch.from_numpy(ref[:, :topk].copy()).to(torch.int32)
    qd, kd, vd, lod, hid, pd = (t.cuda() for t in (q, k, v, lo, hi, p))
    assert _small(qd, kd, topk, topk, lod) == (n <= 128)
    res = step.speculative_step(qd, kd, vd, lod, hid, pd, topk)
    torch.cuda.synchronize()
    assert res.selected.cpu().numpy().tolist() == ref.tolist()


@pytest.mark.parametrize("n,topk,sp,union", [(64, 6, 12, False), (100, 14, 5, True),
                                            (128, 16, 16, True), (30, 3, 16, False)])
def test_small_step_rows_differ(n, topk, sp, union):
    """Predicted rows of a width other than K (SP above and below 8, both
    row counts of the kernel): IDs, states and output against the oracle."""
    from stk_harness.configs import make_qkv, perturb
    from strict_topk import step
    hq, hkv, d = 8, 4, 64
    q, k, v, lo, hi = make_qkv(hq, hkv, d, 32, n, torch.bfloat16, True, 31 + n + sp)
    ids = O.select_blocks(C.f64(q), lo.numpy(), hi.numpy(), topk)
    p = perturb(torch.from_numpy(ids), n, sp, 0.6, n + sp)
    assert p.shape == (hq, sp)
    qd, kd, vd, lod, hid, pd = (t.cuda() for t in (q, k, v, lo, hi, p))
    assert _small(qd, kd, topk, sp, lod)
    res = step.speculative_step(qd, kd, vd, lod, hid, pd, topk, union=union)
    torch.cuda.synchronize()
    _check(res, (q, k, v, lo, hi), p, topk, union, (n, topk, sp, union))
