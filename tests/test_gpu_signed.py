"""The drop-in signed repair with inline fallback on its one-launch path.

signed_fused.repair_signed_fused over saved and hybrid predictions on bf16 /
fp16 with D in {64, 128, 256} runs as one kernel per call (schedule,
corrections and guarded merge; the wrong blocks' corrections from the
prediction's block states, the misses from their tiles).  Each case builds
the prediction on the GPU with kernels.speculate and gives the oracle the
same prediction (as FP64), so the repair itself is pinned: job counts, the
job queue (misses in selected-slot order, then the wrong low blocks in
predicted-slot order, reference strict_topk/signed_repair.py:18-82), guard
flags and the budget fields exact, outputs within |err| <= 3e-4 + 3e-4 |ref|
(tests/check_correctness.py:22).  The shapes cover both per-slot paths
(SP <= 64 and up to 256), whole-block and multi-chunk tiles, int64 IDs,
block IDs past the LDS maps' range, the skip budget, the strict fallback
and the cancellation guard.
"""
import numpy as np
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


def _ids(h, n, sa, sp, overlap, idtype, gen):
    """Per head: A of sa distinct blocks, P of sp distinct blocks sharing
    round(overlap * min(sa, sp)) of them, both in shuffled order."""
    share = int(round(overlap * min(sa, sp)))
    a_rows, p_rows = [], []
    for _ in range(h):
        perm = torch.randperm(n, generator=gen)
        a = perm[:sa]
        p = torch.cat((a[:share], perm[sa:sa + sp - share]))
        a_rows.append(a[torch.randperm(sa, generator=gen)])
        p_rows.append(p[torch.randperm(sp, generator=gen)])
    return torch.stack(a_rows).to(idtype), torch.stack(p_rows).to(idtype)


def _oracle_pred(pred):
    """The GPU prediction as the oracle's FP64 container."""
    f = lambda t: None if t is None else t.cpu().double().numpy()
    st = O.State(f(pred.state.m), f(pred.state.l), f(pred.state.u))
    low = None if pred.low is None else O.State(f(pred.low.m), f(pred.low.l), f(pred.low.u))
    high = None if pred.high is None else pred.high.cpu().numpy().astype(bool)
    return O.Prediction(st, pred.mode, high, low, low_abs=f(pred.low_abs),
                        mass_m=f(pred.mass_m), mass_l=f(pred.mass_l))


def _call_with_queue(q, k, v, a, p, pred, min_rem, tol, eps):
    """stk_repair_signed through the C ABI with the queue kept."""
    from strict_topk import _lib
    from strict_topk.kernels import _args, prediction_args
    h, d = q.shape
    sa, sp = a.shape[1], p.shape[1]
    hybrid = pred.mode == "hybrid"
    cap = sa + sp if hybrid else sa
    pa = prediction_args(pred, q)
    queue = torch.full((h, cap), -7, device=DEV, dtype=torch.promote_types(a.dtype, p.dtype))
    pos = torch.empty((h,), device=DEV, dtype=torch.int32)
    total = torch.empty_like(pos)
    out = torch.empty((h, d), device=DEV, dtype=torch.float32)
    bad = torch.empty((h,), device=DEV, dtype=torch.bool)
    rem = torch.empty((h,), device=DEV, dtype=torch.float32)
    approx = torch.empty_like(bad) if eps > 0 else None
    extra = torch.empty_like(rem) if eps > 0 else None
    ws = _lib.workspace(_lib.size("stk_signed_workspace_bytes", h, sa, sp, pa[1], d, pa[0]),
                        q.device)
    _lib.call("stk_repair_signed", *_args(q, k, v), _lib.ptr(a), _lib.id_code(a), sa,
              _lib.ptr(p), _lib.id_code(p), sp, *pa, _lib.ptr(pred.mass_m), _lib.ptr(pred.mass_l),
              float(min_rem), float(tol), float(eps), 1, _lib.ptr(queue), _lib.id_code(queue),
              _lib.ptr(pos), _lib.ptr(total), _lib.ptr(out), _lib.ptr(bad), _lib.ptr(rem),
              _lib.ptr(approx), _lib.ptr(extra), _lib.ptr(ws), ws.numel(), _lib.stream(q.device))
    return queue, pos, total, out, bad, rem, approx, extra


# hq, hkv, n, b, d, sa, sp, overlap, dtype, mode, tau, eps, min_rem, tol, idtype
CASES = [
    (8, 4, 300, 32, 128, 64, 64, 0.5, torch.bfloat16, "hybrid", 0.2, 0.0, 1e-3, 1e-5,
     torch.int32),                                                          # c5's widths
    (8, 4, 300, 32, 128, 64, 64, 0.75, torch.bfloat16, "hybrid", 0.2, 0.01, 1e-3, 1e-5,
     torch.int32),                                                          # budget
    (8, 4, 300, 32, 128, 64, 64, 0.5, torch.bfloat16, "hybrid", 0.05, 1.0, 1e-3, 1e-5,
     torch.int32),                                                          # skip every head
    (8, 4, 300, 32, 128, 64, 64, 0.5, torch.bfloat16, "hybrid", 0.05, 0.0, 1.0, 1e-5,
     torch.int32),                                                          # strict fallback
    (8, 4, 300, 64, 128, 32, 32, 0.5, torch.bfloat16, "hybrid", 0.05, 0.01, 1e-3, 2.0,
     torch.int32),                                                          # cancel, 2 chunks
    (4, 4, 200, 16, 64, 24, 100, 0.6, torch.float16, "hybrid", 0.02, 0.0, 1e-3, 1e-5,
     torch.int64),                                                          # SP > 64, int64
    (4, 2, 120, 32, 256, 40, 40, 0.5, torch.float16, "saved", 0.1, 0.0, 1e-3, 1e-5,
     torch.int32),                                                          # D = 256, saved
    (4, 1, 9000, 16, 64, 48, 48, 0.5, torch.bfloat16, "hybrid", 0.1, 0.0, 1e-3, 1e-5,
     torch.int64),                                                          # IDs past the maps
    (8, 8, 400, 32, 128, 256, 256, 0.9, torch.bfloat16, "hybrid", 0.01, 0.0, 1e-3, 1e-5,
     torch.int32),                                                          # widest rows
]


@pytest.mark.parametrize("hq,hkv,n,b,d,sa,sp,overlap,dtype,mode,tau,eps,min_rem,tol,idtype",
                         CASES)
def test_signed_fused_one_launch(hq, hkv, n, b, d, sa, sp, overlap, dtype, mode, tau, eps,
                                 min_rem, tol, idtype):
    from strict_topk.kernels import speculate
    from strict_topk.signed_fused import repair_signed_fused
    gen = torch.Generator().manual_seed(hq * 1000 + n + sp)
    q = torch.randn((hq, d), generator=gen).to(dtype)
    k = (torch.randn((hkv, n, b, d), generator=gen) * 1.5).to(dtype)
    v = torch.randn((hkv, n, b, d), generator=gen).to(dtype)
    a, p = _ids(hq, n, sa, sp, overlap, idtype, gen)
    qd, kd, vd, ad, pd = (t.to(DEV) for t in (q, k, v, a, p))
    pred = speculate(qd, kd, vd, pd, mode=mode, mass_threshold=tau, keep_mass=True)
    opred = _oracle_pred(pred)
    qn, kn, vn = (C.f64(t) for t in (q, k, v))
    ref = O.repair_signed_fused(qn, kn, vn, a.numpy(), p.numpy(), opred, min_rem, tol, eps)
    res = repair_signed_fused(qd, kd, vd, ad, pd, pred, min_rem, tol, eps)
    what = (mode, n, sp, eps, min_rem, tol)
    assert res.positive_jobs.cpu().numpy().tolist() == ref.positive_jobs.tolist(), what
    assert res.total_jobs.cpu().numpy().tolist() == ref.total_jobs.tolist(), what
    assert res.fallback.cpu().numpy().tolist() == ref.fallback.tolist(), what
    np.testing.assert_allclose(res.remaining.cpu().double().numpy(), ref.remaining, rtol=1e-4,
                               atol=1e-6)
    if eps > 0:
        assert res.approximate_heads.cpu().numpy().tolist() == ref.approximate_heads.tolist()
        np.testing.assert_allclose(res.extra_mass_bound.cpu().double().numpy(),
                                   ref.extra_mass_bound, rtol=1e-4, atol=1e-7)
    m = C.error_metrics(C.f64(res.output), ref.output)
    assert m["passed"], (what, m)
    if min_rem == 1.0:
        assert res.fallback.any()
    # the job queue through the C ABI
    sch = O.schedule(a.numpy(), p.numpy(), opred, eps)
    queue, pos, total, out, *_ = _call_with_queue(qd, kd, vd, ad, pd, pred, min_rem, tol, eps)
    torch.cuda.synchronize()
    qh = queue.cpu().numpy()
    for h in range(hq):
        assert qh[h, :int(sch.total[h])].tolist() == [int(x) for x in sch.queue[h]], (what, h)
    assert torch.equal(out, res.output)
