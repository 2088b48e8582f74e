"""GPU parity at the benchmark configurations' real shapes.

Every input is drawn from seeded CPU generators (identical on every machine)
and moved to the device; the FP64 oracle checks the GPU results on the same
values.  Bars: block IDs bit-exact; outputs within the reference tolerance
|err| <= 3e-4 + 3e-4 |ref| (tests/check_correctness.py:22); guard flags and
job counts exact.

  c3  the drop-in two-stream composition of the reference's overlap_run
      (benchmarks/run_benchmark.py:99-118): gqa.select_blocks ||
      gqa.partials(P), joined, then gqa_light.repair_saved_auto, eager and
      replayed from a captured graph with the inputs changed in place.
  c4  Hq=48, Hkv=4, D=128, B=4, N=8192: the shared top-2048 of the QSA
      indexer (benchmarks/selector_window.py:76-84), P at 80 % overlap,
      gqa_hierarchical.partials -> repair_saved_shared
      (strict_topk/gqa_hierarchical.py:115-144) and exact, also through
      overlap_run.
  c5  16 requests, contexts 32 * U{256..4096} tokens, overlap U[0.5, 1],
      in one page pool: paged.speculative_signed_step with
      max_extra_mass 0.01 and 0 against the oracle's select ||
      speculate('hybrid', 0.2, keep_mass) -> repair_signed_fused
      (strict_topk/signed_fused.py:148-193) per request.
"""
import functools

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
    _lib.lib()   # fail loudly if the HIP library is missing


def check(out, expected, what=""):
    m = C.error_metrics(C.f64(out), expected)
    assert m["passed"], (what, m)


def restrict(k, v, *id_rows):
    """K/V reduced to the blocks some ID row names, and the rows renumbered
    into it (an increasing map, so ascending rows stay ascending): the oracle
    then converts megabytes to FP64 instead of gigabytes."""
    need = np.unique(np.concatenate([np.asarray(r, np.int64).ravel() for r in id_rows]))
    remap = np.full(k.shape[1], -1, np.int64)
    remap[need] = np.arange(len(need))
    idx = torch.from_numpy(need)
    return (C.f64(k[:, idx]), C.f64(v[:, idx]),
            *[remap[np.asarray(r, np.int64)] for r in id_rows])


# ------------------------------------------------------------------ c3
@pytest.mark.parametrize("overlap", [0.9, 0.75])
def test_c3_overlap_run_composition(overlap):
    from stk_harness.configs import CONFIGS, make_qkv, perturb
    from stk_harness.timing import overlap_run
    from strict_topk import gqa, gqa_light
    c = CONFIGS["c3"]
    q, k, v, lo, hi = make_qkv(c.hq, c.hkv, c.dim, c.block, c.blocks, c.dtype, c.hot, 20261103)
    qn = C.f64(q)
    ref_ids = O.select_blocks(qn, lo.numpy(), hi.numpy(), c.topk)
    p = perturb(torch.from_numpy(ref_ids), c.blocks, c.sp, overlap, 20261103)
    kn, vn, a_r = restrict(k, v, ref_ids)
    expected = O.attention(qn, kn, vn, a_r)
    qd, kd, vd, lod, hid, pd = (t.to(DEV) for t in (q, k, v, lo, hi, p))
    ss, ps = torch.cuda.Stream(), torch.cuda.Stream()

    def run(emf):
        return overlap_run(lambda: gqa.select_blocks(qd, lod, hid, c.topk),
                           lambda: gqa.partials(qd, kd, vd, pd),
                           lambda a, st: (a, gqa_light.repair_saved_auto(qd, kd, vd, a, pd, st,
                                                                         emf)), ss, ps)

    # 0.03 * 64 <= 2 takes the light repair, 0.25 the split saved repair
    for emf in (0.03, 0.25):
        sel, out = run(emf)
        torch.cuda.synchronize()
        assert sel.cpu().numpy().tolist() == ref_ids.tolist()
        check(out, expected, ("c3 composition", overlap, emf))
    # the same composition replayed from a captured graph while the query
    # changes in place between replays (with eager work in between)
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        for _ in range(2):
            run(0.03)
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        gsel, gout = run(0.03)
    q0 = qd.clone()
    for scale in (1.0, -1.0, 0.5):
        qd.copy_(q0 * scale)
        g.replay()
        torch.cuda.synchronize()
        qs = qd.cpu()
        ids_s = O.select_blocks(C.f64(qs), lo.numpy(), hi.numpy(), c.topk)
        assert gsel.cpu().numpy().tolist() == ids_s.tolist(), scale
        ks, vs, a_s = restrict(k, v, ids_s)
        check(gout, O.attention(C.f64(qs), ks, vs, a_s), ("c3 graph", overlap, scale))
        torch.cuda.synchronize()
        eager_sel, _ = run(0.25)   # eager work between replays
        torch.cuda.synchronize()
        assert torch.equal(eager_sel, gsel)


@pytest.mark.parametrize("overlap,seed", [
    (1.0, 20261103), (1.0, 20261104), (1.0, 20261105),
    (0.9, 20261104), (0.9, 20261105), (0.75, 20261104), (0.75, 20261105),
])
def test_c3_step_and_composition(overlap, seed):
    """c3 at every hit rate and seed of the sweep: the fused step (one launch)
    and the drop-in composition (gqa_light.repair_saved_auto behind
    overlap_run, with the bench's expected-miss fraction 1 - overlap) against
    the oracle."""
    from stk_harness.configs import CONFIGS, make_qkv, perturb
    from stk_harness.timing import overlap_run
    from strict_topk import gqa, gqa_light, step
    c = CONFIGS["c3"]
    q, k, v, lo, hi = make_qkv(c.hq, c.hkv, c.dim, c.block, c.blocks, c.dtype, c.hot, seed)
    qn = C.f64(q)
    ref_ids = O.select_blocks(qn, lo.numpy(), hi.numpy(), c.topk)
    p = perturb(torch.from_numpy(ref_ids), c.blocks, c.sp, overlap, seed)
    kn, vn, a_r = restrict(k, v, ref_ids)
    expected = O.attention(qn, kn, vn, a_r)
    qd, kd, vd, lod, hid, pd = (t.to(DEV) for t in (q, k, v, lo, hi, p))
    res = step.speculative_step(qd, kd, vd, lod.to(c.dtype), hid.to(c.dtype), pd, c.topk)
    ss, ps = torch.cuda.Stream(), torch.cuda.Stream()
    sel, out = overlap_run(lambda: gqa.select_blocks(qd, lod, hid, c.topk),
                           lambda: gqa.partials(qd, kd, vd, pd),
                           lambda a, st: (a, gqa_light.repair_saved_auto(
                               qd, kd, vd, a, pd, st, 1.0 - overlap)), ss, ps)
    torch.cuda.synchronize()
    assert res.selected.cpu().numpy().tolist() == ref_ids.tolist()
    assert sel.cpu().numpy().tolist() == ref_ids.tolist()
    check(res.output, expected, ("c3 step", overlap, seed))
    check(out, expected, ("c3 composition", overlap, seed))


# ------------------------------------------------------------------ c2
def test_c2_repair_saved():
    """c2's own strategy at its shape: gqa.select_blocks || gqa.partials, then
    gqa.repair_saved (strict_topk/gqa.py:164-188), eagerly and through
    overlap_run."""
    from stk_harness.configs import CONFIGS, make_qkv, perturb
    from stk_harness.timing import overlap_run
    from strict_topk import gqa
    c = CONFIGS["c2"]
    q, k, v, lo, hi = make_qkv(c.hq, c.hkv, c.dim, c.block, c.blocks, c.dtype, c.hot, 20261103)
    qn = C.f64(q)
    ref_ids = O.select_blocks(qn, lo.numpy(), hi.numpy(), c.topk)
    p = perturb(torch.from_numpy(ref_ids), c.blocks, c.sp, 0.9, 20261103)
    kn, vn, a_r = restrict(k, v, ref_ids)
    expected = O.attention(qn, kn, vn, a_r)
    qd, kd, vd, lod, hid, pd = (t.to(DEV) for t in (q, k, v, lo, hi, p))
    sel = gqa.select_blocks(qd, lod, hid, c.topk)
    st = gqa.partials(qd, kd, vd, pd)
    out = gqa.repair_saved(qd, kd, vd, sel, pd, st)
    ss, ps = torch.cuda.Stream(), torch.cuda.Stream()
    out2 = overlap_run(lambda: gqa.select_blocks(qd, lod, hid, c.topk),
                       lambda: gqa.partials(qd, kd, vd, pd),
                       lambda a, s: gqa.repair_saved(qd, kd, vd, a, pd, s), ss, ps)
    torch.cuda.synchronize()
    assert sel.cpu().numpy().tolist() == ref_ids.tolist()
    check(out, expected, "c2 repair_saved")
    check(out2, expected, "c2 repair_saved (overlap_run)")


# ------------------------------------------------------------------ c4
def test_c4_real_shape():
    from stk_harness.configs import CONFIGS, make_qkv, perturb
    from stk_harness.timing import overlap_run
    from strict_topk import gqa_hierarchical as hier, indexer
    c = CONFIGS["c4"]
    seed = 20261103
    q, k, v, _, _ = make_qkv(c.hq, c.hkv, c.dim, c.block, c.blocks, c.dtype, c.hot, seed)
    gen = torch.Generator().manual_seed(seed + 4)
    iq = torch.randn((4, 128), generator=gen).to(c.dtype)
    ik = torch.randn((c.blocks, 128), generator=gen).to(c.dtype)
    ref_sel = O.indexer_select(C.f64(iq), C.f64(ik), c.topk, c.hq)
    prow = perturb(torch.from_numpy(ref_sel[:1]), c.blocks, c.sp, c.overlaps[0], seed)
    p = prow.expand(c.hq, -1).contiguous()
    assert len(np.intersect1d(prow[0].numpy(), ref_sel[0])) == round(0.8 * c.topk)
    qn = C.f64(q)
    kn, vn, a_r = restrict(k, v, ref_sel)
    expected = O.attention(qn, kn, vn, a_r)
    qd, kd, vd, pd, iqd, ikd = (t.to(DEV) for t in (q, k, v, p, iq, ik))
    sel = indexer.select_shared(iqd, ikd, c.topk, c.hq)
    assert sel.cpu().numpy().tolist() == ref_sel.tolist()
    st = hier.partials(qd, kd, vd, pd)
    check(hier.repair_saved_shared(qd, kd, vd, sel, pd, st), expected, "c4 repair_saved_shared")
    check(hier.repair_saved(qd, kd, vd, sel, pd, st), expected, "c4 repair_saved")
    check(hier.exact(qd, kd, vd, sel), expected, "c4 exact")
    ss, ps = torch.cuda.Stream(), torch.cuda.Stream()
    out = overlap_run(lambda: indexer.select_shared(iqd, ikd, c.topk, c.hq),
                      lambda: hier.partials(qd, kd, vd, pd),
                      lambda a, s: hier.repair_saved_shared(qd, kd, vd, a, pd, s), ss, ps)
    torch.cuda.synchronize()
    check(out, expected, "c4 two-stream composition")


# ------------------------------------------------------------------ c5
@functools.lru_cache(maxsize=1)
def _c5_requests(seed):
    from stk_harness.configs import C5, make_qkv, perturb
    rng = np.random.default_rng(seed)
    blocks = rng.integers(C5["min_blocks"], C5["max_blocks"] + 1, size=C5["requests"])
    overlaps = rng.uniform(C5["min_overlap"], C5["max_overlap"], size=C5["requests"])
    reqs = []
    for r in range(C5["requests"]):
        n = int(blocks[r])
        q, k, v, lo, hi = make_qkv(C5["hq"], C5["hkv"], C5["dim"], C5["block"], n, C5["dtype"],
                                   True, seed + 101 * r)
        ids = O.select_blocks(C.f64(q), lo.numpy(), hi.numpy(), C5["topk"])
        p = perturb(torch.from_numpy(ids), n, C5["topk"], float(overlaps[r]), seed + r)
        reqs.append(dict(q=q, k=k, v=v, lo=lo, hi=hi, ids=ids, p=p, n=n))
        print(f"c5 request {r}: {n} blocks, overlap {overlaps[r]:.3f}", flush=True)
    return reqs


def test_c5_real_batch():
    from stk_harness.configs import C5
    from strict_topk import paged
    reqs = _c5_requests(20261103)
    kv = paged.pack([(r["k"].to(DEV), r["v"].to(DEV)) for r in reqs])
    qb = torch.stack([r["q"] for r in reqs]).to(DEV)
    pb = torch.stack([r["p"] for r in reqs]).to(DEV)
    # the oracle per request over the blocks P u A only
    refs = []
    for r in reqs:
        kn, vn, a_r, p_r = restrict(r["k"], r["v"], r["ids"], r["p"].numpy())
        qn = C.f64(r["q"])
        pred = O.speculate(qn, kn, vn, p_r, "hybrid", 0.2, keep_mass=True)
        refs.append((qn, kn, vn, a_r, p_r, pred))
    for eps in (0.01, 0.0):
        res = paged.speculative_signed_step(qb, kv, pb, C5["topk"], "hybrid", 0.2,
                                            max_extra_mass=eps)
        torch.cuda.synchronize()
        out = res.result
        for i, (r, (qn, kn, vn, a_r, p_r, pred)) in enumerate(zip(reqs, refs)):
            assert res.selected[i].cpu().numpy().tolist() == r["ids"].tolist(), i
            ref = O.repair_signed_fused(qn, kn, vn, a_r, p_r, pred, max_extra_mass=eps)
            assert out.fallback[i].cpu().numpy().tolist() == ref.fallback.tolist(), (eps, i)
            assert out.positive_jobs[i].cpu().numpy().tolist() == ref.positive_jobs.tolist()
            assert out.total_jobs[i].cpu().numpy().tolist() == ref.total_jobs.tolist()
            if eps > 0:
                assert out.approximate_heads[i].cpu().numpy().tolist() == \
                    ref.approximate_heads.tolist(), i
            check(out.output[i], ref.output, ("c5 paged signed", eps, i, r["n"]))
            if eps == 0:
                check(out.output[i], O.attention(qn, kn, vn, a_r), ("c5 strict", i))


def test_c5_dropin_signed_composition():
    """The reference API's own c5 composition on three of the requests
    (smallest, median and largest context): overlap_run(gqa.select_blocks ||
    kernels.speculate('hybrid', 0.2, keep_mass=True)), then
    signed_fused.repair_signed_fused (strict_topk/signed_fused.py:148-193)
    with max_extra_mass 0.01 and 0, against the oracle."""
    from stk_harness.configs import C5
    from stk_harness.timing import overlap_run
    from strict_topk import gqa, kernels, signed_fused
    reqs = _c5_requests(20261103)
    order = sorted(range(len(reqs)), key=lambda i: reqs[i]["n"])
    ss, ps = torch.cuda.Stream(), torch.cuda.Stream()
    for i in (order[0], order[len(order) // 2], order[-1]):
        r = reqs[i]
        qd, kd, vd, lod, hid, pd = (t.to(DEV) for t in (r["q"], r["k"], r["v"], r["lo"],
                                                        r["hi"], r["p"]))
        kn, vn, a_r, p_r = restrict(r["k"], r["v"], r["ids"], r["p"].numpy())
        qn = C.f64(r["q"])
        pred_ref = O.speculate(qn, kn, vn, p_r, "hybrid", 0.2, keep_mass=True)
        sel, pred = overlap_run(lambda: gqa.select_blocks(qd, lod, hid, C5["topk"]),
                                lambda: kernels.speculate(qd, kd, vd, pd, "hybrid", 0.2,
                                                          keep_mass=True),
                                lambda a, st: (a, st), ss, ps)
        assert sel.cpu().numpy().tolist() == r["ids"].tolist(), i
        for eps in (0.01, 0.0):
            out = signed_fused.repair_signed_fused(qd, kd, vd, sel, pd, pred, max_extra_mass=eps)
            torch.cuda.synchronize()
            ref = O.repair_signed_fused(qn, kn, vn, a_r, p_r, pred_ref, max_extra_mass=eps)
            assert out.fallback.cpu().numpy().tolist() == ref.fallback.tolist(), (eps, i)
            assert out.positive_jobs.cpu().numpy().tolist() == ref.positive_jobs.tolist()
            assert out.total_jobs.cpu().numpy().tolist() == ref.total_jobs.tolist()
            if eps > 0:
                assert out.approximate_heads.cpu().numpy().tolist() == \
                    ref.approximate_heads.tolist(), i
            check(out.output, ref.output, ("c5 drop-in signed", eps, i, r["n"]))
            if eps == 0:
                check(out.output, O.attention(qn, kn, vn, a_r), ("c5 drop-in strict", i))
