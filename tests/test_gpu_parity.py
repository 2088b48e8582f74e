"""GPU parity: the HIP path against the FP64 oracle on identical inputs.

Bars: block IDs bit-exact (ties toward the lower index, canonical order);
FP32 scores bit-exact to float32(oracle FP64 score); outputs within the
reference tolerance |err| <= 3e-4 + 3e-4 |ref| (tests/check_correctness.py:22);
discrete flags exact on the reference's known-answer inputs.
"""
import math

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


def dev(*ts):
    return [t.to(DEV) for t in ts]


def np_(*ts):
    return [C.f64(t) if t.is_floating_point() else C.ids_np(t) for t in ts]


def check(out, expected, what=""):
    m = C.error_metrics(C.f64(out), expected)
    assert m["passed"], (what, m)


# --------------------------------------------------------------- selection
def test_selector_scores_and_ids_bit_exact():
    from strict_topk.selector import block_scores, select_blocks
    gen = torch.Generator().manual_seed(C.SEED)
    q = torch.randn((3, 70), generator=gen).half()
    keys = torch.randn((3, 37, 7, 70), generator=gen).half()
    lo, hi = keys.amin(dim=2).float(), keys.amax(dim=2).float()
    q[0].zero_()
    ref = O.bound_scores(*np_(q, lo, hi))
    qd, lod, hid = dev(q, lo, hi)
    scores = block_scores(qd, lod, hid)
    assert scores.dtype == torch.float32 and scores.shape == (3, 37)
    assert np.array_equal(scores.cpu().numpy(), ref.astype(np.float32))
    for topk in (1, 11, 37):
        ids = select_blocks(qd, lod, hid, topk)
        assert ids.shape == (3, topk) and ids.dtype == torch.int32 and ids.is_contiguous()
        assert ids.cpu().numpy().tolist() == O.topk_ids(ref, topk).tolist()
    assert select_blocks(qd, lod, hid, 11)[0].cpu().tolist() == list(range(11))


def test_gqa_select_ids_bit_exact():
    from strict_topk import gqa
    for hq, hkv, n, b, d, topk in [(6, 2, 23, 7, 13, 5), (16, 8, 512, 32, 128, 64),
                                   (48, 4, 300, 4, 128, 200), (4, 4, 64, 32, 64, 8),
                                   (2, 1, 5000, 2, 32, 700)]:
        gen = torch.Generator().manual_seed(hq * 1000 + n)
        q = torch.randn((hq, d), generator=gen).bfloat16()
        k = torch.randn((hkv, n, b, d), generator=gen).bfloat16()
        lo, hi = k.amin(2).float(), k.amax(2).float()
        q[0].zero_()
        ref = O.select_blocks(*np_(q, lo, hi), topk)
        ids = gqa.select_blocks(*dev(q, lo, hi), topk)
        assert ids.cpu().numpy().tolist() == ref.tolist(), (hq, n, topk)


@pytest.mark.parametrize("n,topk", [(7, 7), (1000, 1), (2048, 64), (3000, 3000), (4096, 64),
                                    (8192, 2048), (16384, 100), (20000, 333)])
def test_select_ties_and_row_lengths(n, topk):
    """Many exactly tied scores (small-integer q and bounds), every register
    tile size of the top-K kernel and the long-row path, k == n."""
    from strict_topk import gqa
    gen = torch.Generator().manual_seed(n + topk)
    hq, hkv, d = 4, 2, 16
    q = torch.randint(-2, 3, (hq, d), generator=gen).to(torch.bfloat16)
    lo = torch.randint(-3, 1, (hkv, n, d), generator=gen).float()
    hi = lo + torch.randint(0, 3, (hkv, n, d), generator=gen).float()
    q[1].zero_()
    ref = O.select_blocks(*np_(q, lo, hi), topk)
    ids = gqa.select_blocks(*dev(q, lo, hi), topk)
    assert ids.cpu().numpy().tolist() == ref.tolist()
    assert ids[1].cpu().tolist() == list(range(topk))


@pytest.mark.parametrize("hq,hkv,n,topk", [(16, 4, 1025, 64), (16, 4, 2048, 2048),
                                            (16, 4, 3000, 64), (16, 4, 4096, 1000),
                                            (16, 4, 4097, 64), (16, 4, 6000, 700),
                                            (16, 4, 8192, 8192), (288, 4, 2048, 64),
                                            (288, 4, 4000, 300), (288, 4, 8000, 64)])
def test_select_ties_many_rows(hq, hkv, n, topk):
    """Up to 256 rows of 1024 < n <= 8192 keys take four or eight keys per
    thread, more rows the 256-thread kernels: tied scores, every row length
    bracket, k == n."""
    from strict_topk import gqa
    gen = torch.Generator().manual_seed(7 * n + topk + hq)
    d = 16
    q = torch.randint(-2, 3, (hq, d), generator=gen).to(torch.bfloat16)
    lo = torch.randint(-3, 1, (hkv, n, d), generator=gen).float()
    hi = lo + torch.randint(0, 3, (hkv, n, d), generator=gen).float()
    q[3].zero_()
    ref = O.select_blocks(*np_(q, lo, hi), topk)
    ids = gqa.select_blocks(*dev(q, lo, hi), topk)
    assert ids.cpu().numpy().tolist() == ref.tolist()
    assert ids[3].cpu().tolist() == list(range(topk))


def test_select_nonfinite_bounds():
    """-inf/+inf bounds and NaN scores: NaN ranks below -inf."""
    from strict_topk import gqa
    gen = torch.Generator().manual_seed(11)
    q = torch.randn((2, 8), generator=gen).half()
    lo = torch.randn((2, 40, 8), generator=gen)
    hi = lo + 1
    lo[0, 3] = float("-inf")
    hi[1, 5] = float("inf")
    lo[1, 7, 0] = float("nan")
    hi[1, 7, 0] = float("nan")
    ref = O.select_blocks(*np_(q, lo, hi), 39)
    ids = gqa.select_blocks(*dev(q, lo, hi), 39)
    assert ids.cpu().numpy().tolist() == ref.tolist()


@pytest.mark.parametrize("dtype,b,d", [(torch.bfloat16, 32, 128), (torch.float16, 4, 64),
                                     (torch.bfloat16, 16, 256), (torch.float32, 8, 48),
                                     (torch.float16, 5, 13), (torch.bfloat16, 32, 256),
                                     (torch.float16, 7, 192), (torch.bfloat16, 100, 128)])
def test_block_bounds_and_append(dtype, b, d):
    """Block metadata bit-exact against the oracle (min / max are exact), NaN
    keys included; appending a block's tokens one by one gives the same
    bounds as building them from the block."""
    from strict_topk import bounds
    gen = torch.Generator().manual_seed(b * d)
    hkv, n = 3, 41
    k = (torch.randn((hkv, n, b, d), generator=gen) * 3).to(dtype)
    k[2, 7, b - 1, d // 2] = float("nan")
    lo_ref, hi_ref = O.block_bounds(C.f64(k))
    lo, hi = bounds.block_bounds(k.to(DEV))
    assert np.array_equal(lo.cpu().numpy(), lo_ref.astype(np.float32), equal_nan=True)
    assert np.array_equal(hi.cpu().numpy(), hi_ref.astype(np.float32), equal_nan=True)
    # decode appends into a copy, block by block (positions 0 .. b-1)
    lo2 = torch.full_like(lo, 123.0)
    hi2 = torch.full_like(hi, -123.0)
    kd = k.to(DEV)
    for blk in (0, 7, n - 1):
        for t in range(b):
            bounds.append(lo2, hi2, kd[:, blk, t].contiguous(), blk, t)
        assert torch.equal(lo2[:, blk].isnan(), lo[:, blk].isnan())
        fin = ~lo[:, blk].isnan()
        assert torch.equal(lo2[:, blk][fin], lo[:, blk][fin])
        assert torch.equal(hi2[:, blk][fin], hi[:, blk][fin])
    with pytest.raises(ValueError):
        bounds.append(lo2, hi2, kd[:, 0, 0].contiguous(), n, 0)


@pytest.mark.parametrize("dtype,h,n,d,topk", [(torch.float16, 4, 8192, 128, 2048),
                                            (torch.bfloat16, 4, 3000, 128, 64),
                                            (torch.float32, 3, 50, 13, 7),
                                            (torch.float16, 16, 700, 256, 700)])
def test_indexer_scores_and_shared_select(dtype, h, n, d, topk):
    """QSA indexer (benchmarks/selector_window.py:126-142): FP32 scores
    bit-exact to float32(oracle FP64 score), shared IDs bit-exact in every
    row; integer-valued keys make many exact ties (lower index wins); a NaN
    key ranks last."""
    from strict_topk import indexer
    gen = torch.Generator().manual_seed(n + d)
    iq = torch.randn((h, d), generator=gen).to(dtype)
    ik = torch.randn((n, d), generator=gen).to(dtype)
    t = min(40, n // 6)
    ik[n // 3: n // 3 + t] = torch.randint(-1, 2, (t, d), generator=gen).to(dtype)
    ik[n // 2: n // 2 + t] = ik[n // 3: n // 3 + t]
    ik[5, 1] = float("nan")
    ref = O.indexer_scores(C.f64(iq), C.f64(ik))
    got = indexer.scores(iq.to(DEV), ik.to(DEV))
    assert np.array_equal(got.cpu().numpy(), ref.astype(np.float32), equal_nan=True)
    ids = indexer.select_shared(iq.to(DEV), ik.to(DEV), topk, 6)
    assert ids.shape == (6, topk) and ids.dtype == torch.int32
    assert ids.cpu().numpy().tolist() == O.indexer_select(C.f64(iq), C.f64(ik), topk, 6).tolist()


def _indexer_inputs(dtype, n, seed, ties=True):
    gen = torch.Generator().manual_seed(seed)
    iq = torch.randn((4, 128), generator=gen).to(dtype)
    ik = torch.randn((n, 128), generator=gen).to(dtype)
    if ties and n >= 12:
        t = min(40, n // 6)
        ik[n // 3: n // 3 + t] = torch.randint(-1, 2, (t, 128), generator=gen).to(dtype)
        ik[n // 2: n // 2 + t] = ik[n // 3: n // 3 + t]
    return iq, ik


@pytest.mark.parametrize("dtype,n,topk,rows", [
    (torch.bfloat16, 8192, 2048, 48),    # c4's shape: 12 workgroups write 4 rows each
    (torch.float16, 16384, 8192, 5),     # the largest shape of k_topk_shared (16 keys per thread)
    (torch.bfloat16, 16384, 1, 1),
    (torch.bfloat16, 1, 1, 1),
    (torch.float16, 100, 37, 9),         # topk not a multiple of 4: 4-byte stores
    (torch.bfloat16, 1025, 1025, 3),     # topk = n
    (torch.bfloat16, 4099, 4000, 13),
    (torch.bfloat16, 1000, 100, 300),    # 64 workgroups, some writing five rows
    (torch.float16, 20000, 300, 2),      # past 16384 keys: top-K, then the row copy
    (torch.float16, 20000, 300, 70),
])
def test_shared_select_rows(dtype, n, topk, rows):
    """The shared selection (benchmarks/selector_window.py:76-84): every
    workgroup of k_topk_shared ranks the whole row and writes its share of
    the rows; past its shapes the top-K writes row 0 and k_rows_copy the
    rest.  IDs bit-exact against the oracle in every row, with exact ties in
    the keys."""
    from strict_topk import indexer
    iq, ik = _indexer_inputs(dtype, n, n + topk)
    ids = indexer.select_shared(iq.to(DEV), ik.to(DEV), topk, rows)
    torch.cuda.synchronize()
    assert ids.shape == (rows, topk)
    assert ids.cpu().numpy().tolist() == \
        O.indexer_select(C.f64(iq), C.f64(ik), topk, rows).tolist()


def test_shared_select_in_a_graph():
    """The selection captured in a graph and replayed while the indexer
    query changes in place: every replay equals the eager call on the same
    inputs, and the last one the oracle."""
    from strict_topk import indexer
    iq, ik = _indexer_inputs(torch.bfloat16, 8192, 7)
    iqd, ikd = iq.to(DEV), ik.to(DEV)
    indexer.select_shared(iqd, ikd, 2048, 48)
    g = torch.cuda.CUDAGraph()
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        with torch.cuda.graph(g, stream=s):
            out = indexer.select_shared(iqd, ikd, 2048, 48)
    torch.cuda.current_stream().wait_stream(s)
    gen = torch.Generator().manual_seed(11)
    for _ in range(4):
        iqd.copy_(torch.randn((4, 128), generator=gen).to(torch.bfloat16))
        g.replay()
        torch.cuda.synchronize()
        eager = indexer.select_shared(iqd, ikd, 2048, 48)
        torch.cuda.synchronize()
        assert torch.equal(out, eager)
    ref = O.indexer_select(C.f64(iqd.cpu()), C.f64(ik), 2048, 48)
    assert out.cpu().numpy().tolist() == ref.tolist()


def test_select_rejects_bad_k():
    from strict_topk import gqa
    q = torch.randn((4, 8), device=DEV)
    lo = torch.zeros((2, 10, 8), device=DEV)
    with pytest.raises(RuntimeError):
        gqa.select_blocks(q, lo, lo, 11)
    assert gqa.select_blocks(q, lo, lo, 0).shape == (4, 0)


# ----------------------------------------------------------------- kernels
REPAIRS = ["split", "fused", "signed", "signed_fused"]


def _repair_fn(name):
    from strict_topk import fused, kernels, signed_fused, signed_repair
    return {"split": kernels.repair, "fused": fused.repair_fused,
            "signed": signed_repair.repair_signed,
            "signed_fused": signed_fused.repair_signed_fused}[name]


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
def test_kernels_strict_paths(dtype):
    from strict_topk.kernels import exact_attention, speculate
    for name, *ts in C.correctness_cases(dtype):
        expected = O.attention(*np_(ts[0], ts[1], ts[2], ts[4]))
        q, k, v, p, a = dev(*ts)
        check(exact_attention(q, k, v, a), expected, (name, "exact"))
        for mode, thr in [("saved", .1), ("hybrid", .05), ("hybrid", .2), ("hybrid", 1.),
                          ("compact", .05), ("compact", .2), ("compact", 1.)]:
            st = speculate(q, k, v, p, mode=mode, mass_threshold=thr)
            for impl in REPAIRS:
                res = _repair_fn(impl)(q, k, v, a, p, st)
                check(res.output, expected, (name, mode, thr, impl))
                if mode != "saved" and thr == 1. and name in C.EXPECTED_FALLBACK:
                    assert int(res.fallback.sum()) == C.EXPECTED_FALLBACK[name], (name, mode, impl)
                if impl in ("signed", "signed_fused"):
                    assert res.approximate_heads is None


def test_block_partials_and_merge_match_oracle():
    from strict_topk.kernels import block_partials, merge_partials
    for name, *ts in C.correctness_cases(torch.bfloat16):
        qn, kn, vn, pn, an = np_(*ts)
        q, k, v, p, a = dev(*ts)
        st = block_partials(q, k, v, a)
        ref = O.block_states(qn, kn, vn, an)
        np.testing.assert_allclose(st.m.cpu().double().numpy(), ref.m, rtol=1e-5, atol=1e-5)
        # compare normalised states to be frame-independent
        lu = st.u.cpu().double().numpy() / st.l.cpu().double().numpy()[..., None]
        np.testing.assert_allclose(lu, ref.u / ref.l[..., None], rtol=1e-3, atol=3e-4)
        mask = torch.zeros(a.shape, dtype=torch.bool, device=DEV)
        mask[:, ::2] = True
        st2 = block_partials(q, k, v, a, mask)
        assert torch.isinf(st2.m[:, 1::2]).all() and (st2.l[:, 1::2] == 0).all()
        inc = mask.clone()
        check(merge_partials(st, inc), O.attention(qn, kn, vn, an, inc.cpu().numpy()), name)
        head = torch.zeros(a.shape[0], dtype=torch.bool, device=DEV)
        head[0] = True
        st3 = block_partials(q, k, v, a, head)
        assert torch.isinf(st3.m[1:]).all()


def test_speculate_fields_match_oracle():
    from strict_topk.kernels import speculate
    gen = torch.Generator().manual_seed(99)
    h, n, b, d, s = 4, 40, 16, 64, 12
    q = torch.randn(h, d, generator=gen).half()
    k = (torch.randn(h, n, b, d, generator=gen) * 2).half()
    v = torch.randn(h, n, b, d, generator=gen).half()
    p = torch.stack([torch.randperm(n, generator=gen)[:s] for _ in range(h)]).int()
    qn, kn, vn, pn = np_(q, k, v, p)
    qd, kd, vd, pd = dev(q, k, v, p)
    for mode in ("hybrid", "compact"):
        for thr in (.05, .1, .3):
            ref = O.speculate(qn, kn, vn, pn, mode=mode, mass_threshold=thr, keep_mass=True)
            got = speculate(qd, kd, vd, pd, mode=mode, mass_threshold=thr, keep_mass=True)
            # decisions are exact unless a mass sits within 1e-5 of the threshold
            st = O.block_states(qn, kn, vn, pn)
            mass = np.exp(st.m - st.m.max(1, keepdims=True)) * st.l
            frac = mass / mass.sum(1, keepdims=True)
            safe = np.abs(frac - thr) > 1e-5
            assert (got.high.cpu().numpy() == ref.high)[safe].all(), (mode, thr)
            if safe.all():
                assert np.array_equal(got.high.cpu().numpy(), ref.high)
                if mode == "compact":
                    assert got.retained_ids.cpu().numpy().tolist() == ref.retained_ids.tolist()
                    assert got.overflow.cpu().numpy().tolist() == ref.overflow.tolist()
                    assert got.retained_ids.dtype == pd.dtype
                np.testing.assert_allclose(got.low.m.cpu().numpy(), ref.low.m, rtol=1e-5, atol=1e-5)
                np.testing.assert_allclose(got.low.l.cpu().numpy(), ref.low.l, rtol=1e-4)
                np.testing.assert_allclose(got.low.u.cpu().numpy(), ref.low.u, rtol=1e-3, atol=1e-4)
                np.testing.assert_allclose(got.low_abs.cpu().numpy(), ref.low_abs, rtol=1e-3, atol=1e-4)
            np.testing.assert_allclose(got.mass_m.cpu().numpy(), ref.mass_m, rtol=1e-5, atol=1e-5)
            np.testing.assert_allclose(got.mass_l.cpu().numpy(), ref.mass_l, rtol=1e-4)


@pytest.mark.parametrize("mode", ["hybrid", "compact"])
@pytest.mark.parametrize("impl", ["fused", "signed", "signed_fused"])
def test_extra_mass_budget(mode, impl):
    from strict_topk.kernels import speculate
    q, k, v, p, a, extra_set = C.budget_case()
    strict = O.attention(*np_(q, k, v, a))
    with_extra = O.attention(*np_(q, k, v, extra_set))
    extra_mass = math.exp(-3) / (2 + math.exp(-3))
    q, k, v, p, a = dev(q, k, v, p, a)
    fn = _repair_fn(impl)
    st = speculate(q, k, v, p, mode=mode, mass_threshold=.2, keep_mass=True)
    low = fn(q, k, v, a, p, st, max_extra_mass=.01)
    assert not low.approximate_heads.item() and low.extra_mass_bound.item() == 0.
    check(low.output, strict)
    high = fn(q, k, v, a, p, st, max_extra_mass=.1)
    assert high.approximate_heads.item()
    assert extra_mass <= high.extra_mass_bound.item() <= .1
    assert abs(high.extra_mass_bound.item() - math.exp(-3) / (1 + math.exp(-3))) < 1e-6
    check(high.output, with_extra)
    forced = fn(q, k, v, a, p, st, cancellation_tol=2., max_extra_mass=.1)
    assert forced.fallback.item() and not forced.approximate_heads.item()
    assert forced.extra_mass_bound.item() == 0.
    check(forced.output, strict)
    if impl != "fused":
        assert low.positive_jobs.item() == 1 and low.total_jobs.item() == 2
        assert high.positive_jobs.item() == 1 and high.total_jobs.item() == 1
        assert low.positive_jobs.dtype == torch.int32


def test_budget_requires_keep_mass():
    from strict_topk.fused import repair_fused
    from strict_topk.kernels import speculate
    from strict_topk.signed_fused import repair_signed_fused
    q, k, v, p, a, _ = dev(*C.budget_case())
    st = speculate(q, k, v, p, mode="hybrid", mass_threshold=.2)
    for fn in (repair_fused, repair_signed_fused):
        with pytest.raises(ValueError):
            fn(q, k, v, a, p, st, max_extra_mass=.1)
        with pytest.raises(ValueError):
            fn(q, k, v, a, p, st, max_extra_mass=1.5)


def test_signed_fused_underflow_regression():
    from strict_topk.kernels import speculate
    from strict_topk.signed_fused import repair_signed_fused
    ts = C.underflow_case()
    expected = O.attention(*np_(ts[0], ts[1], ts[2], ts[4]))
    q, k, v, p, a = dev(*ts)
    pred = speculate(q, k, v, p, mode="hybrid", mass_threshold=1.)
    res = repair_signed_fused(q, k, v, a, p, pred)
    check(res.output, expected)
    assert res.fallback.item()


def test_schedule_queue_order():
    """Queue = misses in selected order, then wrong-low blocks in predicted order."""
    from strict_topk.kernels import speculate
    from strict_topk.signed_fused import repair_signed_fused
    for name, *ts in C.correctness_cases(torch.float16):
        if not name.startswith("random_unordered"):
            continue
        qn, kn, vn, pn, an = np_(*ts)
        q, k, v, p, a = dev(*ts)
        for mode in ("saved", "hybrid"):
            st = speculate(q, k, v, p, mode=mode, mass_threshold=.2)
            res = repair_signed_fused(q, k, v, a, p, st)
            for h in range(pn.shape[0]):
                _, miss = O.membership(pn[h], an[h])
                assert res.positive_jobs[h].item() == int(miss.sum())
            if mode == "hybrid":
                high = st.high.cpu().numpy()
                for h in range(pn.shape[0]):
                    hit, _ = O.membership(pn[h], an[h])
                    low_hit = (hit & ~high[h]).any()
                    wrong = (~hit & ~high[h]) & low_hit
                    assert res.total_jobs[h].item() == int(res.positive_jobs[h].item() + wrong.sum())


# --------------------------------------------------------------------- GQA
def test_tiny_gqa_known_answers():
    from strict_topk import gqa, gqa_light
    q, k, v, p = dev(*C.tiny_gqa())
    union = (8 * math.e ** 5 - 5) / (math.e ** 5 + 1)
    st = gqa.partials(q, k, v, p)
    assert gqa.exact(q, k, v, p).cpu()[:, 0].tolist() == pytest.approx([8., -5.], abs=1e-6)
    assert gqa.repair_saved(q, k, v, 1 - p, p, st).cpu()[:, 0].tolist() == pytest.approx([-5., 8.], abs=1e-6)
    assert gqa.repair_union(q, k, v, 1 - p, p, st).cpu()[:, 0].tolist() == pytest.approx([union] * 2, rel=1e-6)
    assert gqa_light.repair_saved_light(q, k, v, 1 - p, p, st).cpu()[:, 0].tolist() == pytest.approx([-5., 8.], abs=1e-6)


@pytest.mark.parametrize("hq", [6, 16])
def test_gqa_paths(hq):
    from strict_topk import gqa, gqa_light
    for name, *ts in C.gqa_cases(hq=hq, hkv=2 if hq == 6 else 4):
        qn, kn, vn, pn, an = np_(*ts)
        expected = O.attention(qn, kn, vn, an)
        hit = (an[:, :, None] == pn[:, None, :]).any(-1)
        q, k, v, p, a = dev(*ts)
        st = gqa.partials(q, k, v, p)
        ref = O.block_states(qn, kn, vn, pn)
        np.testing.assert_allclose(st.m.cpu().double().numpy(), ref.m, rtol=1e-5, atol=1e-4)
        check(gqa.exact(q, k, v, a), expected, (name, "exact"))
        check(gqa.repair_saved(q, k, v, a, p, st), expected, (name, "saved"))
        union = O.attention(qn, kn, vn, [np.concatenate((pn[h], an[h][~hit[h]]))
                                         for h in range(len(pn))])
        check(gqa.repair_union(q, k, v, a, p, st), union, (name, "union"))
        check(gqa_light.repair_saved_light(q, k, v, a, p, st), expected, (name, "light"))
        for emf in (0., 1.):
            check(gqa_light.repair_saved_auto(q, k, v, a, p, st, emf), expected, (name, "auto", emf))
    with pytest.raises(ValueError):
        gqa_light.repair_saved_auto(q, k, v, a, p, st, 1.5)


@pytest.mark.parametrize("hq,hkv,n,b,d,sa,sp,hits,dtype", [
    (8, 2, 300, 32, 128, 64, 64, 58, torch.bfloat16),     # grouped rows sharing blocks
    (8, 2, 300, 64, 128, 40, 40, 0, torch.bfloat16),      # no hits, two-chunk tiles
    (4, 1, 9000, 8, 256, 100, 120, 100, torch.float16),   # all hits, wide rows, big N
    (6, 3, 12000, 5, 70, 37, 29, 11, torch.float32),      # odd D and B, brute-force membership
    (16, 4, 2048, 32, 128, 64, 64, 48, torch.bfloat16),   # c3-like, 16 misses per head
    (8, 4, 500, 48, 64, 30, 30, 20, torch.float16),       # three 16-token chunks per block
    (8, 8, 400, 16, 128, 24, 24, 12, torch.bfloat16),     # G = 1, one 16-token chunk
])
def test_gqa_states_and_repair_shapes(hq, hkv, n, b, d, sa, sp, hits, dtype):
    """GQA states (one wave per (query head, slot); heads of a KV group that
    list the same block each read its tile) and the single-launch saved /
    union / light repair against the oracle."""
    from strict_topk import gqa, gqa_light
    gen = torch.Generator().manual_seed(hq * 7 + n)
    q = torch.randn((hq, d), generator=gen).to(dtype)
    k = torch.randn((hkv, n, b, d), generator=gen).to(dtype)
    v = torch.randn(k.shape, generator=gen).to(dtype)
    g = hq // hkv
    rows_a, rows_p = [], []
    for kv in range(hkv):
        pool = torch.randperm(n, generator=gen)[:sa + sp + 8]
        for _ in range(g):
            # heads of a group draw from one pool, so their rows overlap
            a_row = pool[torch.randperm(sa + 8, generator=gen)[:sa]]
            others = pool[sa + 8:]
            keep = a_row[torch.randperm(sa, generator=gen)[:hits]]
            p_row = torch.cat((keep, others[torch.randperm(len(others), generator=gen)[:sp - hits]]))
            rows_a.append(a_row)
            rows_p.append(p_row[torch.randperm(sp, generator=gen)])
    a = torch.stack(rows_a).to(torch.int64)
    p = torch.stack(rows_p).to(torch.int32)
    qn, kn, vn, an, pn = np_(q, k, v, a, p)
    ref = O.block_states(qn, kn, vn, pn)
    qd, kd, vd, ad, pd = dev(q, k, v, a, p)
    st = gqa.partials(qd, kd, vd, pd)
    np.testing.assert_allclose(st.m.cpu().double().numpy(), ref.m, rtol=1e-5, atol=1e-5)
    np.testing.assert_allclose(st.l.cpu().double().numpy(), ref.l, rtol=1e-4, atol=1e-5)
    np.testing.assert_allclose(st.u.cpu().double().numpy(), ref.u, rtol=1e-4, atol=1e-4)
    expected = O.attention(qn, kn, vn, an)
    check(gqa.exact(qd, kd, vd, ad), expected, "exact")
    check(gqa.repair_saved(qd, kd, vd, ad, pd, st), expected, "saved")
    check(gqa_light.repair_saved_light(qd, kd, vd, ad, pd, st), expected, "light")
    hit = (an[:, :, None] == pn[:, None, :]).any(-1)
    union = O.attention(qn, kn, vn, [np.concatenate((pn[r], an[r][~hit[r]])) for r in range(hq)])
    check(gqa.repair_union(qd, kd, vd, ad, pd, st), union, "union")


def test_gqa_validation_messages():
    from strict_topk import gqa
    q = torch.randn((6, 13), device=DEV, dtype=torch.float16)
    k = torch.randn((4, 23, 7, 13), device=DEV, dtype=torch.float16)
    ids = torch.zeros((6, 3), device=DEV, dtype=torch.int32)
    with pytest.raises(ValueError, match="Hq divisible"):
        gqa.partials(q, k, k, ids)
    with pytest.raises(ValueError, match="nonempty int32/int64"):
        gqa.partials(q, k[:2], k[:2], ids.float())


# ------------------------------------------------- packed small-block states
@pytest.mark.parametrize("b,d,dtype,itype,hq,shared", [
    (4, 128, torch.bfloat16, torch.int32, 6, False),
    (8, 64, torch.float16, torch.int64, 6, False),
    (4, 256, torch.bfloat16, torch.int64, 6, False),
    (8, 128, torch.bfloat16, torch.int32, 6, False),
    (4, 128, torch.bfloat16, torch.int32, 24, True),    # G = 12: four heads per wave
    (8, 64, torch.float16, torch.int64, 8, False),      # G = 4, rows differ
    (4, 128, torch.float16, torch.int32, 12, True),     # G = 6: two heads per wave
])
def test_packed_small_block_states(b, d, dtype, itype, hq, shared):
    """Blocks of 4 or 8 tokens run 32-token packs per wave: per-block states
    against the oracle, with a ragged row, invalid IDs, both active-mask
    kinds, and the hierarchical exact / saved repair (skip mode) on top.
    With G a multiple of 2, a wave serves several heads of a KV group: rows
    shared by the group (one pack load), with single entries changed so that
    some packs differ between heads, and rows that differ everywhere."""
    from strict_topk import gqa_hierarchical as hier
    from strict_topk.kernels import block_partials
    gen = torch.Generator().manual_seed(11 + b + d + hq)
    hkv, n, s = 2, 300, 37   # 37 positions: the last pack is partial
    g = hq // hkv
    q = torch.randn((hq, d), generator=gen).to(dtype)
    k = torch.randn((hkv, n, b, d), generator=gen).to(dtype)
    v = torch.randn(k.shape, generator=gen).to(dtype)
    if shared:
        base = [torch.randperm(n, generator=gen)[:s] for _ in range(hkv)]
        valid = torch.stack([base[h // g] for h in range(hq)]).to(itype)
    else:
        valid = torch.stack([torch.randperm(n, generator=gen)[:s] for _ in range(hq)]).to(itype)
    ids = valid.clone()
    ids[1, 5] = -1
    ids[2, 36] = -1
    qn, kn, vn = np_(q, k, v)
    ref = O.block_states(qn, kn, vn, C.ids_np(ids))
    qd, kd, vd, idd = dev(q, k, v, ids)

    def same(st, r, what):
        m, l, u = (x.cpu().double().numpy() for x in (st.m, st.l, st.u))
        off = np.isinf(r.m)
        assert np.isinf(m[off]).all() and (m[off] < 0).all(), what
        assert (l[off] == 0).all() and (u[off] == 0).all(), what
        np.testing.assert_allclose(m[~off], r.m[~off], rtol=1e-5, atol=1e-5, err_msg=what)
        np.testing.assert_allclose(l, r.l, rtol=1e-4, atol=1e-6, err_msg=what)
        np.testing.assert_allclose(u, r.u, rtol=1e-4, atol=1e-4, err_msg=what)

    same(block_partials(qd, kd, vd, idd), ref, "states")
    big = idd.clone()
    big[0, 3] = n + 7   # out of range: empty state, no memory read
    st = block_partials(qd, kd, vd, big)
    assert torch.isinf(st.m[0, 3]) and st.l[0, 3] == 0 and (st.u[0, 3] == 0).all()
    mask = torch.zeros((hq, s), dtype=torch.bool)
    mask[:, ::3] = True
    same(block_partials(qd, kd, vd, idd, mask.to(DEV)),
         O.block_states(qn, kn, vn, C.ids_np(ids), mask.numpy()), "slot mask")
    head = torch.tensor([h % 3 != 1 for h in range(hq)])
    same(block_partials(qd, kd, vd, idd, head.to(DEV)),
         O.block_states(qn, kn, vn, C.ids_np(ids), head.numpy()), "head mask")
    an = C.ids_np(valid)
    expected = O.attention(qn, kn, vn, an)
    a = valid.to(DEV)
    check(hier.exact(qd, kd, vd, a), expected, "packed exact")
    for hits in (0, s // 2, s):
        p = C.prediction_rows(valid, n, s, hits).to(itype).to(DEV)
        check(hier.repair_saved(qd, kd, vd, a, p, hier.partials(qd, kd, vd, p)), expected,
              ("packed saved", hits))


# ------------------------------------------------------------ hierarchical
@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
def test_hierarchical_paths(dtype):
    from strict_topk import gqa_hierarchical as impl
    for (h, hkv, n, b, d, sa), *ts in C.hier_cases(dtype):
        qn, kn, vn, an = np_(*ts)
        expected = O.attention(qn, kn, vn, an)
        q, k, v, a = dev(*ts)
        check(impl.exact(q, k, v, a), expected, "exact")
        for hits in [0, sa // 2, sa - 1, sa]:
            p = C.prediction_rows(a.cpu(), n, sa, hits).to(DEV)
            st = impl.partials(q, k, v, p)
            check(impl.repair_saved(q, k, v, a, p, st), expected, ("saved", hits))
        shared = a[:1].expand(h, -1).contiguous()
        exp_shared = O.attention(qn, kn, vn, C.ids_np(shared))
        for hits in (0, sa // 2, sa):
            pred = C.prediction_rows(shared.cpu(), n, max(1, sa // 2), min(hits, sa // 2)).to(DEV)
            out = impl.repair_saved_shared(q, k, v, shared, pred, impl.partials(q, k, v, pred))
            check(out, exp_shared, ("shared", hits))


@pytest.mark.parametrize("dtype,b,g,shared,itype,sharp", [
    (torch.bfloat16, 4, 12, True, torch.int32, 1.0),      # c4's group tile
    (torch.bfloat16, 4, 12, True, torch.int32, 8.0),      # near one-hot rows
    (torch.bfloat16, 8, 16, False, torch.int64, 1.0),     # per-head rows: one pass per head
    (torch.float16, 4, 8, False, torch.int32, 8.0),
    (torch.float16, 8, 12, True, torch.int64, 1.0),
    (torch.float16, 4, 16, True, torch.int32, 0.01),      # nearly flat rows
])
def test_hierarchical_exact_group_tile(dtype, b, g, shared, itype, sharp):
    """gqa_hierarchical.exact, .partials and the repairs on the matrix-core group tile
    (D = 128, 8-16 query heads per KV head, B = 4 or 8): selections shared by
    the group (one tile per pack) or per head (the block states then take the
    layout whose MFMA rows are one head's blocks), a ragged last pack, sharp
    and flat softmax rows (the P.V weights travel as a high and a low 16-bit
    part).  Outputs against the FP64 oracle at |err| <= 3e-4 + 3e-4 |ref|
    (tests/check_correctness.py:22); block states as in the packed-states test."""
    from strict_topk import gqa_hierarchical as impl
    hkv, n, d, sa = 2, 300, 128, 45
    h = hkv * g
    gen = torch.Generator().manual_seed(g * 100 + b + int(shared))
    q = (torch.randn((h, d), generator=gen) * sharp).to(dtype)
    k = torch.randn((hkv, n, b, d), generator=gen).to(dtype)
    v = torch.randn((hkv, n, b, d), generator=gen).to(dtype)
    if shared:
        a = torch.randperm(n, generator=gen)[:sa].expand(h, -1).contiguous()
    else:
        a = torch.stack([torch.randperm(n, generator=gen)[:sa] for _ in range(h)])
    a = a.to(itype)
    qn, kn, vn, an = np_(q, k, v, a)
    expected = O.attention(qn, kn, vn, an)
    what = ("group tile", dtype, b, g, shared, sharp)
    check(impl.exact(*dev(q, k, v, a)), expected, what)
    st = impl.partials(*dev(q, k, v, a))
    ref = O.block_states(qn, kn, vn, an)
    m, l, u = (x.cpu().double().numpy() for x in (st.m, st.l, st.u))
    np.testing.assert_allclose(m, ref.m, rtol=1e-5, atol=1e-5, err_msg=str(what))
    np.testing.assert_allclose(l, ref.l, rtol=1e-4, atol=1e-6, err_msg=str(what))
    np.testing.assert_allclose(u, ref.u, rtol=1e-4, atol=1e-4, err_msg=str(what))
    # the repair on the same tile: misses from K/V, hits from the prediction's
    # block states at their slots (predictions of 40 blocks: none, some or
    # all of the selection, the rest wrong)
    qd, kd, vd, ad = dev(q, k, v, a)
    for hits in (0, 20, 40):
        pd = C.prediction_rows(a, n, 40, hits).to(DEV)
        st = impl.partials(qd, kd, vd, pd)
        check(impl.repair_saved(qd, kd, vd, ad, pd, st), expected, what + ("saved", hits))
        if shared:
            check(impl.repair_saved_shared(qd, kd, vd, ad, pd, st), expected,
                  what + ("saved_shared", hits))


@pytest.mark.parametrize("n", [300, 8192])
def test_hier_shared_repair_slots(n):
    """repair_saved_shared's hits use the prediction's state at the highest
    slot holding the block (gqa_hierarchical.py:10-19, _match_ids).  The
    predicted row repeats some selected blocks, and the state at each
    repeat's lower slot is overwritten with a wrong one, which a lower-slot
    match would merge; it also holds invalid IDs (-1, n + 3), which match
    nothing."""
    from strict_topk import gqa_hierarchical as impl
    h, hkv, b, d, sa = 24, 2, 4, 128, 64
    gen = torch.Generator().manual_seed(n)
    q = torch.randn((h, d), generator=gen).to(torch.bfloat16)
    k = torch.randn((hkv, n, b, d), generator=gen).to(torch.bfloat16)
    v = torch.randn((hkv, n, b, d), generator=gen).to(torch.bfloat16)
    a = torch.randperm(n, generator=gen)[:sa].to(torch.int32)
    sel = a.expand(h, -1).contiguous()
    others = torch.tensor([x for x in torch.randperm(n, generator=gen)[:200].tolist()
                           if x not in set(a.tolist())][:12], dtype=torch.int32)
    # slots: 0..7 the blocks a[0:8] (later repeated), then hits a[8:40],
    # wrong blocks, invalid IDs, and the repeats of a[0:8] at the top
    prow = torch.cat([a[:8], a[8:40], others, torch.tensor([-1, n + 3], dtype=torch.int32),
                      a[:8]])
    pred = prow.expand(h, -1).contiguous()
    qn, kn, vn, an = np_(q, k, v, sel)
    expected = O.attention(qn, kn, vn, an)
    qd, kd, vd, sd, pd = dev(q, k, v, sel, pred)
    st = impl.partials(qd, kd, vd, pd)
    st.m[:, :8] = 50.0      # the lower copies: a merge of these would dominate
    st.l[:, :8] = 1.0
    st.u[:, :8] = 1000.0
    check(impl.repair_saved_shared(qd, kd, vd, sd, pd, st), expected, ("shared slots", n))


# ----------------------------------------------------------- graph replays
def _capture(fn):
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        for _ in range(3):
            fn()
    torch.cuda.current_stream().wait_stream(s)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        out = fn()
    g.replay()
    torch.cuda.synchronize()
    return g, out


def test_graph_mutation_signed_fused():
    """tests/check_signed_fused.py:31-49: capture, scale V in place, replay."""
    from strict_topk.kernels import speculate
    from strict_topk.signed_fused import repair_signed_fused
    gen = torch.Generator().manual_seed(817)
    for dtype in (torch.float16, torch.bfloat16):
        q = torch.randn((3, 7), generator=gen).to(dtype)
        k = torch.randn((3, 17, 5, 7), generator=gen).to(dtype)
        v = torch.randn(k.shape, generator=gen).to(dtype)
        p = torch.tensor([[0, 1, 2, 3, 4], [3, 4, 5, 6, 7], [8, 9, 10, 11, 12]], dtype=torch.int64)
        a = torch.tensor([[1, 2, 8], [4, 9, 15], [0, 5, 16]], dtype=torch.int32)
        q, k, v, p, a = dev(q, k, v, p, a)
        for mode in ("saved", "hybrid", "compact"):
            g, res = _capture(lambda: repair_signed_fused(
                q, k, v, a, p, speculate(q, k, v, p, mode=mode, mass_threshold=.2)))
            for scale in (1., -.5, 2.):
                v.mul_(scale)
                g.replay()
                torch.cuda.synchronize()
                check(res.output, O.attention(*np_(q, k, v, a)), (dtype, mode, scale))


def test_graph_mutation_hierarchical_ids():
    """tests/check_gqa_hierarchical.py:28-32: captured IDs change in place."""
    from strict_topk import gqa_hierarchical as impl
    gen = torch.Generator().manual_seed(5)
    h, hkv, n, b, d, sa = 6, 2, 96, 5, 96, 37
    q = torch.randn((h, d), generator=gen).bfloat16()
    k = torch.randn((hkv, n, b, d), generator=gen).bfloat16()
    v = torch.randn(k.shape, generator=gen).bfloat16()
    a = torch.stack([torch.randperm(n, generator=gen)[:sa] for _ in range(h)]).int()
    p = C.prediction_rows(a, n, sa, sa // 2)
    q, k, v, a, p = dev(q, k, v, a, p)
    g, out = _capture(lambda: impl.repair_saved(q, k, v, a, p, impl.partials(q, k, v, p)))
    a.copy_((a + 1) % n)
    for _ in range(3):
        g.replay()
        torch.cuda.synchronize()
        check(out, O.attention(*np_(q, k, v, a)), "hier graph")


def test_touch_kv_checksums():
    from strict_topk.kernels import touch_kv
    gen = torch.Generator().manual_seed(4)
    k = torch.randn((2, 9, 40, 64), generator=gen).half()
    v = torch.randn(k.shape, generator=gen).half()
    p = torch.tensor([[0, 3, 8], [1, 2, 7]], dtype=torch.int32)
    ref = O.touch_kv(*np_(k, v, p))
    got = touch_kv(*dev(k, v, p))
    assert got.shape == ref.shape
    np.testing.assert_allclose(got.cpu().numpy(), ref, rtol=1e-4, atol=1e-3)


# ------------------------------------------------------- fused decode step
@pytest.mark.parametrize("hq,hkv,n,b,d,topk,overlap,dtype,union", [
    (32, 8, 2048, 32, 128, 64, 0.9, torch.bfloat16, False),   # c3 shape
    (16, 8, 512, 32, 128, 64, 0.9, torch.bfloat16, True),     # c2 shape, union repair
    (4, 4, 64, 32, 64, 8, 0.75, torch.float16, False),        # c1 shape (G = 1)
    (8, 4, 300, 16, 256, 40, 0.5, torch.bfloat16, False),     # D = 256, one-pass tiles
    (6, 3, 5000, 32, 128, 80, 1.0, torch.float16, False),     # long rows, all hits
    (12, 1, 700, 16, 64, 20, 0.0, torch.bfloat16, False),     # G = 12, no hits, B = 16
    (8, 2, 400, 64, 128, 32, 0.9, torch.bfloat16, False),     # B = 64: two streamed chunks
    (4, 2, 300, 48, 64, 16, 0.75, torch.float16, False),      # B = 48: three 16-token chunks
    (32, 2, 1000, 32, 128, 64, 0.9, torch.bfloat16, True),    # G = 16: G * SP = 1024
    (8, 2, 200, 16, 64, 20, 0.75, torch.float16, True),       # state rows past SP (D = 64)
])
def test_speculative_step(hq, hkv, n, b, d, topk, overlap, dtype, union):
    """speculative_step: selected IDs bit-exact, prediction states and the
    strict (or union) output against the oracle on the same inputs."""
    from stk_harness.configs import make_qkv, perturb
    from strict_topk import step
    q, k, v, lo, hi = make_qkv(hq, hkv, d, b, n, dtype, True, 20261103 + n)
    qn, kn, vn = np_(q, k, v)
    ref_ids = O.select_blocks(qn, lo.numpy(), hi.numpy(), topk)
    p = perturb(torch.from_numpy(ref_ids), n, topk, overlap, 7)
    pn = p.numpy().astype(np.int64)
    qd, kd, vd, lod, hid, pd = dev(q, k, v, lo, hi, p)
    assert step.supported(qd, kd, lod, topk, pd)
    res = step.speculative_step(qd, kd, vd, lod, hid, pd, topk, union=union)
    assert res.selected.cpu().numpy().tolist() == ref_ids.tolist()
    st = O.block_states(qn, kn, vn, pn)
    np.testing.assert_allclose(res.state.m.cpu().double().numpy(), st.m, rtol=1e-5, atol=1e-5)
    np.testing.assert_allclose(res.state.l.cpu().double().numpy(), st.l, rtol=1e-4, atol=1e-5)
    np.testing.assert_allclose(res.state.u.cpu().double().numpy(), st.u, rtol=1e-4, atol=1e-4)
    if union:
        expected = O.gqa_repair(qn, kn, vn, ref_ids, pn, st, union=True)
    else:
        expected = O.attention(qn, kn, vn, ref_ids)
    check(res.output, expected, ("step", hq, n, union))


@pytest.mark.parametrize("hq,hkv,n,b,d,topk,overlap,dtype,mode,tau,eps,min_rem,tol", [
    (32, 8, 1000, 32, 128, 64, 0.75, torch.bfloat16, "hybrid", 0.2, 0.01, 1e-3, 1e-5),  # c5 shape
    (32, 8, 1000, 32, 128, 64, 0.75, torch.bfloat16, "hybrid", 0.2, 0.0, 1e-3, 1e-5),   # strict
    (8, 2, 3000, 32, 128, 64, 0.6, torch.bfloat16, "hybrid", 0.2, 0.01, 1e-3, 1e-5),    # n > 2048
    (8, 2, 400, 16, 64, 20, 0.5, torch.float16, "hybrid", 0.1, 0.0, 1e-3, 1e-5),        # B = 16
    (16, 8, 512, 32, 128, 64, 0.9, torch.bfloat16, "saved", 0.2, 0.0, 1e-3, 1e-5),      # saved
    (8, 4, 300, 32, 128, 32, 0.5, torch.bfloat16, "hybrid", 0.05, 1.0, 1e-3, 1e-5),     # skip all
    (8, 4, 300, 32, 128, 32, 0.5, torch.bfloat16, "hybrid", 0.05, 0.0, 1.0, 1e-5),      # fallback
    (8, 4, 300, 64, 128, 32, 0.5, torch.bfloat16, "hybrid", 0.05, 0.01, 1e-3, 2.0),     # cancel
])
def test_signed_step(hq, hkv, n, b, d, topk, overlap, dtype, mode, tau, eps, min_rem, tol):
    """speculative_signed_step against the oracle's select || speculate ->
    repair_signed_fused on the same inputs: IDs and job counts exact, guard
    flags exact, outputs within tolerance."""
    from stk_harness.configs import make_qkv, perturb
    from strict_topk import step
    q, k, v, lo, hi = make_qkv(hq, hkv, d, b, n, dtype, True, 20261201 + n + hq)
    qn, kn, vn = np_(q, k, v)
    ref_ids = O.select_blocks(qn, lo.numpy(), hi.numpy(), topk)
    p = perturb(torch.from_numpy(ref_ids), n, topk, overlap, 11)
    pn = p.numpy().astype(np.int64)
    qd, kd, vd, lod, hid, pd = dev(q, k, v, lo, hi, p)
    assert step.supported(qd, kd, lod, topk, pd)
    got = step.speculative_signed_step(qd, kd, vd, lod, hid, pd, topk, mode, tau, min_rem, tol,
                                       eps)
    assert got.selected.cpu().numpy().tolist() == ref_ids.tolist()
    pred = O.speculate(qn, kn, vn, pn, mode, tau, keep_mass=True)
    np.testing.assert_allclose(got.state.m.cpu().double().numpy(), pred.state.m, rtol=1e-5,
                               atol=1e-5)
    np.testing.assert_allclose(got.state.l.cpu().double().numpy(), pred.state.l, rtol=1e-4)
    ref = O.repair_signed_fused(qn, kn, vn, ref_ids, pn, pred, min_rem, tol, eps)
    res = got.result
    assert res.fallback.cpu().numpy().tolist() == ref.fallback.tolist()
    assert res.positive_jobs.cpu().numpy().tolist() == ref.positive_jobs.tolist()
    assert res.total_jobs.cpu().numpy().tolist() == ref.total_jobs.tolist()
    np.testing.assert_allclose(res.remaining.cpu().double().numpy(), ref.remaining, rtol=1e-4,
                               atol=1e-6)
    if eps > 0:
        assert res.approximate_heads.cpu().numpy().tolist() == ref.approximate_heads.tolist()
        np.testing.assert_allclose(res.extra_mass_bound.cpu().double().numpy(),
                                   ref.extra_mass_bound, rtol=1e-4, atol=1e-7)
    else:
        assert res.approximate_heads is None and res.extra_mass_bound is None
    check(res.output, ref.output, ("signed step", mode, n, eps))
    if min_rem == 1.0:
        assert res.fallback.any()


@pytest.mark.parametrize("dtype,b", [(torch.float32, 8), (torch.bfloat16, 8)])
def test_speculative_step_composed_fallback(dtype, b):
    """fp32 inputs with int64 predictions, and blocks whose token count is not
    a multiple of 16, run through the individual kernels."""
    from strict_topk import step
    gen = torch.Generator().manual_seed(9)
    d = 48 if dtype == torch.float32 else 64
    q = torch.randn((4, d), generator=gen).to(dtype)
    k = torch.randn((2, 30, b, d), generator=gen).to(dtype)
    v = torch.randn(k.shape, generator=gen).to(dtype)
    lo, hi = k.amin(2).float(), k.amax(2).float()
    p = torch.stack([torch.randperm(30, generator=gen)[:6] for _ in range(4)])
    qn, kn, vn = np_(q, k, v)
    ref_ids = O.select_blocks(qn, lo.numpy(), hi.numpy(), 6)
    qd, kd, vd, lod, hid, pd = dev(q, k, v, lo, hi, p)
    assert not step.supported(qd, kd, lod, 6, pd)
    res = step.speculative_step(qd, kd, vd, lod, hid, pd, 6)
    assert res.selected.cpu().numpy().tolist() == ref_ids.tolist()
    check(res.output, O.attention(qn, kn, vn, ref_ids), "composed step")


# ------------------------------------------------- paged, batched decode steps
def _paged_batch(hq, hkv, b, d, counts, dtype, seed, topk, sp, overlap=0.75, spare=5):
    """Seeded requests packed into one page pool in a shuffled page order;
    per request: host q, k, v, lo, hi, predicted rows [Hq, sp] and whether
    the dense fused step can serve it (n_r >= topk)."""
    from stk_harness.configs import make_qkv, perturb
    from strict_topk import paged
    reqs = []
    for r, n in enumerate(counts):
        q, k, v, lo, hi = make_qkv(hq, hkv, d, b, n, dtype, True, seed + 97 * r)
        g = torch.Generator().manual_seed(seed + r)
        if n >= topk + sp:
            ref = O.select_blocks(C.f64(q), lo.numpy(), hi.numpy(), topk)
            p = perturb(torch.from_numpy(ref), n, sp, overlap, seed + r)
        else:
            # short request: unique in-range IDs where possible, one slot past
            # the request's blocks (empty state)
            p = torch.stack([torch.randperm(max(n, sp), generator=g)[:sp] for _ in range(hq)])
            p = p.to(torch.int32)
        reqs.append(dict(q=q, k=k, v=v, lo=lo, hi=hi, p=p.to(torch.int32), n=n))
    total = hkv * sum(counts)
    order = torch.randperm(total, generator=torch.Generator().manual_seed(seed))
    kv = paged.pack([(r_["k"].to(DEV), r_["v"].to(DEV)) for r_ in reqs], order=order,
                    spare=spare)
    q = torch.stack([r_["q"] for r_ in reqs]).to(DEV)
    p = torch.stack([r_["p"] for r_ in reqs]).to(DEV)
    return reqs, kv, q, p


def _oracle_ids(p, n):
    pn = C.ids_np(p).copy()
    pn[pn >= n] = -1
    return pn


@pytest.mark.parametrize("hq,hkv,b,d,counts,topk,sp,dtype,union", [
    (32, 8, 32, 128, (1000, 64, 40, 2100, 300), 64, 64, torch.bfloat16, False),  # c5-like
    (8, 2, 16, 64, (200, 17, 700), 20, 24, torch.float16, True),        # union, B = 16
    (12, 1, 64, 128, (130, 500), 32, 32, torch.bfloat16, False),        # G = 12, B = 64
])
def test_paged_step(hq, hkv, b, d, counts, topk, sp, dtype, union):
    """The batched paged step: per request, IDs bit-exact against the oracle
    (a short request selects all its blocks, then -1), states and output
    bit-identical to the dense fused step on the request's own blocks where
    that step applies, and the output against FP64 attention over the
    selected blocks (or the oracle's union repair) everywhere."""
    from strict_topk import paged, step
    reqs, kv, q, p = _paged_batch(hq, hkv, b, d, counts, dtype, 20261215 + hq, topk, sp)
    res = paged.speculative_step(q, kv, p, topk, union=union)
    torch.cuda.synchronize()
    assert res.selected.shape == (len(counts), hq, topk)
    for r, rq in enumerate(reqs):
        qn, kn, vn = np_(rq["q"], rq["k"], rq["v"])
        n = rq["n"]
        pn = _oracle_ids(rq["p"], n)
        lo_p, hi_p = (t.cpu().numpy() for t in (kv.lo_pages, kv.hi_pages))
        tab, nbk = kv.block_table.cpu().numpy(), kv.nblocks.cpu().numpy()
        ids = O.paged_select(qn, lo_p, hi_p, tab, nbk, r, topk)
        assert res.selected[r].cpu().numpy().tolist() == ids.tolist(), r
        st = O.block_states(qn, kn, vn, pn)
        np.testing.assert_allclose(res.state.m[r].cpu().double().numpy(), st.m, rtol=1e-5,
                                   atol=1e-5)
        np.testing.assert_allclose(res.state.l[r].cpu().double().numpy(), st.l, rtol=1e-4,
                                   atol=1e-5)
        sel = [row[row >= 0] for row in ids]
        if union:
            expected = O.gqa_repair(qn, kn, vn, np.stack(sel), pn, st, union=True)
        else:
            expected = O.attention(qn, kn, vn, sel)
        check(res.output[r], expected, ("paged", r, n))
        if n >= topk:
            qd, kd, vd, lod, hid, pd = dev(rq["q"], rq["k"], rq["v"], rq["lo"], rq["hi"],
                                           rq["p"])
            dense = step.speculative_step(qd, kd, vd, lod, hid, pd, topk, union=union)
            assert torch.equal(dense.selected, res.selected[r])
            assert torch.equal(dense.state.m, res.state.m[r])
            assert torch.equal(dense.state.l, res.state.l[r])
            assert torch.equal(dense.state.u, res.state.u[r])
            assert torch.equal(dense.output, res.output[r]), ("dense vs paged", r)


@pytest.mark.parametrize("eps", [0.01, 0.0])
def test_paged_signed_step(eps):
    """The batched signed step against the dense signed step (bit-identical
    fields) and, for a request shorter than K, against the oracle's
    select || speculate -> repair_signed_fused over all its blocks."""
    from strict_topk import paged, step
    hq, hkv, b, d, topk, sp, tau = 32, 8, 32, 128, 64, 32, 0.2
    counts = (900, 40, 2500, 256)
    reqs, kv, q, p = _paged_batch(hq, hkv, b, d, counts, torch.bfloat16, 20261222, topk, sp,
                                  overlap=0.6)
    res = paged.speculative_signed_step(q, kv, p, topk, "hybrid", tau, max_extra_mass=eps)
    torch.cuda.synchronize()
    out = res.result
    for r, rq in enumerate(reqs):
        n = rq["n"]
        if n >= topk:
            qd, kd, vd, lod, hid, pd = dev(rq["q"], rq["k"], rq["v"], rq["lo"], rq["hi"],
                                           rq["p"])
            dn = step.speculative_signed_step(qd, kd, vd, lod, hid, pd, topk, "hybrid", tau,
                                              max_extra_mass=eps)
            assert torch.equal(dn.selected, res.selected[r])
            assert torch.equal(dn.state.u, res.state.u[r])
            for f in ("output", "fallback", "remaining", "positive_jobs", "total_jobs"):
                assert torch.equal(getattr(dn.result, f), getattr(out, f)[r]), (r, f)
            if eps > 0:
                assert torch.equal(dn.result.approximate_heads, out.approximate_heads[r])
                assert torch.equal(dn.result.extra_mass_bound, out.extra_mass_bound[r])
        qn, kn, vn = np_(rq["q"], rq["k"], rq["v"])
        pn = C.ids_np(rq["p"])
        sel = np.tile(np.arange(n), (hq, 1)) if n < topk else \
            O.select_blocks(qn, rq["lo"].numpy(), rq["hi"].numpy(), topk)
        assert res.selected[r, :, :min(n, topk)].cpu().numpy().tolist() == sel.tolist()
        pred = O.speculate(qn, kn, vn, pn, "hybrid", tau, keep_mass=True)
        ref = O.repair_signed_fused(qn, kn, vn, sel, pn, pred, max_extra_mass=eps)
        assert out.fallback[r].cpu().numpy().tolist() == ref.fallback.tolist(), r
        check(out.output[r], ref.output, ("paged signed", r, n))


def test_paged_exact_invalid_pages_and_graph():
    """The serial path over a paged batch (no prediction); invalid pages
    (-1 and past the pool) are never read and score lowest; one captured
    graph serves new block counts and tables written on the device between
    replays."""
    from strict_topk import paged
    hq, hkv, b, d, topk = 8, 2, 32, 128, 16
    counts = (120, 9, 300)
    reqs, kv, q, _ = _paged_batch(hq, hkv, b, d, counts, torch.bfloat16, 20261229, topk, 8)

    def expect(r, sel_ids, tab, nbk, invalid=None):
        rq = reqs[r]
        qn, kn, vn = np_(rq["q"], rq["k"], rq["v"])
        ids = O.paged_select(qn, *(t.cpu().numpy() for t in (kv.lo_pages, kv.hi_pages)), tab,
                             nbk, r, topk, invalid=invalid)
        assert sel_ids.cpu().numpy().tolist() == ids.tolist(), r
        n = int(nbk[r])
        return O.attention(qn, kn[:, :n], vn[:, :n], [row[row >= 0] for row in ids])

    sel, out = paged.exact(q, kv, topk)
    tab, nbk = kv.block_table.cpu().numpy(), kv.nblocks.cpu().numpy()
    for r in range(len(counts)):
        check(out[r], expect(r, sel[r], tab, nbk), ("exact", r))
    # invalid pages in request 2: block 5 of KV head 1 (-1), block 2 of KV
    # head 0 (past the pool); they must never be chosen, nor read
    kv.block_table[2, 1, 5] = -1
    kv.block_table[2, 0, 2] = kv.pages + 7
    inv = np.zeros((hkv, counts[2]), bool)
    inv[1, 5] = inv[0, 2] = True
    sel, out = paged.exact(q, kv, topk)
    tab = kv.block_table.cpu().numpy()
    tab_ok = tab.copy()
    tab_ok[tab_ok < 0] = 0
    tab_ok[tab_ok >= kv.pages] = 0
    check(out[2], expect(2, sel[2], tab_ok, nbk, invalid=inv), "invalid pages")
    # graph: capture once, then shorten request 0 and lengthen nothing else
    g, (gsel, gout) = _capture(lambda: paged.exact(q, kv, topk))
    for n0 in (120, 50, 16, 5):
        kv.nblocks[0] = n0
        g.replay()
        torch.cuda.synchronize()
        nbk = kv.nblocks.cpu().numpy()
        check(gout[0], expect(0, gsel[0], tab_ok, nbk), ("graph", n0))


def test_paged_append_matches_packing():
    """Decode appends into a paged pool: writing each request's last block
    token by token (one launch per token for the whole batch, the positions a
    device tensor advanced between the calls of one captured graph) leaves
    the pages, the lo/hi pages and the block counts equal to packing the
    complete caches; after a partial block, that page's bounds are the
    min / max of its tokens so far."""
    from strict_topk import paged
    hkv, b, d = 2, 16, 64
    counts = (5, 2, 9)
    gen = torch.Generator().manual_seed(77)
    full = [(torch.randn((hkv, n, b, d), generator=gen).half(),
             torch.randn((hkv, n, b, d), generator=gen).half()) for n in counts]
    order = torch.randperm(hkv * sum(counts), generator=gen)
    ref = paged.pack([(k.to(DEV), v.to(DEV)) for k, v in full], order=order, spare=3)
    # the same pool with every last block zeroed and the counts one short
    part = []
    for k, v in full:
        k2, v2 = k.clone(), v.clone()
        k2[:, -1].zero_()
        v2[:, -1].zero_()
        part.append((k2.to(DEV), v2.to(DEV)))
    kv = paged.pack(part, order=order, spare=3)
    kv.nblocks.sub_(1)
    start = torch.tensor([(n - 1) * b for n in counts], dtype=torch.int32, device=DEV)
    pos = start.clone()
    kn = torch.empty((len(counts), hkv, d), dtype=torch.float16, device=DEV)
    vn = torch.empty_like(kn)

    def feed(t):
        kn.copy_(torch.stack([k[:, -1, t] for k, _ in full]))
        vn.copy_(torch.stack([v[:, -1, t] for _, v in full]))

    feed(0)
    g, _ = _capture(lambda: paged.append(kv, kn, vn, pos))   # writes token 0 (capture + replay)
    for t in range(1, b):
        pos.copy_(start + t)
        feed(t)
        g.replay()
        torch.cuda.synchronize()
        if t == 6:
            for r, n in enumerate(counts):
                for h in range(hkv):
                    page = int(kv.block_table[r, h, n - 1])
                    toks = full[r][0][h, -1, :t + 1].float()
                    assert torch.equal(kv.lo_pages[page].cpu(), toks.amin(0))
                    assert torch.equal(kv.hi_pages[page].cpu(), toks.amax(0))
    assert kv.nblocks.cpu().tolist() == list(counts)
    assert torch.equal(kv.k_pages, ref.k_pages) and torch.equal(kv.v_pages, ref.v_pages)
    assert torch.equal(kv.lo_pages, ref.lo_pages) and torch.equal(kv.hi_pages, ref.hi_pages)
    # a position past the table writes nothing
    before = kv.k_pages.clone()
    paged.append(kv, kn, vn, torch.full_like(pos, max(counts) * b))
    torch.cuda.synchronize()
    assert torch.equal(before, kv.k_pages)


def test_poisoned_workspace(monkeypatch):
    """Every workspace handed to the library is filled with 0xFF bytes (NaN as
    floats, the highest key as integers) instead of left as it comes: a
    kernel that read scratch it did not write, even with a zero weight,
    would turn the output into NaN here.  Covers the hierarchical repairs
    (a partial last group of positions), the fused and signed steps and a
    paged batch."""
    from stk_harness.configs import make_qkv, perturb
    from strict_topk import _lib, gqa_hierarchical as impl, paged, step
    monkeypatch.setattr(_lib, "workspace", lambda nbytes, device: torch.full(
        (max(int(nbytes), 1),), 255, dtype=torch.uint8, device=device))
    for (h, hkv, n, b, d, sa), *ts in C.hier_cases(torch.bfloat16):
        qn, kn, vn, an = np_(*ts)
        expected = O.attention(qn, kn, vn, an)
        q, k, v, a = dev(*ts)
        check(impl.exact(q, k, v, a), expected, ("poisoned exact", n, sa))
        for hits in (1, sa // 2, sa):
            p = C.prediction_rows(a.cpu(), n, sa, hits).to(DEV)
            check(impl.repair_saved(q, k, v, a, p, impl.partials(q, k, v, p)), expected,
                  ("poisoned saved", n, sa, hits))
    for hq, hkv, n, b, d, topk, dt in [(32, 8, 2048, 32, 128, 64, torch.bfloat16),
                                       (8, 2, 200, 16, 64, 20, torch.float16)]:
        q, k, v, lo, hi = make_qkv(hq, hkv, d, b, n, dt, True, 99 + n)
        qn, kn, vn = np_(q, k, v)
        ids = O.select_blocks(qn, lo.numpy(), hi.numpy(), topk)
        p = perturb(torch.from_numpy(ids), n, topk, 0.75, 5)
        qd, kd, vd, lod, hid, pd = dev(q, k, v, lo, hi, p)
        res = step.speculative_step(qd, kd, vd, lod, hid, pd, topk)
        check(res.output, O.attention(qn, kn, vn, ids), ("poisoned step", n))
        sres = step.speculative_signed_step(qd, kd, vd, lod, hid, pd, topk, "hybrid", 0.2,
                                            max_extra_mass=0.01)
        assert torch.isfinite(sres.result.output).all()
    reqs, kv, q, p = _paged_batch(8, 2, 16, 64, (200, 17, 700), torch.float16, 4242, 20, 24)
    sel, out = paged.exact(q, kv, 20)
    assert torch.isfinite(out).all()
    res = paged.speculative_step(q, kv, p, 20)
    assert torch.isfinite(res.output).all()
    assert torch.equal(res.selected, sel)


def _poisoned_caches(hq, hkv, b, d, counts, tokens, dtype, seed, hot_last=True):
    """Per request q, k, v with every token at or past its token count set to
    NaN (so any weight on such a token would show), the partly filled last
    block's live keys pointed along the query so that it ranks high."""
    from stk_harness.configs import make_qkv
    out = []
    for r, (n, t) in enumerate(zip(counts, tokens)):
        q, k, v, _, _ = make_qkv(hq, hkv, d, b, n, dtype, True, seed + 31 * r)
        part = t - (n - 1) * b
        if hot_last:
            qm = q.float().view(hkv, hq // hkv, d).mean(1)
            k[:, n - 1, :part] = (k[:, n - 1, :part].float() +
                                  60.0 * (qm / qm.norm(dim=-1, keepdim=True))[:, None]).to(dtype)
        k[:, n - 1, part:] = float("nan")
        v[:, n - 1, part:] = float("nan")
        out.append((q, k, v, n, t))
    return out


def test_paged_partial_last_block():
    """A request whose last block is partly filled (ntokens): the tokens past
    its count hold NaN and must get no weight anywhere -- the pool's bounds,
    the selection, the predicted states (the last block is a hit for some
    heads and a miss for others), the serial path, the saved step and the
    strict signed step all match the oracle restricted to the live tokens."""
    from strict_topk import paged
    hq, hkv, b, d, topk, sp = 8, 2, 32, 128, 16, 16
    counts = (60, 20, 130)
    tokens = (59 * 32 + 5, 19 * 32 + 31, 129 * 32 + 1)
    reqs = _poisoned_caches(hq, hkv, b, d, counts, tokens, torch.bfloat16, 20261301)
    order = torch.randperm(hkv * sum(counts), generator=torch.Generator().manual_seed(3))
    kv = paged.pack([(k.to(DEV), v.to(DEV)) for _, k, v, _, _ in reqs], order=order, spare=2,
                    tokens=tokens)
    assert kv.ntokens.cpu().tolist() == list(tokens)
    gen = torch.Generator().manual_seed(8)
    preds = []
    for _, _, _, n, _ in reqs:
        rows = []
        for h in range(hq):
            row = torch.randperm(n - 1, generator=gen)[:sp - 1]
            # the partial block predicted for even heads only
            extra = n - 1 if h % 2 == 0 else int(torch.randperm(n - 1, generator=gen)[0])
            while h % 2 and extra in row.tolist():
                extra = (extra + 1) % (n - 1)
            rows.append(torch.cat([row, torch.tensor([extra])]))
        preds.append(torch.stack(rows).to(torch.int32))
    q = torch.stack([r[0] for r in reqs]).to(DEV)
    p = torch.stack(preds).to(DEV)
    lo_p, hi_p = (t.cpu().numpy() for t in (kv.lo_pages, kv.hi_pages))
    tab, nbk = kv.block_table.cpu().numpy(), kv.nblocks.cpu().numpy()
    sel_x, out_x = paged.exact(q, kv, topk)
    res = paged.speculative_step(q, kv, p, topk)
    sres = paged.speculative_signed_step(q, kv, p, topk, "hybrid", 0.2)
    torch.cuda.synchronize()
    for r, (qh, k, v, n, t) in enumerate(reqs):
        qn, kn, vn = np_(qh, k, v)
        part = t - (n - 1) * b
        for h in range(hkv):
            page = int(tab[r, h, n - 1])
            np.testing.assert_array_equal(lo_p[page], kn[h, n - 1, :part].min(0))
            np.testing.assert_array_equal(hi_p[page], kn[h, n - 1, :part].max(0))
        ids = O.paged_select(qn, lo_p, hi_p, tab, nbk, r, topk)
        assert (ids == n - 1).any(), "the partial block should be selected somewhere"
        expected = O.attention(qn, kn, vn, ids, tokens=t)
        assert sel_x[r].cpu().numpy().tolist() == ids.tolist(), r
        assert res.selected[r].cpu().numpy().tolist() == ids.tolist(), r
        check(out_x[r], expected, ("paged exact, partial block", r))
        check(res.output[r], expected, ("paged step, partial block", r))
        check(sres.result.output[r], expected, ("paged signed strict, partial block", r))
        st = O.block_states(qn, kn, vn, C.ids_np(preds[r]), tokens=t)
        np.testing.assert_allclose(res.state.m[r].cpu().double().numpy(), st.m, rtol=1e-5,
                                   atol=1e-5)
        np.testing.assert_allclose(res.state.l[r].cpu().double().numpy(), st.l, rtol=1e-4,
                                   atol=1e-5)
        np.testing.assert_allclose(res.state.u[r].cpu().double().numpy(), st.u, rtol=1e-4,
                                   atol=1e-4)


def test_paged_append_then_step_on_a_partial_block():
    """Decode loop: append six tokens into a fresh last block (the rest of its
    page holds NaN), then run the serial path and the saved step: both equal
    the oracle over the live tokens, and the counts say six tokens."""
    from strict_topk import paged
    hq, hkv, b, d, topk = 4, 2, 16, 64, 8
    counts = (40, 12)
    gen = torch.Generator().manual_seed(21)
    full = [(torch.randn((hkv, n, b, d), generator=gen).half(),
             torch.randn((hkv, n, b, d), generator=gen).half()) for n in counts]
    q = torch.randn((len(counts), hq, d), generator=gen).half()
    part = []
    for k, v in full:
        k2, v2 = k.clone(), v.clone()
        k2[:, -1] = float("nan")
        v2[:, -1] = float("nan")
        part.append((k2.to(DEV), v2.to(DEV)))
    kv = paged.pack(part)
    kv.nblocks.sub_(1)
    kv.ntokens.copy_(kv.nblocks * b)
    kn_ = torch.empty((len(counts), hkv, d), dtype=torch.float16, device=DEV)
    vn_ = torch.empty_like(kn_)
    live = 6
    for t in range(live):
        kn_.copy_(torch.stack([k[:, -1, t] for k, _ in full]))
        vn_.copy_(torch.stack([v[:, -1, t] for _, v in full]))
        pos = torch.tensor([(n - 1) * b + t for n in counts], dtype=torch.int32, device=DEV)
        paged.append(kv, kn_, vn_, pos)
    torch.cuda.synchronize()
    assert kv.nblocks.cpu().tolist() == list(counts)
    assert kv.ntokens.cpu().tolist() == [(n - 1) * b + live for n in counts]
    lo_p, hi_p = (t.cpu().numpy() for t in (kv.lo_pages, kv.hi_pages))
    tab, nbk = kv.block_table.cpu().numpy(), kv.nblocks.cpu().numpy()
    qd = q.to(DEV)
    p = torch.stack([torch.stack([torch.randperm(n, generator=gen)[:topk] for _ in range(hq)])
                     for n in (min(counts),) * len(counts)]).to(torch.int32)
    p[:, 0, 0] = torch.tensor([n - 1 for n in counts], dtype=torch.int32)   # predicted partial
    p[:, 0, 1:] = torch.arange(1, topk, dtype=torch.int32)
    sel, out = paged.exact(qd, kv, topk)
    res = paged.speculative_step(qd, kv, p.to(DEV), topk)
    torch.cuda.synchronize()
    for r, (k, v) in enumerate(full):
        n = counts[r]
        tok = (n - 1) * b + live
        qn = C.f64(q[r])
        kn, vn = C.f64(k), C.f64(v)
        ids = O.paged_select(qn, lo_p, hi_p, tab, nbk, r, topk)
        expected = O.attention(qn, kn, vn, ids, tokens=tok)
        assert sel[r].cpu().numpy().tolist() == ids.tolist()
        assert res.selected[r].cpu().numpy().tolist() == ids.tolist()
        check(out[r], expected, ("append then exact", r))
        check(res.output[r], expected, ("append then step", r))


def test_masks_and_bounds_reject_host_tensors():
    """Masks and bound arrays that are not on the query's device (or not
    contiguous) are rejected before any launch."""
    from strict_topk import bounds, kernels
    gen = torch.Generator().manual_seed(2)
    q = torch.randn((2, 64), generator=gen).half().to(DEV)
    k = torch.randn((2, 6, 16, 64), generator=gen).half().to(DEV)
    ids = torch.tensor([[0, 1], [2, 3]], dtype=torch.int32, device=DEV)
    with pytest.raises(ValueError, match="active"):
        kernels.block_partials(q, k, k, ids, active=torch.ones((2,), dtype=torch.bool))
    st = kernels.block_partials(q, k, k, ids)
    with pytest.raises(ValueError, match="include"):
        kernels.merge_partials(st, include=torch.ones((2, 2), dtype=torch.bool))
    with pytest.raises(ValueError, match="include"):
        kernels.merge_partials(st, include=torch.ones((2, 4), dtype=torch.bool,
                                                      device=DEV)[:, ::2])
    lo, hi = bounds.block_bounds(k)
    with pytest.raises(ValueError, match="lo and hi"):
        bounds.append(lo.cpu(), hi.cpu(), k[:, 0, 0].contiguous(), 0, 0)
    with pytest.raises(ValueError, match="lo and hi"):
        bounds.append(lo.transpose(0, 1).contiguous().transpose(0, 1), hi,
                      k[:, 0, 0].contiguous(), 0, 0)


@pytest.mark.parametrize("hq,hkv,n,b,d,topk,dtype", [
    (32, 8, 2048, 32, 128, 64, torch.bfloat16),    # c3
    (8, 4, 300, 16, 64, 20, torch.float16),
    (8, 4, 300, 32, 256, 40, torch.bfloat16),
])
def test_16bit_bounds_give_the_same_results(hq, hkv, n, b, d, topk, dtype):
    """Bounds kept in K's own 16-bit type are exact (min / max of 16-bit keys),
    so every entry point that takes them returns exactly what it returns with
    FP32 bounds: the builder, the append, the selection extension, the saved,
    signed and allocation-free steps, and a paged batch."""
    from stk_harness.configs import make_qkv, perturb
    from strict_topk import bounds, gqa, paged, step
    q, k, v, lo, hi = make_qkv(hq, hkv, d, b, n, dtype, True, 4040 + n)
    ids = O.select_blocks(C.f64(q), lo.numpy(), hi.numpy(), topk)
    p = perturb(torch.from_numpy(ids), n, topk, 0.75, 3)
    qd, kd, vd, pd = dev(q, k, v, p)
    lo32, hi32 = bounds.block_bounds(kd)
    lo16, hi16 = bounds.block_bounds(kd, dtype=dtype)
    assert lo16.dtype == dtype and torch.equal(lo16.float(), lo32) and torch.equal(hi16.float(), hi32)
    assert torch.equal(lo32.cpu(), lo) and torch.equal(hi32.cpu(), hi)
    sel32 = gqa.select_blocks(qd, lo32, hi32, topk)
    assert torch.equal(step.select_blocks(qd, lo16, hi16, topk), sel32)
    assert sel32.cpu().numpy().tolist() == ids.tolist()
    r32 = step.speculative_step(qd, kd, vd, lo32, hi32, pd, topk)
    r16 = step.speculative_step(qd, kd, vd, lo16, hi16, pd, topk)
    for a, b_ in ((r32.selected, r16.selected), (r32.state.u, r16.state.u), (r32.output, r16.output)):
        assert torch.equal(a, b_)
    s32 = step.speculative_signed_step(qd, kd, vd, lo32, hi32, pd, topk, "hybrid", 0.2,
                                       max_extra_mass=0.01)
    s16 = step.speculative_signed_step(qd, kd, vd, lo16, hi16, pd, topk, "hybrid", 0.2,
                                       max_extra_mass=0.01)
    assert torch.equal(s32.selected, s16.selected)
    for f in ("output", "fallback", "remaining", "total_jobs", "extra_mass_bound"):
        assert torch.equal(getattr(s32.result, f), getattr(s16.result, f)), f
    na = step.speculative_step_noalloc(qd, kd, vd, lo16, hi16, pd, topk)
    assert torch.equal(na.selected, r32.selected) and torch.equal(na.output, r32.output)
    ser = step.serial_step(qd, kd, vd, lo16, hi16, topk)
    assert torch.equal(ser[0], sel32)
    check(ser[1], O.attention(*np_(q, k, v), ids), "serial step, 16-bit bounds")
    # a paged pool with 16-bit bounds
    kv32 = paged.pack([(kd, vd)])
    kv16 = paged.pack([(kd, vd)], bounds_dtype=dtype)
    assert torch.equal(kv16.lo_pages.float(), kv32.lo_pages)
    a32 = paged.speculative_step(qd[None], kv32, pd[None], topk)
    a16 = paged.speculative_step(qd[None], kv16, pd[None], topk)
    assert torch.equal(a32.selected, a16.selected) and torch.equal(a32.output, a16.output)
    # append into 16-bit bounds equals append into FP32 bounds
    kn = kd[:, 5, 3].contiguous()
    bounds.append(lo32, hi32, kn, 5, 0)
    bounds.append(lo16, hi16, kn, 5, 0)
    bounds.append(lo32, hi32, kd[:, 5, 7].contiguous(), 5, 1)
    bounds.append(lo16, hi16, kd[:, 5, 7].contiguous(), 5, 1)
    assert torch.equal(lo16.float(), lo32) and torch.equal(hi16.float(), hi32)


def test_16bit_bounds_select_unaligned_dims():
    """The selection extension with 16-bit bounds on a head dimension that is
    not a multiple of 64 (element-wise bound loads)."""
    from strict_topk import gqa, step
    gen = torch.Generator().manual_seed(12)
    q = torch.randn((6, 48), generator=gen).half()
    keys = torch.randn((3, 40, 8, 48), generator=gen).half()
    lo, hi = keys.amin(2), keys.amax(2)
    ref = O.select_blocks(*np_(q, lo.float(), hi.float()), 9)
    qd, lod, hid = dev(q, lo, hi)
    got = step.select_blocks(qd, lod, hid, 9)
    assert got.cpu().numpy().tolist() == ref.tolist()
    assert torch.equal(got, gqa.select_blocks(qd, lod.float(), hid.float(), 9))
    with pytest.raises(ValueError, match="FP32"):
        gqa.select_blocks(qd, lod, hid, 9)   # the reference contract stays FP32
