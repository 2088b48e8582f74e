"""CPU checks that pin the FP64 oracle (oracle/stk_oracle.py).

Pins: the reference's known-answer tests, closed forms (every strict repair
equals FP64 attention over the selected set; epsilon repairs equal attention
over the kept set; merged states equal direct attention), brute force on tiny
inputs, and planted mistakes that must make those checks fail.
"""
import math

import numpy as np
import pytest
import torch

from oracle import stk_oracle as O
from tests import cases as C


def _np(*ts):
    return [C.f64(t) if t.is_floating_point() else C.ids_np(t) for t in ts]


# ------------------------------------------------------------ known answers
def test_tiny_gqa_known_answers():
    """tests/check_gqa.py:65-70: same rows 8 / -5, swapped -5 / 8, union 7.9130."""
    q, k, v, p = _np(*C.tiny_gqa())
    np.testing.assert_allclose(O.attention(q, k, v, p)[:, 0], [8.0, -5.0], rtol=0, atol=1e-12)
    np.testing.assert_allclose(O.attention(q, k, v, 1 - p)[:, 0], [-5.0, 8.0], rtol=0, atol=1e-12)
    union = (8 * math.e ** 5 - 5) / (math.e ** 5 + 1)
    assert abs(union - 7.9130) < 1e-4
    st = O.block_states(q, k, v, p)
    got = O.gqa_repair(q, k, v, 1 - p, p, st, union=True)[:, 0]
    np.testing.assert_allclose(got, [union, union], rtol=1e-12)
    np.testing.assert_allclose(O.gqa_repair(q, k, v, 1 - p, p, st)[:, 0], [-5.0, 8.0], atol=1e-12)
    np.testing.assert_allclose(O.repair_light(q, k, v, 1 - p, p, st)[:, 0], [-5.0, 8.0], atol=1e-12)
    np.testing.assert_allclose(O.repair_light(q, k, v, p, p, st)[:, 0], [8.0, -5.0], atol=1e-12)


@pytest.mark.parametrize("mode", ["hybrid", "compact"])
@pytest.mark.parametrize("impl", ["signed", "signed_fused", "fused"])
def test_extra_mass_budget_known_answers(mode, impl):
    """tests/check_signed_repair.py:29-56."""
    q, k, v, p, a, extra_set = _np(*C.budget_case())
    strict = O.attention(q, k, v, a)
    with_extra = O.attention(q, k, v, extra_set)
    assert abs(strict[0, 0] - 1.5) < 1e-12
    extra_mass = math.exp(-3) / (2 + math.exp(-3))
    assert abs(extra_mass - 0.02429) < 1e-5
    fn = {"signed": O.repair_signed, "signed_fused": O.repair_signed_fused,
          "fused": O.repair_fused}[impl]
    st = O.speculate(q, k, v, p, mode=mode, mass_threshold=.2, keep_mass=True)
    low = fn(q, k, v, a, p, st, max_extra_mass=.01)
    assert not low.approximate_heads[0] and low.extra_mass_bound[0] == 0.0
    np.testing.assert_allclose(low.output, strict, atol=1e-12)
    high = fn(q, k, v, a, p, st, max_extra_mass=.1)
    assert high.approximate_heads[0]
    bound = math.exp(-3) / (1 + math.exp(-3))
    assert abs(high.extra_mass_bound[0] - bound) < 1e-12
    assert extra_mass <= high.extra_mass_bound[0] <= .1
    np.testing.assert_allclose(high.output, with_extra, atol=1e-12)
    forced = fn(q, k, v, a, p, st, cancellation_tol=2., max_extra_mass=.1)
    assert forced.fallback[0] and not forced.approximate_heads[0]
    assert forced.extra_mass_bound[0] == 0.0
    np.testing.assert_allclose(forced.output, strict, atol=1e-12)
    if impl != "fused":
        assert low.positive_jobs[0] == 1 and low.total_jobs[0] == 2
        assert high.positive_jobs[0] == 1 and high.total_jobs[0] == 1


REPAIRS = {"split": O.repair, "fused": O.repair_fused, "signed": O.repair_signed,
           "signed_fused": O.repair_signed_fused}


@pytest.mark.parametrize("impl", list(REPAIRS))
@pytest.mark.parametrize("mode", ["hybrid", "compact"])
def test_expected_fallback_heads(impl, mode):
    """tests/check_correctness.py:128-135 (mass_threshold 1.0)."""
    for name, q, k, v, p, a in C.correctness_cases(torch.float16):
        if name not in C.EXPECTED_FALLBACK:
            continue
        q, k, v, p, a = _np(q, k, v, p, a)
        st = O.speculate(q, k, v, p, mode=mode, mass_threshold=1.0)
        res = REPAIRS[impl](q, k, v, a, p, st)
        assert int(res.fallback.sum()) == C.EXPECTED_FALLBACK[name], (name, impl, mode)
        np.testing.assert_allclose(res.output, O.attention(q, k, v, a), rtol=1e-9, atol=1e-12)


def test_all_zero_query_ties_pick_lower_indices():
    """tests/check_selector.py:13 (q[0] = 0 -> every score ties)."""
    rng = np.random.default_rng(1)
    lo = rng.standard_normal((1, 37, 70)).astype(np.float32)
    hi = lo + 1
    q = np.zeros((1, 70))
    ids = O.select_blocks(q, lo, hi, 11)
    assert ids.tolist() == [list(range(11))]


def test_signed_fused_underflow_regression():
    """tests/check_signed_fused.py:17-30: fallback on the bf16 underflow case."""
    q, k, v, p, a = _np(*C.underflow_case())
    st = O.speculate(q, k, v, p, mode="hybrid", mass_threshold=1.)
    res = O.repair_signed_fused(q, k, v, a, p, st)
    assert res.fallback[0]
    assert C.error_metrics(res.output, O.attention(q, k, v, a))["passed"]


# ------------------------------------------------------------ closed forms
@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
def test_strict_repairs_equal_selected_attention(dtype):
    for name, *ts in C.correctness_cases(dtype):
        q, k, v, p, a = _np(*ts)
        expected = O.attention(q, k, v, a)
        np.testing.assert_allclose(O.exact_attention(q, k, v, a), expected, rtol=1e-9, atol=1e-12)
        for mode, thr in [("saved", .1), ("hybrid", .05), ("hybrid", .2), ("hybrid", 1.),
                          ("compact", .05), ("compact", .2), ("compact", 1.)]:
            st = O.speculate(q, k, v, p, mode=mode, mass_threshold=thr)
            for impl, fn in REPAIRS.items():
                res = fn(q, k, v, a, p, st)
                ok = np.allclose(res.output, expected, rtol=1e-7, atol=1e-9)
                assert ok, (name, mode, thr, impl)


def test_gqa_repairs_equal_closed_forms():
    for name, *ts in C.gqa_cases():
        q, k, v, p, a = _np(*ts)
        st = O.block_states(q, k, v, p)
        expected = O.attention(q, k, v, a)
        hit = (a[:, :, None] == p[:, None, :]).any(-1)
        union_ids = [np.concatenate((p[h], a[h][~hit[h]])) for h in range(len(p))]
        np.testing.assert_allclose(O.gqa_repair(q, k, v, a, p, st, union=True),
                                   O.attention(q, k, v, union_ids), rtol=1e-9, atol=1e-12)
        np.testing.assert_allclose(O.gqa_repair(q, k, v, a, p, st), expected, rtol=1e-9, atol=1e-12)
        np.testing.assert_allclose(O.repair_light(q, k, v, a, p, st), expected, rtol=1e-9, atol=1e-12)
        np.testing.assert_allclose(O.merge_states(O.block_states(q, k, v, a)), expected,
                                   rtol=1e-9, atol=1e-12)


def test_hierarchical_equals_attention():
    for (h, hkv, n, b, d, sa), *ts in C.hier_cases(torch.bfloat16):
        if h > 6:
            continue   # the 24-head shape runs on the GPU tests only
        q, k, v, a = _np(*ts)
        expected = O.attention(q, k, v, a)
        np.testing.assert_allclose(O.hier_reduce(O.block_states(q, k, v, a)), expected,
                                   rtol=1e-9, atol=1e-12)
        for hits in (0, sa // 2, sa):
            p = C.ids_np(C.prediction_rows(torch.from_numpy(a), n, sa, hits))
            st = O.block_states(q, k, v, p)
            np.testing.assert_allclose(O.hier_repair(q, k, v, a, p, st), expected,
                                       rtol=1e-9, atol=1e-12)
        shared = np.repeat(a[:1], h, 0)
        p = C.ids_np(C.prediction_rows(torch.from_numpy(shared), n, max(1, sa // 2), sa // 4))
        st = O.block_states(q, k, v, p)
        np.testing.assert_allclose(O.hier_repair(q, k, v, shared, p, st, shared=True),
                                   O.attention(q, k, v, shared), rtol=1e-9, atol=1e-12)


def test_bound_scores_against_reference_form():
    rng = np.random.default_rng(7)
    for hq, hkv, n, d in [(3, 3, 37, 70), (6, 2, 23, 13), (8, 4, 50, 128), (2, 1, 9, 1)]:
        q = rng.standard_normal((hq, d)).astype(np.float32)
        k = rng.standard_normal((hkv, n, 7, d)).astype(np.float32)
        lo, hi = k.min(2), k.max(2)
        q[0] = 0
        s = O.bound_scores(q, lo, hi)
        np.testing.assert_allclose(s, O.bound_scores_plain(q, lo, hi), rtol=1e-13, atol=1e-12)
        # bf16-representable inputs: every float64 summation order is exact
        qb = torch.from_numpy(q).bfloat16().double().numpy()
        kb = torch.from_numpy(k).bfloat16().double().numpy()
        lo_b, hi_b = kb.min(2), kb.max(2)
        assert np.array_equal(O.bound_scores(qb, lo_b, hi_b), O.bound_scores_plain(qb, lo_b, hi_b))


# ------------------------------------------------------------- brute force
def test_topk_brute_force_with_ties():
    rng = np.random.default_rng(3)
    for _ in range(50):
        n = int(rng.integers(1, 40))
        k = int(rng.integers(0, n + 1))
        s = rng.integers(-3, 4, size=(2, n)).astype(np.float64)
        if rng.random() < .3:
            s[0, rng.integers(0, n)] = np.nan
        got = O.topk_ids(s, k)
        for r in range(2):
            key = [(1 if math.isnan(x) else 0, 0 if math.isnan(x) else -x, i)
                   for i, x in enumerate(s[r])]
            want = sorted(i for _, _, i in sorted(key)[:k])
            assert got[r].tolist() == want


def test_membership_and_slots_brute_force():
    rng = np.random.default_rng(5)
    for _ in range(30):
        n = 40
        p = rng.permutation(n)[:int(rng.integers(1, 12))]
        a = rng.permutation(n)[:int(rng.integers(1, 12))]
        hit, miss = O.membership(p, a)
        assert hit.tolist() == [x in set(a.tolist()) for x in p]
        assert miss.tolist() == [x not in set(p.tolist()) for x in a]
        slots = O.slot_table(p, a)
        for j, x in enumerate(a):
            assert slots[j] == (p.tolist().index(x) if x in p else -1)


def test_compact_capacity_and_ranking():
    assert O.compact_capacity(8, .05) == 8
    assert O.compact_capacity(8, .2) == 6
    assert O.compact_capacity(8, 1.) == 2
    assert O.compact_capacity(8, 0.) == 8
    rng = np.random.default_rng(11)
    q = rng.standard_normal((2, 8))
    k = rng.standard_normal((2, 12, 3, 8)) * 3
    v = rng.standard_normal((2, 12, 3, 8))
    p = np.stack([rng.permutation(12)[:8] for _ in range(2)])
    for tau in (.05, .1, .2, .5):
        pred = O.speculate(q, k, v, p, mode="compact", mass_threshold=tau)
        st = O.block_states(q, k, v, p)
        c = O.compact_capacity(8, tau)
        for h in range(2):
            mass = np.exp(st.m[h] - st.m[h].max()) * st.l[h]
            high = [j for j in range(8) if mass[j] >= tau * mass.sum()]
            assert pred.overflow[h] == (len(high) > c)
            kept = high[:c]
            want = [p[h, j] for j in kept] + [-1] * (c - len(kept))
            assert pred.retained_ids[h].tolist() == want
            assert pred.high[h].tolist() == [j in kept for j in range(8)]


# --------------------------------------------------------- planted mistakes
def test_planted_scale_mistake_is_caught(monkeypatch):
    monkeypatch.setattr(O, "_scale", lambda d: 1.0)
    name, *ts = next(iter(C.correctness_cases(torch.float16)))
    q, k, v, p, a = _np(*ts)
    assert not np.allclose(O.exact_attention(q, k, v, a), O.attention(q, k, v, a), rtol=1e-6)


def test_planted_tie_direction_mistake_is_caught(monkeypatch):
    real = O.topk_ids

    def reversed_ties(scores, k):
        s = np.asarray(scores, dtype=np.float64)
        n = s.shape[1]
        return (n - 1 - real(s[:, ::-1], k))

    lo = np.zeros((1, 20, 4), np.float32)
    ids = reversed_ties(O.bound_scores(np.zeros((1, 4)), lo, lo + 1), 5)
    assert ids.tolist() != [list(range(5))]


def test_planted_low_frame_mistake_is_caught(monkeypatch):
    """Dropping the low-group rescale (alpha) breaks the hybrid closed form."""
    orig = O._hybrid_group

    def broken(state, tau):
        high, low, labs = orig(state, tau)
        low.l[:] = low.l * 2.0
        return high, low, labs

    monkeypatch.setattr(O, "_hybrid_group", broken)
    for name, *ts in C.correctness_cases(torch.float16):
        if name != "many_low_wrong_mass":
            continue
        q, k, v, p, a = _np(*ts)
        st = O.speculate(q, k, v, p, mode="hybrid", mass_threshold=.05)
        res = O.repair_fused(q, k, v, a, p, st)
        assert not np.allclose(res.output, O.attention(q, k, v, a), rtol=1e-6)


def test_block_bounds_pinned_against_torch():
    """Block metadata: the oracle equals torch.amin / amax over the token axis
    (the reference harness's own expression, benchmarks/critical_path.py:186)
    on finite keys and propagates NaN like it; every token lies inside
    [lo, hi] and both bounds are attained."""
    gen = torch.Generator().manual_seed(5)
    k = torch.randn((3, 17, 6, 10), generator=gen).to(torch.bfloat16)
    k[1, 4, 2, 7] = float("nan")
    lo, hi = O.block_bounds(k.float().numpy())
    tl, th = k.amin(dim=2).float().numpy(), k.amax(dim=2).float().numpy()
    assert np.array_equal(lo, tl, equal_nan=True) and np.array_equal(hi, th, equal_nan=True)
    assert np.isnan(lo[1, 4, 7]) and np.isnan(hi[1, 4, 7])
    kf = k.float().numpy()
    ok = ~np.isnan(lo)
    assert ((kf >= lo[:, :, None]) | ~ok[:, :, None]).all()
    assert ((kf <= hi[:, :, None]) | ~ok[:, :, None]).all()
    assert ((kf == lo[:, :, None]).any(2) | ~ok).all()


def test_indexer_scores_pinned_against_reference_formula():
    """QSA indexer: the oracle's fixed-order FP64 scores equal the reference's
    own formula relu(iq @ ik.T).sum(0) / sqrt(D) (benchmarks/selector_window.py:
    78-84, its FP64 check) to FP64 rounding, keep NaN like torch.relu, and the
    shared selection is the brute-force top-K of those scores in every row."""
    gen = torch.Generator().manual_seed(21)
    iq = torch.randn((4, 128), generator=gen).half()
    ik = torch.randn((300, 128), generator=gen).half()
    ref = (torch.relu(iq.double() @ ik.double().T).sum(0) / 128 ** .5).numpy()
    got = O.indexer_scores(iq.numpy(), ik.numpy())
    np.testing.assert_allclose(got, ref, rtol=1e-13, atol=1e-13)
    # an odd width: quarters of ceil(D / 4) dims
    iq2 = torch.randn((3, 13), generator=gen).double()
    ik2 = torch.randn((50, 13), generator=gen).double()
    np.testing.assert_allclose(O.indexer_scores(iq2.numpy(), ik2.numpy()),
                               (torch.relu(iq2 @ ik2.T).sum(0) / 13 ** .5).numpy(),
                               rtol=1e-13, atol=1e-13)
    ik3 = ik.clone().float()
    ik3[7, 3] = float("nan")
    assert np.isnan(O.indexer_scores(iq.float().numpy(), ik3.numpy())[7])
    ids = O.indexer_select(iq.numpy(), ik.numpy(), 20, 5)
    order = sorted(range(300), key=lambda j: (-got[j], j))[:20]
    assert ids.shape == (5, 20) and (ids == np.array(sorted(order))[None, :]).all()


def _pack_np(caches, rng, spare=3):
    """Pack dense caches [(k [Hkv, n_r, B, D]), ...] into pages in a random
    order (numpy, independent of the product's packer)."""
    hkv = caches[0].shape[0]
    total = hkv * sum(c.shape[1] for c in caches)
    width = max(c.shape[1] for c in caches)
    slot = rng.permutation(total)
    pages = np.zeros((total + spare,) + caches[0].shape[2:])
    table = np.full((len(caches), hkv, width), -1, np.int64)
    base = 0
    for r, c in enumerate(caches):
        n = c.shape[1]
        idx = slot[base:base + hkv * n]
        pages[idx] = c.reshape((hkv * n,) + c.shape[2:])
        table[r, :, :n] = idx.reshape(hkv, n)
        base += hkv * n
    return pages, table, np.array([c.shape[1] for c in caches])


def test_paged_gather_and_select_pinned():
    """The paged wire format: gathering a request's pages gives back its dense
    cache (any page order); FlashInfer's mapping (flashinfer_backend.py:35-40,
    page = block + kv_head * N over k.view(hkv * n, b, 1, d)) is the
    one-request table kvh * N + j; the paged selection equals the dense one
    for n_r >= k, is every block plus -1 padding for n_r < k, and never takes
    a block on an invalid page while valid ones remain (brute force)."""
    rng = np.random.default_rng(5)
    hkv, g, b, d = 2, 3, 4, 8
    ks = [rng.standard_normal((hkv, n, b, d)) for n in (9, 3, 14)]
    pages, table, nb = _pack_np(ks, rng)
    for r, k in enumerate(ks):
        assert np.array_equal(O.gather_pages(pages, table, nb, r), k)
    k = ks[2]
    fi = (np.arange(hkv)[:, None] * k.shape[1] + np.arange(k.shape[1])[None, :])[None]
    assert np.array_equal(O.gather_pages(k.reshape(-1, b, d), fi, [k.shape[1]], 0), k)
    lo_p, hi_p = pages.min(1), pages.max(1)
    q = rng.standard_normal((3, hkv * g, d))
    for r, k in enumerate(ks):
        n = k.shape[1]
        for kk in (1, 3, 5, 14):
            got = O.paged_select(q[r], lo_p, hi_p, table, nb, r, kk)
            if kk <= n:
                assert np.array_equal(got, O.select_blocks(q[r], k.min(2), k.max(2), kk))
            else:
                assert np.array_equal(got[:, :n], np.tile(np.arange(n), (hkv * g, 1)))
                assert (got[:, n:] == -1).all()
    # invalid pages: blocks 0 and 5 of KV head 1 of request 2
    inv = np.zeros((hkv, 14), bool)
    inv[1, [0, 5]] = True
    got = O.paged_select(q[2], lo_p, hi_p, table, nb, 2, 6, invalid=inv)
    sc = O.bound_scores(q[2], ks[2].min(2), ks[2].max(2))
    for h in range(hkv * g):
        bad = inv[h // g]
        order = sorted((j for j in range(14) if not bad[j]), key=lambda j: (-sc[h, j], j))[:6]
        assert got[h].tolist() == sorted(order)


def test_token_count_mask_pinned_by_brute_force():
    """attention / block_states with a token count (a partly filled last
    block) equal a token-by-token softmax over exactly the tokens before the
    count, in plain Python; values past the count (NaN here) are ignored;
    with the count at N * B nothing changes."""
    rng = np.random.default_rng(11)
    hkv, g, n, b, d = 2, 2, 5, 4, 3
    q = rng.standard_normal((hkv * g, d))
    k = rng.standard_normal((hkv, n, b, d))
    v = rng.standard_normal((hkv, n, b, d))
    ids = np.array([[4, 0, 2], [1, 4, 3], [4, 2, 0], [3, 1, 4]])
    full = O.attention(q, k, v, ids)
    np.testing.assert_array_equal(O.attention(q, k, v, ids, tokens=n * b), full)
    for tokens in (4 * b + 1, 4 * b + 3, 3 * b + 2):
        kp, vp = k.copy(), v.copy()
        tail = np.arange(n * b).reshape(n, b) >= tokens
        kp[:, tail] = np.nan
        vp[:, tail] = np.nan
        got = O.attention(q, kp, vp, ids, tokens=tokens)
        st = O.block_states(q, kp, vp, ids, tokens=tokens)
        for h in range(hkv * g):
            toks = [(blk, t) for blk in ids[h] for t in range(b) if blk * b + t < tokens]
            logits = [float(np.dot(k[h // g, blk, t], q[h])) / math.sqrt(d) for blk, t in toks]
            mx = max(logits)
            w = [math.exp(x - mx) for x in logits]
            want = sum(wi * v[h // g, blk, t] for wi, (blk, t) in zip(w, toks)) / sum(w)
            np.testing.assert_allclose(got[h], want, rtol=1e-12, atol=1e-12)
            for j, blk in enumerate(ids[h]):
                live = [t for t in range(b) if blk * b + t < tokens]
                if not live:
                    assert st.m[h, j] == -np.inf and st.l[h, j] == 0 and not st.u[h, j].any()
                    continue
                s = [float(np.dot(k[h // g, blk, t], q[h])) / math.sqrt(d) for t in live]
                mm = max(s)
                assert st.m[h, j] == pytest.approx(mm, abs=1e-12)
                assert st.l[h, j] == pytest.approx(sum(math.exp(x - mm) for x in s), rel=1e-12)


@pytest.mark.parametrize("b,d", [(16, 128), (8, 96), (3, 40)])
def test_touch_kv_pinned_against_torch(b, d):
    """touch_kv (reference strict_topk/kernels.py:250-260,553-560): the sum
    of K + V over each 1024-element tile of a predicted block's flattened
    [B, D] rows, the last tile short.  Pinned by a gather + padded view in
    torch (an independent reduction), and by the invariant that a block's
    tiles add up to its whole sum."""
    gen = torch.Generator().manual_seed(b * 1000 + d)
    h, n, s = 3, 9, 4
    k = torch.randn((h, n, b, d), generator=gen, dtype=torch.float64)
    v = torch.randn((h, n, b, d), generator=gen, dtype=torch.float64)
    p = torch.stack([torch.randperm(n, generator=gen)[:s] for _ in range(h)])
    got = O.touch_kv(k.numpy(), v.numpy(), p.numpy())
    nt = -(-b * d // 1024)
    kv = (k + v)[torch.arange(h)[:, None], p].reshape(h, s, b * d)
    ref = torch.nn.functional.pad(kv, (0, nt * 1024 - b * d)).view(h, s, nt, 1024).sum(-1)
    assert got.shape == (h, s, nt)
    np.testing.assert_allclose(got, ref.numpy(), rtol=1e-12, atol=1e-12)
    np.testing.assert_allclose(got.sum(-1), kv.sum(-1).numpy(), rtol=1e-12, atol=1e-12)
