"""FP64 CPU oracle for the speculative block-sparse Top-K decode path.

TEST INFRASTRUCTURE ONLY.  Nothing in the product path imports this module:
only ``tests/``, ``__graft_entry__.smoke()`` and the ``cpu_baseline`` leg of
``bench.py`` use it, and only as the checker.  The HIP library never falls
back to it.

Every function restates one piece of the reference algorithm
(``6Mikao9/strict-topk-overlap``, files under ``strict_topk/``) in float64
numpy and cites the reference lines it follows.  Inputs are the *quantized*
fp16/bf16/fp32 values converted exactly to float64, as in the reference's own
oracle (``tests/check_correctness.py:12-17``).

Layouts (reference ``strict_topk/kernels.py:1-6``, ``strict_topk/gqa.py:1-6``):
  q[Hq, D]; k, v[Hkv, N, B, D] with Hq % Hkv == 0 and query head h reading
  KV head h // (Hq // Hkv); lo, hi[Hkv, N, D]; ids[Hq, S] (unique, valid).

Selection contract (this build's, stricter than the reference's
``torch.topk(sorted=False)``, whose order and tie choice are unspecified):
  * the bound score of ``bound_scores`` is evaluated in float64 in one fixed
    summation order (``SCORE_LANES`` interleaved lane sums, then an xor
    butterfly), so the GPU scorer and this oracle produce identical bits;
  * ``topk_ids`` returns the K entries with the highest score, ties broken
    toward the lower block index, emitted in ascending block index order;
    NaN ranks below -inf.

Pinning: ``tests/test_oracle.py`` checks each function against the
reference's known-answer tests (``tests/check_gqa.py:65-70``,
``tests/check_signed_repair.py:29-56``, ``tests/check_correctness.py:64-135``,
``tests/check_selector.py:13``), against closed forms (strict repairs equal
FP64 attention over the selected set; epsilon repairs equal attention over
the kept set; merged block states equal direct attention) and against brute
force on tiny inputs (membership, compact ranking and capacity, top-K by
exhaustive sort).
"""
from __future__ import annotations

import math
from dataclasses import dataclass

import numpy as np

NEG_INF = -np.inf
SCORE_LANES = 16      # lanes that share one block's dot product in the scorer
SCORE_VEC = 4         # consecutive dims each lane owns per 64-dim pass


# ---------------------------------------------------------------------------
# containers (reference strict_topk/kernels.py:13-39, signed_repair.py:12-15)
# ---------------------------------------------------------------------------
@dataclass
class State:
    m: np.ndarray
    l: np.ndarray
    u: np.ndarray


@dataclass
class Prediction:
    state: State
    mode: str
    high: np.ndarray | None = None
    low: State | None = None
    retained_ids: np.ndarray | None = None
    overflow: np.ndarray | None = None
    low_abs: np.ndarray | None = None
    mass_m: np.ndarray | None = None
    mass_l: np.ndarray | None = None


@dataclass
class Repair:
    output: np.ndarray
    fallback: np.ndarray
    remaining: np.ndarray
    approximate_heads: np.ndarray | None = None
    extra_mass_bound: np.ndarray | None = None
    positive_jobs: np.ndarray | None = None
    total_jobs: np.ndarray | None = None


def _f64(x):
    return np.asarray(x, dtype=np.float64)


def _group(q, k):
    hq, hkv = q.shape[0], k.shape[0]
    assert hq % hkv == 0
    return hq // hkv


def _scale(d):
    # reference: logits * D ** -0.5 (strict_topk/kernels.py:58, gqa.py:272)
    return float(d) ** -0.5


def _exp(x):
    with np.errstate(invalid="ignore", over="ignore"):
        return np.exp(x)


def _sub(a, b):
    """a - b with -inf - -inf treated as -inf (an empty state has weight 0)."""
    with np.errstate(invalid="ignore"):
        r = np.subtract(a, b)
    return np.where(np.isnan(r) & np.isneginf(a), NEG_INF, r)


# ---------------------------------------------------------------------------
# shared-selection indexer (QSA formula), reference
# benchmarks/selector_window.py:126-142 and the shared top-K :76-84
# ---------------------------------------------------------------------------
def indexer_scores(iq, ik):
    """score[n] = sum_h relu(iq_h . ik_n) / sqrt(D), in the build's fixed FP64
    order: 16 partial sums over consecutive sixteenths of the dims
    (ceil(D/16) each, in order), combined as a pairwise tree ((s0 + s1) +
    (s2 + s3) and so on); relu keeps NaN; heads summed in order from 0.0;
    times 1 / sqrt(D) (the reference's D**-.5)."""
    iq = np.asarray(iq, dtype=np.float64)
    ik = np.asarray(ik, dtype=np.float64)
    h, d = iq.shape
    lanes = 16
    qd = (d + lanes - 1) // lanes
    sc = np.zeros(ik.shape[0])
    for hh in range(h):
        parts = []
        for p in range(lanes):
            d0, d1 = min(d, p * qd), min(d, p * qd + qd)
            acc = np.zeros(ik.shape[0])
            for i in range(d0, d1):
                acc = acc + ik[:, i] * iq[hh, i]
            parts.append(acc)
        while len(parts) > 1:
            parts = [parts[i] + parts[i + 1] for i in range(0, len(parts), 2)]
        tot = parts[0]
        sc = sc + np.where((tot > 0) | np.isnan(tot), tot, 0.0)
    return sc * (1.0 / math.sqrt(d))


def indexer_select(iq, ik, topk, rows):
    """The shared selection: top-K of the indexer scores (ties to the lower
    index, ascending IDs), the same row for every query head."""
    ids = topk_ids(indexer_scores(iq, ik)[None, :], topk)[0]
    return np.repeat(ids[None, :], rows, axis=0)


# ---------------------------------------------------------------------------
# block metadata (the reference harness builds it outside the step)
# ---------------------------------------------------------------------------
def block_bounds(k):
    """lo, hi[Hkv, N, D] = per-block minimum / maximum of k[Hkv, N, B, D] over
    the B tokens (reference harness: k.amin(dim=2).float() / k.amax(dim=2),
    benchmarks/critical_path.py:186).  NaN propagates, as in torch."""
    k = np.asarray(k, dtype=np.float64)
    return k.min(axis=2), k.max(axis=2)


# ---------------------------------------------------------------------------
# A1/A2: min/max query-sign bound score
# reference strict_topk/selector.py:8-20 (_score) and strict_topk/gqa.py:15-26
# (_bound_score): score[h,n] = sum_d q_d * (q_d >= 0 ? hi : lo)[h // G, n, d]
# ---------------------------------------------------------------------------
def bound_scores(q, lo, hi):
    """Float64 bound scores in the contract's fixed summation order.

    Products q_d * bound_d are exact in float64 (fp16/bf16/fp32 times fp32).
    Lane c (0..15) sums dims 64*j + 4*c + t (j ascending, then t = 0..3)
    starting from +0.0; lanes then combine by acc[c] += acc[c ^ off] for
    off = 8, 4, 2, 1.  A zero result is canonicalised to +0.0.
    """
    q, lo, hi = _f64(q), _f64(lo), _f64(hi)
    hq, d = q.shape
    hkv, n, d2 = lo.shape
    assert d2 == d and hi.shape == lo.shape and hq % hkv == 0
    g = hq // hkv
    passes = (d + 63) // 64
    lanes = np.arange(SCORE_LANES)
    out = np.empty((hq, n))
    for h in range(hq):
        qh = q[h]
        bound = np.where(qh >= 0, hi[h // g], lo[h // g])
        prod = np.zeros((n, passes * 64))
        prod[:, :d] = bound * qh
        prod = prod.reshape(n, passes, SCORE_LANES, SCORE_VEC)
        acc = np.zeros((n, SCORE_LANES))
        for j in range(passes):
            for t in range(SCORE_VEC):
                acc = acc + prod[:, j, :, t]
        for off in (8, 4, 2, 1):
            acc = acc + acc[:, lanes ^ off]
        s = acc[:, 0]
        out[h] = np.where(s == 0, 0.0, s)
    return out


def bound_scores_plain(q, lo, hi):
    """The reference test oracle's form (tests/check_selector.py:15,
    tests/check_gqa.py:201-202): float64 where/mul/sum, numpy's own order."""
    q, lo, hi = _f64(q), _f64(lo), _f64(hi)
    g = q.shape[0] // lo.shape[0]
    kv = np.arange(q.shape[0]) // g
    qr = q[:, None, :]
    return (np.where(qr >= 0, hi[kv], lo[kv]) * qr).sum(-1)


def topk_ids(scores, k):
    """Top-k block IDs per row, ties toward the lower index, ascending IDs.

    Restates the reference's ``scores.topk(k, sorted=False)``
    (strict_topk/gqa.py:161, selector.py:43) with the lower-index tie rule of
    ``argsort(descending, stable=True)`` (experiments/predictor_rank_trace.py:24-25).
    """
    scores = _f64(scores)
    h, n = scores.shape
    if k > n:
        raise ValueError("k exceeds the number of blocks")
    idx = np.arange(n)
    out = np.empty((h, k), dtype=np.int64)
    for r in range(h):
        s = scores[r]
        nan = np.isnan(s)
        primary = np.where(nan, np.inf, -s)
        order = np.lexsort((idx, nan, primary))
        out[r] = np.sort(order[:k])
    return out


def select_blocks(q, lo, hi, k):
    return topk_ids(bound_scores(q, lo, hi), k)


# ---------------------------------------------------------------------------
# attention over ID sets: tests/check_correctness.py:12-17,
# tests/check_gqa.py:10-17, benchmarks/critical_path.py:16-25 (include mask)
# ---------------------------------------------------------------------------
def _live(rows, b, tokens):
    """[S, B] mask of the tokens that hold data: token t of block j when
    j * B + t < tokens (every token when tokens is None)."""
    if tokens is None:
        return np.ones((len(rows), b), bool)
    return (np.asarray(rows, np.int64)[:, None] * b + np.arange(b)[None, :]) < int(tokens)


def attention(q, k, v, ids, include=None, tokens=None):
    """FP64 softmax attention of each head over its ID row (rows may differ
    in length when ``ids`` is a list).  ``tokens``: the sequence's token
    count, for a partly filled last block (the paged format's ntokens);
    tokens at or past it get no weight and their values are ignored."""
    q, k, v = _f64(q), _f64(k), _f64(v)
    rows = [np.asarray(r, dtype=np.int64) for r in ids]
    g = _group(q, k)
    hq, d = q.shape
    out = np.empty((hq, d))
    for h in range(hq):
        kk = k[h // g][rows[h]]
        vv = v[h // g][rows[h]]
        logits = (kk @ q[h]) / math.sqrt(d)
        live = _live(rows[h], k.shape[2], tokens)
        logits = np.where(live, logits, NEG_INF)
        vv = np.where(live[..., None], vv, 0.0)
        if include is not None:
            logits = np.where(np.asarray(include[h], bool)[:, None], logits, NEG_INF)
        mx = logits.max()
        w = np.exp(logits - mx)
        w = w / w.sum()
        out[h] = np.einsum("sb,sbd->d", w, vv)
    return out


# ---------------------------------------------------------------------------
# A5/A11: per-block softmax states
# reference strict_topk/kernels.py:42-71 (_partial), gqa.py:29-59
# ---------------------------------------------------------------------------
def _one_state(qh, kb, vb, d, live=None):
    s = (kb @ qh) * _scale(d)
    if live is not None:
        if not live.any():
            return NEG_INF, 0.0, np.zeros(d)
        s = np.where(live, s, NEG_INF)
        vb = np.where(live[:, None], vb, 0.0)
    m = s.max()
    w = np.exp(s - m)
    return m, w.sum(), w @ vb


def block_states(q, k, v, ids, active=None, with_values=True, tokens=None):
    """Per-block states of every (head, listed block); ``tokens`` as in
    ``attention`` (a block with no token holding data has the empty state)."""
    q, k, v = _f64(q), _f64(k), _f64(v)
    ids = np.asarray(ids, dtype=np.int64)
    g = _group(q, k)
    hq, d = q.shape
    s = ids.shape[1]
    m = np.full((hq, s), NEG_INF)
    l = np.zeros((hq, s))
    u = np.zeros((hq, s, d))
    for h in range(hq):
        for j in range(s):
            if active is not None:
                act = np.asarray(active, bool)
                on = act[h] if act.ndim == 1 else act[h, j]
                if not on:
                    continue
            b = ids[h, j]
            if b < 0:
                continue
            live = None if tokens is None else _live([b], k.shape[2], tokens)[0]
            mm, ll, uu = _one_state(q[h], k[h // g, b], v[h // g, b], d, live)
            m[h, j], l[h, j] = mm, ll
            if with_values:
                u[h, j] = uu
    return State(m, l, u)


# A6: reference strict_topk/kernels.py:74-91 (_merge), 437-447
def merge_states(state, include=None):
    m, l, u = state.m, state.l, state.u
    h, s, d = u.shape
    mask = np.ones((h, s), bool) if include is None else np.asarray(include, bool)
    mm = np.where(mask, m, NEG_INF)
    ll = np.where(mask, l, 0.0)
    uu = np.where(mask[:, :, None], u, 0.0)
    top = mm.max(axis=1, keepdims=True)
    top = np.where(np.isneginf(top), 0.0, top)
    a = _exp(_sub(mm, top))
    z = (a * ll).sum(1)
    return (a[:, :, None] * uu).sum(1) / np.maximum(z, 1e-30)[:, None]


def exact_attention(q, k, v, selected):
    return merge_states(block_states(q, k, v, selected))


# ---------------------------------------------------------------------------
# A7: speculate saved/hybrid, reference strict_topk/kernels.py:94-117, 450-477
# ---------------------------------------------------------------------------
def _hybrid_group(state, tau):
    m, l, u = state.m, state.l, state.u
    h, s, d = u.shape
    high = np.zeros((h, s), bool)
    lm = np.zeros((h, 1))
    ll = np.zeros((h, 1))
    lu = np.zeros((h, 1, d))
    labs = np.zeros((h, d))
    for r in range(h):
        gm = m[r].max()
        mass = _exp(_sub(m[r], gm)) * l[r]
        total = mass.sum()
        high[r] = mass >= tau * total
        low = ~high[r]
        lmr = m[r][low].max() if low.any() else NEG_INF
        lmr = 0.0 if lmr == NEG_INF else lmr
        alpha = np.where(low, _exp(_sub(m[r], lmr)), 0.0)
        lm[r, 0] = lmr
        ll[r, 0] = (alpha * l[r]).sum()
        lu[r, 0] = (alpha[:, None] * u[r]).sum(0)
        labs[r] = (alpha[:, None] * np.abs(u[r])).sum(0)
    return high, State(lm, ll, lu), labs


def compact_capacity(s, tau):
    """reference strict_topk/kernels.py:485"""
    return s if tau <= 1 / s else min(s, int(1 / tau) + 1)


def speculate(q, k, v, predicted, mode="saved", mass_threshold=0.1, keep_mass=False):
    if mode not in ("saved", "hybrid", "compact"):
        raise ValueError(mode)
    if not 0 <= mass_threshold <= 1:
        raise ValueError("mass_threshold must be in [0,1]")
    if mode == "compact":
        return _speculate_compact(q, k, v, predicted, mass_threshold, keep_mass)
    st = block_states(q, k, v, predicted)
    mm, ml = (st.m, st.l) if keep_mass else (None, None)
    if mode == "saved":
        return Prediction(st, mode, mass_m=mm, mass_l=ml)
    high, low, labs = _hybrid_group(st, mass_threshold)
    return Prediction(st, mode, high, low, low_abs=labs, mass_m=mm, mass_l=ml)


# A8: reference strict_topk/kernels.py:263-356, 480-501
def _speculate_compact(q, k, v, predicted, tau, keep_mass):
    q, k, v = _f64(q), _f64(k), _f64(v)
    predicted = np.asarray(predicted, dtype=np.int64)
    g = _group(q, k)
    hq, d = q.shape
    s = predicted.shape[1]
    c = compact_capacity(s, tau)
    mass_state = block_states(q, k, v, predicted, with_values=False)
    pm, pl = mass_state.m, mass_state.l
    high = np.zeros((hq, s), bool)
    rids = np.full((hq, c), -1, dtype=np.int64)
    overflow = np.zeros(hq, bool)
    lm = np.zeros((hq, 1))
    ll = np.zeros((hq, 1))
    lu = np.zeros((hq, 1, d))
    labs = np.zeros((hq, d))
    for h in range(hq):
        mass = np.exp(pm[h] - pm[h].max()) * pl[h]
        hi_ = mass >= tau * mass.sum()
        rank = np.cumsum(hi_)
        count = int(hi_.sum())
        overflow[h] = count > c
        hi_ = hi_ & (rank <= c)
        high[h] = hi_
        for pos in np.nonzero(hi_)[0]:
            rids[h, rank[pos] - 1] = predicted[h, pos]
        low = ~hi_
        lmr = pm[h][low].max() if low.any() else 0.0
        lm[h, 0] = lmr
        ll[h, 0] = np.where(low, np.exp(pm[h] - lmr) * pl[h], 0.0).sum()
        # slot 0 walks the low blocks in position order, per token, in the
        # low frame, with an absolute envelope (kernels.py:320-336)
        for pos in np.nonzero(low)[0]:
            b = predicted[h, pos]
            s_t = (k[h // g, b] @ q[h]) * _scale(d)
            wv = np.exp(s_t - lmr)[:, None] * v[h // g, b]
            lu[h, 0] += wv.sum(0)
            labs[h] += np.abs(wv).sum(0)
    state = block_states(q, k, v, rids)
    mm, ml = (pm, pl) if keep_mass else (None, None)
    return Prediction(state, "compact", high, State(lm, ll, lu), rids, overflow, labs, mm, ml)


# ---------------------------------------------------------------------------
# membership helpers (reference kernels.py:120-143, 359-381; fused.py:62-66)
# ---------------------------------------------------------------------------
def membership(p_row, a_row):
    """hit[p] = P[p] in A; miss[a] = A[a] not in P (brute-force equality)."""
    p_row = np.asarray(p_row, dtype=np.int64)
    a_row = np.asarray(a_row, dtype=np.int64)
    eq = p_row[:, None] == a_row[None, :]
    return eq.any(1), ~eq.any(0)


def slot_table(p_row, a_row):
    """slot[a] = max{p : P[p] == A[a]} or -1 (gqa.py:42, gqa_hierarchical.py:10-19)."""
    p_row = np.asarray(p_row, dtype=np.int64)
    out = np.full(len(a_row), -1, dtype=np.int64)
    for j, a in enumerate(np.asarray(a_row, dtype=np.int64)):
        hits = np.nonzero(p_row == a)[0]
        if len(hits):
            out[j] = hits.max()
    return out


def _online(qh, k, v, blocks, d, start=(NEG_INF, 0.0, None), fixed_m=None):
    """Sequential online softmax over blocks (kernels.py:223-247, fused.py:10-45).

    With fixed_m, weights are exp(s - fixed_m) without rescaling."""
    m, z, u = start
    u = np.zeros(d) if u is None else u.copy()
    for b in blocks:
        s = (k[b] @ qh) * _scale(d)
        if fixed_m is not None:
            w = np.exp(s - fixed_m)
            z = z + w.sum()
            u = u + w @ v[b]
            continue
        nm = max(m, s.max())
        alpha = 0.0 if m == NEG_INF else math.exp(m - nm)
        w = np.exp(s - nm)
        u = u * alpha + w @ v[b]
        z = z * alpha + w.sum()
        m = nm
    return m, z, u


def _nonfinite(x):
    return not np.all(np.isfinite(x))


# ---------------------------------------------------------------------------
# A9: split repair, reference strict_topk/kernels.py:504-550 with
# _saved_merge :146-168, _hybrid_merge :171-220, _wrong_aggregate :384-407,
# _fallback :223-247
# ---------------------------------------------------------------------------
def repair(q, k, v, selected, predicted, pred, min_remaining=1e-3, cancellation_tol=1e-5):
    q, k, v = _f64(q), _f64(k), _f64(v)
    a_ids = np.asarray(selected, dtype=np.int64)
    p_ids = np.asarray(predicted, dtype=np.int64)
    g = _group(q, k)
    hq, d = q.shape
    out = np.zeros((hq, d))
    bad = np.zeros(hq, bool)
    rem = np.ones(hq)
    hybrid = pred.mode in ("hybrid", "compact")
    for h in range(hq):
        kk, vv = k[h // g], v[h // g]
        phit, miss = membership(p_ids[h], a_ids[h])
        if pred.mode == "compact":
            r = pred.retained_ids[h]
            hit = np.array([(x >= 0) and (x in set(a_ids[h].tolist())) for x in r])
        else:
            hit = phit.copy()
        low_hit = False
        wrong = np.zeros(len(p_ids[h]), bool)
        if hybrid:
            high = pred.high[h]
            low_hit = bool((phit & ~high).any())
            wrong = ~phit & ~high & low_hit
            if pred.mode != "compact":
                hit = phit & high
        # miss states (block_partials with the miss mask)
        am = np.full(len(a_ids[h]), NEG_INF)
        al = np.zeros(len(a_ids[h]))
        au = np.zeros((len(a_ids[h]), d))
        for j in np.nonzero(miss)[0]:
            am[j], al[j], au[j] = _one_state(q[h], kk[a_ids[h, j]], vv[a_ids[h, j]], d)
        pm = np.where(hit, pred.state.m[h], NEG_INF)
        pl = np.where(hit, pred.state.l[h], 0.0)
        pu = np.where(hit[:, None], pred.state.u[h], 0.0)
        if not hybrid:
            mx = max(pm.max(), am.max())
            ap, ax = _exp(_sub(pm, mx)), _exp(_sub(am, mx))
            z = (ap * pl).sum() + (ax * al).sum()
            out[h] = ((ap[:, None] * pu).sum(0) + (ax[:, None] * au).sum(0)) / z
            continue
        lm = pred.low.m[h, 0]
        if pred.mode == "compact":
            # one aggregate of wrong blocks in the low frame
            _, wz, wu = _online(q[h], kk, vv, [p_ids[h, j] for j in np.nonzero(wrong)[0]], d,
                                start=(lm, 0.0, None), fixed_m=lm)
            wm = np.array([lm if low_hit else NEG_INF])
            wl = np.array([wz if low_hit else 0.0])
            wuu = np.array([wu]) if low_hit else np.zeros((1, d))
        else:
            wm = np.full(len(p_ids[h]), NEG_INF)
            wl = np.zeros(len(p_ids[h]))
            wuu = np.zeros((len(p_ids[h]), d))
            if low_hit:
                for j in np.nonzero(wrong)[0]:
                    wm[j], wl[j], wuu[j] = _one_state(q[h], kk[p_ids[h, j]], vv[p_ids[h, j]], d)
        mx = max(pm.max(), am.max())
        mx = max(mx, lm if low_hit else NEG_INF)
        ap, ax, aw = _exp(_sub(pm, mx)), _exp(_sub(am, mx)), _exp(_sub(wm, mx))
        lowalpha = math.exp(lm - mx) if low_hit else 0.0
        ll = (pred.low.l[h, 0] if low_hit else 0.0) * lowalpha
        removed = (aw * wl).sum()
        remaining = ll - removed
        fraction = remaining / max(ll, 1e-30) if ll > 0 else 1.0
        z = remaining + (ap * pl).sum() + (ax * al).sum()
        lu = (pred.low.u[h, 0] if low_hit else np.zeros(d)) * lowalpha
        removed_u = (aw[:, None] * wuu).sum(0)
        residual = lu - removed_u
        labs = (pred.low_abs[h] if low_hit else np.zeros(d)) * lowalpha
        scale = labs + np.abs(removed_u)
        cancel = (np.abs(residual) < cancellation_tol * scale) & (scale > 0) & low_hit
        u = residual + (ap[:, None] * pu).sum(0) + (ax[:, None] * au).sum(0)
        o = u / max(z, 1e-30)
        b = (z <= 0) or (fraction < min_remaining) or math.isnan(fraction) or math.isinf(z)
        b = b or bool(cancel.any()) or _nonfinite(o)
        if b:
            _, fz, fu = _online(q[h], kk, vv, a_ids[h], d)
            o = fu / fz
        out[h], bad[h], rem[h] = o, b, fraction
    return Repair(out, bad, rem)


# ---------------------------------------------------------------------------
# A10: fused repair, reference strict_topk/fused.py:48-173, 176-220
# ---------------------------------------------------------------------------
def repair_fused(q, k, v, selected, predicted, pred, min_remaining=1e-3,
                 cancellation_tol=1e-5, max_extra_mass=0.0):
    if not 0 <= max_extra_mass <= 1:
        raise ValueError("max_extra_mass must be in [0, 1]")
    hybrid = pred.mode in ("hybrid", "compact")
    compact = pred.mode == "compact"
    if hybrid and max_extra_mass > 0 and (pred.mass_m is None or pred.mass_l is None):
        raise ValueError("positive max_extra_mass requires speculate(..., keep_mass=True)")
    q, k, v = _f64(q), _f64(k), _f64(v)
    a_ids = np.asarray(selected, dtype=np.int64)
    p_ids = np.asarray(predicted, dtype=np.int64)
    g = _group(q, k)
    hq, d = q.shape
    out = np.zeros((hq, d))
    bad_all = np.zeros(hq, bool)
    rem = np.ones(hq)
    approx = np.zeros(hq, bool)
    extra = np.zeros(hq)
    for h in range(hq):
        kk, vv = k[h // g], v[h // g]
        hit, missing = membership(p_ids[h], a_ids[h])
        fraction, bad, skip, extra_bound = 1.0, False, False, 0.0
        residual = np.zeros(d)
        mass = 0.0
        lm = NEG_INF
        if hybrid:
            high = pred.high[h]
            low_hit = bool((hit & ~high).any())
            retained_hit = hit & high
        else:
            retained_hit = hit
        if compact:
            aset = set(a_ids[h].tolist())
            keep = np.array([x in aset for x in pred.retained_ids[h].tolist()])
        else:
            keep = retained_hit
        pm = np.where(keep, pred.state.m[h], NEG_INF)
        pl = np.where(keep, pred.state.l[h], 0.0)
        retained_m = pm.max()
        if hybrid and low_hit:
            lm = pred.low.m[h, 0]
            ll = pred.low.l[h, 0]
            lu = pred.low.u[h, 0]
            labs = pred.low_abs[h]
            wrong = ~hit & ~high
            removed, removed_u = 0.0, np.zeros(d)
            if max_extra_mass > 0 and wrong.any():
                ref = max(retained_m, lm)
                wm = np.where(wrong, pred.mass_m[h], NEG_INF)
                wl = np.where(wrong, pred.mass_l[h], 0.0)
                wrong_mass = (_exp(_sub(wm, ref)) * wl).sum()
                denom = math.exp(lm - ref) * ll + (_exp(_sub(pm, ref)) * pl).sum()
                extra_bound = wrong_mass / denom
                skip = extra_bound <= max_extra_mass
            if wrong.any() and not skip:
                _, removed, removed_u = _online(q[h], kk, vv, p_ids[h][wrong], d,
                                                start=(lm, 0.0, None), fixed_m=lm)
            mass = ll - removed
            residual = lu - removed_u
            fraction = mass / ll
            scale = labs + np.abs(removed_u)
            cancel = (np.abs(residual) < cancellation_tol * scale) & (scale > 0)
            bad = (fraction < min_remaining) or math.isnan(fraction) or bool(cancel.any())
        pu = np.where(keep[:, None], pred.state.u[h], 0.0)
        mx = max(retained_m, lm)
        ref = 0.0 if mx == NEG_INF else mx
        alpha = _exp(_sub(pm, ref))
        low_alpha = 0.0 if lm == NEG_INF else math.exp(lm - ref)
        z = (alpha * pl).sum() + low_alpha * mass
        u = (alpha[:, None] * pu).sum(0) + low_alpha * residual
        todo = a_ids[h][missing]
        if hybrid and bad:
            todo, mx, z, u = a_ids[h], NEG_INF, 0.0, np.zeros(d)
        if len(todo):
            mx, z, u = _online(q[h], kk, vv, todo, d, start=(mx, z, u))
        with np.errstate(divide="ignore", invalid="ignore"):
            o = u / z
        if hybrid:
            bad_output = (z <= 0) or math.isinf(z) or _nonfinite(o)
            if bad_output and not bad:
                _, z, u = _online(q[h], kk, vv, a_ids[h], d)
                o = u / z
            bad = bad or bad_output
        out[h], bad_all[h], rem[h] = o, bad, fraction
        if max_extra_mass > 0:
            approx[h] = skip and not bad
            extra[h] = extra_bound if approx[h] else 0.0
    if max_extra_mass > 0:
        return Repair(out, bad_all, rem, approx, extra)
    return Repair(out, bad_all, rem)


# ---------------------------------------------------------------------------
# A14: signed job queue, reference strict_topk/signed_repair.py:18-82
# ---------------------------------------------------------------------------
@dataclass
class Schedule:
    queue: list          # per head: list of block IDs (misses then wrong-low)
    pos: np.ndarray      # positive (miss) job count
    total: np.ndarray
    keep: np.ndarray     # [H, SC]
    low_hit: np.ndarray
    approx: np.ndarray
    extra: np.ndarray


def schedule(selected, predicted, pred, max_extra_mass=0.0):
    a_ids = np.asarray(selected, dtype=np.int64)
    p_ids = np.asarray(predicted, dtype=np.int64)
    hybrid = pred.mode in ("hybrid", "compact")
    compact = pred.mode == "compact"
    hq = a_ids.shape[0]
    sc = pred.state.m.shape[1]
    queue, pos, total = [], np.zeros(hq, np.int64), np.zeros(hq, np.int64)
    keep = np.zeros((hq, sc), bool)
    low_hit = np.zeros(hq, bool)
    approx = np.zeros(hq, bool)
    extra = np.zeros(hq)
    for h in range(hq):
        hit, miss = membership(p_ids[h], a_ids[h])
        jobs = list(a_ids[h][miss])
        pos[h] = len(jobs)
        if hybrid:
            high = pred.high[h]
            low_hit[h] = bool((hit & ~high).any())
            wrong = low_hit[h] & ~hit & ~high
            retained_hit = hit & high
        else:
            retained_hit = hit
        if compact:
            aset = set(a_ids[h].tolist())
            keep[h] = [x in aset for x in pred.retained_ids[h].tolist()]
        else:
            keep[h] = retained_hit
        skip, ex = False, 0.0
        if hybrid:
            if max_extra_mass > 0 and wrong.any():
                lm, ll = pred.low.m[h, 0], pred.low.l[h, 0]
                pm = np.where(keep[h], pred.state.m[h], NEG_INF)
                pl = np.where(keep[h], pred.state.l[h], 0.0)
                wm = np.where(wrong, pred.mass_m[h], NEG_INF)
                wl = np.where(wrong, pred.mass_l[h], 0.0)
                ref = max(lm, pm.max())
                denom = math.exp(lm - ref) * ll + (_exp(_sub(pm, ref)) * pl).sum()
                ex = (_exp(_sub(wm, ref)) * wl).sum() / denom
                skip = ex <= max_extra_mass
            wrong = wrong & (not skip)
            jobs += list(p_ids[h][wrong])
        queue.append(jobs)
        total[h] = len(jobs)
        approx[h] = skip
        extra[h] = ex if skip else 0.0
    return Schedule(queue, pos, total, keep, low_hit, approx, extra)


def _signed_common(q, k, v, selected, predicted, pred, min_remaining,
                   cancellation_tol, max_extra_mass, fused):
    if not 0 <= max_extra_mass <= 1:
        raise ValueError("max_extra_mass must be in [0,1]")
    hybrid = pred.mode in ("hybrid", "compact")
    compact = pred.mode == "compact"
    if hybrid and max_extra_mass > 0 and (pred.mass_m is None or pred.mass_l is None):
        raise ValueError("positive max_extra_mass requires speculate(..., keep_mass=True)")
    q, k, v = _f64(q), _f64(k), _f64(v)
    a_ids = np.asarray(selected, dtype=np.int64)
    g = _group(q, k)
    hq, d = q.shape
    sch = schedule(selected, predicted, pred, max_extra_mass)
    out = np.zeros((hq, d))
    bad_all = np.zeros(hq, bool)
    rem = np.ones(hq)
    approx = sch.approx.copy()
    extra = sch.extra.copy()
    for h in range(hq):
        kk, vv = k[h // g], v[h // g]
        keep = sch.keep[h]
        pm = np.where(keep, pred.state.m[h], NEG_INF)
        pl = np.where(keep, pred.state.l[h], 0.0)
        pu = np.where(keep[:, None], pred.state.u[h], 0.0)
        npos = int(sch.pos[h])
        jobs = sch.queue[h]
        cm = np.full(len(jobs), NEG_INF)
        cl = np.zeros(len(jobs))
        cu = np.zeros((len(jobs), d))
        lm = pred.low.m[h, 0] if hybrid else None
        for j, b in enumerate(jobs):
            negative = hybrid and j >= npos
            s = (kk[b] @ q[h]) * _scale(d)
            bm = s.max()
            if fused and compact and negative:
                # signed_fused.py:44-47: compact negatives in the low frame
                w = np.exp(s - lm)
                den, num, sc_ = w.sum(), w @ vv[b], lm
            else:
                w = np.exp(s - bm)
                den, num, sc_ = w.sum(), w @ vv[b], bm
                if fused and hybrid and not compact and negative:
                    # signed_fused.py:52-61: block-local then rescale
                    f = math.exp(bm - lm)
                    den, num, sc_ = den * f, num * f, lm
            sign = -1.0 if negative else 1.0
            cm[j], cl[j], cu[j] = sc_, sign * den, sign * num
        positive = np.arange(len(jobs)) < npos
        fraction, b_ = 1.0, False
        low_m, low_l, low_u = NEG_INF, 0.0, np.zeros(d)
        if hybrid and sch.low_hit[h]:
            low_m = lm
            ol, ou = pred.low.l[h, 0], pred.low.u[h, 0]
            env = pred.low_abs[h]
            neg = ~positive
            if fused:
                # signed_fused.py:331-336: negatives already in the low frame
                wx = np.where(neg, 1.0, 0.0)
            else:
                # signed_repair.py:145: exp(cm - low_m) for negative jobs
                wx = np.where(neg, _exp(_sub(cm, low_m)), 0.0)
            removed_u = (wx[:, None] * cu).sum(0)
            low_l = ol + (wx * cl).sum()
            low_u = ou + removed_u
            fraction = low_l / ol
            scale = env + np.abs(removed_u)
            cancel = (np.abs(low_u) < cancellation_tol * scale) & (scale > 0)
            b_ = (fraction < min_remaining) or math.isnan(fraction) or bool(cancel.any())
        maxpos = np.where(positive, cm, NEG_INF).max() if len(jobs) else NEG_INF
        cmn = max(pm.max(), maxpos, low_m)
        pw = _exp(_sub(pm, cmn))
        aw = _exp(_sub(np.where(positive, cm, NEG_INF), cmn))
        lw = 0.0 if low_m == NEG_INF else math.exp(low_m - cmn)
        den = (pw * pl).sum() + (aw * cl).sum() + lw * low_l
        num = (pw[:, None] * pu).sum(0) + (aw[:, None] * cu).sum(0) + lw * low_u
        with np.errstate(divide="ignore", invalid="ignore"):
            o = num / den
        if hybrid:
            b_ = b_ or _nonfinite(o) or den <= 0 or math.isinf(den)
            if b_:
                _, fz, fu = _online(q[h], kk, vv, a_ids[h], d)
                o = fu / fz
                approx[h] = False
                extra[h] = 0.0
        out[h], bad_all[h], rem[h] = o, b_, fraction
    res = Repair(out, bad_all, rem, None, None, sch.pos.copy(), sch.total.copy())
    if max_extra_mass > 0:
        res.approximate_heads, res.extra_mass_bound = approx, extra
    return res


def repair_signed(q, k, v, selected, predicted, pred, min_remaining=1e-3,
                  cancellation_tol=1e-5, max_extra_mass=0.0):
    """4-launch signed repair, reference strict_topk/signed_repair.py:85-232."""
    return _signed_common(q, k, v, selected, predicted, pred, min_remaining,
                          cancellation_tol, max_extra_mass, fused=False)


def repair_signed_fused(q, k, v, selected, predicted, pred, min_remaining=1e-3,
                        cancellation_tol=1e-5, max_extra_mass=0.0):
    """3-launch signed repair, reference strict_topk/signed_fused.py:30-193."""
    return _signed_common(q, k, v, selected, predicted, pred, min_remaining,
                          cancellation_tol, max_extra_mass, fused=True)


# ---------------------------------------------------------------------------
# A12: GQA saved / union repair, reference strict_topk/gqa.py:62-104, 384-413
# A13: single-launch light repair, reference strict_topk/gqa_light.py:10-92
# ---------------------------------------------------------------------------
def gqa_repair(q, k, v, selected, predicted, state, union=False):
    q, k, v = _f64(q), _f64(k), _f64(v)
    a_ids = np.asarray(selected, dtype=np.int64)
    p_ids = np.asarray(predicted, dtype=np.int64)
    g = _group(q, k)
    hq, d = q.shape
    out = np.zeros((hq, d))
    for h in range(hq):
        slot = slot_table(p_ids[h], a_ids[h])
        ms, ls, us = [], [], []
        for j, b in enumerate(a_ids[h]):
            if slot[j] >= 0 and not union:
                ms.append(state.m[h, slot[j]]); ls.append(state.l[h, slot[j]])
                us.append(state.u[h, slot[j]])
            elif slot[j] < 0:
                mm, ll, uu = _one_state(q[h], k[h // g, b], v[h // g, b], d)
                ms.append(mm); ls.append(ll); us.append(uu)
        if union:
            ms += list(state.m[h]); ls += list(state.l[h]); us += list(state.u[h])
        ms, ls, us = np.array(ms), np.array(ls), np.array(us)
        w = np.exp(ms - ms.max())
        out[h] = (w[:, None] * us).sum(0) / (w * ls).sum()
    return out


def repair_light(q, k, v, selected, predicted, state):
    q, k, v = _f64(q), _f64(k), _f64(v)
    a_ids = np.asarray(selected, dtype=np.int64)
    p_ids = np.asarray(predicted, dtype=np.int64)
    g = _group(q, k)
    hq, d = q.shape
    out = np.zeros((hq, d))
    for h in range(hq):
        hit, miss = membership(p_ids[h], a_ids[h])
        pm = np.where(hit, state.m[h], NEG_INF)
        mx = pm.max()
        px = _exp(_sub(pm, 0.0 if mx == NEG_INF else mx))
        z = (px * np.where(hit, state.l[h], 0.0)).sum()
        u = (px[:, None] * np.where(hit[:, None], state.u[h], 0.0)).sum(0)
        todo = np.sort(a_ids[h][miss])  # ascending block ID (gqa_light.py:44-47)
        mx, z, u = _online(q[h], k[h // g], v[h // g], todo, d, start=(mx, z, u))
        out[h] = u / z
    return out


# ---------------------------------------------------------------------------
# A16-A18: hierarchical reduction, reference strict_topk/gqa_hierarchical.py
# ---------------------------------------------------------------------------
HIER_TILE = 32


def hier_reduce(state, prediction=None, slot=None, shared=False):
    """_groups (:64-96) then merge_partials (:99-108)."""
    m, l, u = state.m.copy(), state.l.copy(), state.u.copy()
    h, s, d = u.shape
    if prediction is not None:
        for r in range(h):
            sl = slot[0 if shared else r]
            hit = sl >= 0
            m[r, hit] = prediction.m[r, sl[hit]]
            l[r, hit] = prediction.l[r, sl[hit]]
            u[r, hit] = prediction.u[r, sl[hit]]
    groups = (s + HIER_TILE - 1) // HIER_TILE
    om = np.empty((h, groups))
    ol = np.empty((h, groups))
    ou = np.empty((h, groups, d))
    for gi in range(groups):
        sl = slice(gi * HIER_TILE, min(s, (gi + 1) * HIER_TILE))
        mx = m[:, sl].max(1)
        w = _exp(_sub(m[:, sl], mx[:, None]))
        om[:, gi] = mx
        ol[:, gi] = (w * l[:, sl]).sum(1)
        ou[:, gi] = (w[:, :, None] * u[:, sl]).sum(1)
    return merge_states(State(om, ol, ou))


def hier_repair(q, k, v, selected, predicted, state, shared=False):
    a_ids = np.asarray(selected, dtype=np.int64)
    p_ids = np.asarray(predicted, dtype=np.int64)
    rows = [0] if shared else range(a_ids.shape[0])
    slot = np.stack([slot_table(p_ids[r], a_ids[r]) for r in rows])
    hq = a_ids.shape[0]
    active = np.stack([slot[0 if shared else r] < 0 for r in range(hq)])
    scratch = block_states(q, k, v, a_ids, active=active)
    return hier_reduce(scratch, state, slot, shared)


# ---------------------------------------------------------------------------
# touch_kv checksum, reference strict_topk/kernels.py:250-260, 553-560
# ---------------------------------------------------------------------------
def touch_kv(k, v, predicted, tile=1024):
    k, v = _f64(k), _f64(v)
    p_ids = np.asarray(predicted, dtype=np.int64)
    h, n, b, d = k.shape
    s = p_ids.shape[1]
    nt = (b * d + tile - 1) // tile
    out = np.zeros((h, s, nt))
    for r in range(h):
        for j in range(s):
            flat = (k[r, p_ids[r, j]] + v[r, p_ids[r, j]]).reshape(-1)
            for t in range(nt):
                out[r, j, t] = flat[t * tile:(t + 1) * tile].sum()
    return out


# ---------------------------------------------------------------------------
# paged, ragged KV: the wire format's definition.  The reference's only page
# mapping is FlashInfer's (strict_topk/flashinfer_backend.py:35-40: page =
# block + kv_head * N over k.view(hkv * n, b, 1, d)), the special case of one
# request with table[kvh, j] = kvh * N + j.
# ---------------------------------------------------------------------------
def gather_pages(pages, table, nblocks, r):
    """Dense [Hkv, n_r, ...] cache of request r from a page pool
    pages[P, ...] and block table[R, Hkv, NB] (n_r = nblocks[r])."""
    pages = np.asarray(pages)
    t = np.asarray(table, dtype=np.int64)[r, :, :int(nblocks[r])]
    return pages[t]


def paged_select(q, lo_pages, hi_pages, table, nblocks, r, k, invalid=None):
    """The batched step's selection for request r: the top-min(k, n_r) of the
    request's blocks (IDs ascending), padded with -1 to k columns.  Blocks on
    an invalid page (``invalid``: a bool mask [Hkv, n_r]) score lowest, below
    every finite score (their 64-bit key is that of NaN)."""
    lo = gather_pages(lo_pages, table, nblocks, r)
    hi = gather_pages(hi_pages, table, nblocks, r)
    scores = bound_scores(q, lo, hi)
    if invalid is not None:
        g = scores.shape[0] // lo.shape[0]
        scores = np.where(np.repeat(np.asarray(invalid), g, axis=0), np.nan, scores)
    n = lo.shape[1]
    kk = min(int(k), n)
    ids = topk_ids(scores, kk) if kk > 0 else np.zeros((scores.shape[0], 0), np.int64)
    out = np.full((scores.shape[0], int(k)), -1, dtype=np.int64)
    out[:, :kk] = ids
    return out
