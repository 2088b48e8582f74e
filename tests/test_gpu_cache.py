"""The host-backed cache (strict_topk.hostcache, stk_cache_step) on the GPU.

Three decode steps over a two-request batch whose K/V live in pinned host
memory, with C = G * topk device slots per (request, KV head):
  1. nothing resident: every predicted state is empty, every selected block
     is copied in;
  2. the same query: the selection is resident, nothing is copied, the
     resident predicted blocks have their states;
  3. a new query: part of the selection is copied in over the least recently
     used slots not needed now.
Every step: IDs bit-exact and the output within the reference tolerance of
FP64 attention over the selected blocks (the oracle), every selected block
resident afterwards with its device page equal to its host page, table and
slot map consistent, and the bytes counted equal to the pages copied.
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


def _check_cache(cache, reqs, selected, g, b, d):
    hkv = cache.hkv
    table = cache.table.cpu().numpy()
    sblock = cache.slot_block.cpu().numpy()
    htab = cache.host_table.cpu().numpy()
    c = cache.slots_per_group
    ks, vs = cache.k_slots.cpu(), cache.v_slots.cpu()
    for r in range(len(reqs)):
        for kh in range(hkv):
            grp = r * hkv + kh
            row = table[r, kh]
            # table and slot map agree, slots stay inside the group
            for j in np.nonzero(row >= 0)[0]:
                s = row[j]
                assert grp * c <= s < (grp + 1) * c and sblock[s] == j
            for s in range(grp * c, (grp + 1) * c):
                if sblock[s] >= 0:
                    assert row[sblock[s]] == s
            # every selected block of the group's heads is resident and equal
            ids = np.unique(selected[r, kh * g:(kh + 1) * g])
            ids = ids[ids >= 0]
            assert (row[ids] >= 0).all()
            for j in ids:
                hp = htab[r, kh, j]
                assert torch.equal(ks[row[j]], cache.host_k[hp])
                assert torch.equal(vs[row[j]], cache.host_v[hp])


def test_host_cache_steps():
    from stk_harness.configs import make_qkv, perturb
    from strict_topk import hostcache
    hq, hkv, b, d, topk, sp = 8, 2, 32, 128, 16, 16
    g = hq // hkv
    counts = (300, 130)
    reqs = []
    for r, n in enumerate(counts):
        q, k, v, lo, hi = make_qkv(hq, hkv, d, b, n, torch.bfloat16, True, 777 + r)
        reqs.append(dict(q=q, k=k, v=v, lo=lo, hi=hi, n=n))
    cache = hostcache.build([(x["k"], x["v"]) for x in reqs], g * topk, device=DEV,
                            bounds_dtype=torch.bfloat16)
    page = 2 * b * d * 2
    gen = torch.Generator().manual_seed(5)
    queries = [torch.stack([x["q"] for x in reqs])]
    queries.append(queries[0])
    queries.append(torch.randn(queries[0].shape, generator=gen).to(torch.bfloat16))
    resident_before = [np.full((hkv, max(counts)), -1)] * len(reqs)
    h2d_prev = 0
    for step, qb in enumerate(queries):
        print(f"cache step {step}", flush=True)
        ids, preds = [], []
        for r, x in enumerate(reqs):
            a = O.select_blocks(C.f64(qb[r]), x["lo"].numpy(), x["hi"].numpy(), topk)
            ids.append(a)
            preds.append(perturb(torch.from_numpy(a), x["n"], sp, 0.75, 40 + step + r))
        table_before = cache.table.cpu().numpy()
        res = hostcache.speculative_step(qb.to(DEV), cache, torch.stack(preds).to(DEV), topk)
        torch.cuda.synchronize()
        sel = res.selected.cpu().numpy()
        for r, x in enumerate(reqs):
            assert sel[r].tolist() == ids[r].tolist(), (step, r)
            qn, kn, vn = C.f64(qb[r]), C.f64(x["k"]), C.f64(x["v"])
            m = C.error_metrics(C.f64(res.output[r]), O.attention(qn, kn, vn, ids[r]))
            assert m["passed"], (step, r, m)
            # prediction states: those of the blocks resident when the step
            # began, empty for the others
            pn = C.ids_np(preds[r])
            st = O.block_states(qn, kn, vn, pn)
            kv_of = np.arange(hq) // g
            was = table_before[r][kv_of[:, None], pn] >= 0
            got_m = res.state.m[r].cpu().double().numpy()
            np.testing.assert_allclose(got_m[was], st.m[was], rtol=1e-5, atol=1e-5)
            assert np.isneginf(got_m[~was]).all() and (res.state.l[r].cpu().numpy()[~was] == 0).all()
        _check_cache(cache, reqs, sel, g, b, d)
        # bytes copied: the selected blocks that were not resident, once per group
        new = 0
        for r in range(len(reqs)):
            for kh in range(hkv):
                need = np.unique(sel[r, kh * g:(kh + 1) * g])
                need = need[need >= 0]
                new += int((table_before[r, kh, need] < 0).sum())
        h2d = int(cache.h2d_bytes.item())
        assert h2d - h2d_prev == new * page, (step, h2d - h2d_prev, new)
        if step == 1:
            assert new == 0
        h2d_prev = h2d
    assert int(cache.clock.item()) == len(queries)


def test_host_cache_serial_path():
    """hostcache.exact: select, swap-in, then the exact attention (no
    prediction), over a request whose last block is partly filled."""
    from stk_harness.configs import make_qkv
    from strict_topk import hostcache
    hq, hkv, b, d, topk, n = 8, 4, 16, 64, 12, 90
    q, k, v, lo, hi = make_qkv(hq, hkv, d, b, n, torch.float16, True, 31)
    tokens = (n - 1) * b + 5
    live = torch.arange(n * b).view(n, b) < tokens
    lo = torch.where(live[None, :, :, None], k.float(), float("inf")).amin(2)
    hi = torch.where(live[None, :, :, None], k.float(), float("-inf")).amax(2)
    cache = hostcache.build([(k, v)], 2 * topk, device=DEV, tokens=[tokens])
    sel, out = hostcache.exact(q[None].to(DEV), cache, topk)
    torch.cuda.synchronize()
    qn, kn, vn = C.f64(q), C.f64(k), C.f64(v)
    ids = O.select_blocks(qn, lo.numpy(), hi.numpy(), topk)
    assert sel[0].cpu().numpy().tolist() == ids.tolist()
    m = C.error_metrics(C.f64(out[0]), O.attention(qn, kn, vn, ids, tokens=tokens))
    assert m["passed"], m
    assert int(cache.h2d_bytes.item()) > 0


@pytest.mark.parametrize("n", [200, 16])
def test_host_cache_invalid_host_page(n):
    """A block whose host-table entry is -1 has no data: it scores lowest (its
    bounds are indexed by host page), and when it is selected all the same
    (n = topk: every block is) it gets no slot, stays non-resident, adds no
    H2D bytes and has the empty state, as an invalid page has in the paged
    steps."""
    from stk_harness.configs import make_qkv, perturb
    from strict_topk import hostcache
    hq, hkv, b, d, topk, sp = 8, 2, 32, 128, 16, 16
    g = hq // hkv
    q, k, v, lo, hi = make_qkv(hq, hkv, d, b, n, torch.bfloat16, True, 4242)
    cache = hostcache.build([(k, v)], g * topk, device=DEV, bounds_dtype=torch.bfloat16)
    qn, kn, vn = C.f64(q), C.f64(k), C.f64(v)
    dead = int(O.select_blocks(qn, lo.numpy(), hi.numpy(), topk)[0][3])
    cache.host_table[0, 0, dead] = -1
    scores = O.bound_scores(qn, lo.numpy(), hi.numpy())
    scores[:g, dead] = -np.inf        # below every finite score
    ids = O.topk_ids(scores, topk)
    # (with every block selected there is none left to mispredict)
    pred = perturb(torch.from_numpy(ids), n, sp, 0.75 if n > topk else 1.0, 9)
    res = hostcache.speculative_step(q[None].to(DEV), cache, pred[None].to(DEV), topk)
    torch.cuda.synchronize()
    assert res.selected[0].cpu().numpy().tolist() == ids.tolist()
    assert (dead in ids[0]) == (n == topk)
    table = cache.table.cpu().numpy()
    assert table[0, 0, dead] == -1
    rows = [[j for j in ids[h] if not (h // g == 0 and j == dead)] for h in range(hq)]
    m = C.error_metrics(C.f64(res.output[0]), O.attention(qn, kn, vn, rows))
    assert m["passed"], m
    copied = sum(len(set(np.unique(ids[kh * g:(kh + 1) * g])) - ({dead} if kh == 0 else set()))
                 for kh in range(hkv))
    assert int(cache.h2d_bytes.item()) == copied * 2 * b * d * 2
