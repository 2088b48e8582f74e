"""Golden fixtures (tests/golden/, written by tests/golden/make_golden.py).

CPU: the seeded c1 inputs still hash to the stored digests, the FP64 oracle
still reproduces every stored vector, and the stored known-answer table
agrees with the oracle.  GPU (marked): the HIP library matches the stored
vectors through the drop-in API -- block IDs bit-exact, states and outputs
within |err| <= 3e-4 + 3e-4 |ref|.
"""
import json
import math
from pathlib import Path

import numpy as np
import pytest
import torch

from oracle import stk_oracle as O
from tests import cases as C
from tests.golden import make_golden as G

HERE = Path(__file__).resolve().parent / "golden"


def _load(name):
    return np.load(HERE / name, allow_pickle=False)


# ------------------------------------------------------------------ CPU
def test_c1_inputs_hash_to_the_fixture():
    fx = _load("c1.npz")
    _, q, k, v, lo, hi = G.c1_inputs()
    assert [G.sha(x) for x in (q, k, v, lo, hi)] == fx["sha256"].tolist()


def test_oracle_reproduces_c1():
    fx = _load("c1.npz")
    c, q, k, v, lo, hi = G.c1_inputs()
    qn, kn, vn = G.f64(q), G.f64(k), G.f64(v)
    np.testing.assert_array_equal(O.bound_scores(qn, lo.numpy(), hi.numpy()), fx["scores"])
    ids = O.select_blocks(qn, lo.numpy(), hi.numpy(), c.topk)
    np.testing.assert_array_equal(ids, fx["selected"])
    # 6 hits, 2 wrong, 2 missed per row
    for a, p in zip(fx["selected"], fx["predicted"]):
        assert len(set(a.tolist()) & set(p.tolist())) == 6
    st = O.block_states(qn, kn, vn, fx["predicted"])
    np.testing.assert_allclose(st.u, fx["u"], rtol=1e-12, atol=1e-12)
    np.testing.assert_allclose(O.attention(qn, kn, vn, ids), fx["output"], rtol=1e-12, atol=1e-12)
    # the strict repair of the stored prediction gives the stored output
    pred = O.speculate(qn, kn, vn, fx["predicted"], mode="saved")
    res = O.repair(qn, kn, vn, ids, fx["predicted"], pred)
    np.testing.assert_allclose(res.output, fx["output"], rtol=1e-10, atol=1e-12)


def test_oracle_reproduces_tiny():
    fx = _load("tiny.npz")
    q, k, v = (fx[x].astype(np.float64) for x in ("q", "k", "v"))
    ids = O.select_blocks(q, fx["lo"], fx["hi"], int(fx["topk"]))
    np.testing.assert_array_equal(ids, fx["selected"])
    st = O.block_states(q, k, v, fx["predicted"])
    for name in ("m", "l", "u"):
        np.testing.assert_allclose(getattr(st, name), fx[name], rtol=1e-12, atol=1e-12)
    np.testing.assert_allclose(O.gqa_repair(q, k, v, ids, fx["predicted"], st), fx["saved"],
                               rtol=1e-12, atol=1e-12)
    np.testing.assert_allclose(O.gqa_repair(q, k, v, ids, fx["predicted"], st, union=True),
                               fx["union"], rtol=1e-12, atol=1e-12)
    # saved repair = attention over the selected set (closed form)
    np.testing.assert_allclose(fx["saved"], O.attention(q, k, v, ids), rtol=1e-12, atol=1e-12)


def test_known_answer_table():
    kat = json.loads((HERE / "kat.json").read_text())
    t = kat["tiny_gqa"]
    q, k, v, p = (C.f64(x) if x.is_floating_point() else C.ids_np(x) for x in C.tiny_gqa())
    np.testing.assert_allclose(O.attention(q, k, v, p)[:, 0], t["same_rows"], atol=1e-12)
    np.testing.assert_allclose(O.attention(q, k, v, 1 - p)[:, 0], t["swapped_rows"], atol=1e-12)
    st = O.block_states(q, k, v, p)
    np.testing.assert_allclose(O.gqa_repair(q, k, v, 1 - p, p, st, union=True)[:, 0],
                               [t["union"]] * 2, rtol=1e-12)
    b = kat["extra_mass_budget"]
    q, k, v, p, a, _ = (C.f64(x) if x.is_floating_point() else C.ids_np(x) for x in C.budget_case())
    st = O.speculate(q, k, v, p, mode="hybrid", mass_threshold=.2, keep_mass=True)
    low = O.repair_signed(q, k, v, a, p, st, max_extra_mass=.01)
    assert abs(low.output[0, 0] - b["strict_output"]) < 1e-12
    assert (low.positive_jobs[0], low.total_jobs[0]) == (b["positive_jobs"], b["total_jobs"])
    high = O.repair_signed(q, k, v, a, p, st, max_extra_mass=.1)
    assert abs(high.extra_mass_bound[0] - b["extra_mass_bound_eps_0.1"]) < 1e-12
    assert b["extra_mass_bound_min"] <= high.extra_mass_bound[0] <= .1
    assert math.isclose(kat["tolerance"]["abs"], 3e-4) and math.isclose(kat["tolerance"]["rel"], 3e-4)


# ------------------------------------------------------------------ GPU
def _gpu():
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    from strict_topk import _lib
    _lib.lib()   # fail loudly if the HIP library is missing


def _check(out, expected, what):
    m = C.error_metrics(C.f64(out), expected)
    assert m["passed"], (what, m)


@pytest.mark.gpu
def test_hip_matches_c1_fixture():
    _gpu()
    from strict_topk import kernels, selector
    fx = _load("c1.npz")
    c, q, k, v, lo, hi = G.c1_inputs()
    assert [G.sha(x) for x in (q, k, v, lo, hi)] == fx["sha256"].tolist()
    q, k, v, lo, hi = (x.cuda() for x in (q, k, v, lo, hi))
    p = torch.from_numpy(fx["predicted"]).cuda()
    ids = selector.select_blocks(q, lo, hi, c.topk)
    np.testing.assert_array_equal(ids.cpu().numpy(), fx["selected"])
    pred = kernels.speculate(q, k, v, p, mode="saved")
    for name in ("m", "l", "u"):
        _check(getattr(pred.state, name), fx[name], ("c1 state", name))
    res = kernels.repair(q, k, v, ids, p, pred)
    _check(res.output, fx["output"], "c1 repair")
    _check(kernels.exact_attention(q, k, v, ids), fx["output"], "c1 exact")


@pytest.mark.gpu
def test_hip_matches_tiny_fixture():
    _gpu()
    from strict_topk import gqa, step
    fx = _load("tiny.npz")
    q, k, v, lo, hi = (torch.from_numpy(np.ascontiguousarray(fx[x])).cuda()
                       for x in ("q", "k", "v", "lo", "hi"))
    p = torch.from_numpy(fx["predicted"]).cuda()
    topk = int(fx["topk"])
    ids = gqa.select_blocks(q, lo, hi, topk)
    np.testing.assert_array_equal(ids.cpu().numpy(), fx["selected"])
    st = gqa.partials(q, k, v, p)
    for name in ("m", "l", "u"):
        _check(getattr(st, name), fx[name], ("tiny state", name))
    _check(gqa.repair_saved(q, k, v, ids, p, st), fx["saved"], "tiny saved")
    _check(gqa.repair_union(q, k, v, ids, p, st), fx["union"], "tiny union")
    assert step.supported(q, k, lo, topk, p)
    for union, key in ((False, "saved"), (True, "union")):
        res = step.speculative_step(q, k, v, lo, hi, p, topk, union=union)
        np.testing.assert_array_equal(res.selected.cpu().numpy(), fx["selected"])
        _check(res.output, fx[key], ("tiny step", key))
    # the same request as a one-request paged batch, its pages in reverse order
    from strict_topk import paged
    hkv, n = k.shape[:2]
    order = torch.arange(hkv * n - 1, -1, -1)
    kv = paged.pack([(k, v)], order=order, spare=2)
    for union, key in ((False, "saved"), (True, "union")):
        res = paged.speculative_step(q.unsqueeze(0).contiguous(), kv, p.unsqueeze(0).contiguous(),
                                     topk, union=union)
        np.testing.assert_array_equal(res.selected[0].cpu().numpy(), fx["selected"])
        _check(res.output[0], fx[key], ("tiny paged step", key))
