"""kernels.speculate(mode='hybrid') in one launch (k_spec1) against the same
call as two launches (k_states_tok, then k_hybrid_group1) on identical
inputs, and against the oracle.

The one launch hands each head's states to its grouping workgroup through
flags in the stream's slot; the arithmetic is the two launches', so every
output (the states, the high flags, the low aggregate and its envelope) must
agree bit for bit.  A test hook selects the two launches for the reference
run and, for the failure case, withholds the states' flags so that every
bounded wait times out: the launch ends and every head's grouping is NaN.
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


def _hook(spin=2000000, flags=0):
    from strict_topk import _lib
    torch.cuda.synchronize()
    assert _lib.lib().stk_step1_test_hook(spin, flags) == 0


def _inputs(hq, hkv, n, b, d, s, dtype, idt, seed):
    from stk_harness.configs import make_qkv
    q, k, v, _, _ = make_qkv(hq, hkv, d, b, n, dtype, True, seed)
    gen = torch.Generator().manual_seed(seed)
    pred = torch.stack([torch.randperm(n, generator=gen)[:s] for _ in range(hq)]).to(idt)
    return (q, k, v, pred), tuple(t.cuda() for t in (q, k, v, pred))


def _fields(p):
    return (p.state.m, p.state.l, p.state.u, p.high, p.low.m, p.low.l, p.low.u, p.low_abs)


@pytest.mark.parametrize("hq,hkv,n,b,d,s,dtype,idt,tau", [
    (32, 8, 2000, 32, 128, 64, torch.bfloat16, torch.int32, 0.2),   # c5's request shape
    (32, 8, 2000, 32, 128, 64, torch.bfloat16, torch.int64, 0.1),
    (8, 2, 700, 16, 64, 200, torch.float16, torch.int32, 0.05),     # 200 slots, B = 16
    (6, 3, 97, 32, 64, 5, torch.float16, torch.int64, 0.5),         # few slots
])
def test_spec1_matches_two_launches(hq, hkv, n, b, d, s, dtype, idt, tau):
    from strict_topk import _lib, kernels
    host, (q, k, v, p) = _inputs(hq, hkv, n, b, d, s, dtype, idt, 20261209 + n)
    _hook(flags=2)
    try:
        ref = kernels.speculate(q, k, v, p, "hybrid", tau)
        torch.cuda.synchronize()
    finally:
        _hook()
    got = kernels.speculate(q, k, v, p, "hybrid", tau)
    torch.cuda.synchronize()
    for a, r in zip(_fields(got), _fields(ref)):
        assert torch.equal(a, r)
    # the grouping against the FP64 oracle: high decisions exact unless a
    # block's mass share sits within 1e-5 of the threshold
    qn, kn, vn = (C.f64(t) for t in host[:3])
    pn = host[3].numpy()
    want = O.speculate(qn, kn, vn, pn, "hybrid", tau)
    st = O.block_states(qn, kn, vn, pn)
    mass = np.exp(st.m - st.m.max(1, keepdims=True)) * st.l
    safe = np.abs(mass / mass.sum(1, keepdims=True) - tau) > 1e-5
    assert (got.high.cpu().numpy() == want.high)[safe].all()
    if safe.all():
        np.testing.assert_allclose(got.low.m.cpu().numpy(), want.low.m, rtol=1e-5, atol=1e-5)
        np.testing.assert_allclose(got.low.l.cpu().numpy(), want.low.l, rtol=1e-4)
        np.testing.assert_allclose(got.low.u.cpu().numpy(), want.low.u, rtol=1e-3, atol=1e-4)
        np.testing.assert_allclose(got.low_abs.cpu().numpy(), want.low_abs, rtol=1e-3, atol=1e-4)
    assert _lib.lib().stk_step1_timeouts() == 0


def test_spec1_in_a_graph_and_two_streams():
    """Replays of a captured sequence, and calls on two streams, each equal
    to the two launches on the same inputs."""
    from strict_topk import kernels
    from stk_harness import timing
    _, (q, k, v, p) = _inputs(32, 8, 2000, 32, 128, 64, torch.bfloat16, torch.int32, 20261210)
    _hook(flags=2)
    try:
        ref = kernels.speculate(q, k, v, p, "hybrid", 0.2)
        torch.cuda.synchronize()
    finally:
        _hook()
    g, outs = timing.capture(lambda: [kernels.speculate(q, k, v, p, "hybrid", 0.2)
                                      for _ in range(3)])
    for _ in range(3):
        g.replay()
        torch.cuda.synchronize()
        for res in outs:
            for a, r in zip(_fields(res), _fields(ref)):
                assert torch.equal(a, r)
    s1, s2 = torch.cuda.Stream(), torch.cuda.Stream()
    s1.wait_stream(torch.cuda.current_stream())
    s2.wait_stream(torch.cuda.current_stream())
    got = []
    for st in (s1, s2, s1, s2):
        with torch.cuda.stream(st):
            got.append(kernels.speculate(q, k, v, p, "hybrid", 0.2))
    torch.cuda.synchronize()
    for res in got:
        for a, r in zip(_fields(res), _fields(ref)):
            assert torch.equal(a, r)
    from strict_topk import _lib
    assert _lib.lib().stk_step1_timeouts() == 0


def test_spec1_timed_out_waits_fail_loudly():
    """Flags withheld, 20 us limit: the launch ends, every head's low
    aggregate is NaN and no block is high; the next call is exact again."""
    from strict_topk import _lib, kernels
    _, (q, k, v, p) = _inputs(32, 8, 2000, 32, 128, 64, torch.bfloat16, torch.int32, 20261211)
    _hook(flags=2)
    try:
        ref = kernels.speculate(q, k, v, p, "hybrid", 0.2)
        torch.cuda.synchronize()
    finally:
        _hook()
    _hook(spin=2000, flags=1)
    try:
        bad = kernels.speculate(q, k, v, p, "hybrid", 0.2)
        torch.cuda.synchronize()
        assert torch.isnan(bad.low.u).all() and torch.isnan(bad.low_abs).all()
        assert torch.isnan(bad.low.m).all() and not bad.high.any()
        assert _lib.lib().stk_step1_timeouts() >= 1
    finally:
        _hook()
    assert _lib.lib().stk_step1_timeouts() == 0
    got = kernels.speculate(q, k, v, p, "hybrid", 0.2)
    torch.cuda.synchronize()
    for a, r in zip(_fields(got), _fields(ref)):
        assert torch.equal(a, r)
