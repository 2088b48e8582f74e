"""Write the golden fixtures in tests/golden/ from this build's FP64 oracle.

Run from the repository root:  python tests/golden/make_golden.py

The fixtures hold data only (inputs and expected outputs); nothing of the
reference's source.  They freeze the oracle: tests/test_golden.py checks that
the oracle still reproduces them (CPU) and that the HIP library matches them
(GPU).

  c1.npz    config c1 (Hq = Hkv = 4, D = 64,
            64 blocks of 32 tokens, K = 8, fp16, 6 hits / 2 wrong / 2 missed per
            row).  The inputs are regenerated from the seed by
            stk_harness.configs.make_qkv; the fixture stores their sha256
            (so generator drift is detected), the predicted rows, the FP64
            bound scores, the selected IDs (ascending, ties to the lower
            index), the prediction's block states and the strict output.
  tiny.npz  a small GQA case with its inputs stored (fp16 Q/K/V, fp32 lo/hi,
            Hq = 4, Hkv = 2, D = 64, B = 16, N = 12, K = SP = 4): expected IDs,
            prediction states, saved and union repair outputs.
  kat.json  the reference's known-answer values, with the reference lines they
            come from.
"""
from __future__ import annotations

import hashlib
import json
import math
import sys
from pathlib import Path

import numpy as np
import torch

ROOT = Path(__file__).resolve().parents[2]
for p in (ROOT / "strict-topk-overlap_amd", ROOT):
    if str(p) not in sys.path:
        sys.path.insert(0, str(p))

from oracle import stk_oracle as O  # noqa: E402
from stk_harness.configs import CONFIGS, make_qkv, perturb  # noqa: E402

HERE = Path(__file__).resolve().parent
C1_SEED = 20261103
TINY_SEED = 20261104


def sha(t):
    return hashlib.sha256(t.detach().cpu().contiguous().view(torch.uint8).numpy().tobytes()).hexdigest()


def f64(t):
    return t.detach().cpu().double().numpy()


def c1_inputs():
    c = CONFIGS["c1"]
    q, k, v, lo, hi = make_qkv(c.hq, c.hkv, c.dim, c.block, c.blocks, c.dtype, c.hot, C1_SEED)
    return c, q, k, v, lo, hi


def tiny_inputs():
    gen = torch.Generator().manual_seed(TINY_SEED)
    hq, hkv, d, b, n = 4, 2, 64, 16, 12
    q = torch.randn((hq, d), generator=gen).half()
    k = torch.randn((hkv, n, b, d), generator=gen).half()
    v = torch.randn((hkv, n, b, d), generator=gen).half()
    lo, hi = k.float().amin(2), k.float().amax(2)
    return q, k, v, lo, hi


def main():
    c, q, k, v, lo, hi = c1_inputs()
    qn, kn, vn = f64(q), f64(k), f64(v)
    scores = O.bound_scores(qn, lo.numpy(), hi.numpy())
    ids = O.select_blocks(qn, lo.numpy(), hi.numpy(), c.topk)
    pred = perturb(torch.from_numpy(ids), c.blocks, c.sp, c.overlaps[0], C1_SEED).numpy()
    st = O.block_states(qn, kn, vn, pred)
    out = O.attention(qn, kn, vn, ids)
    np.savez(HERE / "c1.npz", seed=np.array(C1_SEED),
             sha256=np.array([sha(x) for x in (q, k, v, lo, hi)]),
             predicted=pred.astype(np.int32), scores=scores, selected=ids.astype(np.int32),
             m=st.m, l=st.l, u=st.u, output=out)

    q, k, v, lo, hi = tiny_inputs()
    qn, kn, vn = f64(q), f64(k), f64(v)
    topk = 4
    ids = O.select_blocks(qn, lo.numpy(), hi.numpy(), topk)
    # two of four predicted blocks kept, two replaced (positions 1 and 3)
    pred = ids.copy()
    for r in range(pred.shape[0]):
        free = [x for x in range(k.shape[1]) if x not in set(ids[r].tolist())]
        pred[r, 1], pred[r, 3] = free[r % len(free)], free[(r + 5) % len(free)]
    st = O.block_states(qn, kn, vn, pred)
    np.savez(HERE / "tiny.npz", q=q.numpy(), k=k.numpy(), v=v.numpy(), lo=lo.numpy(),
             hi=hi.numpy(), topk=np.array(topk), predicted=pred.astype(np.int32),
             selected=ids.astype(np.int32), m=st.m, l=st.l, u=st.u,
             saved=O.gqa_repair(qn, kn, vn, ids, pred, st),
             union=O.gqa_repair(qn, kn, vn, ids, pred, st, union=True))

    kat = {
        "tiny_gqa": {"source": "tests/check_gqa.py:65-70",
                     "q": 1.0, "k": [2.0, -3.0], "v": [8.0, -5.0],
                     "same_rows": [8.0, -5.0], "swapped_rows": [-5.0, 8.0],
                     "union": (8 * math.e ** 5 - 5) / (math.e ** 5 + 1)},
        "extra_mass_budget": {"source": "tests/check_signed_repair.py:29-56",
                              "strict_output": 1.5, "positive_jobs": 1, "total_jobs": 2,
                              "extra_mass_bound_eps_0.1": math.exp(-3) / (1 + math.exp(-3)),
                              "extra_mass_bound_min": 0.02429},
        "zero_query_ties": {"source": "tests/check_selector.py:13",
                            "rule": "all-zero q: the selected IDs are 0..K-1"},
        "tolerance": {"source": "tests/check_correctness.py:22", "abs": 3e-4, "rel": 3e-4},
    }
    (HERE / "kat.json").write_text(json.dumps(kat, indent=1) + "\n")
    print("wrote", *(p.name for p in sorted(HERE.glob("*.npz"))), "kat.json")


if __name__ == "__main__":
    main()
