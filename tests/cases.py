"""Test cases restated from the reference's GPU check scripts.

The structures, shapes and adversarial constructions follow
``tests/check_correctness.py:35-104``, ``tests/check_gqa.py:37-70``,
``tests/check_gqa_light.py:24-48``, ``tests/check_gqa_hierarchical.py:15-32``,
``tests/check_signed_repair.py:29-56`` and ``tests/check_signed_fused.py:17-30``.
Random tensors come from a seeded CPU ``torch.Generator`` (the reference used
a CUDA generator), so the values differ from the reference's but every
machine builds the same ones.  All tensors are created on the CPU; callers
move them to the device.
"""
from __future__ import annotations

import math

import numpy as np
import torch

SEED = 20261103


def f64(t):
    return t.detach().to("cpu").double().numpy()


def ids_np(t):
    return t.detach().to("cpu").long().numpy()


def error_metrics(output, expected):
    """Reference tolerance: |err| <= 3e-4 + 3e-4 |ref| (tests/check_correctness.py:20-32)."""
    out = np.asarray(output, dtype=np.float64)
    diff = np.abs(out - expected)
    tol = 3e-4 + 3e-4 * np.abs(expected)
    finite = bool(np.isfinite(out).all())
    return {"max_abs_error": float(diff.max()) if diff.size else 0.0,
            "finite": finite, "passed": bool((diff <= tol).all() and finite)}


def correctness_cases(dtype=torch.float16):
    """tests/check_correctness.py:35-104 with a CPU generator."""
    gen = torch.Generator().manual_seed(SEED)
    for h, n, b, d, count in [(1, 19, 16, 32, 5), (4, 32, 32, 64, 8), (8, 24, 64, 128, 8)]:
        q = torch.randn(h, d, generator=gen).to(dtype)
        k = torch.randn(h, n, b, d, generator=gen).to(dtype)
        v = torch.randn(h, n, b, d, generator=gen).to(dtype)
        p = torch.arange(count, dtype=torch.int32).expand(h, -1).contiguous()
        for overlap in [0, count // 2, count]:
            a = torch.arange(count - overlap, 2 * count - overlap, dtype=torch.int32)
            yield f"random_h{h}_b{b}_d{d}_overlap{overlap}of{count}", q, k, v, p, a.expand(h, -1).contiguous()

    h, n, b, d = 4, 31, 17, 48
    q = torch.randn(h, d, generator=gen).to(dtype)
    k = torch.randn(h, n, b, d, generator=gen).to(dtype)
    v = torch.randn(h, n, b, d, generator=gen).to(dtype)
    for sp, sa, overlap in [(8, 5, 0), (8, 5, 2), (8, 5, 5), (3, 7, 2)]:
        preds, sels = [], []
        for _ in range(h):
            perm = torch.randperm(n, generator=gen)
            pi = perm[:sp]
            ai = torch.cat((pi[:overlap], perm[sp:sp + sa - overlap]))
            preds.append(pi[torch.randperm(sp, generator=gen)])
            sels.append(ai[torch.randperm(sa, generator=gen)])
        p, a = torch.stack(preds).int(), torch.stack(sels).int()
        yield f"random_unordered_b17_d48_p{sp}_a{sa}_hit{overlap}", q, k, v, p, a

    for name in ["high_wrong_mass", "many_low_wrong_mass", "signed_value_cancellation",
                 "extreme_wrong_logits"]:
        h, n, b, d, count = 2, 24, 16, 32, 8
        q = torch.zeros(h, d, dtype=dtype)
        q[:, 0] = 1
        logits = torch.zeros(h, n)
        if name == "high_wrong_mass":
            logits[:, 0] = 20
        elif name == "many_low_wrong_mass":
            logits.fill_(-8)
            logits[:, :7] = 10
        elif name == "extreme_wrong_logits":
            logits.fill_(-40)
            logits[:, :7] = 80
        k = torch.zeros(h, n, b, d, dtype=dtype)
        k[..., 0] = (logits * math.sqrt(d))[:, :, None]
        v = torch.randn(h, n, b, d, generator=gen).to(dtype)
        if name == "signed_value_cancellation":
            signs = torch.where(torch.arange(d) % 2 == 0, 1., -1.)
            v[:] = signs * .01
            v[:, :7] = signs * 60000.
        p = torch.arange(count, dtype=torch.int32).expand(h, -1).contiguous()
        a = torch.arange(7, 15, dtype=torch.int32).expand(h, -1).contiguous()
        yield name, q, k, v, p, a

    q = torch.ones(1, 1, dtype=dtype)
    k = torch.zeros(1, 4, 1, 1, dtype=dtype)
    v = torch.tensor([60000., .01, -60000., 1.], dtype=dtype).view_as(k)
    p = torch.tensor([[0, 1, 2]], dtype=torch.int32)
    a = torch.tensor([[1]], dtype=torch.int32)
    yield "signed_low_aggregate_cancellation", q, k, v, p, a

    k = k.clone()
    k[:, :3] = 100
    a = torch.tensor([[3]], dtype=torch.int32)
    yield "discard_high_logit_low_group", q, k, v, p, a


# expected fallback heads at mass_threshold 1.0 (tests/check_correctness.py:128-135)
EXPECTED_FALLBACK = {"signed_low_aggregate_cancellation": 1, "discard_high_logit_low_group": 0}


def gqa_cases(hq=6, hkv=2, n=23, b=7, d=13, seed=SEED):
    """tests/check_gqa.py:37-44 / check_gqa_light.py:24-32."""
    gen = torch.Generator().manual_seed(seed)
    q = torch.randn((hq, d), generator=gen).half()
    k = torch.randn((hkv, n, b, d), generator=gen).half()
    v = torch.randn(k.shape, generator=gen).half()
    perms = torch.stack([torch.randperm(n, generator=gen) for _ in range(hq)])
    out = []
    for sp, sa, overlap in [(6, 6, 0), (6, 6, 3), (6, 6, 5), (6, 6, 6), (7, 5, 2), (3, 7, 2)]:
        p = perms[:, :sp].contiguous()
        a = torch.cat((perms[:, :overlap], perms[:, sp:sp + sa - overlap]), dim=1)
        out.append((f"gqa_p{sp}_a{sa}_o{overlap}", q, k, v, p.int(), a.flip(1).int().contiguous()))
    # huge logits, mixed int32/int64 (check_gqa.py:56-63)
    q2 = torch.zeros_like(q)
    q2[:, 0] = 1
    k2 = k.clone()
    k2[..., 0] = -5000
    k2[:, 1, :, 0] = 2000
    k2[:, 3, :, 0] = 5000
    p = torch.tensor([[0, 3, 2]] * hq, dtype=torch.int32)
    a = torch.tensor([[2, 1, 0]] * hq, dtype=torch.int64)
    out.append(("gqa_huge_logits", q2, k2, v, p, a))
    return out


def tiny_gqa():
    """tests/check_gqa.py:65-70: q = 1, k = [2, -3], v = [8, -5]."""
    q = torch.ones((2, 1), dtype=torch.float16)
    k = torch.tensor([[[[2.]], [[-3.]]]], dtype=torch.float16)
    v = torch.tensor([[[[8.]], [[-5.]]]], dtype=torch.float16)
    p = torch.tensor([[0], [1]], dtype=torch.int32)
    return q, k, v, p


def budget_case():
    """tests/check_signed_repair.py:29-56."""
    q = torch.ones((1, 1), dtype=torch.float16)
    k = torch.tensor([3., 0., -3., 0.], dtype=q.dtype).view(1, 4, 1, 1)
    v = torch.tensor([100., 1., 8., 2.], dtype=q.dtype).view_as(k)
    p = torch.tensor([[0, 1, 2]], dtype=torch.int64)
    a = torch.tensor([[1, 3]], dtype=torch.int32)
    extra_set = torch.tensor([[1, 3, 2]], dtype=torch.int32)
    return q, k, v, p, a, extra_set


def underflow_case():
    """tests/check_signed_fused.py:17-30 (bf16; exp(-104) underflows in FP32)."""
    q = torch.ones((1, 1), dtype=torch.bfloat16)
    k = torch.full((1, 3, 8192, 1), -200., dtype=q.dtype)
    k[:, :, 0, 0] = 0.
    k[:, 2, :, 0] = -104.
    k[:, 2, 0, 0] = -80.
    v = torch.zeros_like(k)
    v[:, 2, 1:, 0] = 3.e38
    p = torch.tensor([[0, 1, 2]], dtype=torch.int32)
    a = torch.tensor([[0, 1]], dtype=torch.int32)
    return q, k, v, p, a


def prediction_rows(selected, blocks, predict_k, hits):
    """benchmarks/critical_path.py:170-176: keep the first `hits` selected IDs
    and fill with the lowest non-selected IDs."""
    rows = []
    for row in selected.tolist():
        sel = set(row)
        wrong = [x for x in range(blocks) if x not in sel]
        rows.append(row[:hits] + wrong[:predict_k - hits])
    return torch.tensor(rows, dtype=selected.dtype)


def hier_cases(dtype):
    """tests/check_gqa_hierarchical.py:15-32 shapes (reduced for the oracle)."""
    gen = torch.Generator().manual_seed(317)
    for h, hkv, n, b, d, sa in [(24, 2, 1024, 4, 256, 512), (6, 2, 96, 5, 96, 37),
                                (48, 4, 2048, 4, 128, 320), (12, 1, 700, 8, 64, 200)]:
        q = torch.randn((h, d), generator=gen).to(dtype)
        k = torch.randn((hkv, n, b, d), generator=gen).to(dtype)
        v = torch.randn(k.shape, generator=gen).to(dtype)
        a = torch.stack([torch.randperm(n, generator=gen)[:sa] for _ in range(h)]).int()
        yield (h, hkv, n, b, d, sa), q, k, v, a
