"""Synthetic decode-step inputs for the five benchmark configurations.

Counterpart of the reference's input builders ``benchmarks/critical_path.py:170-186``
(``_prediction``, ``_synthetic_inputs``) and ``benchmarks/run_benchmark.py:36-65``
(``setup``).  Everything is generated from a seeded CPU ``torch.Generator`` so
that this container and the GPU box build bit-identical tensors; tensors are
moved to the device afterwards.

Rules (all seeded):
  * Q, K, V ~ N(0, 1) drawn in float32 and cast to the config dtype.
  * Hot blocks (configs c2, c3, c5): 5 % of the blocks of every KV head get
    ``k += 1.5 * qhat_g`` where ``qhat_g`` is the unit mean query of the KV
    group (float32 arithmetic, then cast).
  * ``lo/hi = k.amin/amax(dim=2).float()`` (reference
    ``benchmarks/critical_path.py:186``), built outside any timing.
  * The selected set A comes from the caller (normally the float64 oracle's
    top-K with the lower-index tie rule); the prediction P is A with
    ``round((1 - overlap) * K)`` seeded positions replaced by seeded blocks
    outside A, per head.  The reference keeps the first ``hits`` IDs of the
    unsorted ``topk`` output instead, which depends on topk order.
"""
from __future__ import annotations

from dataclasses import dataclass, field

import torch

SEEDS = (20261103, 20261104, 20261105)   # benchmarks/critical_path.py:205


@dataclass(frozen=True)
class Config:
    name: str
    hq: int
    hkv: int
    dim: int
    block: int
    blocks: int
    topk: int
    dtype: torch.dtype
    hot: bool
    overlaps: tuple = (0.9,)
    predict_k: int | None = None
    shared: bool = False

    @property
    def group(self):
        return self.hq // self.hkv

    @property
    def context(self):
        return self.blocks * self.block

    @property
    def sp(self):
        return self.predict_k or self.topk


CONFIGS = {
    # c1: tiny strict 'saved' decode (6 hits / 2 wrong / 2 missed of 8)
    "c1": Config("c1", 4, 4, 64, 32, 64, 8, torch.float16, False, (0.75,)),
    # c2: Qwen3-0.6B-like single GQA layer, 16K context
    "c2": Config("c2", 16, 8, 128, 32, 512, 64, torch.bfloat16, True, (0.9,)),
    # c3: Qwen3-4B-like, 64K context, three hit rates
    "c3": Config("c3", 32, 8, 128, 32, 2048, 64, torch.bfloat16, True, (1.0, 0.9, 0.75)),
    # c4: hierarchical small blocks, 12 query heads per KV head, shared selection
    "c4": Config("c4", 48, 4, 128, 4, 8192, 2048, torch.bfloat16, False, (0.8,), shared=True),
}

# c5: batched signed_fused repair over 16 ragged requests
C5 = dict(requests=16, hq=32, hkv=8, dim=128, block=32, topk=64,
          min_blocks=256, max_blocks=4096, min_overlap=0.5, max_overlap=1.0,
          dtype=torch.bfloat16)


def _gen(seed):
    return torch.Generator().manual_seed(int(seed))


def make_qkv(hq, hkv, dim, block, blocks, dtype, hot, seed, device="cpu"):
    """Q[hq,D], K/V[hkv,N,B,D] plus lo/hi[hkv,N,D] float32, on ``device``.

    The large tensors are drawn with a generator on ``device`` (a CPU
    generator gives bit-identical tensors on every machine; a GPU generator
    is much faster for the 64K-context configs).  Hot-block choices always
    come from a CPU generator.
    """
    device = torch.device(device)
    gen = torch.Generator(device=device).manual_seed(int(seed))
    small = _gen(seed + 1)
    q32 = torch.randn((hq, dim), generator=gen, dtype=torch.float32, device=device)
    k32 = torch.randn((hkv, blocks, block, dim), generator=gen, dtype=torch.float32, device=device)
    v = torch.randn((hkv, blocks, block, dim), generator=gen, dtype=torch.float32,
                    device=device).to(dtype)
    q = q32.to(dtype)
    if hot:
        g = hq // hkv
        qmean = q.float().view(hkv, g, dim).mean(1)
        qhat = qmean / qmean.norm(dim=-1, keepdim=True)
        nhot = max(1, round(0.05 * blocks))
        for kv in range(hkv):
            idx = torch.randperm(blocks, generator=small)[:nhot].to(device)
            k32[kv, idx] += 1.5 * qhat[kv]
    k = k32.to(dtype)
    del k32
    lo = k.amin(dim=2).float()
    hi = k.amax(dim=2).float()
    return q, k, v, lo, hi


def perturb(selected, blocks, predict_k, overlap, seed):
    """Prediction rows: A with round((1-overlap)*K) seeded replacements.

    ``selected`` is an int tensor [H, K] on CPU.  Returns int32 [H, predict_k].
    Positions keep A's order; replaced positions get blocks outside A.
    """
    gen = _gen(seed + 7919)
    sel = selected.to(torch.int64)
    h, k = sel.shape
    replace = round((1.0 - overlap) * k)
    rows = []
    for r in range(h):
        row = sel[r].clone()
        taken = torch.zeros(blocks, dtype=torch.bool)
        taken[row] = True
        free = torch.nonzero(~taken).flatten()
        free = free[torch.randperm(len(free), generator=gen)]
        pos = torch.randperm(k, generator=gen)[:replace]
        row[pos] = free[:replace]
        if predict_k > k:
            row = torch.cat((row, free[replace:replace + predict_k - k]))
        elif predict_k < k:
            row = row[:predict_k]
        rows.append(row)
    return torch.stack(rows).to(torch.int32)


def random_selection(h, blocks, k, seed):
    """Seeded unique block IDs per row (used where no selector is timed)."""
    gen = _gen(seed + 104729)
    return torch.stack([torch.randperm(blocks, generator=gen)[:k] for _ in range(h)]).to(torch.int32)


@dataclass
class Request:
    q: torch.Tensor
    k: torch.Tensor
    v: torch.Tensor
    lo: torch.Tensor
    hi: torch.Tensor
    overlap: float
    blocks: int
    extra: dict = field(default_factory=dict)
