"""Decode-step closures and algorithmic byte counts for the benchmark configs.

Counterpart of the reference's synthetic decode cases
(``benchmarks/critical_path.py:65-167,170-236``): the full speculative step
``overlap_run(select, speculate, repair)`` and the same-work serial step
``exact(select())`` (``benchmarks/critical_path.py:110``).

Byte model (HBM-bound path; every figure counts bytes that must cross HBM
once per decode step, from the actual IDs of the run):
  tile      = 2 * B * D * e            K and V of one (KV head, block), e = element bytes
  U_x       = unique (KV head, block) pairs read by pass x
  kv_bytes  = (U_spec + U_miss) * tile              (saved repair reads no wrong blocks)
  meta      = 2 * Hkv * N * D * eb                  lo and hi, read once (eb = 4 for
                                                    FP32 bounds, 2 for bounds in K's type)
  states    = Hq * SP * (D + 2) * 4                 speculative state write
            + Hq * hits * (D + 2) * 4               state read of the hits
  small     = Q + output + ID rows
The serial step reads meta + U_A * tile + small.
"""
from __future__ import annotations

from dataclasses import dataclass

import numpy as np
import torch

from strict_topk import gqa, gqa_light
from strict_topk import step as step_mod

from .configs import CONFIGS, make_qkv, perturb
from .timing import overlap_run

HBM_PEAK = 8.0e12   # MI355X HBM3E bytes/s


def unique_pairs(ids, group):
    """Number of unique (KV head, block) pairs over rows of ``ids`` [Hq, S]."""
    ids = np.asarray(ids, dtype=np.int64)
    hq = ids.shape[0]
    total = 0
    for kv in range(hq // group):
        total += len(np.unique(ids[kv * group:(kv + 1) * group]))
    return total


def misses(selected, predicted):
    """Per-row selected IDs absent from the predicted row (list of arrays)."""
    out = []
    for a, p in zip(np.asarray(selected), np.asarray(predicted)):
        out.append(np.setdiff1d(a, p, assume_unique=True))
    return out


@dataclass
class Bytes:
    kv_spec: int
    kv_miss: int
    meta: int
    states: int
    small: int
    serial_kv: int
    kv_select_only: int = 0

    @property
    def full(self):
        return self.kv_spec + self.kv_miss + self.meta + self.states + self.small

    @property
    def kv_full(self):
        return self.kv_spec + self.kv_miss

    @property
    def serial(self):
        return self.meta + self.serial_kv + self.small


def byte_model(cfg, selected, predicted, elem_bytes, bound_bytes=4):
    g = cfg.hq // cfg.hkv
    tile = 2 * cfg.block * cfg.dim * elem_bytes
    sel = np.asarray(selected, dtype=np.int64)
    pred = np.asarray(predicted, dtype=np.int64)
    miss_rows = misses(sel, pred)
    hits = sum(sel.shape[1] - len(m) for m in miss_rows)
    # unique (kv, block) miss pairs per KV group
    u_miss = 0
    for kv in range(cfg.hkv):
        rows = miss_rows[kv * g:(kv + 1) * g]
        u_miss += len(np.unique(np.concatenate(rows))) if rows else 0
    st = 4 * (cfg.dim + 2)
    small = cfg.hq * cfg.dim * elem_bytes + cfg.hq * cfg.dim * 4 + 4 * (sel.size + pred.size)
    return Bytes(
        kv_spec=unique_pairs(pred, g) * tile,
        kv_miss=u_miss * tile,
        meta=2 * cfg.hkv * cfg.blocks * cfg.dim * bound_bytes,
        states=cfg.hq * pred.shape[1] * st + hits * st,
        small=small,
        serial_kv=unique_pairs(sel, g) * tile,
    )


class GqaStep:
    """c2 / c3: gqa.select_blocks || gqa.partials -> saved repair.

    ``sets`` device copies of (q, k, v, lo, hi) hold identical values at
    different addresses; step i of a captured sequence uses copy i % sets, so
    that a sequence larger than the caches (MI355X: 4 MB L2 per XCD, 256 MB
    Infinity Cache) reads its operands from HBM as a real decode loop does.
    ``bounds``: "keys" keeps lo/hi in K's own 16-bit type (exact, half the
    bytes) for the fused step and the serial path; "fp32" is the reference's
    layout.  The drop-in composition (gqa.select_blocks) always reads the
    FP32 copies (``sets32``), its contract.
    """

    def __init__(self, cfg, overlap, seed, device, repair="auto", sets=1, bounds="keys"):
        self.cfg, self.overlap, self.seed = cfg, overlap, seed
        q, k, v, lo, hi = make_qkv(cfg.hq, cfg.hkv, cfg.dim, cfg.block, cfg.blocks, cfg.dtype,
                                   cfg.hot, seed)
        self.host = (q, k, v, lo, hi)
        self.bounds = bounds
        bdt = cfg.dtype if bounds == "keys" else torch.float32
        first = tuple(t.to(device) for t in (q, k, v, lo, hi))
        self.sets32 = [first] + [tuple(t.clone() for t in first) for _ in range(sets - 1)]
        self.sets = [(q_, k_, v_, lo_.to(bdt), hi_.to(bdt)) for q_, k_, v_, lo_, hi_ in
                     self.sets32]
        self.q, self.k, self.v, self.lo, self.hi = first
        self.selected = gqa.select_blocks(self.q, self.lo, self.hi, cfg.topk)
        self.predicted = perturb(self.selected.cpu(), cfg.blocks, cfg.sp, overlap, seed).to(device)
        self.emf = 1.0 - overlap
        self.repair = repair
        self.ss = torch.cuda.Stream()
        self.ps = torch.cuda.Stream()
        torch.cuda.synchronize()

    # -- phases on input copy i
    def select(self, i=0):
        """The drop-in selection (FP32 bounds, the reference contract)."""
        q, k, v, lo, hi = self.sets32[i % len(self.sets32)]
        return gqa.select_blocks(q, lo, hi, self.cfg.topk)

    def speculate(self, i=0):
        q, k, v, lo, hi = self.sets[i % len(self.sets)]
        return gqa.partials(q, k, v, self.predicted)

    def finish(self, a, state, i=0):
        q, k, v, lo, hi = self.sets[i % len(self.sets)]
        if self.repair == "light":
            return gqa_light.repair_saved_light(q, k, v, a, self.predicted, state)
        if self.repair == "saved":
            return gqa.repair_saved(q, k, v, a, self.predicted, state)
        return gqa_light.repair_saved_auto(q, k, v, a, self.predicted, state, self.emf)

    # -- whole steps on input copy i
    def full(self, i=0):
        """The drop-in composition: overlap_run over two side streams."""
        return overlap_run(lambda: self.select(i), lambda: self.speculate(i),
                           lambda a, st: self.finish(a, st, i), self.ss, self.ps)

    def fused(self, i=0, sets=None):
        """The same step on one stream (strict_topk.step: one launch at c2 / c3)."""
        sets = self.sets if sets is None else sets
        q, k, v, lo, hi = sets[i % len(sets)]
        return step_mod.speculative_step(q, k, v, lo, hi, self.predicted, self.cfg.topk).output

    def serial(self, i=0, sets=None):
        """The same-work serial path: selection, then attention over it."""
        sets = self.sets if sets is None else sets
        q, k, v, lo, hi = sets[i % len(sets)]
        return step_mod.serial_step(q, k, v, lo, hi, self.cfg.topk)[1]

    def fused32(self, i=0):
        return self.fused(i, self.sets32)

    def serial32(self, i=0):
        return self.serial(i, self.sets32)

    def bound_bytes(self):
        return self.sets[0][3].element_size()

    def bytes(self):
        e = torch.tensor([], dtype=self.cfg.dtype).element_size()
        return byte_model(self.cfg, self.selected.cpu().numpy(), self.predicted.cpu().numpy(), e,
                          self.bound_bytes())

    def front_bytes(self):
        """Algorithmic bytes of the select || speculate launch (k_front)."""
        by = self.bytes()
        c = self.cfg
        e = torch.tensor([], dtype=c.dtype).element_size()
        return (by.meta + by.kv_spec + c.hq * c.sp * 4 * (c.dim + 2) + c.hq * c.blocks * 8
                + c.hq * c.dim * e + c.hq * c.sp * 4)


def gqa_step(name="c3", overlap=0.9, seed=20261103, device="cuda", repair="auto", sets=1,
             bounds="keys"):
    return GqaStep(CONFIGS[name], overlap, seed, device, repair, sets, bounds)
