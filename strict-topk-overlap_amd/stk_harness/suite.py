"""Timed decode steps for configs c1, c2, c4, c5 and a c3 sweep (c3 is bench.py's headline).

Each case builds its seeded inputs on the device, captures its speculative
path and the same-work serial path into HIP graphs, and times them with
randomized ABBA pairs (``timing.paired``).  The reference strategy each
config exercises (BASELINE.json ``configs``):

  c1  selector.select_blocks || kernels.speculate('saved') -> kernels.repair,
      the same with fused.repair_fused (two streams, the drop-in
      composition), and strict_topk.step.speculative_step (fused);
      serial = exact_attention(select).
  c2  gqa.select_blocks || gqa.partials -> gqa.repair_saved (two streams, the
      drop-in composition) and strict_topk.step.speculative_step (fused);
      serial = gqa.exact(select).
  c4  gqa_hierarchical.partials(P) -> repair_saved_shared, selection given:
      the reference's shared selector is the QSA indexer, outside this path,
      so the selected set (top-2048 of the bound score summed over all heads,
      ties to the lower index, one row shared by every head as
      repair_saved_shared requires) is built once outside timing and both the
      speculative and the serial path (gqa_hierarchical.exact) start from it.
  c5  16 requests with 8K-128K contexts and overlap U[0.5, 1]: per request
      gqa.select_blocks || kernels.speculate('hybrid', 0.2, keep_mass=True)
      -> signed_fused.repair_signed_fused with max_extra_mass 0.01 and 0
      (strict); serial = gqa.exact(select) per request; and the whole batch
      in one page pool (strict_topk.paged: the batched signed step against the
      batched serial path, two launches each), the primary pair.
  c3 sweep  the fused step against the serial path at every c3 hit rate
      (overlap 1.0, 0.9, 0.75), three seeds each.

No checking happens here: every case keeps host copies of its inputs and the
device outputs of its captured graphs, which bench.py's CPU leg compares with
the FP64 oracle.
"""
from __future__ import annotations

from dataclasses import dataclass, field

import numpy as np
import torch

from strict_topk import (fused, gqa, gqa_hierarchical, indexer, kernels, paged, selector,
                         signed_fused)
from strict_topk import step as step_mod

from . import timing
from .configs import C5, CONFIGS, make_qkv, perturb
from .decode import HBM_PEAK, GqaStep, byte_model, unique_pairs


@dataclass
class Case:
    name: str
    strategy: str
    graphs: dict                     # name -> captured graph (M steps each)
    steps_per_graph: int
    bytes_full: int
    bytes_kv: int
    bytes_serial: int
    primary: str = ""                # the path reported as the speculative step
    check: list = field(default_factory=list)   # (label, kind, data) for the CPU leg
    notes: str = ""
    pairs: dict = field(default_factory=dict)   # label -> (speculative, serial) also reported
    baseline: str = "serial"         # the serial path the primary is compared with
    # Everything on the device that the graphs read but do not own (inputs,
    # prediction rows, side streams).  A captured graph holds raw addresses,
    # not tensor references, and every torch.cuda.graph capture starts with
    # torch.cuda.empty_cache(): an input dropped after its graph was captured
    # goes back to the driver at the next capture, and replaying the graph
    # then reads unmapped memory.  Released together with the graphs.
    keep: object = None
    after: object = None             # measurements taken after the timing (dict)

    def release(self):
        self.graphs = {}
        self.keep = None

    def measure(self, replays=20, rounds=3, seed=20261103):
        med, _ = timing.paired(self.graphs, replays=replays, rounds=rounds, seed=seed,
                               warm_ms=50.0)
        per = {k: v / self.steps_per_graph for k, v in med.items()}
        full = per[self.primary]
        extra = self.after() if self.after else {}
        return {
            **extra,
            "strategy": self.strategy, "primary": self.primary,
            "us_per_step": {k: round(v, 3) for k, v in per.items()},
            "speedup_vs_serial": round(per[self.baseline] / full, 4),
            **({"speedups": {k: round(per[b] / per[a], 4) for k, (a, b) in self.pairs.items()}}
               if self.pairs else {}),
            "algorithmic_bytes": self.bytes_full, "kv_bytes": self.bytes_kv,
            "serial_bytes": self.bytes_serial,
            "frac": round(self.bytes_full / (full * 1e-6) / HBM_PEAK, 4),
            "kv_frac": round(self.bytes_kv / (full * 1e-6) / HBM_PEAK, 4),
            "notes": self.notes,
        }


def _host(*ts):
    return tuple(t.detach().cpu() for t in ts)


def _seq(fn, m):
    return lambda: [fn(i) for i in range(m)]


# ------------------------------------------------------------------ c1
def case_c1(dev, seed=20261103):
    c = CONFIGS["c1"]
    q, k, v, lo, hi = (t.to(dev) for t in make_qkv(c.hq, c.hkv, c.dim, c.block, c.blocks,
                                                    c.dtype, c.hot, seed))
    sel = selector.select_blocks(q, lo, hi, c.topk)
    p = perturb(sel.cpu(), c.blocks, c.sp, c.overlaps[0], seed).to(dev)
    ss, ps = torch.cuda.Stream(), torch.cuda.Stream()

    def full(repair):
        return lambda i: timing.overlap_run(
            lambda: selector.select_blocks(q, lo, hi, c.topk),
            lambda: kernels.speculate(q, k, v, p, "saved"),
            lambda a, st: repair(q, k, v, a, p, st).output, ss, ps)

    m = 4
    graphs, outs = {}, {}
    for name, fn in (("split", full(kernels.repair)), ("fused", full(fused.repair_fused)),
                     ("step", lambda i: step_mod.speculative_step(q, k, v, lo, hi, p,
                                                                  c.topk).output),
                     ("serial", lambda i: kernels.exact_attention(
                         q, k, v, selector.select_blocks(q, lo, hi, c.topk)))):
        graphs[name], outs[name] = timing.capture(_seq(fn, m))
    tile = 2 * c.block * c.dim * 2
    pa, sa = p.cpu().numpy(), sel.cpu().numpy()
    kv = (unique_pairs(pa, 1) + sum(len(np.setdiff1d(a, b)) for a, b in zip(sa, pa))) * tile
    meta = 2 * c.hkv * c.blocks * c.dim * 4
    states = c.hq * c.sp * (c.dim + 2) * 4 * 2
    small = c.hq * c.dim * (2 + 4) + 4 * (sa.size + pa.size)
    case = Case("c1", "select || speculate('saved') -> repair (split / repair_fused, two "
                "streams; and the fused step)", graphs, m,
                kv + meta + states + small, kv, meta + unique_pairs(sa, 1) * tile + small,
                primary="step")
    case.keep = (q, k, v, lo, hi, sel, p, ss, ps)
    hq_, hk_, hv_ = _host(q, k, v)
    case.check = [("ids", "select", (hq_, *_host(lo, hi), c.topk, sel.cpu()))]
    for name in graphs:
        case.check.append((name, "attention", (hq_, hk_, hv_, sel.cpu(), outs[name][-1].cpu())))
    return case


# ------------------------------------------------------------------ c2
def case_c2(dev, seed=20261103):
    m = 12
    st = GqaStep(CONFIGS["c2"], 0.9, seed, dev, repair="saved", sets=m)
    graphs, outs = {}, {}
    for name, fn in (("composed", st.full), ("fused", st.fused), ("serial", st.serial)):
        graphs[name], outs[name] = timing.capture(_seq(fn, m))
    by = st.bytes()
    case = Case("c2", "gqa.select_blocks || gqa.partials -> gqa.repair_saved (composed, two "
                "streams; and the fused step)", graphs, m, by.full, by.kv_full, by.serial,
                primary="fused", notes=f"inputs rotated over {m} device copies")
    case.keep = st
    q, k, v, lo, hi = st.host
    case.check = [("ids", "select", (q, lo, hi, st.cfg.topk, st.selected.cpu()))]
    for name in graphs:
        case.check.append((name, "attention", (q, k, v, st.selected.cpu(), outs[name][-1].cpu())))
    return case


# ------------------------------------------------------------------ c4
def _shared_selection(q, lo, hi, g, topk):
    """Top-k blocks of the bound score summed over every query head (FP32
    torch, ties to the lower index), one row repeated for all heads:
    repair_saved_shared's contract is identical rows for every head
    (reference strict_topk/gqa_hierarchical.py:137-143), as a per-layer
    indexer produces."""
    qg = q.float().view(lo.shape[0], g, -1)
    s = (torch.einsum("kgd,knd->kgn", qg.clamp(min=0), hi) +
         torch.einsum("kgd,knd->kgn", qg.clamp(max=0), lo)).sum((0, 1))
    order = torch.sort(-s, stable=True).indices[:topk]
    ids = torch.sort(order).values.to(torch.int32)
    return ids.expand(q.shape[0], -1).contiguous()


def case_c4(dev, seed=20261103):
    c = CONFIGS["c4"]
    g = c.group
    # CPU generators: the same inputs on every machine
    q, k, v, lo, hi = (t.to(dev) for t in make_qkv(c.hq, c.hkv, c.dim, c.block, c.blocks,
                                                   c.dtype, c.hot, seed))
    # the shared selection: the QSA indexer formula over 4 synthetic indexer
    # heads and one 128-dim indexer key per block (no trained weights), as
    # the reference's QSA probe does (benchmarks/selector_window.py:76-84)
    gen = torch.Generator().manual_seed(seed + 4)
    iq = torch.randn((4, 128), generator=gen).to(c.dtype).to(dev)
    ik = torch.randn((c.blocks, 128), generator=gen).to(c.dtype).to(dev)

    def select():
        return indexer.select_shared(iq, ik, c.topk, c.hq)

    sel = select()
    prow = perturb(sel[:1].cpu(), c.blocks, c.sp, c.overlaps[0], seed)
    p = prow.expand(c.hq, -1).contiguous().to(dev)
    m = 2
    ss, ps = torch.cuda.Stream(), torch.cuda.Stream()

    def full(i):
        return timing.overlap_run(
            select, lambda: gqa_hierarchical.partials(q, k, v, p),
            lambda a, st: gqa_hierarchical.repair_saved_shared(q, k, v, a, p, st), ss, ps)

    def given(i):
        st = gqa_hierarchical.partials(q, k, v, p)
        return gqa_hierarchical.repair_saved_shared(q, k, v, sel, p, st)

    graphs, outs = {}, {}
    for name, fn in (("speculative", full),
                     ("serial", lambda i: gqa_hierarchical.exact(q, k, v, select())),
                     ("speculative_given_selection", given),
                     ("serial_given_selection", lambda i: gqa_hierarchical.exact(q, k, v, sel))):
        graphs[name], outs[name] = timing.capture(_seq(fn, m))
    tile = 2 * c.block * c.dim * 2
    sa, pa = sel.cpu().numpy(), p.cpu().numpy()
    u_p = unique_pairs(pa, g)
    u_miss = sum(len(np.setdiff1d(sa[x * g], pa[x * g])) for x in range(c.hkv))
    states = c.hq * c.sp * (c.dim + 2) * 4
    hits = sum(len(np.intersect1d(a, b)) for a, b in zip(sa, pa))
    small = c.hq * c.dim * (2 + 4) + 4 * (sa.size + pa.size) + ik.numel() * ik.element_size()
    kv = (u_p + u_miss) * tile
    case = Case("c4", "indexer.select_shared || gqa_hierarchical.partials(P) -> "
                "repair_saved_shared (two streams); serial: select, then gqa_hierarchical.exact",
                graphs, m, kv + states + hits * (c.dim + 2) * 4 + small, kv,
                unique_pairs(sa, g) * tile + small, primary="speculative",
                notes="selection shared by all heads: QSA indexer formula over 4 synthetic "
                      "indexer heads (no trained weights); *_given_selection: selection built "
                      "outside timing",
                pairs={"with_selection": ("speculative", "serial"),
                       "selection_given": ("speculative_given_selection",
                                           "serial_given_selection")})
    case.keep = (q, k, v, lo, hi, iq, ik, sel, p, ss, ps)
    hq_, hk_, hv_ = _host(q, k, v)
    for name in graphs:
        case.check.append((name, "attention", (hq_, hk_, hv_, sel.cpu(), outs[name][-1].cpu())))
    return case


# ------------------------------------------------------------------ c5
def case_c5(dev, seed=20261103):
    cf = C5
    rng = np.random.default_rng(seed)
    blocks = rng.integers(cf["min_blocks"], cf["max_blocks"] + 1, size=cf["requests"])
    overlaps = rng.uniform(cf["min_overlap"], cf["max_overlap"], size=cf["requests"])
    reqs = []
    # Context lengths, overlaps and hot blocks come from CPU generators; the
    # K/V values (about 2.3 G elements over the batch) from the device's
    # generator, which takes seconds where a CPU draw takes minutes.  The
    # parity checks compare the device path with the oracle on these same
    # tensors, so they hold on any machine; the values themselves are the
    # device's.
    for r in range(cf["requests"]):
        q, k, v, lo, hi = make_qkv(cf["hq"], cf["hkv"], cf["dim"], cf["block"], int(blocks[r]),
                                   cf["dtype"], True, seed + 101 * r, device=dev)
        sel = gqa.select_blocks(q, lo, hi, cf["topk"])
        p = perturb(sel.cpu(), int(blocks[r]), cf["topk"], float(overlaps[r]), seed + r).to(dev)
        reqs.append((q, k, v, lo, hi, sel, p))
    ss, ps = torch.cuda.Stream(), torch.cuda.Stream()

    def full(eps):
        def run(i):
            outs = []
            for q, k, v, lo, hi, _, p in reqs:
                outs.append(timing.overlap_run(
                    lambda: gqa.select_blocks(q, lo, hi, cf["topk"]),
                    lambda: kernels.speculate(q, k, v, p, "hybrid", 0.2, keep_mass=True),
                    lambda a, st: signed_fused.repair_signed_fused(
                        q, k, v, a, p, st, max_extra_mass=eps).output, ss, ps))
            return outs
        return run

    def fused_step(eps):
        def run(i):
            return [step_mod.speculative_signed_step(q, k, v, lo, hi, p, cf["topk"], "hybrid",
                                                     0.2, max_extra_mass=eps).result.output
                    for q, k, v, lo, hi, _, p in reqs]
        return run

    def serial(i):
        return [gqa.exact(q, k, v, gqa.select_blocks(q, lo, hi, cf["topk"]))
                for q, k, v, lo, hi, _, _ in reqs]

    # the same independent requests of one batched step spread over four
    # streams (one fork and one join per step; four hardware queues per
    # process): one request's latency-bound kernels overlap the next one's
    # bandwidth-bound ones, for both paths alike
    rs = [torch.cuda.Stream() for _ in range(4)]

    def fused_step_conc(eps):
        def run(i):
            return timing.across_streams(
                [lambda r=r: step_mod.speculative_signed_step(
                    r[0], r[1], r[2], r[3], r[4], r[6], cf["topk"], "hybrid", 0.2,
                    max_extra_mass=eps).result.output for r in reqs], rs)
        return run

    def serial_conc(i):
        return timing.across_streams(
            [lambda r=r: gqa.exact(r[0], r[1], r[2], gqa.select_blocks(r[0], r[3], r[4],
                                                                       cf["topk"]))
             for r in reqs], rs)

    # the whole batch in one paged pool: every request's front in one grid,
    # every (request, head) tail in one launch, for the speculative step and
    # for the serial path (top-K, then exact attention) alike
    kvp = paged.pack([(k, v) for _, k, v, _, _, _, _ in reqs])
    qb = torch.stack([r[0] for r in reqs])
    pb = torch.stack([r[6] for r in reqs])

    def paged_step(eps):
        return lambda i: paged.speculative_signed_step(qb, kvp, pb, cf["topk"], "hybrid", 0.2,
                                                       max_extra_mass=eps).result.output

    def paged_serial(i):
        return paged.exact(qb, kvp, cf["topk"])[1]

    graphs, outs = {}, {}
    for name, fn in (("step_eps0.01", fused_step(0.01)), ("step_strict", fused_step(0.0)),
                     ("signed_eps0.01", full(0.01)), ("signed_strict", full(0.0)),
                     ("serial", serial), ("step_eps0.01_4streams", fused_step_conc(0.01)),
                     ("serial_4streams", serial_conc), ("paged_step_eps0.01", paged_step(0.01)),
                     ("paged_step_strict", paged_step(0.0)), ("paged_serial", paged_serial)):
        graphs[name], outs[name] = timing.capture(lambda fn=fn: fn(0))
    g = cf["hq"] // cf["hkv"]
    tile = 2 * cf["block"] * cf["dim"] * 2
    full_b = kv_b = ser_b = 0
    for (q, k, v, lo, hi, sel, p), n in zip(reqs, blocks):
        sa, pa = sel.cpu().numpy(), p.cpu().numpy()
        u_p, u_a = unique_pairs(pa, g), unique_pairs(sa, g)
        u_union = unique_pairs(np.concatenate([sa, pa], axis=1), g)
        meta = 2 * cf["hkv"] * int(n) * cf["dim"] * 4
        small = cf["hq"] * cf["dim"] * (2 + 4) + 4 * (sa.size + pa.size)
        # misses are added and wrong blocks subtracted: every tile of P u A is read
        kv = u_union * tile
        kv_b += kv
        full_b += kv + meta + cf["hq"] * cf["topk"] * (cf["dim"] + 2) * 4 * 2 + small
        ser_b += meta + u_a * tile + small
    case = Case("c5", "per request: gqa.select_blocks || kernels.speculate('hybrid', 0.2, "
                "keep_mass) -> signed_fused.repair_signed_fused (eps 0.01 and strict): the "
                "fused two-launch step (step_*) and the two-stream composition (signed_*)",
                graphs, 1, full_b, kv_b, ser_b, primary="paged_step_eps0.01",
                baseline="paged_serial",
                notes=f"16 requests, contexts {int(blocks.min()) * 32}-{int(blocks.max()) * 32} "
                      "tokens; one graph replay = one batched decode step; *_4streams: the "
                      "requests spread over four streams; paged_*: the whole batch in one page "
                      "pool, two launches per step (strict_topk.paged)",
                pairs={"sequential": ("step_eps0.01", "serial"),
                       "four_streams": ("step_eps0.01_4streams", "serial_4streams"),
                       "batched_paged": ("paged_step_eps0.01", "paged_serial")})
    case.keep = (reqs, ss, ps, rs, kvp, qb, pb)
    for r, (q, k, v, lo, hi, sel, p) in enumerate(reqs):
        hq_, hlo, hhi = _host(q, lo, hi)
        case.check.append((f"ids[{r}]", "select", (hq_, hlo, hhi, cf["topk"], sel.cpu())))
        need = torch.unique(torch.cat([sel.flatten(), p.flatten()]).long())
        ks, vs = _host(k[:, need], v[:, need])
        remap = torch.full((int(blocks[r]),), -1, dtype=torch.int64)
        remap[need.cpu()] = torch.arange(len(need))
        sel_r = remap[sel.cpu().long()].to(torch.int32)
        p_r = remap[p.cpu().long()].to(torch.int32)
        case.check.append((f"strict[{r}]", "attention",
                           (hq_, ks, vs, sel_r, outs["signed_strict"][r].cpu())))
        case.check.append((f"serial[{r}]", "attention",
                           (hq_, ks, vs, sel_r, outs["serial"][r].cpu())))
        case.check.append((f"eps0.01[{r}]", "signed_fused",
                           (hq_, ks, vs, sel_r, p_r, 0.01, outs["signed_eps0.01"][r].cpu())))
        case.check.append((f"step_strict[{r}]", "attention",
                           (hq_, ks, vs, sel_r, outs["step_strict"][r].cpu())))
        case.check.append((f"step_eps0.01[{r}]", "signed_fused",
                           (hq_, ks, vs, sel_r, p_r, 0.01, outs["step_eps0.01"][r].cpu())))
        case.check.append((f"step_eps0.01_4streams[{r}]", "signed_fused",
                           (hq_, ks, vs, sel_r, p_r, 0.01,
                            outs["step_eps0.01_4streams"][r].cpu())))
        case.check.append((f"serial_4streams[{r}]", "attention",
                           (hq_, ks, vs, sel_r, outs["serial_4streams"][r].cpu())))
        case.check.append((f"paged_step_eps0.01[{r}]", "signed_fused",
                           (hq_, ks, vs, sel_r, p_r, 0.01, outs["paged_step_eps0.01"][r].cpu())))
        case.check.append((f"paged_step_strict[{r}]", "attention",
                           (hq_, ks, vs, sel_r, outs["paged_step_strict"][r].cpu())))
        case.check.append((f"paged_serial[{r}]", "attention",
                           (hq_, ks, vs, sel_r, outs["paged_serial"][r].cpu())))
    return case


# ------------------------------------------------------------------ c3 sweep
def case_c3sweep(dev, seed=20261103):
    """c3 at every prediction hit rate of its definition (100, 90, 75 %), each
    over three seeds: the fused step against the serial path, cold (12
    device copies of the inputs per seed)."""
    c = CONFIGS["c3"]
    graphs, outs, pairs, checks, steps = {}, {}, {}, [], []
    m = 12
    for ov in c.overlaps:
        for k_ in range(3):
            st = GqaStep(c, ov, seed + k_, dev, sets=m)
            steps.append(st)   # its graphs read its device copies until measured
            tag = f"{ov:g}/s{k_}"
            # the reference API's own two-stream composition (overlap_run of
            # gqa.select_blocks || gqa.partials, then repair_saved_auto) on
            # the first seed of every hit rate
            paths = (("fused", st.fused), ("serial", st.serial)) + \
                ((("composed", st.full),) if k_ == 0 else ())
            for name, fn in paths:
                graphs[f"{name}@{tag}"], outs[f"{name}@{tag}"] = timing.capture(_seq(fn, m))
            pairs[tag] = (f"fused@{tag}", f"serial@{tag}")
            if k_ == 0:
                pairs[f"composed@{tag}"] = (f"composed@{tag}", f"serial@{tag}")
            if ov == 0.9 and k_ == 0:
                by = st.bytes()
            q, k, v, lo, hi = st.host
            sel = st.selected.cpu()
            need = torch.unique(sel.flatten().long())
            remap = torch.full((c.blocks,), -1, dtype=torch.int64)
            remap[need] = torch.arange(len(need))
            sel_r = remap[sel.long()].to(torch.int32)
            ks, vs = k[:, need], v[:, need]
            for name in ("fused", "serial") + (("composed",) if k_ == 0 else ()):
                checks.append((f"{name}@{tag}", "attention",
                               (q, ks, vs, sel_r, outs[f"{name}@{tag}"][-1].cpu())))
    case = Case("c3_sweep", "c3 fused step vs serial at overlap 1.0 / 0.9 / 0.75, seeds "
                f"{seed}..{seed + 2}; the drop-in two-stream composition (repair_saved_auto) "
                "on the first seed", graphs, m, by.full, by.kv_full, by.serial,
                primary="fused@0.9/s0", baseline="serial@0.9/s0", pairs=pairs,
                notes="byte counts and fractions: the 0.9 / first-seed case")
    case.keep = steps
    case.check = checks
    return case


# ------------------------------------------------------------------ host cache
def case_cache(dev, seed=20261103):
    """c3's shape with its KV in pinned host memory (strict_topk.hostcache):
    C = 2 * G * K device slots per KV head (a quarter of the context
    resident), a decode sequence of 12 correlated queries (q_i = q_0 + 0.5 *
    noise_i) whose prediction is the previous step's selection.  The cache
    step (select || speculate on the resident predicted blocks, swap-in of
    the selected blocks, repair) against the cache's serial path (select,
    swap-in, exact attention), each on a cache of its own that evolves over
    the replays; H2D bytes per step counted by the swap-in kernel."""
    from strict_topk import hostcache
    c = CONFIGS["c3"]
    g = c.group
    q, k, v, lo, hi = make_qkv(c.hq, c.hkv, c.dim, c.block, c.blocks, c.dtype, c.hot, seed)
    m = 12
    gen = torch.Generator().manual_seed(seed + 12)
    qs = [(q.float() + 0.5 * torch.randn(q.shape, generator=gen)).to(c.dtype) for _ in range(m)]
    qd = [x.to(dev)[None].contiguous() for x in qs]
    lod, hid = lo.to(dev), hi.to(dev)
    sels = [step_mod.select_blocks(x[0], lod, hid, c.topk) for x in qd]
    preds = [sels[(i - 1) % m][None].contiguous() for i in range(m)]
    slots = 2 * g * c.topk
    spec = hostcache.build([(k, v)], slots, device=dev, bounds_dtype=c.dtype)
    ser = hostcache.build([(k, v)], slots, device=dev, bounds_dtype=c.dtype)

    def full(i):
        return hostcache.speculative_step(qd[i], spec, preds[i], c.topk).output

    def serial(i):
        return hostcache.exact(qd[i], ser, c.topk)[1]

    graphs, outs = {}, {}
    for name, fn in (("cache_step", full), ("cache_serial", serial)):
        graphs[name], outs[name] = timing.capture(_seq(fn, m))
    tile = 2 * c.block * c.dim * 2
    sa = torch.stack(sels).cpu().numpy()
    u_a = sum(unique_pairs(x, g) for x in sa) / m
    meta = 2 * c.hkv * c.blocks * c.dim * 2
    # The speculative path's device-side bytes: the prediction is the
    # previous step's selection, which that step swapped in (C >= G * K
    # slots), so every predicted block is resident (P n R = P): the front
    # reads P's tiles and writes their states, the repair reads the hits'
    # states and the tiles of A \ P (swapped in where not resident).  The
    # bounds of every block are read once, as in the serial path.  H2D
    # copies are counted apart, on both paths.
    spec_models = [byte_model(c, sels[i].cpu().numpy(), preds[i][0].cpu().numpy(), 2, 2)
                   for i in range(m)]
    spec_bytes = int(sum(b.full for b in spec_models) / m)
    spec_kv = int(sum(b.kv_full for b in spec_models) / m)

    def after():
        out = {}
        for name, cache in (("cache_step", spec), ("cache_serial", ser)):
            g_ = graphs[name]
            for _ in range(3):
                g_.replay()
            torch.cuda.synchronize()
            b0 = int(cache.h2d_bytes.item())
            reps = 10
            for _ in range(reps):
                g_.replay()
            torch.cuda.synchronize()
            out[f"h2d_bytes_per_step_{name}"] = (int(cache.h2d_bytes.item()) - b0) // (reps * m)
        out["resident_fraction"] = round(slots / c.blocks, 4)
        return out

    case = Case("cache", "host-backed cache (pinned host pool, swap-in, P n R speculation): "
                "hostcache.speculative_step against hostcache.exact", graphs, m,
                spec_bytes, spec_kv, int(meta + u_a * tile),
                primary="cache_step", baseline="cache_serial",
                notes=f"c3 shape, {slots} device slots per KV head of {c.blocks} blocks, 12 "
                      "correlated queries, prediction = previous step's selection; bytes: the "
                      "device-side algorithmic bytes, the speculative path's with the "
                      "predicted blocks' tiles and states (H2D reported separately)")
    case.after = after
    case.keep = (qd, lod, hid, sels, preds, spec, ser)
    for i in (0, m - 1):
        sel = sels[i].cpu()
        need = torch.unique(sel.flatten().long())
        remap = torch.full((c.blocks,), -1, dtype=torch.int64)
        remap[need] = torch.arange(len(need))
        sel_r = remap[sel.long()].to(torch.int32)
        for name in ("cache_step", "cache_serial"):
            case.check.append((f"{name}[{i}]", "attention",
                               (qs[i], k[:, need], v[:, need], sel_r,
                                outs[name][i][0].cpu())))
    return case


CASES = {"c1": case_c1, "c2": case_c2, "c4": case_c4, "c5": case_c5, "c3sweep": case_c3sweep,
         "cache": case_cache}
