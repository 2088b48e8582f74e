#!/usr/bin/env python3
"""Benchmark: one speculative block-sparse Top-K decode step on one MI355X.

A step is select (fused bound scorer + exact top-K) concurrently with
speculative GQA attention over the predicted blocks, joined, then the strict
repair -- the full path of the reference's ``overlap_run``
(``benchmarks/run_benchmark.py:99-118``), captured once into a HIP graph and
replayed.  The workload is config c3 (Qwen3-4B-like shape, 64K context, K=64,
90 % prediction overlap, bf16), the configuration
the north-star target is stated on.

Printed JSON line (rank 0 only, one GPU):
  value / ms_per_step   microseconds per full decode step (lower is better),
                        timed over exactly --steps graph replays bracketed by
                        torch.cuda.synchronize(), inputs resident in HBM;
  serial_us             the same-work serial step (select, then attention over
                        the selected blocks), paired ABBA replay timing;
  roofline              dominant kernel, algorithmic bytes / average launch
                        duration measured here with HIP events on its stream;
  path_roofline         the whole step's algorithmic bytes against 8 TB/s;
  cpu_baseline          this repository's torch-CPU port of the reference's
                        serial path on a bounded sample of the same workload.
"""
from __future__ import annotations

import argparse
import json
import os
import sys
import time
from pathlib import Path

ROOT = Path(__file__).resolve().parent
for _p in (ROOT / "strict-topk-overlap_amd", ROOT):
    if str(_p) not in sys.path:
        sys.path.insert(0, str(_p))

import numpy as np  # noqa: E402
import torch  # noqa: E402


def log(msg):
    print(msg, file=sys.stderr, flush=True)


def parse():
    ap = argparse.ArgumentParser(description=__doc__.splitlines()[0])
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=2000)
    ap.add_argument("--warmup", type=int, default=200)
    ap.add_argument("--config", default="c3", choices=("c2", "c3"))
    ap.add_argument("--overlap", type=float, default=0.9)
    ap.add_argument("--seed", type=int, default=20261103)
    ap.add_argument("--cpu-seconds", type=float, default=10.0)
    ap.add_argument("--no-cpu", action="store_true")
    return ap.parse_args()


def main():
    args = parse()
    if args.gpus != 1:
        sys.exit("bench.py: this path runs on one GPU; --gpus %d is not supported "
                 "(the decode step shards by KV head with no exchange; see DESIGN.md)" % args.gpus)
    if int(os.environ.get("WORLD_SIZE", "1")) > 1:
        sys.exit("bench.py: multi-rank launch is not supported; run with one GPU")
    if not torch.cuda.is_available():
        sys.exit("bench.py: no HIP device visible")

    from oracle import stk_oracle as O
    from stk_harness import decode, timing
    from strict_topk import _lib

    _lib.lib()   # fail loudly if the HIP library is missing
    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)
    log(f"bench: building {args.config} inputs (seed {args.seed}, overlap {args.overlap})")
    step = decode.gqa_step(args.config, args.overlap, args.seed, dev)
    cfg = step.cfg
    q, k, v, lo, hi = step.host

    # ---- parity of the measured configuration against the FP64 oracle
    log("bench: oracle selection and attention")
    qn, kn, vn = (t.double().numpy() for t in (q, k, v))
    ref_ids = O.select_blocks(qn, lo.numpy(), hi.numpy(), cfg.topk)
    ids_exact = bool(np.array_equal(step.selected.cpu().numpy(), ref_ids))
    expected = O.attention(qn, kn, vn, ref_ids)

    log("bench: capturing graphs")
    g_full, out_full = timing.capture(step.full)
    g_serial, out_serial = timing.capture(step.serial)
    g_select, _ = timing.capture(step.select)
    g_spec, st_spec = timing.capture(step.speculate)
    a_fixed = step.selected
    g_repair, _ = timing.capture(lambda: step.finish(a_fixed, st_spec))

    def err(out):
        o = out.double().cpu().numpy()
        d = np.abs(o - expected)
        return float(d.max()), float((d / np.maximum(np.abs(expected), 1e-30)).max()), \
            bool((d <= 3e-4 + 3e-4 * np.abs(expected)).all() and np.isfinite(o).all())

    abs_full, rel_full, ok_full = err(out_full)
    abs_ser, _, ok_ser = err(out_serial)
    if not (ids_exact and ok_full and ok_ser):
        sys.exit(f"bench: parity failed (ids exact {ids_exact}, full err {abs_full:.3g}, "
                 f"serial err {abs_ser:.3g})")

    # ---- the timed region: exactly --steps full decode steps
    log(f"bench: {args.warmup} warm-up + {args.steps} timed full steps")
    for _ in range(args.warmup):
        g_full.replay()
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record()
    for _ in range(args.steps):
        g_full.replay()
    e1.record()
    torch.cuda.synchronize()
    wall_ms = (time.perf_counter() - t0) * 1e3
    ms_per_step = e0.elapsed_time(e1) / args.steps
    # the replay output must still be right after the timed region
    if not err(out_full)[2]:
        sys.exit("bench: full-path output changed during timing")

    log("bench: paired ABBA intervals (full, serial, phases)")
    med, _ = timing.paired({"full": g_full, "serial": g_serial, "select": g_select,
                            "speculate": g_spec, "repair": g_repair}, replays=100, rounds=5,
                           seed=args.seed)

    # ---- dominant-kernel roofline: speculative states kernel (k_states),
    # one launch per call of gqa.partials, events on its stream
    by = step.bytes()
    kernels = {}
    st_us = timing.launch_us(step.speculate, launches=500)
    spec_bytes = by.kv_spec + cfg.hq * cfg.sp * 4 * (cfg.dim + 2) + cfg.hq * cfg.dim * 2 \
        + cfg.hq * cfg.sp * 4
    kernels["k_states(speculate)"] = {"us": st_us, "bytes": spec_bytes}
    sel_us = timing.launch_us(step.select, launches=500)
    kernels["select(k_score_sort+k_topk_merge)"] = {"us": sel_us, "bytes": by.meta}
    dominant = "k_states(speculate)"
    dk = kernels[dominant]
    achieved = dk["bytes"] / (dk["us"] * 1e-6) / 1e9
    roofline = {"kernel": dominant, "bound": "hbm", "achieved": round(achieved, 1),
                "peak": 8000.0, "unit": "GB/s", "frac": round(achieved / 8000.0, 4),
                "traffic": None, "bytes_per_launch": dk["bytes"], "us_per_launch": round(dk["us"], 3)}

    full_us = ms_per_step * 1e3
    path = {"algorithmic_bytes": by.full, "kv_bytes": by.kv_full,
            "frac": round(by.full / (full_us * 1e-6) / decode.HBM_PEAK, 4),
            "kv_frac": round(by.kv_full / (full_us * 1e-6) / decode.HBM_PEAK, 4),
            "serial_bytes": by.serial,
            "serial_frac": round(by.serial / (med["serial"] * 1e-6) / decode.HBM_PEAK, 4)}

    cpu = None
    if not args.no_cpu:
        from oracle import cpu_path
        log(f"bench: CPU baseline (~{args.cpu_seconds:.0f} s)")
        us, steps, threads = cpu_path.time_serial(q, k, v, lo, hi, cfg.topk,
                                                  budget_s=args.cpu_seconds)
        cpu = {"value": round(us, 1), "unit": "us/step", "cores": threads, "kind": "port",
               "sample": f"{steps} serial decode steps of {cfg.name} (torch fp32 CPU: "
                         "where/sum bound score, topk, gather-softmax attention)"}

    line = {
        "metric": "us/decode step full path (select+spec+repair) vs serial; HBM GB/s % of peak",
        "value": round(full_us, 3), "unit": "us/step", "n_gpus": 1, "steps": args.steps,
        "warmup": args.warmup, "ms_per_step": round(ms_per_step, 6), "higher_is_better": False,
        "scaling": "weak", "vs_baseline": None, "dtype": "bf16",
        "data": "synthetic (seeded CPU generator, hot blocks +1.5 along the group-mean query)",
        "config": {"workload": f"{cfg.name}: Hq={cfg.hq} Hkv={cfg.hkv} D={cfg.dim} "
                               f"B={cfg.block} N={cfg.blocks} K={cfg.topk} "
                               f"overlap={args.overlap} gqa_light auto repair",
                   "context": cfg.context, "topk": cfg.topk, "overlap": args.overlap,
                   "seed": args.seed},
        "serial_us": round(med["serial"], 3),
        "speedup_vs_serial": round(med["serial"] / med["full"], 4),
        "paired_us": {k_: round(v_, 3) for k_, v_ in med.items()},
        "roofline": roofline,
        "path_roofline": path,
        "kernels": {k_: {"us": round(v_["us"], 3), "bytes": v_["bytes"],
                         "GB/s": round(v_["bytes"] / (v_["us"] * 1e-6) / 1e9, 1)}
                    for k_, v_ in kernels.items()},
        "parity": {"ids_bit_exact": ids_exact, "max_abs_err": abs_full, "max_rel_err": rel_full,
                   "serial_max_abs_err": abs_ser},
        "wall_ms_timed_region": round(wall_ms, 2),
        "cpu_baseline": cpu,
    }
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
