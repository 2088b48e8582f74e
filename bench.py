#!/usr/bin/env python3
"""Benchmark: one speculative block-sparse Top-K decode step on one MI355X.

A step is select (fused bound scorer + exact top-K) concurrently with
speculative GQA attention over the already-known predicted blocks, then the
strict repair -- the full path of the reference's ``overlap_run``
(``benchmarks/run_benchmark.py:99-118``).  It runs as ``strict_topk.step``:
one launch (k_step1) whose workgroups score blocks, compute the predicted
blocks' states, or -- one per query head -- run the top-K and the repair as
soon as their head's scores are published, while the states still stream.
The headline workload is config c3 (Qwen3-4B-like shape, 64K context, K=64,
90 % prediction overlap, bf16), the configuration the north-star target is
stated on.

Timing.  M consecutive decode steps are captured into one HIP graph, step i
reading the i % M-th of M device copies of the inputs (identical values,
different addresses), so the touched working set (~45 MB a step) exceeds
the L2 and Infinity Cache and operands come from HBM, as in a decode loop
where every layer's KV is touched once per token.  The timed region is
exactly --steps steps (--steps / M replays) bracketed by
torch.cuda.synchronize().  The same construction times the same-work serial
path (select, then attention over the selected blocks) and the drop-in
two-stream composition; "hot" variants replay all M steps on one input copy
(the reference's own method, caches warm).  Configs c1, c2, c4 and c5 are
timed the same way (stk_harness/suite.py) and reported under "configs".

CPU leg (skipped with --no-cpu): the repository's torch-CPU port of the
reference's serial path is timed on a bounded sample on all host cores, and
the FP64 oracle checks every output the GPU legs produced (block IDs
bit-exact, outputs within |err| <= 3e-4 + 3e-4 |ref|).

Printed JSON line (one GPU):
  value / ms_per_step   microseconds per full c3 decode step (lower is better);
  serial_us             the serial path, paired ABBA replay timing;
  roofline              the dominant kernel, k_step1 (the whole step):
                        the step's algorithmic bytes / average launch time
                        measured here with HIP events on its stream; traffic
                        from the committed rocprof counter runs of the c3
                        path; beside it, the same figures for k_front, the
                        first of the two launches that shapes outside the
                        one-launch step run;
  path_roofline         the whole step's algorithmic bytes against 8 TB/s;
  configs               c1, c2, c4, c5: speculative path vs serial;
  parity                oracle check of every measured output (CPU leg);
  cpu_baseline          the torch-CPU port of the serial path.
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

TOL = "|err| <= 3e-4 + 3e-4 |ref| vs FP64"


def log(msg):
    print(msg, file=sys.stderr, flush=True)


def parse():
    ap = argparse.ArgumentParser(description=__doc__.splitlines()[0])
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=2400)
    ap.add_argument("--warmup", type=int, default=240)
    ap.add_argument("--config", default="c3", choices=("c2", "c3"))
    ap.add_argument("--bounds", default="keys", choices=("keys", "fp32"),
                    help="lo/hi of the fused step and the serial path: in K's own 16-bit "
                         "type (exact, half the bytes) or FP32 (the reference's layout)")
    ap.add_argument("--overlap", type=float, default=0.9)
    ap.add_argument("--seed", type=int, default=20261103)
    ap.add_argument("--graph-steps", type=int, default=12,
                    help="decode steps per captured graph (and input copies)")
    ap.add_argument("--cpu-seconds", type=float, default=10.0)
    ap.add_argument("--no-cpu", action="store_true",
                    help="skip the CPU leg (CPU baseline and oracle parity)")
    ap.add_argument("--no-suite", action="store_true", help="time c3 only")
    ap.add_argument("--suite", default="c1,c2,c4,c5,c3sweep,cache",
                    help="comma-separated configs timed beside c3")
    return ap.parse_args()


def divisor_at_most(k, m):
    for x in range(min(k, m), 0, -1):
        if k % x == 0:
            return x
    return 1


def traffic_record(workload):
    """HBM bytes per k_front launch from the committed rocprof counter runs
    (FETCH_SIZE and WRITE_SIZE, each scaled by its reading for a plain copy of
    known size), or None when no run covers this workload."""
    path = ROOT / "profiles" / "k_front_traffic.json"
    if not path.exists():
        return None
    return json.loads(path.read_text()).get(workload)


def path_traffic(config):
    """The committed counter record of a config's paths (profiles/traffic.json,
    written by stk_harness/profile_traffic.py): HBM bytes per decode step of
    the speculative and the serial path, and their ratio to the algorithmic
    bytes.  None when no run covers the config."""
    path = ROOT / "profiles" / "traffic.json"
    if not path.exists():
        return None
    rec = json.loads(path.read_text()).get(config)
    if not rec:
        return None
    return {name: {"traffic": p["traffic_per_step"],
                   "traffic_over_algorithmic": p["traffic_over_algorithmic"]}
            for name, p in rec["paths"].items()}


def cpu_leg(args, step, c3_outs, cases):
    """The CPU side: the FP64 oracle as the checker of every GPU output, and
    the torch-CPU port of the serial path timed as the baseline."""
    from oracle import cpu_path
    from oracle import stk_oracle as O

    def f64(t):
        return t.double().numpy() if isinstance(t, torch.Tensor) else np.asarray(t, np.float64)

    def err(out, expected):
        o = out.double().numpy()
        d = np.abs(o - expected)
        return {"max_abs_err": float(d.max()),
                "passed": bool((d <= 3e-4 + 3e-4 * np.abs(expected)).all() and
                               np.isfinite(o).all())}

    log("bench: oracle check of the c3 outputs")
    cfg = step.cfg
    q, k, v, lo, hi = step.host
    qn, kn, vn = f64(q), f64(k), f64(v)
    ref_ids = O.select_blocks(qn, lo.numpy(), hi.numpy(), cfg.topk)
    ids_exact = bool(np.array_equal(step.selected.cpu().numpy(), ref_ids))
    expected = O.attention(qn, kn, vn, ref_ids)
    c3 = {key: err(out, expected) for key, out in c3_outs.items()}
    parity = {"c3": {"ids_bit_exact": ids_exact,
                     "max_abs_err": {k_: v_["max_abs_err"] for k_, v_ in c3.items()},
                     "passed": ids_exact and all(v_["passed"] for v_ in c3.values())}}
    for case in cases:
        log(f"bench: oracle check of {case.name}")
        res = {}
        for label, kind, data in case.check:
            if kind == "select":
                cq, clo, chi, topk, ids = data
                res[label] = {"passed": bool(np.array_equal(
                    ids.numpy(), O.select_blocks(f64(cq), clo.numpy(), chi.numpy(), topk)))}
            elif kind == "attention":
                cq, ck, cv, ids, out = data
                res[label] = err(out, O.attention(f64(cq), f64(ck), f64(cv), ids.numpy()))
            elif kind == "signed_fused":
                cq, ck, cv, sel, p, eps, out = data
                cq, ck, cv = f64(cq), f64(ck), f64(cv)
                st = O.speculate(cq, ck, cv, p.numpy(), mode="hybrid", mass_threshold=0.2,
                                 keep_mass=True)
                ref = O.repair_signed_fused(cq, ck, cv, sel.numpy(), p.numpy(), st,
                                            max_extra_mass=eps)
                res[label] = err(out, ref.output)
        parity[case.name] = {
            "passed": all(r["passed"] for r in res.values()),
            "checks": len(res),
            "max_abs_err": max((r.get("max_abs_err", 0.0) for r in res.values()), default=0.0),
            "failed": sorted(l_ for l_, r in res.items() if not r["passed"]),
        }
        if not parity[case.name]["passed"]:
            log(f"bench: {case.name} parity FAILED: {parity[case.name]['failed']}")
    parity["tolerance"] = TOL

    log(f"bench: CPU baseline (~{args.cpu_seconds:.0f} s)")
    us, steps, threads = cpu_path.time_serial(q, k, v, lo, hi, cfg.topk, budget_s=args.cpu_seconds)
    cpu = {"value": round(us, 1), "unit": "us/step", "cores": threads, "kind": "port",
           "sample": f"{steps} serial decode steps of {cfg.name} (torch fp32 CPU: "
                     "where/sum bound score, topk, gather-softmax attention)"}
    log("bench: FP64 oracle cost (~5 s)")
    o_us, o_steps = cpu_path.time_oracle(q, k, v, lo, hi, cfg.topk, budget_s=5.0)
    cpu["fp64_oracle"] = {"value": round(o_us, 1), "unit": "us/step", "steps": o_steps,
                          "sample": f"{o_steps} serial decode steps of {cfg.name} through the "
                                    "FP64 numpy oracle (bound scores, top-K, attention)"}
    return parity, cpu


def main():
    args = parse()
    if args.gpus != 1:
        sys.exit("bench.py: this path runs on one GPU; --gpus %d is not supported "
                 "(the decode step would shard by KV head, with no exchange between GPUs)" % args.gpus)
    if int(os.environ.get("WORLD_SIZE", "1")) > 1:
        sys.exit("bench.py: multi-rank launch is not supported; run with one GPU")
    if not torch.cuda.is_available():
        sys.exit("bench.py: no HIP device visible")

    from stk_harness import decode, timing
    from strict_topk import _lib

    _lib.lib()   # fail loudly if the HIP library is missing
    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)
    M = divisor_at_most(args.steps, args.graph_steps)
    log(f"bench: {args.config} inputs, {M} device copies (seed {args.seed}, "
        f"overlap {args.overlap})")
    step = decode.gqa_step(args.config, args.overlap, args.seed, dev, sets=M,
                           bounds=args.bounds)
    cfg = step.cfg

    def seq(fn, hot):
        return lambda: [fn(0 if hot else i) for i in range(M)]

    log("bench: capturing graphs")
    graphs, outs = {}, {}
    for name, fn in (("fused", step.fused), ("serial", step.serial), ("composed", step.full)):
        for hot in (False, True):
            key = name + ("_hot" if hot else "")
            graphs[key], outs[key] = timing.capture(seq(fn, hot))
    if args.bounds == "keys":
        # the same two paths on the reference's FP32 bounds
        for name, fn in (("fused_fp32_bounds", step.fused32), ("serial_fp32_bounds", step.serial32)):
            graphs[name], outs[name] = timing.capture(seq(fn, False))

    # ---- the timed region: exactly --steps fused decode steps (cold)
    g = graphs["fused"]
    warm = max(1, -(-args.warmup // M))   # whole replays, at least the requested steps
    reps = args.steps // M
    log(f"bench: {warm * M} warm-up + {reps * M} timed steps ({M} per graph replay)")
    for _ in range(warm):
        g.replay()
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record()
    for _ in range(reps):
        g.replay()
    e1.record()
    torch.cuda.synchronize()
    wall_ms = (time.perf_counter() - t0) * 1e3
    ms_per_step = e0.elapsed_time(e1) / (reps * M)
    # outputs of the last step of every captured sequence, for the CPU leg
    c3_outs = {key: out[-1].cpu() for key, out in outs.items()}

    log("bench: paired ABBA intervals")
    med, _ = timing.paired(graphs, replays=max(1, 120 // M), rounds=5, seed=args.seed)
    per_step = {key: round(us / M, 3) for key, us in med.items()}

    # ---- dominant-kernel roofline: the step is one kernel (k_step1: select ||
    # speculate, top-K and repair) where stk_step1_supported says so; one
    # launch per stk_speculative_step call, HIP events on its stream, input
    # copies rotated, the launches captured so the host's call rate does not
    # bound the measurement
    from strict_topk import step as step_mod  # noqa: F401  (loads the symbols)
    c = cfg
    st = step.speculate(0)
    ws = _lib.workspace(_lib.size("stk_step_workspace_bytes", c.hq, c.hkv, c.blocks, c.dim,
                                  c.topk), dev)
    L = _lib.lib()
    one_launch = bool(L.stk_step1_supported(_lib.dtype_code(step.q), c.hq, c.hkv, c.blocks,
                                            c.block, c.dim, c.topk, c.sp, 0))
    sel1 = torch.empty((c.hq, c.topk), dtype=torch.int32, device=dev)
    out1 = torch.empty((c.hq, c.dim), dtype=torch.float32, device=dev)
    sstate = [0]

    def whole_step():
        i = sstate[0] % M
        sstate[0] += 1
        sq, sk, sv, slo, shi = step.sets[i]
        rc = L.stk_speculative_step(sq.data_ptr(), sk.data_ptr(), sv.data_ptr(),
                                    _lib.dtype_code(sq), c.hq, c.hkv, c.blocks, c.block, c.dim,
                                    slo.data_ptr(), shi.data_ptr(), _lib.bounds_code(slo, sq),
                                    c.topk, step.predicted.data_ptr(), 0, c.sp, 0,
                                    sel1.data_ptr(), st.m.data_ptr(), st.l.data_ptr(),
                                    st.u.data_ptr(), out1.data_ptr(), ws.data_ptr(), ws.numel(),
                                    _lib.stream(dev))
        assert rc == 0, L.stk_last_error()

    nstep = 4 * M
    g_step, _ = timing.capture(lambda: [whole_step() for _ in range(nstep)])
    timing.warm([g_step], ms=50.0)
    step_us = min(timing.interval_us(g_step, 20) for _ in range(5)) / nstep
    del g_step
    by0 = step.bytes()
    tr_c3 = path_traffic("c3")
    state = [0]

    def front():
        i = state[0] % M
        state[0] += 1
        sq, sk, sv, slo, shi = step.sets[i]
        rc = L.stk_step_front(sq.data_ptr(), sk.data_ptr(), sv.data_ptr(), _lib.dtype_code(sq),
                              c.hq, c.hkv, c.blocks, c.block, c.dim, slo.data_ptr(),
                              shi.data_ptr(), _lib.bounds_code(slo, sq), c.topk,
                              step.predicted.data_ptr(), 0, c.sp,
                              st.m.data_ptr(), st.l.data_ptr(), st.u.data_ptr(), ws.data_ptr(),
                              ws.numel(), _lib.stream(dev))
        assert rc == 0, L.stk_last_error()

    # the launches are captured (4 per input copy) so the host's call rate
    # does not bound the measurement; per launch = replay interval / launches
    nfront = 4 * M
    g_front, _ = timing.capture(lambda: [front() for _ in range(nfront)])
    timing.warm([g_front], ms=50.0)
    front_us = min(timing.interval_us(g_front, 20) for _ in range(5)) / nfront
    fb = step.front_bytes()
    achieved = fb / (front_us * 1e-6) / 1e9
    workload = f"{cfg.name}@{args.overlap}"
    tr = traffic_record(workload)
    front = {"kernel": "k_front (select || speculate; the first of the two launches "
                       "that shapes outside the one-launch step run)", "bound": "hbm",
             "achieved": round(achieved, 1), "peak": 8000.0, "unit": "GB/s",
             "frac": round(achieved / 8000.0, 4),
             "traffic": tr["traffic"] if tr else None,
             "traffic_over_algorithmic": tr["traffic_over_algorithmic"] if tr else None,
             "bytes_per_launch": fb, "us_per_launch": round(front_us, 3)}
    if one_launch and args.overlap == 0.9 and args.config == "c3" and args.bounds == "keys":
        trs = tr_c3["fused"] if tr_c3 and "fused" in tr_c3 else None
    else:
        trs = None
    s_ach = by0.full / (step_us * 1e-6) / 1e9
    roofline = {"kernel": "k_step1 (the whole step in one launch: select || speculate, "
                          "top-K, repair, merge)" if one_launch else
                          "k_front + k_tail (two launches)",
                "bound": "hbm", "achieved": round(s_ach, 1), "peak": 8000.0, "unit": "GB/s",
                "frac": round(s_ach / 8000.0, 4),
                "traffic": trs["traffic"] if trs else None,
                "traffic_over_algorithmic": trs["traffic_over_algorithmic"] if trs else None,
                "bytes_per_launch": by0.full, "us_per_launch": round(step_us, 3),
                "k_front": front}

    # ---- block metadata (lo/hi from K at prefill, and one decode append) on
    # c3's K, rotating over the input copies; checked against torch.amin /
    # amax of the same K
    from strict_topk import bounds
    bstate = [0]

    def build():
        i = bstate[0] % M
        bstate[0] += 1
        return bounds.block_bounds(step.sets[i][1])

    g_b, lohi = timing.capture(lambda: [build() for _ in range(M)])
    timing.warm([g_b], ms=50.0)
    b_us = min(timing.interval_us(g_b, 5) for _ in range(3)) / M
    kk = step.sets[M - 1][1]
    b_exact = bool(torch.equal(lohi[-1][0], kk.amin(dim=2).float()) and
                   torch.equal(lohi[-1][1], kk.amax(dim=2).float()))
    knew = kk[:, 0, 0].contiguous()
    blo, bhi = lohi[-1][0].clone(), lohi[-1][1].clone()
    g_a, _ = timing.capture(lambda: [bounds.append(blo, bhi, knew, cfg.blocks - 1, 5)
                                     for _ in range(M)])
    timing.warm([g_a], ms=20.0)
    a_us = min(timing.interval_us(g_a, 20) for _ in range(3)) / M
    b_bytes = kk.numel() * kk.element_size() + 2 * lohi[-1][0].numel() * 4
    tr_meta = path_traffic("metadata")
    metadata = {"kernel": "k_bounds (lo/hi from K)", "bytes_per_launch": b_bytes,
                "traffic": tr_meta["block_bounds"] if tr_meta else None,
                "us_per_launch": round(b_us, 3),
                "achieved_GBps": round(b_bytes / (b_us * 1e-6) / 1e9, 1),
                "frac": round(b_bytes / (b_us * 1e-6) / decode.HBM_PEAK, 4),
                "bit_exact_vs_torch": b_exact, "append_us": round(a_us, 3)}
    del g_b, g_a, lohi

    by = step.bytes()
    full_us = ms_per_step * 1e3
    path = {"algorithmic_bytes": by.full, "kv_bytes": by.kv_full,
            "frac": round(by.full / (full_us * 1e-6) / decode.HBM_PEAK, 4),
            "kv_frac": round(by.kv_full / (full_us * 1e-6) / decode.HBM_PEAK, 4),
            "serial_bytes": by.serial,
            "traffic": path_traffic("c3"),
            "serial_frac": round(by.serial / (per_step["serial"] * 1e-6) / decode.HBM_PEAK, 4)}
    del graphs, g, g_front

    # ---- the other configurations
    cases, configs = [], {}
    if not args.no_suite:
        from stk_harness import suite
        for name in [x for x in args.suite.split(",") if x]:
            make = suite.CASES[name]
            log(f"bench: config {name}")
            case = make(dev, args.seed)
            configs[name] = case.measure(seed=args.seed)
            tr = path_traffic(name)
            if tr:
                configs[name]["traffic"] = tr
            case.release()   # the graphs, then the device inputs they read
            cases.append(case)
            torch.cuda.synchronize()
            torch.cuda.empty_cache()

    parity, cpu = None, None
    if not args.no_cpu:
        parity, cpu = cpu_leg(args, step, c3_outs, cases)
        if not parity["c3"]["passed"]:
            sys.exit(f"bench: c3 parity failed: {json.dumps(parity['c3'])}")

    line = {
        "metric": "us/decode step full path (select+spec+repair) vs serial; HBM GB/s % of peak",
        "value": round(full_us, 3), "unit": "us/step", "n_gpus": 1, "steps": reps * M,
        "warmup": args.warmup, "ms_per_step": round(ms_per_step, 6), "higher_is_better": False,
        "scaling": "weak", "vs_baseline": None, "dtype": "bf16",
        "warmup_steps_run": warm * M,
        "data": "synthetic (seeded generators, hot blocks +1.5 along the group-mean query)",
        "config": {"workload": f"{cfg.name}: Hq={cfg.hq} Hkv={cfg.hkv} D={cfg.dim} "
                               f"B={cfg.block} N={cfg.blocks} K={cfg.topk} "
                               f"overlap={args.overlap}, fused select||speculate + "
                               "top-K/repair, inputs rotated over "
                               f"{M} HBM copies, lo/hi "
                               f"{'in K dtype' if args.bounds == 'keys' else 'FP32'}",
                   "context": cfg.context, "topk": cfg.topk, "overlap": args.overlap,
                   "seed": args.seed, "steps_per_graph": M, "bounds": args.bounds},
        "serial_us": per_step["serial"],
        "speedup_vs_serial": round(per_step["serial"] / per_step["fused"], 4),
        "paired_us_per_step": per_step,
        "roofline": roofline,
        "path_roofline": path,
        "metadata": metadata,
        "configs": configs,
        "parity": parity,
        "wall_ms_timed_region": round(wall_ms, 2),
        "cpu_baseline": cpu,
    }
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
