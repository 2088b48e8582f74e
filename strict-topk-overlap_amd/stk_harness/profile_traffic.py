"""HBM traffic of the benchmark paths from rocprofv3 counters.

Builds one benchmark case (``suite.CASES``; ``c3``: the headline step and
its serial path at 90 % overlap; ``metadata``: the block-bounds builder on
c3's K), replays its speculative (primary) and serial (baseline)
graphs ``--replays`` times each between marker kernels, then launches
``--launches`` plain device copies of ``--copy-mib`` MiB whose bytes are
known.  Run it twice under rocprofv3, one counter per run:

    rocprofv3 --pmc FETCH_SIZE -d gpurun_out/tr_f -o f --output-format csv \\
        -- python3 -u strict-topk-overlap_amd/stk_harness/profile_traffic.py --config c4
    rocprofv3 --pmc WRITE_SIZE -d gpurun_out/tr_w -o w --output-format csv \\
        -- python3 -u strict-topk-overlap_amd/stk_harness/profile_traffic.py --config c4

then (no GPU needed)

    python3 strict-topk-overlap_amd/stk_harness/profile_traffic.py --config c4 \\
        --summarize gpurun_out/tr_f/f_counter_collection.csv gpurun_out/tr_w/w_counter_collection.csv

which writes the path's calibrated traffic per decode step (every dispatch
between its markers, FETCH_SIZE and WRITE_SIZE each scaled by bytes copied /
reading of the calibration copies), the traffic of each kernel per dispatch,
and the path's algorithmic bytes per step into ``profiles/traffic.json``
(bench.py reports them under ``configs``).
"""
from __future__ import annotations

import argparse
import json
import sys
from pathlib import Path

ROOT = Path(__file__).resolve().parents[2]
for _p in (ROOT / "strict-topk-overlap_amd", ROOT):
    if str(_p) not in sys.path:
        sys.path.insert(0, str(_p))

OUT = ROOT / "profiles" / "traffic.json"
MARK = 20000     # spin cycles of the marker kernel


def _marker():
    import torch
    torch.cuda._sleep(MARK)


def run(args):
    import torch
    from stk_harness import suite, timing
    if not torch.cuda.is_available():
        sys.exit("profile_traffic: no HIP device visible")
    dev = torch.device("cuda:0")
    if args.config == "metadata":
        from stk_harness import decode
        from strict_topk import bounds
        st = decode.gqa_step("c3", 0.9, args.seed, dev, sets=12)
        state = [0]

        def build():
            i = state[0] % 12
            state[0] += 1
            return bounds.block_bounds(st.sets[i][1])

        g, _ = timing.capture(lambda: [build() for _ in range(12)])
        k = st.sets[0][1]
        alg = k.numel() * k.element_size() + 2 * st.cfg.hkv * st.cfg.blocks * st.cfg.dim * 4
        paths = {"block_bounds": (g, 12, alg)}
        keep = st
    elif args.config == "c3":
        from stk_harness import decode
        st = decode.gqa_step("c3", 0.9, args.seed, dev, sets=12)
        paths = {}
        for name, fn in (("fused", st.fused), ("serial", st.serial)):
            g, _ = timing.capture(lambda fn=fn: [fn(i) for i in range(12)])
            by = st.bytes()
            paths[name] = (g, 12, by.full if name == "fused" else by.serial)
        keep = st
    else:
        case = suite.CASES[args.config](dev, args.seed)
        m = case.steps_per_graph
        paths = {case.primary: (case.graphs[case.primary], m, case.bytes_full),
                 case.baseline: (case.graphs[case.baseline], m, case.bytes_serial)}
        keep = case
    for g, _, _ in paths.values():
        timing.warm([g], ms=20.0)
    torch.cuda.synchronize()
    info = {"config": args.config, "replays": args.replays, "paths": {}}
    for name, (g, m, alg) in paths.items():
        _marker()
        for _ in range(args.replays):
            g.replay()
        _marker()
        torch.cuda.synchronize()
        info["paths"][name] = {"steps": args.replays * m, "algorithmic_bytes": int(alg)}
    n = args.copy_mib * (1 << 20) // 4
    src = torch.ones(n, device=dev)
    dst = torch.empty_like(src)
    for _ in range(args.launches):
        dst.copy_(src)
    torch.cuda.synchronize()
    del keep
    (ROOT / "gpurun_out").mkdir(exist_ok=True)
    (ROOT / "gpurun_out" / f"traffic_{args.config}.json").write_text(json.dumps(info))
    print("profile_traffic: " + json.dumps(info), flush=True)


def _rows(path):
    import csv
    with open(path, newline="") as f:
        return [(int(r["Dispatch_Id"]), r["Kernel_Name"], int(r["Grid_Size"]),
                 float(r["Counter_Value"])) for r in csv.DictReader(f)]


def _regions(rows, copies):
    """Per measured path (in launch order) the {kernel: [readings]} between
    its two markers, and the mean reading of the calibration copies."""
    rows = sorted(rows)
    marks = [i for i, (_, k, _, _) in enumerate(rows) if "sleep" in k.lower() or "spin" in k.lower()]
    if len(marks) % 2:
        raise SystemExit("profile_traffic: unpaired marker kernels")
    regions = []
    for a, b in zip(marks[::2], marks[1::2]):
        per = {}
        for _, k, _, v in rows[a + 1:b]:
            per.setdefault(k, []).append(v)
        regions.append(per)
    tail = [(g, v) for d, k, g, v in rows[marks[-1] + 1:] if "copyBuffer" in k]
    big = max((g for g, _ in tail), default=0)
    cal = [v for g, v in tail if g == big]
    if len(cal) != copies:
        raise SystemExit(f"profile_traffic: {len(cal)} calibration copies, expected {copies}")
    return regions, sum(cal) / len(cal)


def summarize(fetch_csv, write_csv, args):
    info = json.loads((ROOT / "gpurun_out" / f"traffic_{args.config}.json").read_text())
    fr, f_cal = _regions(_rows(fetch_csv), args.launches)
    wr, w_cal = _regions(_rows(write_csv), args.launches)
    copy_bytes = args.copy_mib * (1 << 20)
    ff, wf = copy_bytes / (f_cal * 1024), copy_bytes / (w_cal * 1024)
    names = list(info["paths"])
    if len(fr) != len(names) or len(wr) != len(names):
        raise SystemExit("profile_traffic: marker regions do not match the paths")
    rec = {"calibration": f"torch copy_ of {args.copy_mib} MiB: fetch factor {ff:.5f}, "
                          f"write factor {wf:.5f}", "paths": {}}
    for name, fd, wd in zip(names, fr, wr):
        steps = info["paths"][name]["steps"]
        alg = info["paths"][name]["algorithmic_bytes"]
        kernels = {}
        tf = tw = 0.0
        for k in fd:
            f = sum(fd[k]) * 1024 * ff
            w = sum(wd.get(k, [0.0])) * 1024 * wf
            tf, tw = tf + f, tw + w
            kernels[k] = {"dispatches_per_step": round(len(fd[k]) / steps, 3),
                          "traffic_per_dispatch": int((f + w) / len(fd[k])),
                          "fetch_per_dispatch": int(f / len(fd[k])),
                          "write_per_dispatch": int(w / len(fd[k]))}
        per_step = (tf + tw) / steps
        rec["paths"][name] = {"steps": steps, "traffic_per_step": int(per_step),
                              "fetch_per_step": int(tf / steps),
                              "write_per_step": int(tw / steps),
                              "algorithmic_bytes": alg,
                              "traffic_over_algorithmic": round(per_step / alg, 4),
                              "kernels": kernels}
    data = json.loads(OUT.read_text()) if OUT.exists() else {}
    data[args.config] = rec
    OUT.write_text(json.dumps(data, indent=1) + "\n")
    print(json.dumps(rec, indent=1))


def main():
    ap = argparse.ArgumentParser(description=__doc__.splitlines()[0])
    ap.add_argument("--config", required=True)
    ap.add_argument("--seed", type=int, default=20261103)
    ap.add_argument("--replays", type=int, default=4)
    ap.add_argument("--launches", type=int, default=8)
    ap.add_argument("--copy-mib", type=int, default=256)
    ap.add_argument("--summarize", nargs=2, metavar=("FETCH_CSV", "WRITE_CSV"))
    args = ap.parse_args()
    if args.summarize:
        return summarize(*args.summarize, args)
    run(args)


if __name__ == "__main__":
    main()
