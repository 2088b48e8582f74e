"""Kernel timeline of the drop-in two-stream composition in a HIP graph.

The reference's full step is ``overlap_run``
(``benchmarks/run_benchmark.py:99-118``): ``gqa.select_blocks`` on one
stream while ``gqa.partials`` speculates on another, joined, then
``gqa_light.repair_saved_auto``.  Captured into a graph, the two branches may
or may not run concurrently on the device; this tool records it.

    rocprofv3 --kernel-trace --output-format csv -d OUT -o compose -- \\
        python3 -m stk_harness.profile_compose --overlap 1.0 --replays 50

replays a graph of 12 composed c3 steps (inputs rotated over 12 device
copies, as bench.py times them); then

    python3 -m stk_harness.profile_compose --summarize OUT/.../compose_kernel_trace.csv

(no GPU needed) groups each step's kernels and prints, as medians over the
steps: the select branch's span (k_score .. the top-K), the speculation
branch's span (k_states_tok), how long the two overlap, the repair, and the
step from its first kernel's start to the repair's end.
"""
from __future__ import annotations

import argparse
import csv
import statistics
import sys
from pathlib import Path

ROOT = Path(__file__).resolve().parents[2]
for _p in (ROOT / "strict-topk-overlap_amd", ROOT):
    if str(_p) not in sys.path:
        sys.path.insert(0, str(_p))

SELECT = ("k_score", "k_topk")
SPEC = ("k_states_tok",)
REPAIR = ("k_repair_fast", "k_gqa_repair")


def _role(name):
    for tag, keys in (("select", SELECT), ("spec", SPEC), ("repair", REPAIR)):
        if any(k in name for k in keys):
            return tag
    return None


def summarize(path):
    with open(path, newline="") as f:
        rows = [(int(r["Start_Timestamp"]), int(r["End_Timestamp"]), r["Kernel_Name"],
                 r.get("Queue_Id", "")) for r in csv.DictReader(f)]
    rows.sort()
    steps, cur = [], []
    for start, end, name, queue in rows:
        role = _role(name)
        if role is None:
            continue
        cur.append((role, start, end, queue))
        if role == "repair":
            steps.append(cur)
            cur = []
    stats = {"select_us": [], "spec_us": [], "overlap_us": [], "repair_us": [], "step_us": [],
             "gap_before_repair_us": []}
    queues = set()
    for st in steps:
        sel = [(s, e) for r, s, e, _ in st if r == "select"]
        spc = [(s, e) for r, s, e, _ in st if r == "spec"]
        rep = [(s, e) for r, s, e, _ in st if r == "repair"]
        if not sel or not spc or not rep:
            continue
        queues.update((r, q) for r, _, _, q in st)
        s0, s1 = min(s for s, _ in sel), max(e for _, e in sel)
        p0, p1 = min(s for s, _ in spc), max(e for _, e in spc)
        r0, r1 = rep[-1]
        stats["select_us"].append((s1 - s0) / 1e3)
        stats["spec_us"].append((p1 - p0) / 1e3)
        stats["overlap_us"].append(max(0, min(s1, p1) - max(s0, p0)) / 1e3)
        stats["repair_us"].append((r1 - r0) / 1e3)
        stats["gap_before_repair_us"].append((r0 - max(s1, p1)) / 1e3)
        stats["step_us"].append((r1 - min(s0, p0)) / 1e3)
    out = {k: round(statistics.median(v), 3) for k, v in stats.items() if v}
    out["steps"] = len(stats["step_us"])
    out["queues"] = sorted({f"{r}:{q}" for r, q in queues})
    print(out)
    return out


def main():
    ap = argparse.ArgumentParser(description=__doc__.splitlines()[0])
    ap.add_argument("--overlap", type=float, default=1.0)
    ap.add_argument("--seed", type=int, default=20261103)
    ap.add_argument("--replays", type=int, default=50)
    ap.add_argument("--summarize", metavar="KERNEL_TRACE_CSV")
    args = ap.parse_args()
    if args.summarize:
        return summarize(args.summarize)
    import torch
    from stk_harness import decode, timing
    dev = torch.device("cuda:0")
    step = decode.gqa_step("c3", args.overlap, args.seed, dev, sets=12)
    g, _ = timing.capture(lambda: [step.full(i) for i in range(12)])
    for _ in range(args.replays):
        g.replay()
    torch.cuda.synchronize()
    print(f"profile_compose: {args.replays} replays of 12 composed c3 steps at overlap "
          f"{args.overlap}", flush=True)


if __name__ == "__main__":
    main()
