"""Launch sequence for rocprofv3 counter runs on the dominant kernel.

Runs ``--launches`` launches of the fused step's select || speculate kernel
(k_front) on the c3 workload, rotating over device copies of the inputs so
that every launch reads from HBM, then ``--launches`` launches of a plain
device copy of ``--copy-mib`` MiB (torch ``copy_``), whose bytes are known:
the copy kernel's FETCH_SIZE / WRITE_SIZE readings calibrate the counters.
No timing is done here; run it under ``rocprofv3 --pmc FETCH_SIZE`` and
``rocprofv3 --pmc WRITE_SIZE`` (one counter block per run).

    python3 -m stk_harness.profile_front --launches 48

``--summarize FETCH_CSV WRITE_CSV --alg-bytes N`` (no GPU needed) turns the
two runs' counter_collection.csv files into the traffic record that
bench.py reports: each counter's mean k_front reading (KiB per dispatch)
scaled by bytes copied / reading of the calibration copies; N is the
algorithmic byte count the counter runs printed.
"""
from __future__ import annotations

import argparse
import sys
from pathlib import Path

ROOT = Path(__file__).resolve().parents[2]
for _p in (ROOT / "strict-topk-overlap_amd", ROOT):
    if str(_p) not in sys.path:
        sys.path.insert(0, str(_p))

import torch  # noqa: E402


def _readings(path, launches):
    """Mean k_front reading and mean calibration-copy reading (KiB) of one
    rocprofv3 counter_collection.csv.  The calibration copies are the
    copyBuffer dispatches after the last k_front launch with the largest
    grid (smaller copies, such as reading results back, are skipped)."""
    import csv
    with open(path, newline="") as f:
        rows = [(int(r["Dispatch_Id"]), r["Kernel_Name"], int(r["Grid_Size"]),
                 float(r["Counter_Value"])) for r in csv.DictReader(f)]
    front = [(d, k, v) for d, k, g, v in rows if "k_front" in k]
    if not front:
        raise SystemExit(f"profile_front: {path} holds no k_front dispatch")
    last = max(d for d, _, _ in front)
    after = [(g, v) for d, k, g, v in rows if d > last and "copyBuffer" in k]
    big = max((g for g, _ in after), default=0)
    copies = [v for g, v in after if g == big]
    if len(copies) != launches:
        raise SystemExit(f"profile_front: {path}: {len(copies)} calibration copies, "
                         f"expected {launches}")
    vals = [v for _, _, v in front]
    return front[-1][1], len(vals), sum(vals) / len(vals), sum(copies) / len(copies)


def summarize(fetch_csv, write_csv, args):
    import json
    if not args.alg_bytes:
        raise SystemExit("profile_front: --summarize needs --alg-bytes")
    copy_bytes = args.copy_mib * (1 << 20)
    name, disp, f_raw, f_cal = _readings(fetch_csv, args.launches)
    _, _, w_raw, w_cal = _readings(write_csv, args.launches)
    ff, wf = copy_bytes / (f_cal * 1024), copy_bytes / (w_cal * 1024)
    fetch, write = f_raw * 1024 * ff, w_raw * 1024 * wf
    alg = args.alg_bytes
    key = f"{args.config}@{args.overlap:g}"
    rec = {"kernel": name, "traffic": int(fetch + write), "fetch_bytes": int(fetch),
           "write_bytes": int(write), "fetch_kib_raw": round(f_raw, 1),
           "write_kib_raw": round(w_raw, 1), "dispatches": disp,
           "fetch_factor": round(ff, 5), "write_factor": round(wf, 5),
           "calibration": f"torch copy_ of {args.copy_mib} MiB (__amd_rocclr_copyBuffer): "
                          f"FETCH_SIZE {f_cal:.1f} KiB, WRITE_SIZE {w_cal:.1f} KiB per dispatch",
           "algorithmic_bytes": alg, "traffic_over_algorithmic": round((fetch + write) / alg, 4)}
    out = ROOT / "profiles" / "k_front_traffic.json"
    data = json.loads(out.read_text()) if out.exists() else {}
    rec["commands"] = data.get(key, {}).get("commands", [])
    data[key] = rec
    out.write_text(json.dumps(data, indent=1) + "\n")
    print(json.dumps(rec, indent=1))


def main():
    ap = argparse.ArgumentParser(description=__doc__.splitlines()[0])
    ap.add_argument("--config", default="c3")
    ap.add_argument("--overlap", type=float, default=0.9)
    ap.add_argument("--seed", type=int, default=20261103)
    ap.add_argument("--launches", type=int, default=48)
    ap.add_argument("--sets", type=int, default=12)
    ap.add_argument("--copy-mib", type=int, default=256)
    ap.add_argument("--summarize", nargs=2, metavar=("FETCH_CSV", "WRITE_CSV"))
    ap.add_argument("--alg-bytes", type=int, default=0)
    args = ap.parse_args()
    if args.summarize:
        return summarize(*args.summarize, args)
    if not torch.cuda.is_available():
        sys.exit("profile_front: no HIP device visible")
    from stk_harness import decode
    from strict_topk import _lib

    dev = torch.device("cuda:0")
    step = decode.gqa_step(args.config, args.overlap, args.seed, dev, sets=args.sets)
    c = step.cfg
    st = step.speculate(0)
    ws = _lib.workspace(_lib.size("stk_step_workspace_bytes", c.hq, c.hkv, c.blocks, c.dim,
                                  c.topk), dev)
    L = _lib.lib()
    for i in range(args.launches):
        sq, sk, sv, slo, shi = step.sets[i % args.sets]
        rc = L.stk_step_front(sq.data_ptr(), sk.data_ptr(), sv.data_ptr(), _lib.dtype_code(sq),
                              c.hq, c.hkv, c.blocks, c.block, c.dim, slo.data_ptr(),
                              shi.data_ptr(), _lib.bounds_code(slo, sq), c.topk,
                              step.predicted.data_ptr(), 0, c.sp,
                              st.m.data_ptr(), st.l.data_ptr(), st.u.data_ptr(), ws.data_ptr(),
                              ws.numel(), _lib.stream(dev))
        if rc:
            sys.exit("profile_front: " + L.stk_last_error().decode())
    n = args.copy_mib * (1 << 20) // 4
    src = torch.ones(n, device=dev)
    dst = torch.empty_like(src)
    for _ in range(args.launches):
        dst.copy_(src)
    torch.cuda.synchronize()
    by = step.front_bytes()
    print(f"profile_front: {args.launches} k_front launches ({by} algorithmic bytes each), "
          f"{args.launches} copies of {args.copy_mib} MiB", flush=True)


if __name__ == "__main__":
    main()
