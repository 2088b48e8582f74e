"""Launch sequence for rocprofv3 counter runs on the dominant kernel.

Runs ``--launches`` launches of the fused step's select || speculate kernel
(k_front) on the c3 workload, rotating over device copies of the inputs so
that every launch reads from HBM, then ``--launches`` launches of a plain
device copy of ``--copy-mib`` MiB (torch ``copy_``), whose bytes are known:
the copy kernel's FETCH_SIZE / WRITE_SIZE readings calibrate the counters.
No timing is done here; run it under ``rocprofv3 --pmc FETCH_SIZE`` and
``rocprofv3 --pmc WRITE_SIZE`` (one counter block per run).

    python3 -m stk_harness.profile_front --launches 48
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


def main():
    ap = argparse.ArgumentParser(description=__doc__.splitlines()[0])
    ap.add_argument("--config", default="c3")
    ap.add_argument("--overlap", type=float, default=0.9)
    ap.add_argument("--seed", type=int, default=20261103)
    ap.add_argument("--launches", type=int, default=48)
    ap.add_argument("--sets", type=int, default=12)
    ap.add_argument("--copy-mib", type=int, default=256)
    args = ap.parse_args()
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
                              shi.data_ptr(), c.topk, step.predicted.data_ptr(), 0, c.sp,
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
