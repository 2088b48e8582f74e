"""Build libstrict_topk_hip.so for gfx950 with hipcc (in-tree).

Usage: python strict-topk-overlap_amd/build_lib.py [--jobs N]

Objects go to strict-topk-overlap_amd/_build/, the shared library next to the
Python package (strict_topk/libstrict_topk_hip.so), so it travels with the
source tree.
"""
from __future__ import annotations

import argparse
import concurrent.futures as cf
import os
import shutil
import subprocess
import sys
from pathlib import Path

ROOT = Path(__file__).resolve().parent
CSRC = ROOT / "csrc"
OUT = ROOT / "strict_topk" / "libstrict_topk_hip.so"
BUILD = ROOT / "_build"
ARCH = "gfx950"
SOURCES = ["api.cpp", "states.hip", "select.hip", "repair.hip", "signed.hip", "hier.hip", "sstep.hip",
           "bounds.hip", "indexer.hip", "paged.hip", "step.hip", "tail_dense.hip", "front_pg.hip",
           "tail_pg.hip", "stail_pg.hip", "cache.hip", "srepair.hip",
           "hier_mfma.hip", "step1.hip", "repair_fast.hip", "step_small.hip"]

FLAGS = [
    f"--offload-arch={ARCH}", "-O3", "-std=c++17", "-fPIC",
    "-Wall", "-Wno-unused-function", "-Wno-unknown-warning-option",
    # packed FP32 ops stay disabled for every HIP translation unit
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
]


def hipcc():
    for cand in (os.environ.get("HIPCC"), shutil.which("hipcc"), "/opt/rocm/bin/hipcc"):
        if cand and Path(cand).exists():
            return cand
    raise RuntimeError("hipcc not found")


def _up_to_date(src: str, obj: Path) -> bool:
    """STK_INCREMENTAL=1 (development only): an object newer than its source
    and every header is kept."""
    if not os.environ.get("STK_INCREMENTAL") or not obj.exists():
        return False
    deps = [CSRC / src, *CSRC.glob("*.hpp"), ROOT.parent / "include" / "strict_topk.h"]
    return obj.stat().st_mtime > max(d.stat().st_mtime for d in deps)


def _compile(src: str) -> Path:
    obj = BUILD / (Path(src).stem + ".o")
    if _up_to_date(src, obj):
        return obj
    lang = ["-x", "hip"] if src.endswith(".hip") else []
    cmd = [hipcc(), *FLAGS, *lang, "-c", str(CSRC / src), "-o", str(obj)]
    res = subprocess.run(cmd, capture_output=True, text=True)
    noise = "packed-fp32-ops"
    err = "\n".join(l for l in res.stderr.splitlines() if noise not in l)
    if res.returncode != 0:
        raise RuntimeError(f"hipcc failed for {src}:\n{err}")
    if err.strip():
        sys.stderr.write(err + "\n")
    return obj


def build(jobs: int | None = None) -> Path:
    BUILD.mkdir(exist_ok=True)
    jobs = jobs or min(len(SOURCES), os.cpu_count() or 4)
    with cf.ThreadPoolExecutor(max_workers=jobs) as ex:
        objs = list(ex.map(_compile, SOURCES))
    tmp = OUT.with_suffix(".so.tmp")
    cmd = [hipcc(), f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", str(tmp),
           *map(str, objs)]
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"link failed:\n{res.stderr}")
    os.replace(tmp, OUT)
    return OUT


if __name__ == "__main__":
    ap = argparse.ArgumentParser()
    ap.add_argument("--jobs", type=int, default=None)
    args = ap.parse_args()
    print(build(args.jobs))
