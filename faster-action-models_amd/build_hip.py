"""Build libfam_hip.so (the gfx950 kernels + C ABI) in-tree.

    python faster-action-models_amd/build_hip.py [--jobs N]

Each csrc/*.hip is compiled by hipcc for gfx950 into _build/, then linked into
fam/libfam_hip.so next to the Python package that loads it.  Packed-fp32 instruction
selection is disabled for device code (-packed-fp32-ops); hipcc's host pass warns that it
does not know the feature, which is harmless and filtered from the log.  Floating-point
contraction is limited to single expressions (-ffp-contract=on) so that the explicit bf16
roundings the kernels perform to mirror the reference are kept.
"""
from __future__ import annotations

import argparse
import concurrent.futures as cf
import glob
import os
import shutil
import subprocess
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
CSRC = os.path.join(HERE, "csrc")
BUILD = os.path.join(HERE, "_build")
OUT = os.path.join(HERE, "fam", "libfam_hip.so")
ARCH = "gfx950"

HIPCC_FLAGS = [
    f"--offload-arch={ARCH}", "-O3", "-fPIC", "-std=c++17",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    # contraction only inside one expression: HIP's default (fast) also fuses across an
    # explicit float -> bf16 -> float round trip, dropping a rounding the reference performs
    "-ffp-contract=on",
    "-Wall", "-Wno-unused-function", "-Wno-unused-variable",
]


def hipcc() -> str:
    for cand in (os.environ.get("HIPCC"), "/opt/rocm/bin/hipcc", shutil.which("hipcc")):
        if cand and os.path.exists(cand):
            return cand
    raise RuntimeError("hipcc not found (expected /opt/rocm/bin/hipcc)")


def _filter(log: str) -> str:
    return "\n".join(l for l in log.splitlines() if "packed-fp32-ops" not in l)


def _compile(src: str) -> str:
    obj = os.path.join(BUILD, os.path.basename(src).replace(".hip", ".o"))
    cmd = [hipcc(), *HIPCC_FLAGS, "-c", src, "-o", obj]
    p = subprocess.run(cmd, capture_output=True, text=True)
    log = _filter(p.stdout + p.stderr)
    if p.returncode != 0:
        raise RuntimeError(f"hipcc failed for {src}:\n{log}")
    if log.strip():
        print(log, file=sys.stderr)
    return obj


def build(jobs: int = 4, verbose: bool = True) -> str:
    os.makedirs(BUILD, exist_ok=True)
    srcs = sorted(glob.glob(os.path.join(CSRC, "*.hip")))
    if not srcs:
        raise RuntimeError(f"no HIP sources under {CSRC}")
    with cf.ThreadPoolExecutor(max_workers=max(1, jobs)) as ex:
        objs = list(ex.map(_compile, srcs))
    tmp = OUT + ".tmp"
    cmd = [hipcc(), f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", tmp, *objs]
    p = subprocess.run(cmd, capture_output=True, text=True)
    if p.returncode != 0:
        raise RuntimeError(f"link failed:\n{_filter(p.stdout + p.stderr)}")
    os.replace(tmp, OUT)
    if verbose:
        print(f"built {OUT} from {len(srcs)} sources")
    return OUT


if __name__ == "__main__":
    ap = argparse.ArgumentParser()
    ap.add_argument("--jobs", type=int, default=min(8, os.cpu_count() or 4))
    build(ap.parse_args().jobs)
