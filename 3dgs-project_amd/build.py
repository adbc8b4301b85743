"""Builds the gfx950 C-ABI library `amdsplat/libamdsplat.so` with hipcc.

    python 3dgs-project_amd/build.py            # build (always recompiles)
    python 3dgs-project_amd/build.py --check    # only report whether the library is stale

Flags: -O3 for gfx950 only; -ffp-contract=off (every FMA is an explicit fmaf, so the
kernels and the CPU oracle round identically); IEEE division and sqrt; packed-FP32
instruction selection disabled; hardware float atomics (global_atomic_add_f32).
"""
from __future__ import annotations

import argparse
import os
import shutil
import subprocess
import sys
from pathlib import Path

HERE = Path(__file__).resolve().parent
CSRC = HERE / "csrc"
OUT = HERE / "amdsplat" / "libamdsplat.so"
SOURCES = ["capi.hip", "preprocess.hip", "binning.hip", "blend.hip", "raster2d.hip", "adam.hip", "loss.hip",
           "probe.hip"]

HIPCC_FLAGS = [
    "-O3",
    "--offload-arch=gfx950",
    "-std=c++17",
    "-fPIC",
    "-shared",
    "-ffp-contract=off",
    "-fhip-fp32-correctly-rounded-divide-sqrt",
    "-munsafe-fp-atomics",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Wall",
    "-Wno-unused-function",
]


def hipcc() -> str:
    for cand in (os.environ.get("HIPCC"), "/opt/rocm/bin/hipcc", shutil.which("hipcc")):
        if cand and Path(cand).exists():
            return cand
    raise RuntimeError("hipcc not found (set HIPCC or install ROCm)")


def sources() -> list[Path]:
    return [CSRC / s for s in SOURCES if (CSRC / s).exists()]


def stale() -> bool:
    if not OUT.exists():
        return True
    t = OUT.stat().st_mtime
    deps = list(CSRC.glob("*.h")) + list(CSRC.glob("*.hip")) + [HERE.parent / "include" / "amdsplat.h"]
    return any(p.stat().st_mtime > t for p in deps if p.exists())


def build(verbose: bool = False) -> Path:
    tmp = OUT.with_suffix(".so.tmp")
    cmd = [hipcc(), *HIPCC_FLAGS, *map(str, sources()), "-o", str(tmp)]
    if verbose:
        print(" ".join(cmd), flush=True)
    res = subprocess.run(cmd, capture_output=True, text=True)
    # the host pass does not know the packed-fp32 target feature; that warning is harmless
    noise = "'-packed-fp32-ops' is not a recognized feature"
    err = "\n".join(l for l in res.stderr.splitlines() if noise not in l)
    if res.returncode != 0:
        raise RuntimeError(f"hipcc failed ({res.returncode}):\n{err}")
    if verbose and err.strip():
        print(err)
    os.replace(tmp, OUT)
    return OUT


def main() -> int:
    ap = argparse.ArgumentParser()
    ap.add_argument("--check", action="store_true")
    ap.add_argument("-v", "--verbose", action="store_true")
    a = ap.parse_args()
    if a.check:
        print("stale" if stale() else "fresh")
        return 0
    print(build(verbose=a.verbose))
    return 0


if __name__ == "__main__":
    sys.exit(main())
