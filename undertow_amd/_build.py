"""Builds libundertow_hip.so (the gfx950 backend) in-tree with hipcc.

Every ``csrc/*.hip`` file is compiled to an object for gfx950 only and the
objects are linked into ``undertow_amd/lib/libundertow_hip.so``.  Packed
FP32 instructions are disabled for all device code, and floating-point
contraction is off (FMAs are written explicitly where wanted).
"""
from __future__ import annotations

import concurrent.futures as cf
import os
import shutil
import subprocess
from pathlib import Path

HERE = Path(__file__).resolve().parent
CSRC = HERE / "csrc"
OBJ = HERE / "lib" / "obj"
LIB = HERE / "lib" / "libundertow_hip.so"

HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")
# Tuning switches of the sources (``#ifndef UT_...`` macros), e.g.
# UT_BUILD_DEFINES="-DUT_MOE_FOLD_COMBINE=1" to rebuild a measured variant.
DEFINES = os.environ.get("UT_BUILD_DEFINES", "").split()
ARCH = "gfx950"
FLAGS = [
    f"--offload-arch={ARCH}", "-O3", "-fPIC", "-std=c++17", "-ffp-contract=off",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Wall", "-Wno-unused-function", "-Wno-unused-variable", "-Wno-unused-result",
]


def _compile(src: Path) -> Path:
    obj = OBJ / (src.stem + ".o")
    cmd = [HIPCC, *FLAGS, *DEFINES, "-c", str(src), "-o", str(obj)]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"hipcc failed for {src.name}:\n{r.stdout}\n{r.stderr}")
    return obj


def build(jobs: int = 8) -> Path:
    """Compile every HIP source and link the shared library (always rebuilds)."""
    bad = [d for d in DEFINES if not d.startswith("-DUT_")]
    if bad:
        raise RuntimeError(f"UT_BUILD_DEFINES takes -DUT_* switches only, got {bad}")
    if not Path(HIPCC).exists() and shutil.which("hipcc") is None:
        raise RuntimeError("hipcc not found; cannot build the gfx950 backend")
    OBJ.mkdir(parents=True, exist_ok=True)
    srcs = sorted(CSRC.glob("*.hip"))
    with cf.ThreadPoolExecutor(max_workers=max(1, min(jobs, len(srcs)))) as ex:
        objs = list(ex.map(_compile, srcs))
    tmp = LIB.with_suffix(".so.tmp")
    cmd = [HIPCC, f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", str(tmp),
           *map(str, objs)]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"link failed:\n{r.stdout}\n{r.stderr}")
    os.replace(tmp, LIB)
    return LIB


if __name__ == "__main__":
    print(build())
