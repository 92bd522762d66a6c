"""Builds libkf_int4.so in-tree for gfx950 with hipcc.

    python -m kernelforge.build            # from kernel-forge_amd/
    python kernel-forge_amd/kernelforge/build.py

Each .hip translation unit is compiled to an object in parallel, then linked
into ``kernelforge/libkf_int4.so``, where ``kernelforge._lib`` loads it.
"""

from __future__ import annotations

import os
import re
import shutil
import subprocess
import sys
from concurrent.futures import ThreadPoolExecutor
from pathlib import Path

PKG_DIR = Path(__file__).resolve().parent
SRC_DIR = PKG_DIR.parent / "csrc"
REPO_ROOT = PKG_DIR.parent.parent
INCLUDE_DIR = REPO_ROOT / "include"
BUILD_DIR = PKG_DIR.parent / "_build"
LIB_NAME = "libkf_int4.so"
LIB_PATH = PKG_DIR / LIB_NAME
ARCH = "gfx950"

SOURCES = ("kf_abi.hip", "kf_gemv.hip", "kf_gemm.hip", "kf_skinny.hip", "kf_quant.hip", "kf_aux.hip")

# Packed fp32 VALU ops stay disabled: the kernels never need them and some of
# their forms are not trusted on the target machines.  The first 16 dwords of
# kernel arguments are preloaded into SGPRs (gfx950 kernarg preloading; the
# code object keeps a fallback prologue for firmware without it), which
# removes a scalar memory round trip from the start of every wavefront.
DEVICE_FLAGS = ["-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
                "-mllvm", "-amdgpu-kernarg-preload-count=16"]
COMMON_FLAGS = ["-O3", "-std=c++17", "-fPIC", f"--offload-arch={ARCH}", "-Wall", "-Wno-unused-result"]


def device_flags() -> list[str]:
    """DEVICE_FLAGS, plus -DKF_DMA_WAIT_ALL when KF_DMA_WAIT_ALL=1 is set: every counted wait for
    an LDS-DMA copy becomes a wait for all outstanding vector-memory operations (kf_device.h)."""
    extra = ["-DKF_DMA_WAIT_ALL"] if os.environ.get("KF_DMA_WAIT_ALL", "0") not in ("", "0") else []
    return DEVICE_FLAGS + extra


def hipcc() -> str:
    for cand in (os.environ.get("HIPCC"), "/opt/rocm/bin/hipcc", shutil.which("hipcc")):
        if cand and Path(cand).exists():
            return cand
    raise RuntimeError("hipcc not found: the MI355X library needs ROCm's hipcc to build")


def _run(cmd: list[str], quiet_remarks: bool = False) -> str:
    proc = subprocess.run(cmd, capture_output=True, text=True)
    # hipcc's host pass warns that it does not know the packed-fp32 feature; drop that noise.
    noise = "is not a recognized feature for this target"
    err = "\n".join(line for line in proc.stderr.splitlines() if noise not in line)
    if proc.returncode != 0:
        raise RuntimeError(f"command failed ({proc.returncode}): {' '.join(cmd)}\n{err}")
    shown = err
    if quiet_remarks:
        shown = "\n".join(line for line in err.splitlines()
                          if "kernel-resource-usage" not in line and not line.lstrip().startswith(("|", "^"))
                          and not line.lstrip()[:1].isdigit())
    if shown.strip():
        print(shown, file=sys.stderr)
    return err


# Kernels whose launch plan counts on an occupancy (kf_gemv.hip, gemv_plan: the grouped M = 1
# launches, mixed and shaped, fit one resident round of 8 wavefronts per SIMD).
MIN_OCCUPANCY = {
    "gemv_grouped_kernelILi1ELi3ELi1ELb1E": 8,
    "gemv_grouped_kernelILi1ELi4ELi1ELb1E": 8,
}


def _check_resources(remarks: str, src: str) -> None:
    """Every kernel must run from registers: no scratch (private segment) and no spills.  A
    kernel whose accumulators fall to scratch still gives right answers, 10-20x slower."""
    bad, name = [], None
    for line in remarks.splitlines():
        m = re.search(r"Function Name: (\S+)", line)
        if m:
            name = m.group(1)
            continue
        m = re.search(r"(ScratchSize \[bytes/lane\]|VGPRs Spill|SGPRs Spill): (\d+)", line)
        if m and int(m.group(2)) > 0:
            bad.append(f"{name}: {m.group(1)} = {m.group(2)}")
        m = re.search(r"Occupancy \[waves/SIMD\]: (\d+)", line)
        if m and name:
            for pattern, need in MIN_OCCUPANCY.items():
                if pattern in name and int(m.group(1)) < need:
                    bad.append(f"{name}: occupancy {m.group(1)} waves per SIMD, the launch plan assumes {need}")
    if bad:
        raise RuntimeError(f"{src}: kernels use scratch memory or spill registers:\n  " + "\n  ".join(bad))


def build_library(verbose: bool = False, resource_usage: bool = False) -> Path:
    """Compiles every kernel source and links libkf_int4.so; returns its path."""
    cc = hipcc()
    BUILD_DIR.mkdir(parents=True, exist_ok=True)
    extra = ["-Rpass-analysis=kernel-resource-usage"]

    def compile_one(src: str) -> Path:
        obj = BUILD_DIR / (Path(src).stem + ".o")
        cmd = [cc, *COMMON_FLAGS, *device_flags(), *extra, "-I", str(INCLUDE_DIR), "-I", str(SRC_DIR),
               "-c", str(SRC_DIR / src), "-o", str(obj)]
        if verbose:
            print(" ".join(cmd))
        remarks = _run(cmd, quiet_remarks=not resource_usage)
        _check_resources(remarks, src)
        return obj

    with ThreadPoolExecutor(max_workers=min(len(SOURCES), 4)) as pool:
        objs = list(pool.map(compile_one, SOURCES))
    tmp = LIB_PATH.with_suffix(".so.tmp")
    _run([cc, f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", str(tmp), *map(str, objs)])
    os.replace(tmp, LIB_PATH)
    return LIB_PATH


if __name__ == "__main__":
    path = build_library(verbose="-v" in sys.argv, resource_usage="--resource-usage" in sys.argv)
    print(f"built {path}")
