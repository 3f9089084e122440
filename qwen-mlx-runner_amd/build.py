"""Builds libqmr_hip.so (HIP kernels + C ABI) for gfx950 with hipcc, in-tree.

Usage: python qwen-mlx-runner_amd/build.py [-j N]
Objects go to qwen-mlx-runner_amd/_build/, the library next to this file.
"""
from __future__ import annotations

import argparse
import os
import shutil
import subprocess
import sys
from concurrent.futures import ThreadPoolExecutor
from pathlib import Path

PKG = Path(__file__).resolve().parent
CSRC = PKG / "csrc"
BUILD = PKG / "_build"
LIB = PKG / "libqmr_hip.so"
ARCH = os.environ.get("QMR_OFFLOAD_ARCH", "gfx950")

# Packed FP32 instructions are disabled for all device code; hipcc's host
# pass warns that it does not know the feature, which is harmless.
DEVICE_FLAGS = ["-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops"]
COMMON = ["-O3", "-fPIC", "-std=c++17", "-Wall", f"--offload-arch={ARCH}"]

# The band kernel's source compiles once per weight format (bits x scale
# type), each object holding that format's instances, plus once without the
# format macros for its planner; these are the longest compiles, so they are
# queued first.
BAND_FORMATS = [(bits, meta) for bits in (4, 8) for meta in (0, 1, 2)]

SOURCES = [
    *[("affine_tile.hip", ["-x", "hip", f"-DQMR_BAND_BITS={bits}", f"-DQMR_BAND_META={meta}"],
       f"affine_tile_q{bits}_m{meta}.o") for bits, meta in BAND_FORMATS],
    ("contract.cpp", ["-x", "c++"]),
    ("checkpoint.cpp", ["-x", "c++"]),
    ("runtime.cpp", ["-x", "hip"]),
    ("affine_gemv.hip", ["-x", "hip"]),
    ("affine_mfma.hip", ["-x", "hip"]),
    ("affine_rows.hip", ["-x", "hip"]),
    ("affine_tile.hip", ["-x", "hip"]),
    ("dense_mfma.hip", ["-x", "hip"]),
    ("misc_kernels.hip", ["-x", "hip"]),
    # MFMA accumulators in VGPRs: the wide kernel's FP32 epilogue adds into
    # the same registers its bias MFMAs accumulate into.
    ("wide_mfma.hip", ["-x", "hip", "-mllvm", "-amdgpu-mfma-vgpr-form"]),
]


def hipcc() -> str:
    for cand in (os.environ.get("HIPCC"), "/opt/rocm/bin/hipcc", shutil.which("hipcc")):
        if cand and Path(cand).exists():
            return cand
    raise RuntimeError("hipcc not found (expected /opt/rocm/bin/hipcc)")


def _compile(src: str, lang: list[str], obj_name: str | None = None) -> Path:
    obj = BUILD / (obj_name or src + ".o")
    cmd = [hipcc(), *COMMON, *lang, "-c", str(CSRC / src), "-o", str(obj)]
    if lang[:2] == ["-x", "hip"]:
        cmd[1:1] = DEVICE_FLAGS
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"compile failed: {' '.join(cmd)}\n{res.stdout}\n{res.stderr}")
    return obj


def build(jobs: int | None = None) -> Path:
    BUILD.mkdir(exist_ok=True)
    jobs = jobs or min(len(SOURCES), os.cpu_count() or 4)
    with ThreadPoolExecutor(max_workers=jobs) as ex:
        objs = list(ex.map(lambda s: _compile(*s), SOURCES))
    tmp = LIB.with_suffix(".so.tmp")
    cmd = [hipcc(), f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", str(tmp), *map(str, objs)]
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"link failed: {' '.join(cmd)}\n{res.stdout}\n{res.stderr}")
    os.replace(tmp, LIB)
    return LIB


def build_oracle() -> Path:
    oracle = PKG.parent / "oracle"
    res = subprocess.run(["make", "-C", str(oracle), "-B", "liboracle.so"], capture_output=True,
                         text=True)
    if res.returncode != 0:
        raise RuntimeError(f"oracle build failed\n{res.stdout}\n{res.stderr}")
    return oracle / "liboracle.so"


if __name__ == "__main__":
    ap = argparse.ArgumentParser()
    ap.add_argument("-j", type=int, default=None)
    args = ap.parse_args()
    print(build(args.j))
    print(build_oracle())
    sys.exit(0)
