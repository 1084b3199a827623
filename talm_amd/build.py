"""Build libtalm.so (the gfx950 kernels behind include/talm.h) in-tree with hipcc.

    python -m talm_amd.build          # compile every csrc/*.hip for gfx950 and link

Each source compiles to its own object in parallel under talm_amd/_build/, then one link makes
talm_amd/libtalm.so. Only the `extern "C"` entry points are exported (-fvisibility=hidden).
"""

import concurrent.futures
import os
import shutil
import subprocess
import sys
from pathlib import Path

PKG = Path(__file__).resolve().parent
CSRC = PKG / "csrc"
BUILD = PKG / "_build"
LIB = PKG / "libtalm.so"
ARCH = "gfx950"

# Packed fp32 VALU ops are switched off for every kernel (the compiler must not form
# v_pk_{add,mul,fma}_f32); hipcc's host pass warns that it does not know the feature.
DEVICE_FLAGS = ["-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops"]
COMMON_FLAGS = [f"--offload-arch={ARCH}", "-O3", "-std=c++17", "-fPIC", "-fvisibility=hidden",
                "-Wall", "-Wno-unused-function"]


def hipcc():
    path = shutil.which("hipcc") or "/opt/rocm/bin/hipcc"
    if not Path(path).exists():
        raise RuntimeError("hipcc not found: the ROCm toolchain is needed to build libtalm.so")
    return path


def _compile(src, obj):
    cmd = [hipcc(), *COMMON_FLAGS, *DEVICE_FLAGS, "-c", str(src), "-o", str(obj)]
    proc = subprocess.run(cmd, capture_output=True, text=True)
    errors = "\n".join(line for line in (proc.stdout + proc.stderr).splitlines()
                       if "packed-fp32-ops" not in line)
    if proc.returncode != 0:
        raise RuntimeError(f"hipcc failed on {src.name}:\n{errors}")
    return errors.strip()


def build(verbose=False):
    """Compile every csrc/*.hip and link talm_amd/libtalm.so; returns the library path."""
    BUILD.mkdir(exist_ok=True)
    sources = sorted(CSRC.glob("*.hip"))
    if not sources:
        raise RuntimeError(f"no HIP sources under {CSRC}")
    objects = [BUILD / (src.stem + ".o") for src in sources]
    workers = min(len(sources), max(1, min(8, os.cpu_count() or 1)))
    with concurrent.futures.ThreadPoolExecutor(workers) as pool:
        for src, warnings in zip(sources, pool.map(_compile, sources, objects)):
            if warnings and verbose:
                print(f"[talm build] {src.name}:\n{warnings}", file=sys.stderr)
    tmp = LIB.with_suffix(".so.tmp")
    cmd = [hipcc(), f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", str(tmp),
           *map(str, objects)]
    proc = subprocess.run(cmd, capture_output=True, text=True)
    if proc.returncode != 0:
        raise RuntimeError(f"link of libtalm.so failed:\n{proc.stdout}{proc.stderr}")
    os.replace(tmp, LIB)
    return LIB


if __name__ == "__main__":
    print(build(verbose=True))
