"""Build libtalm.so (the gfx950 kernels behind include/talm.h) and libtalm_torch.so (the
torch.ops.talm.* custom ops over it) in-tree.

    python -m talm_amd.build          # compile every csrc/*.hip for gfx950, link, then the ops

Each HIP source compiles to its own object in parallel under talm_amd/_build/, then one link makes
talm_amd/libtalm.so; only the `extern "C"` entry points are exported (-fvisibility=hidden).
csrc/torch_ops.cpp is host code only: g++ against PyTorch's headers, linked to libtalm.so.
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
OPS_LIB = PKG / "libtalm_torch.so"
BENCH_LIB = PKG / "libtalm_bench.so"  # bench.py's streaming probes (csrc/bench/), not the product
INCLUDE = PKG.parent / "include"
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
    build_ops()
    build_bench()
    return LIB


def build_bench():
    """Compile csrc/bench/*.hip into libtalm_bench.so (bench.py's HBM streaming probes)."""
    sources = sorted((CSRC / "bench").glob("*.hip"))
    tmp = BENCH_LIB.with_suffix(".so.tmp")
    cmd = [hipcc(), *COMMON_FLAGS, *DEVICE_FLAGS, "-shared", *map(str, sources), "-o", str(tmp)]
    proc = subprocess.run(cmd, capture_output=True, text=True)
    if proc.returncode != 0:
        raise RuntimeError(f"build of libtalm_bench.so failed:\n{proc.stdout}{proc.stderr}")
    os.replace(tmp, BENCH_LIB)
    return BENCH_LIB


def build_ops():
    """Compile csrc/torch_ops.cpp into libtalm_torch.so (needs libtalm.so); returns its path."""
    import torch
    from torch.utils import cpp_extension

    torch_lib = Path(torch.__file__).resolve().parent / "lib"
    includes = [INCLUDE, *map(Path, cpp_extension.include_paths()), Path("/opt/rocm/include")]
    abi = int(torch._C._GLIBCXX_USE_CXX11_ABI)
    tmp = OPS_LIB.with_suffix(".so.tmp")
    cmd = [shutil.which("g++") or "g++", "-O2", "-std=c++17", "-fPIC", "-shared",
           "-fvisibility=hidden", f"-D_GLIBCXX_USE_CXX11_ABI={abi}", "-DUSE_ROCM",
           "-D__HIP_PLATFORM_AMD__=1", *[f"-I{p}" for p in includes],
           str(CSRC / "torch_ops.cpp"), "-o", str(tmp), f"-L{PKG}", "-ltalm", f"-L{torch_lib}",
           "-lc10", "-lc10_hip", "-ltorch_cpu", "-ltorch_hip", "-lhipblaslt", "-Wl,-rpath,$ORIGIN",
           f"-Wl,-rpath,{torch_lib}"]
    proc = subprocess.run(cmd, capture_output=True, text=True)
    if proc.returncode != 0:
        raise RuntimeError(f"build of libtalm_torch.so failed:\n{proc.stdout}{proc.stderr}")
    os.replace(tmp, OPS_LIB)
    return OPS_LIB


if __name__ == "__main__":
    print(build(verbose=True))
