"""The C-ABI library: it loads, it exports every entry point include/talm.h declares with the
arity the Python binding uses, and argument rejection returns TALM_EINVAL with a message before
anything touches a GPU (no compute call runs here)."""

import ctypes
import re
from pathlib import Path

import pytest

from talm_amd import _lib

HEADER = Path(__file__).resolve().parents[1] / "include" / "talm.h"


def declared():
    """{name: number of parameters} of every function declared in include/talm.h."""
    text = re.sub(r"/\*.*?\*/", "", HEADER.read_text(), flags=re.S)
    out = {}
    for m in re.finditer(r"\b(talm_\w+)\s*\(([^)]*)\)\s*;", text):
        params = m.group(2).strip()
        out[m.group(1)] = 0 if params in ("", "void") else len(params.split(","))
    return out


def test_library_builds_loads_and_reports_abi():
    lib = _lib.lib()
    assert lib.talm_abi_version() == _lib.ABI_VERSION


def test_every_declared_symbol_is_exported_with_the_bound_arity():
    lib = _lib.lib()
    decl = declared()
    assert {"talm_last_error", "talm_abi_version", "talm_nf4_group_dequant"} <= set(decl)
    for name, arity in decl.items():
        assert hasattr(lib, name), f"{name} declared in talm.h but not exported"
        bound = {**_lib.SIGNATURES, **_lib.SIZE_FUNCTIONS}
        if name in bound:
            assert len(bound[name]) == arity, name
    assert set(_lib.SIGNATURES) | set(_lib.SIZE_FUNCTIONS) <= set(decl)


def test_argument_rejection_needs_no_gpu():
    lib = _lib.lib()
    status = lib.talm_nf4_group_dequant(None, None, None, None, None, None, 4, 3, 256, None)
    assert status == _lib.TALM_EINVAL
    assert b"qblock" in lib.talm_last_error()
    status = lib.talm_rmsnorm(None, None, None, None, None, None, None, 1, 8, 7, 1, 0,
                              ctypes.c_float(1e-6), 0, 0, None)
    assert status == _lib.TALM_EINVAL and b"dtype" in lib.talm_last_error()
    with pytest.raises(ValueError, match="even"):
        _lib.check(lib.talm_nf4_dequant(None, None, None, 3, 64, None), "nf4_dequant")
    assert lib.talm_swiglu_fwd(None, None, None, 0, None) == _lib.TALM_OK  # empty: no launch
    assert lib.talm_last_error() == b""
    # the transposed head weight: ldwt below the vocabulary, then a stride that is not 16-byte
    assert lib.talm_head_weight_t(None, 64, 100, 64, None, 96, None) == _lib.TALM_EINVAL
    assert b"ldwt" in lib.talm_last_error()
    assert lib.talm_head_weight_t(None, 64, 100, 64, None, 100, None) == _lib.TALM_EINVAL
    # the head rejects a workspace that is not 256-byte aligned before any launch
    ws, out = 1 << 4, 1 << 12  # fake addresses: never dereferenced on rejection
    status = lib.talm_head_ce(out, 64, out, 64, out, 4, 64, 1000, 256, 2, 1, out, out,
                              out, out, out, ws, 1 << 30, None)
    assert status == _lib.TALM_EINVAL and b"256-byte" in lib.talm_last_error()


def test_custom_ops_are_registered_for_the_gpu_only():
    import torch

    from talm_amd import _ops

    assert _ops.OPS_PATH.exists()
    for name in _ops.OPS:
        assert hasattr(torch.ops.talm, name)
        # the schema is the one the C++ layer defines, with the outputs marked as mutated
        assert "!" in str(getattr(torch.ops.talm, name).default._schema), name
    x = torch.zeros(8, dtype=torch.float16)
    with pytest.raises(NotImplementedError):
        torch.ops.talm.swiglu_fwd(x, x, x)  # CPU tensors: no kernel, no fallback


def test_nf4_kernels_have_no_fused_multiply_add():
    """The grouped NF4 kernel must round code * absmax2 before adding the offset (the reference
    compiles without FMA, solution/qgroup.py:99): the gfx950 assembly of the NF4 kernels holds no
    fused multiply-add instruction."""
    import shutil
    import subprocess
    import tempfile

    hipcc = shutil.which("hipcc") or "/opt/rocm/bin/hipcc"
    if not Path(hipcc).exists():
        pytest.skip("hipcc not available")
    src = Path(__file__).resolve().parents[1] / "talm_amd" / "csrc" / "nf4.hip"
    with tempfile.TemporaryDirectory() as tmp:
        asm = Path(tmp) / "nf4.s"
        subprocess.run([hipcc, "--offload-arch=gfx950", "-O3", "-std=c++17", "--cuda-device-only",
                        "-S", str(src), "-o", str(asm)], check=True, capture_output=True)
        text = asm.read_text()
    bodies = re.findall(r"^(_Z\w*nf4_\w+_kernel\w*):[^\n]*\n(.*?)^\.Lfunc_end", text,
                        flags=re.S | re.M)
    # group (chunks x 4: two second-level layouts x two store kinds; words; transposed x 2),
    # per-projection (words, bytes), block scales
    assert len(bodies) == 10
    for name, body in bodies:
        if "block_scales" not in name:
            assert "v_cvt_pk_f16_f32" in body or "v_cvt_f16_f32" in body, name
        assert not re.search(r"\bv_(pk_)?fma", body), f"{name} contains a fused multiply-add"
