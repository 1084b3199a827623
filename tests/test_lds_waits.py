"""The attention kernels read LDS through inline assembly the compiler does not track
(talm_amd/csrc/attn.hip: read_tr_untracked, read_f4_untracked) and wait for the results
themselves (lgkm_wait8, lgkm_wait_f4). Nothing may touch those destination registers before the
wait, not even a copy the register allocator might insert between the asm blocks. This checks
the gfx950 assembly of every kernel with such reads (and of the other LDS-heavy kernels, whose
reads the compiler tracks) with tests/lds_waits.py, after first checking that the scan catches
a planted early use."""

import shutil
import subprocess
import tempfile
from pathlib import Path

import pytest

from lds_waits import kernel_bodies, violations
from talm_amd import build

CSRC = Path(__file__).resolve().parents[1] / "talm_amd" / "csrc"


def test_scan_catches_an_early_use():
    early = "ds_read_b64_tr_b16 v[4:5], v1\nv_mov_b32 v10, v5\ns_waitcnt lgkmcnt(0)\n"
    assert len(violations(early)) == 1
    waited = "ds_read_b64_tr_b16 v[4:5], v1\ns_waitcnt lgkmcnt(0)\nv_mov_b32 v10, v5\n"
    assert violations(waited) == []
    # LDS returns in order: lgkmcnt(1) completes the first of two reads, not the second
    two = ("ds_read_b128 v[8:11], v1\nds_read_b128 v[12:15], v2\ns_waitcnt lgkmcnt(1)\n"
           "v_mov_b32 v20, v8\nv_mov_b32 v21, v12\n")
    assert [ins for _, ins, _ in violations(two)] == ["v_mov_b32 v21, v12"]
    # a scalar load may return before an earlier LDS read: lgkmcnt(1) after both completes
    # neither for sure
    smem = ("ds_read_b64 v[2:3], v0\ns_load_dword s4, s[0:1], 0x0\ns_waitcnt lgkmcnt(1)\n"
            "v_add_u32 v6, v2, v3\n")
    assert len(violations(smem)) == 1
    # an overwrite of the destination before the wait is a hazard too
    over = "ds_read_b32 v7, v0\nv_mov_b32 v7, 0\ns_waitcnt lgkmcnt(0)\n"
    assert len(violations(over)) == 1


@pytest.mark.parametrize("source,pattern,untracked", [
    ("attn.hip", r"attn_(fwd|bwd)_kernel", True),
    ("w4gemm.hip", r"w4_gemm_kernel", False),
    ("head_ce.hip", r"head_(logits|grad)_kernel", False),
])
def test_no_lds_result_is_used_before_its_wait(source, pattern, untracked):
    hipcc = shutil.which("hipcc") or "/opt/rocm/bin/hipcc"
    if not Path(hipcc).exists():
        pytest.skip("hipcc not available")
    with tempfile.TemporaryDirectory() as tmp:
        asm = Path(tmp) / "k.s"
        subprocess.run([hipcc, f"--offload-arch={build.ARCH}", "-O3", "-std=c++17",
                        *build.DEVICE_FLAGS, "--cuda-device-only", "-S", str(CSRC / source),
                        "-o", str(asm)], check=True, capture_output=True)
        bodies = kernel_bodies(asm.read_text(), pattern)
    assert bodies, f"no kernel matching {pattern} in {source}"
    for name, body in bodies.items():
        if untracked:
            assert "ds_read_b64_tr_b16" in body, name
        bad = violations(body)
        assert not bad, f"{name}: {bad[:3]}"
