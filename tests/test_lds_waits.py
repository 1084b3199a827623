"""The attention kernels read LDS through inline assembly the compiler does not track
(talm_amd/csrc/attn.hip: read_tr_untracked, read_f4_untracked) and wait for the results
themselves (lgkm_wait8, lgkm_wait_f4). Nothing may touch those destination registers before the
wait, not even a copy the register allocator might insert between the asm blocks. This checks
the gfx950 assembly of every kernel with such reads (and of the other LDS-heavy kernels, whose
reads the compiler tracks) with tests/lds_waits.py, after first checking that the scan catches
a planted early use.

A second scan checks the rings of the direct-to-LDS kernels: the next tile's loads stay in
flight while the current tile is read (no vmcnt wait between issuing them and the LDS reads)."""

import shutil
import subprocess
import tempfile
from pathlib import Path

import pytest

from lds_waits import drained_prefetches, kernel_bodies, violations
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


def test_scan_catches_a_drained_prefetch():
    # the ring's shape: wait for the current tile, barrier, issue the next tile, read the current
    ring = ("s_waitcnt vmcnt(0)\ns_barrier\nbuffer_load_dwordx4 v1, s[0:3], 0 offen lds\n"
            "buffer_load_dwordx4 v2, s[0:3], 0 offen lds\nds_read_b128 v[4:7], v3\n")
    assert drained_prefetches(ring) == []
    # a wait that keeps both prefetches in flight (an older register load completes) is fine
    partial = ring.replace("ds_read_b128", "s_waitcnt vmcnt(2)\nds_read_b128")
    assert drained_prefetches(partial) == []
    # vmcnt(1) completes the first prefetch, vmcnt(0) both
    for n in (1, 0):
        drained = ring.replace("ds_read_b128", f"s_waitcnt vmcnt({n})\nds_read_b128")
        assert len(drained_prefetches(drained)) == 1
    # a later load counts: vmcnt(2) after a third operation completes the first prefetch
    late = ring.replace("ds_read_b128", "global_load_dword v8, v[0:1], off\n"
                        "s_waitcnt vmcnt(2)\nds_read_b128")
    assert len(drained_prefetches(late)) == 1
    # a barrier closes the window (the epilogue's __syncthreads)
    closed = ring.replace("ds_read_b128", "s_waitcnt vmcnt(0)\ns_barrier\nds_read_b128")
    assert drained_prefetches(closed) == []


def _device_asm(source):
    hipcc = shutil.which("hipcc") or "/opt/rocm/bin/hipcc"
    if not Path(hipcc).exists():
        pytest.skip("hipcc not available")
    with tempfile.TemporaryDirectory() as tmp:
        asm = Path(tmp) / "k.s"
        subprocess.run([hipcc, f"--offload-arch={build.ARCH}", "-O3", "-std=c++17",
                        *build.DEVICE_FLAGS, "--cuda-device-only", "-S", str(CSRC / source),
                        "-o", str(asm)], check=True, capture_output=True)
        return asm.read_text()


@pytest.mark.parametrize("source,pattern", [
    ("attn.hip", r"attn_(fwd|bwd)_kernel"),
    ("head_ce.hip", r"head_(logits|grad)_kernel"),
    ("qkv.hip", r"proj_ext_kernel"),
    ("w4gemm.hip", r"w4_gemm_kernel"),
    ("gemm.hip", r"gemm_splitk_kernel"),
])
def test_no_ring_waits_for_its_prefetch(source, pattern):
    """Every kernel that streams tiles into an LDS ring with direct-to-LDS loads reads the
    current tile while the next one's loads are in flight: no vmcnt wait between issuing them and
    the reads (the compiler inserts one when it cannot tell the slots apart, or when a register
    load issued after the prefetch is waited for)."""
    bodies = kernel_bodies(_device_asm(source), pattern)
    assert bodies, f"no kernel matching {pattern} in {source}"
    for name, body in bodies.items():
        assert " lds" in body, name
        bad = drained_prefetches(body)
        assert not bad, f"{name}: {bad[:3]}"


@pytest.mark.parametrize("source,pattern,untracked", [
    ("attn.hip", r"attn_(fwd|bwd)_kernel", True),
    ("w4gemm.hip", r"w4_gemm_kernel", False),
    ("head_ce.hip", r"head_(logits|grad)_kernel", False),
])
def test_no_lds_result_is_used_before_its_wait(source, pattern, untracked):
    bodies = kernel_bodies(_device_asm(source), pattern)
    assert bodies, f"no kernel matching {pattern} in {source}"
    for name, body in bodies.items():
        if untracked:
            assert "ds_read_b64_tr_b16" in body, name
        bad = violations(body)
        assert not bad, f"{name}: {bad[:3]}"
