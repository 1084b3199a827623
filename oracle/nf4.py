"""NF4 dequantization oracle (test infrastructure): the C restatement (oracle/nf4_oracle.c, built
by oracle/Makefile) and a numpy twin of the same arithmetic.

- `group_dequant`: solution/qgroup.py:72-91 — per block r of `qblock` weights,
  scale = fl32(fl32(code[absmax8[r]] * absmax2[r // qblock2]) + offset2[r // qblock2]),
  out = fp16_rne(fl32(level[nibble] * scale)), high nibble first.
- `dequant`: solution/nf4_dequant.py:38-80 (= solution/test_fuzz.py:860-868 `_nf4_manual`).
"""

import ctypes
import subprocess
from pathlib import Path

import numpy as np

from .codebook import NF4_LEVELS

_HERE = Path(__file__).resolve().parent
_LIB_PATH = _HERE / "_build" / "libnf4_oracle.so"
_lib = None


def build():
    """Compile the C oracle (gcc, oracle/Makefile)."""
    subprocess.run(["make", "-s", "-C", str(_HERE)], check=True)
    return _LIB_PATH


def _load():
    global _lib
    if _lib is None:
        if not _LIB_PATH.exists():
            build()
        lib = ctypes.CDLL(str(_LIB_PATH))
        p = ctypes.c_void_p
        lib.oracle_nf4_group_dequant.argtypes = [p, p, p, p, p, p, ctypes.c_int64, ctypes.c_int32,
                                                 ctypes.c_int32]
        lib.oracle_nf4_dequant.argtypes = [p, p, p, ctypes.c_int64, ctypes.c_int32]
        lib.oracle_f32_to_f16_array.argtypes = [p, p, ctypes.c_int64]
        lib.oracle_f32_to_f16.argtypes = [ctypes.c_float]
        lib.oracle_f32_to_f16.restype = ctypes.c_uint16
        _lib = lib
    return _lib


def _ptr(a):
    return a.ctypes.data_as(ctypes.c_void_p)


def f32_to_f16_bits(values):
    """The C oracle's binary32 -> binary16 (RNE) conversion, as uint16 bit patterns."""
    src = np.ascontiguousarray(values, dtype=np.float32)
    out = np.empty(src.shape, dtype=np.uint16)
    _load().oracle_f32_to_f16_array(_ptr(src), _ptr(out), src.size)
    return out


def group_dequant(packed, absmax8, code, absmax2, offset2, qblock=64, qblock2=256):
    """C oracle of the grouped kernel: fp16 bit patterns (uint16) of every weight."""
    packed = np.ascontiguousarray(packed, dtype=np.uint8)
    absmax8 = np.ascontiguousarray(absmax8, dtype=np.uint8)
    code = np.ascontiguousarray(code, dtype=np.float32)
    absmax2 = np.ascontiguousarray(absmax2, dtype=np.float32)
    offset2 = np.ascontiguousarray(offset2, dtype=np.float32)
    n_rows = absmax8.size
    assert packed.size == n_rows * qblock // 2
    assert absmax2.size >= -(-n_rows // qblock2) and offset2.size == absmax2.size
    out = np.empty(n_rows * qblock, dtype=np.uint16)
    _load().oracle_nf4_group_dequant(_ptr(packed), _ptr(absmax8), _ptr(code), _ptr(absmax2),
                                     _ptr(offset2), _ptr(out), n_rows, qblock, qblock2)
    return out


def block_scales_np(absmax8, code, absmax2, offset2, qblock2=256):
    """The decoded absmax of every block, fl32(fl32(code[absmax8] * absmax2) + offset2)
    (solution/qgroup.py:82-83): what `group_dequant` multiplies block r's levels by."""
    absmax8 = np.asarray(absmax8)
    block2 = np.arange(absmax8.size) // qblock2
    prod = np.asarray(code, np.float32)[absmax8] * np.asarray(absmax2, np.float32)[block2]
    return (prod + np.asarray(offset2, np.float32)[block2]).astype(np.float32)


def group_dequant_np(packed, absmax8, code, absmax2, offset2, qblock=64, qblock2=256):
    """numpy twin of `group_dequant` (float32 ops round one at a time; numpy's float16 cast is
    IEEE round-to-nearest-even)."""
    packed = np.asarray(packed, dtype=np.uint8)
    scale = block_scales_np(absmax8, code, absmax2, offset2, qblock2)
    scale = np.repeat(scale, qblock // 2)
    first = NF4_LEVELS[packed >> 4] * scale
    second = NF4_LEVELS[packed & 15] * scale
    vals = np.stack([first, second], axis=1).reshape(-1)
    return vals.astype(np.float16).view(np.uint16)


def dequant(packed, absmax, blocksize, n):
    """C oracle of the per-projection kernel: fp16 bit patterns of n weights."""
    packed = np.ascontiguousarray(packed, dtype=np.uint8).reshape(-1)
    absmax = np.ascontiguousarray(absmax, dtype=np.float32)
    assert n % 2 == 0 and packed.size >= n // 2
    out = np.empty(n, dtype=np.uint16)
    _load().oracle_nf4_dequant(_ptr(packed), _ptr(absmax), _ptr(out), n, blocksize)
    return out


def dequant_np(packed, absmax, blocksize, n):
    """numpy twin of `dequant` (the reference's `_nf4_manual`)."""
    codes = np.asarray(packed, dtype=np.uint8).reshape(-1)
    vals = np.stack([NF4_LEVELS[codes >> 4], NF4_LEVELS[codes & 15]], axis=1).reshape(-1)[:n]
    scale = np.repeat(np.asarray(absmax, np.float32), blocksize)[:n]
    return (vals * scale).astype(np.float16).view(np.uint16)


def dequant_state_torch(packed, state):
    """The reference's CPU eager dequantization of one 4-bit projection with PyTorch CPU ops (the
    `cpu_baseline` leg of bench.py times the unpatched step with it): bitsandbytes'
    dequantize_4bit as the reference's tests restate it (`_nf4_manual`, solution/test_fuzz.py:
    860-868) after the double-quant absmax is rebuilt (code[absmax8] * absmax2 + offset, each
    rounded in fp32: solution/qgroup.py:12-14). Returns fp16 [out, in], bit-identical to
    `group_dequant` on the same bytes (tests/test_oracle.py). Runs on the device of `packed` (the
    GPU tests' unpatched baselines use it there, so that their 4-bit layers do not run this
    build's kernels)."""
    import torch

    dev = packed.device
    codes = packed.reshape(-1).to(torch.int64)
    levels = torch.tensor(NF4_LEVELS, dtype=torch.float32, device=dev)
    inner = state.state2
    blk2 = torch.arange(state.absmax.numel(), device=dev) // inner.blocksize
    absmax = inner.code[state.absmax.to(torch.int64)] * inner.absmax[blk2] + state.offset
    vals = torch.stack((levels[codes >> 4], levels[codes & 15]), 1).reshape(-1)
    vals = vals * absmax.repeat_interleave(state.blocksize)[:vals.numel()]
    return vals.to(torch.float16).view(state.shape)
