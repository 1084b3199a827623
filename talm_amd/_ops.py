"""`torch.ops.talm.*`: the PyTorch custom ops over the C-ABI of libtalm.so.

The ops are defined and implemented in C++ (csrc/torch_ops.cpp, built as libtalm_torch.so next
to libtalm.so): each validates device, dtype and layout, passes raw data pointers and the current
HIP stream of the tensors' device to one `extern "C"` entry point, and returns nothing (outputs
are the caller's tensors, annotated as mutated). They are registered for the CUDA (= HIP on ROCm)
dispatch key only: a CPU tensor raises NotImplementedError from the dispatcher, never a CPU
fallback. Importing this module loads both libraries or raises (no fallback).

The workspace sizes of head_ce, lora_wgrad, attn_bwd and gemm_splitk are plain functions over the
C-ABI's size queries.
"""

import threading
from pathlib import Path

import torch

from . import _lib

OPS_PATH = Path(__file__).resolve().parent / "libtalm_torch.so"
OPS = ("nf4_group_dequant", "nf4_group_dequant_streaming", "nf4_dequant", "rmsnorm", "rope",
       "swiglu_fwd", "swiglu_bwd", "swiglu_fwd_rows", "swiglu_bwd_rows",
       "head_weight_t", "head_ce", "lora_down", "qkv_lora_fwd", "qkv_lora_fwd_down", "qkv_bwd_prep", "qkv_lora_bwd_dx",
       "lora_wgrad", "gemm", "gemm_ex", "attn_fwd", "attn_bwd", "attn_bwd_rope", "lora_mirror",
       "lora_adamw", "nf4_gemm", "nf4_block_scales", "nf4_group_dequant_t", "gemm_splitk",
       "pack_rows", "row_stats", "head_loss", "scatter_rows", "scale_rows",
       "gemm_splitk_partials", "nf4_gemm_partials", "splitk_add_rmsnorm", "splitk_rmsnorm_bwd",
       "rope_table", "lora_grad_norm", "lora_adamw_clipped")

_load_lock = threading.Lock()
_loaded = False


def load():
    """Load libtalm.so (ABI-checked) and the op library that registers torch.ops.talm.*."""
    global _loaded
    if _loaded:
        return
    with _load_lock:
        if _loaded:
            return
        _lib.lib()
        if not OPS_PATH.exists():
            raise _lib.LibraryMissing(f"{OPS_PATH} is not built: run `python -m talm_amd.build`")
        try:
            torch.ops.load_library(str(OPS_PATH))
        except OSError as exc:
            raise _lib.LibraryMissing(f"{OPS_PATH} does not load: {exc}") from exc
        _loaded = True


load()


def _require(cond, message):
    if not cond:
        raise ValueError(message)


def head_ce_workspace_bytes(n_rows, hidden, vocab, vchunk, n_grad, group):
    size = _lib.lib().talm_head_ce_workspace(n_rows, hidden, vocab, vchunk, n_grad, group)
    if size < 0:
        raise ValueError(f"head_ce: unsupported shape rows={n_rows} hidden={hidden} "
                         f"vocab={vocab} vchunk={vchunk} n_grad={n_grad} group={group}")
    return int(size)


def lora_wgrad_workspace_bytes(n_tokens, hidden, seg0, seg1):
    size = _lib.lib().talm_lora_wgrad_workspace(n_tokens, hidden, seg0, seg1)
    _require(size >= 0, "lora_wgrad: unsupported shape")
    return int(size)


def attn_bwd_workspace_bytes(n_tokens, n_q_heads):
    size = _lib.lib().talm_attn_bwd_workspace(n_tokens, n_q_heads)
    _require(size >= 0, "attn_bwd: unsupported shape")
    return int(size)


def gemm_splitk_workspace_bytes(m, n, k):
    size = _lib.lib().talm_gemm_splitk_workspace(m, n, k)
    if size < 0:
        raise ValueError(f"gemm_splitk: unsupported shape m={m} n={n} k={k}")
    return size


def nf4_gemm_workspace_bytes(n_tokens, rows, cols, transpose):
    size = _lib.lib().talm_nf4_gemm_workspace(n_tokens, rows, cols, 1 if transpose else 0)
    if size < 0:
        raise ValueError(f"nf4_gemm: unsupported shape tokens={n_tokens} W=[{rows}, {cols}]")
    return size


def gemm_splitk_parts(m, n, k):
    """K parts of the split-K GEMM's plan for [m, k] x [n, k]^T (its partials: parts x m x n)."""
    parts = _lib.lib().talm_gemm_splitk_parts(m, n, k)
    if parts < 1:
        raise ValueError(f"gemm_splitk: unsupported shape m={m} n={n} k={k}")
    return int(parts)


def nf4_gemm_parts(n_tokens, rows, cols, transpose):
    """K parts of the W4A16 GEMM's plan (its partials: parts x n_tokens x out columns)."""
    parts = _lib.lib().talm_nf4_gemm_parts(n_tokens, rows, cols, 1 if transpose else 0)
    if parts < 1:
        raise ValueError(f"nf4_gemm: unsupported shape tokens={n_tokens} W=[{rows}, {cols}]")
    return int(parts)


def lora_grad_norm_workspace_bytes(n_tensors, max_numel):
    size = _lib.lib().talm_lora_grad_norm_workspace(n_tensors, max_numel)
    _require(size >= 0, "lora_grad_norm: unsupported table")
    return int(size)
