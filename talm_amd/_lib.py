"""Loader of libtalm.so (the C-ABI declared in include/talm.h) and its status convention.

There is no fallback here: if the library is missing or fails to load, `lib()` raises, so a
product path can never run without the HIP kernels. A nonzero status of an entry point raises
ValueError (TALM_EINVAL: arguments rejected before any launch) or RuntimeError (TALM_EHIP).
"""

import ctypes
import threading
from pathlib import Path

LIB_PATH = Path(__file__).resolve().parent / "libtalm.so"
ABI_VERSION = 20

TALM_OK, TALM_EINVAL, TALM_EHIP = 0, 1, 2
TALM_F32, TALM_F16 = 0, 1

_P = ctypes.c_void_p
_I64 = ctypes.c_int64
_I32 = ctypes.c_int32
_F32 = ctypes.c_float

# Every exported entry point with its argument types (all return int status).
SIGNATURES = {
    "talm_nf4_group_dequant": [_P, _P, _P, _P, _P, _P, _I64, _I32, _I32, _P],
    "talm_nf4_group_dequant_streaming": [_P, _P, _P, _P, _P, _P, _I64, _I32, _I32, _P],
    "talm_nf4_group_dequant_t": [_P, _P, _P, _P, _P, _P, _I32, _I32, _I32, _P, _I64, _P],
    "talm_nf4_dequant": [_P, _P, _P, _I64, _I32, _P],
    "talm_rmsnorm": [_P, _P, _P, _P, _P, _P, _P, _I64, _I64, _I32, _I32, _I32, _F32, _I32, _I32,
                     _P],
    "talm_rope": [_P, _P, _P, _P, _P, _P, _I64, _I32, _I32, _I32, _I64, _I64, _I64, _I64, _I64,
                  _I64, _I64, _I64, _I64, _I32, _P],
    "talm_swiglu_fwd": [_P, _P, _P, _I64, _P],
    "talm_swiglu_bwd": [_P, _P, _P, _P, _P, _I64, _P],
    "talm_swiglu_fwd_rows": [_P, _I64, _P, _I64, _P, _I64, _I64, _I64, _P],
    "talm_swiglu_bwd_rows": [_P, _I64, _P, _I64, _P, _I64, _P, _I64, _P, _I64, _I64, _I64, _P],
    "talm_head_weight_t": [_P, _I64, _I64, _I64, _P, _I64, _P],
    "talm_lora_down": [_P, _I64, _I64, _I64, _I64, _I64, _I64, _P, _P, _I32, _I32, _F32, _F32, _P,
                       _P, _I64, _P],
    "talm_lora_wgrad": [_P, _I64, _P, _I64, _P, _I64, _P, _I64, _I64, _I64, _I32, _I64, _I64, _F32,
                        _P, _P, _I64, _I64, _F32, _P, _P, _P, _I64, _P],
    "talm_lora_wgrad_noalloc": [_P, _I64, _P, _I64, _P, _I64, _P, _I64, _I64, _I64, _I32, _I64,
                                _I64, _F32, _P, _P, _I64, _I64, _F32, _P, _P, _P],
    "talm_qkv_bwd_prep": [_P, _I64, _P, _I64, _P, _I64, _I64, _I64, _I64, _I64, _P, _P, _I64, _P,
                          _I64, _P],
    "talm_qkv_lora_bwd_dx": [_P, _I64, _I64, _I64, _P, _I64, _I64, _P, _I64, _I64, _P, _I64, _P,
                             _I64, _P],
    "talm_qkv_lora_fwd": [_P, _I64, _I64, _I64, _P, _I64, _I64, _P, _P, _I64, _I32, _P, _I64, _I64,
                          _P, _I64, _I64, _P, _P, _I64, _I64, _P, _I64, _P],
    "talm_qkv_lora_fwd_down": [_P, _I64, _I64, _I64, _P, _I64, _I64, _P, _I32, _P, _P, _I64, _F32,
                               _F32, _P, _I64, _I64, _P, _I64, _I64, _P, _P, _I64, _I64, _P, _I64,
                               _P, _I64, _P],
    "talm_head_ce": [_P, _I64, _P, _I64, _P, _I64, _I64, _I64, _I64, _I64, _I32, _P, _P,
                     _P, _P, _P, _P, _I64, _P],
    "talm_attn_fwd": [_P, _I64, _I64, _P, _I64, _I64, _P, _I64, _I64, _P, _I32, _I32, _I64, _I32,
                      _I32, _I32, _F32, _P, _I64, _I64, _P, _P],
    "talm_attn_bwd": [_P, _I64, _I64, _P, _I64, _I64, _P, _I64, _I64, _P, _I64, _I64, _P, _I64,
                      _I64, _P, _P, _I32, _I32, _I64, _I32, _I32, _I32, _F32, _P, _I64, _I64, _P,
                      _I64, _I64, _P, _I64, _I64, _P, _I64, _P],
    "talm_attn_bwd_rope": [_P, _I64, _I64, _P, _I64, _I64, _P, _I64, _I64, _P, _I64, _I64, _P,
                           _I64, _I64, _P, _P, _I32, _I32, _I64, _I32, _I32, _I32, _F32, _P, _P,
                           _I64, _P, _I64, _I64, _P, _I64, _I64, _P, _I64, _I64, _P, _I64, _P],
    "talm_lora_mirror": [_P, _I32, _I64, _P, _P],
    "talm_rope_table": [_P, _I64, _P, _I32, _F32, _P, _P, _P],
    "talm_pack_rows": [_P, _P, _P, _I32, _I32, _I64, _P, _P, _P, _P, _P, _P],
    "talm_row_stats": [_P, _P, _I32, _I32, _P, _P],
    "talm_head_loss": [_P, _P, _P, _I64, _P, _F32, _I32, _P, _P, _P, _P],
    "talm_scatter_rows": [_P, _P, _P, _P, _P, _I64, _I64, _P, _P, _P, _P],
    "talm_scale_rows": [_P, _I64, _P, _P, _P, _P],
    "talm_lora_adamw": [_P, _I32, _I64, _F32, _F32, _F32, _F32, _F32, _P, _P, _P, _P, _P, _P],
    "talm_lora_grad_norm": [_P, _I32, _I64, _P, _F32, _P, _I64, _P, _P],
    "talm_lora_adamw_clipped": [_P, _I32, _I64, _F32, _F32, _F32, _F32, _F32, _P, _P, _P, _P, _P,
                                _P],
    "talm_nf4_gemm": [_P, _I64, _I64, _P, _P, _I64, _I64, _I32, _I32, _P, _I64, _P, _I64, _P],
    "talm_nf4_block_scales": [_P, _P, _P, _P, _I64, _I32, _P, _P],
    "talm_gemm_splitk": [_P, _I64, _P, _I64, _P, _I64, _I64, _I64, _I64, _P, _I64, _P],
    "talm_gemm_splitk_partials": [_P, _I64, _P, _I64, _I64, _I64, _I64, _P, _I64, _P],
    "talm_nf4_gemm_partials": [_P, _I64, _I64, _P, _P, _I64, _I64, _I32, _I32, _P, _I64, _P],
    "talm_splitk_add_rmsnorm": [_P, _I32, _P, _P, _I32, _F32, _I64, _I64, _P, _P, _P, _P, _P],
    "talm_splitk_rmsnorm_bwd": [_P, _I32, _P, _P, _P, _I32, _P, _I64, _I64, _P, _P, _P],
}

# Entry points that return a size instead of a status.
SIZE_FUNCTIONS = {
    "talm_head_ce_workspace": [_I64, _I64, _I64, _I64, _I64, _I32],
    "talm_lora_wgrad_workspace": [_I64, _I64, _I64, _I64],
    "talm_attn_bwd_workspace": [_I64, _I32],
    "talm_gemm_splitk_workspace": [_I64, _I64, _I64],
    "talm_nf4_gemm_workspace": [_I64, _I64, _I64, _I32],
    "talm_gemm_splitk_parts": [_I64, _I64, _I64],
    "talm_lora_grad_norm_workspace": [_I32, _I64],
    "talm_nf4_gemm_parts": [_I64, _I64, _I64, _I32],
}

_lock = threading.Lock()
_lib = None


class LibraryMissing(ImportError):
    """libtalm.so is not built (or does not load): the kernels cannot run."""


def lib():
    """The loaded libtalm.so with argument types set (loaded once per process)."""
    global _lib
    if _lib is not None:
        return _lib
    with _lock:
        if _lib is None:
            if not LIB_PATH.exists():
                raise LibraryMissing(f"{LIB_PATH} is not built: run `python -m talm_amd.build` "
                                     "(hipcc, gfx950)")
            try:
                handle = ctypes.CDLL(str(LIB_PATH))
            except OSError as exc:
                raise LibraryMissing(f"{LIB_PATH} does not load: {exc}") from exc
            handle.talm_last_error.restype = ctypes.c_char_p
            handle.talm_last_error.argtypes = []
            handle.talm_abi_version.restype = ctypes.c_int
            version = handle.talm_abi_version()
            if version != ABI_VERSION:
                raise LibraryMissing(f"{LIB_PATH} has ABI {version}, expected {ABI_VERSION}: "
                                     "rebuild it")
            for name, argtypes in SIGNATURES.items():
                fn = getattr(handle, name)
                fn.argtypes = argtypes
                fn.restype = ctypes.c_int
            for name, argtypes in SIZE_FUNCTIONS.items():
                fn = getattr(handle, name)
                fn.argtypes = argtypes
                fn.restype = ctypes.c_int64
            _lib = handle
    return _lib


def check(status, what):
    """Raise for a nonzero status of entry point `what`."""
    if status == TALM_OK:
        return
    message = lib().talm_last_error().decode(errors="replace") or f"{what}: status {status}"
    if status == TALM_EINVAL:
        raise ValueError(message)
    raise RuntimeError(message)


def dtype_code(dtype):
    import torch

    if dtype == torch.float32:
        return TALM_F32
    if dtype == torch.float16:
        return TALM_F16
    raise ValueError(f"libtalm: unsupported dtype {dtype}")
