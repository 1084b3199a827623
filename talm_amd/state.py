"""Graceful degradation, as the reference's solution/state.py:1-123 defines it.

An unexpected error in one fast path turns that component off for the rest of the process
(`DISABLED`), prints one line the first time:
    [solution] fallback: <component>: <exception type>: <message>
and the call that failed runs again through the original code. Out-of-memory errors and
PyTorch's own control flow (the early stop of a checkpoint's recomputation) always propagate
(solution/state.py:83-112).

Two additions, so native code can never be silently replaced:
- `LibraryMissing` (libtalm.so not built or not loadable) always propagates: without the HIP
  kernels the product refuses to run instead of degrading.
- With TALM_STRICT=1 (the test suite sets it) nothing is absorbed: every error propagates, so a
  test can only pass on the kernels themselves.
"""

import contextlib
import os

import torch

from ._lib import LibraryMissing

DISABLED = {}

STRICT = os.environ.get("TALM_STRICT") == "1"

COMPONENTS = {
    "fused_head": "fused causal-LM forward (patches.py, fused_head.py) -> transformers' forward",
    "unpad": "padding removal (unpad.py, patches.py) -> the fused head on the padded batch",
    "rmsnorm": "RMSNorm kernel -> transformers' Qwen2RMSNorm.forward",
    "addnorm": "residual add folded into the norm -> the plain add, then the norm",
    "rope": "RoPE kernel -> transformers' apply_rotary_pos_emb",
    "swiglu": "SwiGLU kernels and the in-place backward -> act_fn(gate) * up",
    "qgroup": "grouped NF4 dequantization -> the 4-bit linear's own forward",
    "lora": "the LoRA projection node -> the LoRA linear's own forward",
    "fused_proj": "q|k|v as one GEMM node -> transformers' attention forward",
    "qkv_mfma": "q|k|v + LoRA + RoPE forward on MFMA -> the node's hipBLASLt GEMMs",
    "nf4_dequant": "per-projection NF4 dequantization kernel",
    "mlp_save_up": "opt-in MLP keeping only up and its input -> the MLP forward before it",
    "fused_mlp": "the MLP as one node on the layer group -> the per-projection MLP",
    "attn_block": "q|k|v, attention and o_proj as one node -> the per-node attention",
    "gemm_table": "measured hipBLASLt solutions (gemm_tuning.py) -> hipBLASLt's heuristic",
}


def _text(exc):
    try:
        return str(exc)
    except Exception:  # noqa: BLE001 - a broken __str__ must not hide the original error
        return "<message unavailable>"


def _one_line(exc, limit=500):
    text = " ".join(_text(exc).split())
    return text if len(text) <= limit else text[:limit - 3] + "..."


def is_out_of_memory(exc):
    if isinstance(exc, torch.cuda.OutOfMemoryError):
        return True
    text = _text(exc).lower()
    return "out of memory" in text or "out_of_memory" in text


def is_control_flow(exc):
    """torch.utils.checkpoint's `_StopRecomputationError` passing through a fast path."""
    return type(exc).__name__ == "_StopRecomputationError"


def fallback(component, exc):
    """For `except Exception as exc:` around a fast path. Returns False when `exc` must
    propagate (out of memory, control flow, a missing kernel library, strict mode); otherwise
    turns `component` off, prints one `[solution] fallback:` line the first time, and returns
    True: the caller then runs the original code path."""
    if (STRICT or not isinstance(exc, Exception) or isinstance(exc, LibraryMissing)
            or is_out_of_memory(exc) or is_control_flow(exc)):
        return False
    if component not in DISABLED:
        reason = f"{type(exc).__name__}: {_one_line(exc)}"
        DISABLED[component] = reason
        try:
            print(f"[solution] fallback: {component}: {reason}", flush=True)
        except Exception:  # noqa: BLE001 - printing must never fail a training step
            pass
    return True


@contextlib.contextmanager
def installing(component):
    """Around one patch installation in apply(): an unexpected error leaves that component off
    (one fallback line) instead of failing the run."""
    try:
        yield
    except Exception as exc:  # noqa: BLE001 - the convention is to absorb and report
        if not fallback(component, exc):
            raise
