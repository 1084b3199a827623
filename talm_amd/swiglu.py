"""Fused SwiGLU, silu(gate) * up, for the Qwen2 MLP on the HIP kernels (talm_swiglu_fwd/bwd).

Mirrors solution/swiglu.py: forward gate * sigmoid(gate) * up in fp32 (:23-30); backward
sig = sigmoid(gate), dup = g * gate * sig, dgate = g * up * sig * (1 + gate * (1 - sig))
(:33-45, `reference_grads` :48-54). The launch sites keep the reference kernels' argument order:
`swiglu_fwd(gate, up, out)` and `swiglu_bwd(grad, gate, up, dgate, dup)`, where `out` may be
`gate` and dgate / dup may be gate / up (the in-place backward, swiglu_inplace.py, and the
save-up MLP, mlp_save_up.py).

Graceful degradation (state.py): an error in a launch turns "swiglu" off; the forward then
computes transformers' `act_fn(gate) * up` and the backward the same formula in PyTorch ops.
"""

import torch
import torch.nn.functional as F

from . import _ops  # noqa: F401 - registers torch.ops.talm.*
from .engaged import FELL_BACK
from .state import DISABLED, fallback


def swiglu_fwd(gate, up, out):
    torch.ops.talm.swiglu_fwd(gate, up, out)
    return out


def swiglu_bwd(grad, gate, up, dgate, dup):
    torch.ops.talm.swiglu_bwd(grad, gate, up, dgate, dup)
    return dgate, dup


def reference_grads(grad, gate, up):
    """The backward kernel's formulas in PyTorch ops (fp32), for a launch that failed."""
    FELL_BACK["swiglu"] += 1
    g, a, b = grad.float(), gate.float(), up.float()
    sig = torch.sigmoid(a)
    dgate = g * b * sig * (1.0 + a * (1.0 - sig))
    return dgate.to(gate.dtype), (g * a * sig).to(up.dtype)


class SwiGLU(torch.autograd.Function):
    """silu(gate) * up in one launch each way."""

    @staticmethod
    def forward(ctx, gate, up):
        gate = gate.contiguous()
        up = up.to(gate.dtype).contiguous()
        out = torch.empty_like(gate)
        swiglu_fwd(gate, up, out)
        ctx.save_for_backward(gate, up)
        return out

    @staticmethod
    def backward(ctx, grad):
        gate, up = ctx.saved_tensors
        grad = grad.to(gate.dtype).contiguous()
        if "swiglu" not in DISABLED:
            try:
                dgate, dup = torch.empty_like(gate), torch.empty_like(up)
                swiglu_bwd(grad, gate, up, dgate, dup)
                return dgate, dup
            except Exception as exc:  # noqa: BLE001 - state.py convention
                if not fallback("swiglu", exc):
                    raise
        return reference_grads(grad, gate, up)


def swiglu(gate, up):
    return SwiGLU.apply(gate, up)


def activate(mlp, gate, up, fused):
    """`fused(gate, up)`; on an unexpected error the MLP's own `act_fn(gate) * up`."""
    try:
        return fused(gate, up)
    except Exception as exc:  # noqa: BLE001 - state.py convention
        if not fallback("swiglu", exc):
            raise
    FELL_BACK["swiglu"] += 1
    return getattr(mlp, "act_fn", F.silu)(gate) * up


def patch_qwen2_mlp():
    """Qwen2MLP.forward through the fused kernels (solution/swiglu.py:103-116)."""
    from transformers.models.qwen2 import modeling_qwen2

    original = modeling_qwen2.Qwen2MLP.forward
    if getattr(original, "_solution_swiglu", False):
        return

    def forward(self, x):
        act = getattr(getattr(self, "config", None), "hidden_act", "silu")
        if act != "silu" or not x.is_cuda or "swiglu" in DISABLED:
            return original(self, x)
        return self.down_proj(activate(self, self.gate_proj(x), self.up_proj(x), swiglu))

    forward._solution_swiglu = True
    forward._original = original
    modeling_qwen2.Qwen2MLP.forward = forward
