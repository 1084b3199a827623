"""SwiGLU with its backward written in place (solution/swiglu_inplace.py:22-47).

The node keeps `gate` and `up` ([N, 8960] fp16 each) for its backward and, since nothing else
reads them after it, the backward kernel writes dgate over gate and dup over up (each thread
loads its elements before storing at the same offsets): two [N, 8960] buffers fewer at the start
of the backward pass. Same kernels and arithmetic as swiglu.py, the same values.
"""

import torch

from .engaged import FELL_BACK, ON, RAN
from .fused_mlp import fused_mlp_forward
from .state import DISABLED, fallback
from .swiglu import activate, reference_grads, swiglu, swiglu_bwd, swiglu_fwd


class SwiGLUInPlaceGrad(torch.autograd.Function):
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
                swiglu_bwd(grad, gate, up, gate, up)
                return gate, up
            except Exception as exc:  # noqa: BLE001 - state.py convention
                if not fallback("swiglu", exc):
                    raise
        return reference_grads(grad, gate, up)


def patch_qwen2_mlp_inplace():
    """Qwen2MLP.forward as one FusedMLP node on a packed layer group (fused_mlp.py), else through
    the in-place-backward node when gate and up are separate fresh tensors of the same dtype
    (solution/swiglu_inplace.py:50-77)."""
    install_mlp_forward()
    ON.add("swiglu_inplace")


def install_mlp_forward():
    """The one Qwen2MLP.forward wrapper of this package. Which node takes a call depends on
    what is installed (engaged.ON): the FusedMLP node (in save-up mode when mlp_save_up.py is
    installed and the call records autograd), else, with the in-place patch, the in-place
    SwiGLU node, else the forward found at install time."""
    from transformers.models.qwen2 import modeling_qwen2

    from .patches import _in_chain

    cls = modeling_qwen2.Qwen2MLP
    previous = cls.forward
    if _in_chain(previous, "_solution_inplace"):
        return

    def forward(self, x):
        act = getattr(getattr(self, "config", None), "hidden_act", "silu")
        if act != "silu" or not x.is_cuda or "swiglu" in DISABLED:
            FELL_BACK["swiglu_inplace"] += 1
            return previous(self, x)
        y = fused_mlp_forward(self, x)
        if y is not None:
            return y
        if "swiglu_inplace" not in ON:
            return previous(self, x)
        gate, up = self.gate_proj(x), self.up_proj(x)
        if gate.dtype != up.dtype or gate.data_ptr() == up.data_ptr():
            FELL_BACK["swiglu_inplace"] += 1
            return self.down_proj(activate(self, gate, up, swiglu))
        RAN["swiglu_inplace"] += 1
        return self.down_proj(activate(self, gate, up, SwiGLUInPlaceGrad.apply))

    forward._solution_inplace = True
    forward._previous = previous
    cls.forward = forward
