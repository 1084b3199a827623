"""Qwen2 MLP that keeps `up` and the MLP input for its backward and recomputes `gate` there
(solution/mlp_save_up.py:51-140; opt-in, SOLUTION_MLP_SAVE_UP=1).

The node saves x ([N, 1536] fp16) and up instead of gate and up; the forward writes
silu(gate) * up over gate (the forward kernel with out = gate); the backward recomputes
gate = x W_gate^T with the weight the backward dequantizes anyway, writes dgate over gate and
dup over up (the in-place backward kernel), and returns dx = dgate W_gate + dup W_up.
"""

import torch
import torch.nn.functional as F

from .state import DISABLED, fallback
from .swiglu import swiglu_bwd, swiglu_fwd

GATE, UP = 4, 5


class SwiGLUSaveUp(torch.autograd.Function):
    """silu(x W_gate^T) * (x W_up^T) on a packed 4-bit layer group; saves x and up only."""

    @staticmethod
    def forward(ctx, x, group):
        weight = group.weight(GATE)
        gate = F.linear(x, weight, group.biases[GATE])
        del weight
        up = F.linear(x, group.weight(UP), group.biases[UP])
        swiglu_fwd(gate, up, gate)
        ctx.group = group
        ctx.save_for_backward(x, up)
        return gate

    @staticmethod
    def backward(ctx, grad):
        x, up = ctx.saved_tensors
        group = ctx.group
        weight = group.weight(GATE)
        gate = F.linear(x, weight, group.biases[GATE])
        grad = grad.to(gate.dtype).contiguous()
        swiglu_bwd(grad, gate, up, gate, up)
        del grad
        dx = torch.matmul(gate, weight)
        del gate, weight
        dx += torch.matmul(up, group.weight(UP))
        return dx, None


def save_up_group(mlp, x):
    """The layer group when `SwiGLUSaveUp` can take this MLP call, else None."""
    if not (x.is_cuda and x.dtype == torch.float16 and torch.is_grad_enabled()
            and x.requires_grad):
        return None
    if getattr(getattr(mlp, "config", None), "hidden_act", "silu") != "silu":
        return None
    gate, up = getattr(mlp, "gate_proj", None), getattr(mlp, "up_proj", None)
    tag_gate = getattr(gate, "_solution_group", None)
    tag_up = getattr(up, "_solution_group", None)
    if tag_gate is None or tag_up is None or tag_gate[0] is not tag_up[0] \
            or tag_gate[1] != GATE or tag_up[1] != UP:
        return None
    if any(m._forward_hooks or m._forward_pre_hooks for m in (gate, up)):
        return None
    return tag_gate[0]


def patch_qwen2_mlp_save_up():
    from transformers.models.qwen2 import modeling_qwen2

    from .engaged import FELL_BACK, ON, RAN
    from .patches import _in_chain

    cls = modeling_qwen2.Qwen2MLP
    previous = cls.forward
    ON.add("mlp_save_up")
    if _in_chain(previous, "_solution_save_up"):
        return

    def forward(self, x):
        group = None if "mlp_save_up" in DISABLED else save_up_group(self, x)
        if group is not None:
            try:
                act = SwiGLUSaveUp.apply(x, group)
            except Exception as exc:  # noqa: BLE001 - state.py convention
                if not fallback("mlp_save_up", exc):
                    raise
            else:
                RAN["mlp_save_up"] += 1
                return self.down_proj(act)
        FELL_BACK["mlp_save_up"] += 1
        return previous(self, x)

    forward._solution_save_up = True
    forward._previous = previous
    cls.forward = forward
