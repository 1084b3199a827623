"""The opt-in save-up MLP (SOLUTION_MLP_SAVE_UP=1): the decoder MLP keeps its input and `up` for
the backward and recomputes `gate` there, trading one gate product per layer for the activation
memory of gate (the reference's option, solution/mlp_save_up.py:51-140).

In this build it is a mode of the one-node MLP, `fused_mlp.FusedMLP(x, group, save_up=True)`:
the forward's two products go into separate buffers so that gate can be freed with the forward;
the backward recomputes gate on the layer's NF4 codes (talm_nf4_gemm, into the left half of the
buffer the input-gradient product reads), runs the SwiGLU backward from it and the kept up into
that buffer's halves, and then takes the same input-gradient product over both halves as the
default mode. Saved per token and layer: x (1536) + up (8960) fp16 values instead of gate|up
(17920).

Installing it marks the component on (engaged.ON) and makes sure the package's one MLP wrapper
is in place (swiglu_inplace.install_mlp_forward); `fused_mlp.fused_mlp_forward` then picks the
save-up mode for every call that records autograd on a packed layer group. Calls it does not
take (no autograd recording: nothing would be saved; a layer that is not one packed group; the
component switched off, state.py) go on as without it.
"""

import torch

from .engaged import ON
from .fused_mlp import mlp_plan


def save_up_group(mlp, x):
    """The layer group when the save-up mode can take this MLP call (a recorded call on a packed
    group), else None."""
    if "mlp_save_up" not in ON or not (torch.is_grad_enabled() and x.requires_grad):
        return None
    return mlp_plan(mlp, x, component="mlp_save_up")


def patch_qwen2_mlp_save_up():
    """Switch the MLP node's save-up mode on (the reference's installer name)."""
    from .swiglu_inplace import install_mlp_forward

    install_mlp_forward()
    ON.add("mlp_save_up")
