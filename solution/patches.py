"""`apply()` and the patch installers under the reference's module name (solution/patches.py,
solution/__init__.py:229): each name below is the `talm_amd` function that installs the MI355X
kernel behind the same transformers class the reference patches.

    apply()                     every patch, idempotent; raises when libtalm.so is missing
    unapply()                   restores every original method (A/B runs in one process)
    patch_qwen2_causal_lm()     fused LM head + cross-entropy with padding removal
    patch_qwen2_rmsnorm()       RMSNorm kernel
    patch_qwen2_add_norm()      residual adds folded into the norms
    patch_qwen2_rope()          in-place RoPE kernel
    patch_qwen2_mlp_inplace()   SwiGLU with the in-place backward (and the fused MLP node)
    patch_qwen2_mlp_save_up()   the save-up MLP (opt-in, SOLUTION_MLP_SAVE_UP=1 in apply())
    patch_group_dequant()       one NF4 dequantization launch per decoder layer and pass
    patch_lora()                the LoRA projection node
    patch_qwen2_attention()     q|k|v + LoRA + RoPE node, varlen attention, o_proj
    patch_sdpa_rows()           per-row causal attention on the packed batch
    patch_sft_compute_loss()    TRL's SFTTrainer.compute_loss on the fused head (apply() installs
                                it when trl imports; its metrics from the head's per-token outputs)
"""

from talm_amd.fused_proj import patch_qwen2_attention
from talm_amd.lora import patch_lora
from talm_amd.mlp_save_up import patch_qwen2_mlp_save_up
from talm_amd.patches import LAST_STEP, apply, patch_qwen2_causal_lm, unapply
from talm_amd.qgroup import patch_group_dequant
from talm_amd.rmsnorm import patch_qwen2_add_norm, patch_qwen2_rmsnorm
from talm_amd.rope import patch_qwen2_rope
from talm_amd.sft_loss import patch_sft_compute_loss
from talm_amd.swiglu_inplace import patch_qwen2_mlp_inplace
from talm_amd.unpad import patch_sdpa_rows

__all__ = ["LAST_STEP", "apply", "unapply", "patch_qwen2_causal_lm", "patch_qwen2_rmsnorm",
           "patch_qwen2_add_norm", "patch_qwen2_rope", "patch_qwen2_mlp_inplace",
           "patch_qwen2_mlp_save_up", "patch_group_dequant", "patch_lora",
           "patch_qwen2_attention", "patch_sdpa_rows", "patch_sft_compute_loss"]
