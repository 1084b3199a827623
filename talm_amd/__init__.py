"""talm_amd — the Talm QLoRA kernel set, MI355X-native (gfx950 / CDNA4).

Hand-written HIP kernels (talm_amd/csrc, built into talm_amd/libtalm.so, C-ABI in
include/talm.h) reached through `torch.ops.talm.*` custom ops, behind the reference's patch API:
`talm_amd.apply()` installs them into transformers' Qwen2 exactly where the reference's
`solution.apply()` installs its Triton kernels.

Modules keep the reference's names: qgroup, nf4_dequant, rmsnorm, rope, swiglu, swiglu_inplace,
mlp_save_up, fused_head, lora, fused_proj, patches, state, engaged.
"""

__version__ = "0.1.0"


def apply():
    from .patches import apply as _apply

    return _apply()
