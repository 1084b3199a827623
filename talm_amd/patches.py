"""`apply()`: install the MI355X kernels into transformers' Qwen2 (the reference's patch API).

Mirrors solution.apply() (solution/__init__.py:229-408): class-level patches, looked up at call
time, each installed once (`_in_chain`, :119-129) under `state.installing`, each falling back to
the original code outside the exact situation it was written for. Installed here:

- RMSNorm and the residual adds folded into the norms (rmsnorm.py);
- RoPE (rope.py);
- SwiGLU with the in-place backward (swiglu.py, swiglu_inplace.py), or the save-up MLP
  (mlp_save_up.py, opt-in SOLUTION_MLP_SAVE_UP=1);
- grouped NF4 dequantization of the 4-bit projections (qgroup.py);
- the fused LM head + cross-entropy of the causal LM (fused_head.py, below).

Switches: SOLUTION_DISABLE_<PART>=1 leaves a part out (RMSNORM, ADDNORM, ROPE, SWIGLU_INPLACE,
GROUP, FUSED_HEAD), as in the reference (solution/__init__.py:51-84).
"""

import os

from .engaged import ON
from .state import installing


def _in_chain(fn, marker):
    """Whether a wrapper carrying `marker` is in the patch chain of `fn` (each wrapper keeps the
    function it wraps in `_original` or `_previous`)."""
    seen = set()
    while fn is not None and id(fn) not in seen:
        seen.add(id(fn))
        if getattr(fn, marker, False):
            return True
        fn = getattr(fn, "_previous", None) or getattr(fn, "_original", None)
    return False


def _off(name):
    return os.environ.get(f"SOLUTION_DISABLE_{name}") == "1"


def apply():
    """Install every patch (idempotent). Loads libtalm.so first: without the kernels nothing is
    installed and the error propagates (there is no CPU fallback)."""
    from . import _lib

    _lib.lib()
    if not _off("SWIGLU_INPLACE"):
        with installing("swiglu"):
            from .swiglu_inplace import patch_qwen2_mlp_inplace

            patch_qwen2_mlp_inplace()
    if os.environ.get("SOLUTION_MLP_SAVE_UP") == "1":
        with installing("mlp_save_up"):
            from .mlp_save_up import patch_qwen2_mlp_save_up

            patch_qwen2_mlp_save_up()
    if not _off("RMSNORM"):
        with installing("rmsnorm"):
            from .rmsnorm import patch_qwen2_add_norm, patch_qwen2_rmsnorm

            patch_qwen2_rmsnorm()
            if not _off("ADDNORM"):
                patch_qwen2_add_norm()
    if not _off("ROPE"):
        with installing("rope"):
            from .rope import patch_qwen2_rope

            patch_qwen2_rope()
    if not _off("GROUP"):
        with installing("qgroup"):
            from .qgroup import patch_group_dequant

            patch_group_dequant()
    return sorted(ON)
