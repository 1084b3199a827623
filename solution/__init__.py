"""The reference's package name and entry point over this build: `import solution;
solution.apply()` installs the MI355X kernels exactly where the reference's `solution.apply()`
(solution/__init__.py:229) installs its Triton kernels, with the same patch names, switches
(SOLUTION_DISABLE_<PART>=1) and fallback convention.

The implementation lives in the `talm_amd` package. The reference's module names on the hot path
resolve to the same module objects here (`solution.qgroup is talm_amd.qgroup`, and so on), so
code written against the reference's launch sites (`solution.qgroup.launch`,
`solution.rmsnorm.launch`, `solution.rope._launch`, `solution.fused_head.fused_head_loss`,
`solution.state.DISABLED`, ...) runs unchanged. `solution.patches` holds `apply()` and the
`patch_*` installers. Modules outside the hot path (start-up trims, Triton build and warm-up,
host bookkeeping, the bf16 and fp16-embedding plumbing) have no counterpart.
"""

import importlib
import sys

_SAME_MODULES = ("state", "engaged", "qgroup", "nf4_dequant", "rmsnorm", "rope", "swiglu",
                 "swiglu_inplace", "mlp_save_up", "fused_head", "lora", "fused_proj", "unpad")

for _name in _SAME_MODULES:
    _module = importlib.import_module(f"talm_amd.{_name}")
    sys.modules[f"{__name__}.{_name}"] = _module
    globals()[_name] = _module

from . import patches  # noqa: E402
from .patches import apply, unapply  # noqa: E402

__all__ = ["apply", "unapply", "patches", *_SAME_MODULES]
