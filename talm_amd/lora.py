"""LoRA adapters on the 4-bit projections: PEFT's module layout, the fp16 adapter copies, and the
fast path of a LoRA projection outside the fused q|k|v node.

`LoraLinear` stands in for PEFT's LoRA wrapper of a 4-bit layer (PEFT and bitsandbytes are not
available here): the attributes the reference reads (`base_layer`, `lora_A` / `lora_B` /
`lora_dropout` keyed by adapter name, `scaling`, `active_adapters`, `disable_adapters`, `merged`)
and PEFT's forward under fp16 autocast, result = base(x) + scaling * B(A(dropout(x))), as its own
forward (the eager path every patched path is checked against).

The reference runs such a projection as its own autograd node with PEFT's ops
(`LoraProjectionTorch`, solution/lora.py:151-231). Here it is the q|k|v node of fused_proj.py
with ONE projection and one adapter (`patch_lora`): without dropout, two MFMA launches forward —
t = x A^T (talm_lora_down) and y = [x | s t] [W | B]^T + b (talm_qkv_lora_fwd: the adapter term
accumulated with the base product and rounded once) — and on the backward u = s dy B
(talm_lora_down), dx = dy W + u A (talm_qkv_lora_bwd_dx) and dA, dB (talm_lora_wgrad); with
dropout, the node's PyTorch ops with the mask replayed from the saved generator state.

The fp16 copies of the fp32 adapter weights come from `adapters.COPIES` (one launch per
optimizer step for every adapter; solution/lora.py:57-114 keeps a cast cache instead).
"""

import math
from collections import namedtuple

import torch
import torch.nn as nn

from .adapters import COPIES
from .engaged import FELL_BACK, ON, RAN
from .state import DISABLED, fallback

_hooks = []


def _to_half(lora_a, lora_b):
    if not _hooks:
        return lora_a.to(torch.float16), lora_b.to(torch.float16)
    return COPIES.half(lora_a), COPIES.half(lora_b)


def adapters_t(lora_as):
    """A^T of a q|k|v node's adapters side by side ([hidden, 16 per adapter] fp16)."""
    if not _hooks:
        return torch.cat([a.detach() for a in lora_as], 0).t().to(torch.float16).contiguous()
    return COPIES.pair_t(tuple(lora_as))


def install_cast_cache():
    """The optimizer step post-hook that retires the fp16 copies (once per process)."""
    if not _hooks:
        from torch.optim.optimizer import register_optimizer_step_post_hook

        _hooks.append(register_optimizer_step_post_hook(COPIES.invalidate))


def _power_of_two(value):
    """Whether `value` is a power of two >= 1: then branch * value is exact in fp16, and one
    rounding of out + value * branch equals PEFT's rounded product followed by a rounded add."""
    mantissa, _ = math.frexp(value)
    return value >= 1 and mantissa == 0.5


class LoraLinear(nn.Module):
    """A LoRA adapter on a 4-bit base layer, with PEFT's attribute layout and fp16-autocast
    forward (PEFT's bnb Linear4bit: result = base(x); result + scaling * B(A(dropout(x))))."""

    def __init__(self, base_layer, r=16, alpha=32, dropout=0.0, name="default"):
        super().__init__()
        self.base_layer = base_layer
        in_f, out_f = base_layer.in_features, base_layer.out_features
        device = base_layer.weight.device
        self.lora_A = nn.ModuleDict({name: nn.Linear(in_f, r, bias=False, device=device)})
        self.lora_B = nn.ModuleDict({name: nn.Linear(r, out_f, bias=False, device=device)})
        self.lora_dropout = nn.ModuleDict({name: nn.Dropout(dropout) if dropout > 0
                                           else nn.Identity()})
        self.scaling = {name: alpha / r}
        self.active_adapters = [name]
        self.disable_adapters = False
        self.merged = False
        self.lora_variant = {}
        self.lora_bias = {}
        # PEFT's init: A Kaiming-uniform (nn.Linear's default, a = sqrt(5)), B zero
        nn.init.kaiming_uniform_(self.lora_A[name].weight, a=math.sqrt(5))
        nn.init.zeros_(self.lora_B[name].weight)

    def forward(self, x):
        result = self.base_layer(x)
        result = result.clone()
        for name in self.active_adapters:
            lora_a, lora_b = self.lora_A[name], self.lora_B[name]
            dropout, scaling = self.lora_dropout[name], self.scaling[name]
            requires_conversion = not torch.is_autocast_enabled("cuda")
            if requires_conversion:
                expected = result.dtype
                x = x.to(lora_a.weight.dtype)
            output = lora_b(lora_a(dropout(x)))
            if requires_conversion:
                output = output.to(expected)
            result = result + output * scaling
        return result


# What the fast path needs of one LoRA projection: its packed base (group, index in the group),
# the fp32 adapter weights, the scaling and the dropout rate in force.
Adapter = namedtuple("Adapter", "group idx lora_a lora_b scaling p")


def _dropout_rate(module):
    """The dropout rate in force (0 for Identity or in eval mode), None for another module."""
    if isinstance(module, nn.Identity):
        return 0.0
    if isinstance(module, nn.Dropout):
        return float(module.p) if module.training else 0.0
    return None


def _single_adapter(module):
    """The one plain adapter (name) the LoRA layer applies, or None: exactly one active adapter,
    not merged, not disabled, without a weight-decomposition variant or a bias."""
    if getattr(module, "disable_adapters", True) or getattr(module, "merged", True):
        return None
    active = list(module.active_adapters)
    if len(active) != 1:
        return None
    name = active[0]
    if name not in module.lora_A or name in getattr(module, "lora_variant", {}) \
            or getattr(module, "lora_bias", {}).get(name, False):
        return None
    return name


def lora_plan(module, x):
    """An `Adapter` when the LoRA layer's forward on `x` can run as the package's node: fp16
    CUDA input under fp16 autocast, a packed 4-bit base whose shape matches, one plain rank-r
    adapter with bias-free fp32 A [r, in] and B [out, r], a dropout rate in [0, 1). Else None
    (the layer's own forward runs; the reference's conditions, solution/lora.py:241-281)."""
    if not (x.is_cuda and x.dtype == torch.float16 and x.dim() >= 2) or "qgroup" in DISABLED:
        return None
    if not (torch.is_autocast_enabled("cuda")
            and torch.get_autocast_dtype("cuda") == torch.float16):
        return None
    name = _single_adapter(module)
    tag = getattr(module.base_layer, "_solution_group", None)
    if name is None or tag is None:
        return None
    down, up = module.lora_A[name], module.lora_B[name]
    if not (isinstance(down, nn.Linear) and isinstance(up, nn.Linear)) \
            or down.bias is not None or up.bias is not None:
        return None
    lora_a, lora_b = down.weight, up.weight
    group, idx = tag
    rank, n_in = lora_a.shape
    if lora_a.dtype != torch.float32 or lora_b.dtype != torch.float32 or not lora_a.is_cuda \
            or tuple(lora_b.shape) != (group.shapes[idx][0], rank) or n_in != x.shape[-1] \
            or group.shapes[idx][1] != n_in:
        return None
    p = _dropout_rate(module.lora_dropout[name])
    if p is None or not 0.0 <= p < 1.0:
        return None
    return Adapter(group, idx, lora_a, lora_b, float(module.scaling[name]), p)


def lora_projection(x, plan):
    """y = x W^T + b + scaling * B(A(dropout(x))) as the q|k|v node on one projection."""
    from .fused_proj import FusedProjections

    (y,) = FusedProjections.apply(x, plan.group, plan.idx, plan.idx + 1,
                                  ((0, plan.scaling, plan.p),), (), None, 0, plan.lora_a,
                                  plan.lora_b)
    return y


def patch_lora():
    """`LoraLinear.forward` through `lora_projection` when `lora_plan` takes the call; the
    layer's own forward otherwise (a failure turns "lora" off, state.py)."""
    install_cast_cache()
    ON.add("lora")
    if getattr(LoraLinear.forward, "_solution_lora", False):
        return True
    original = LoraLinear.forward

    def forward(self, x, *args, **kwargs):
        plan = None
        if not (args or kwargs) and "lora" not in DISABLED:
            plan = lora_plan(self, x)
        if plan is not None:
            try:
                y = lora_projection(x, plan)
            except Exception as exc:  # noqa: BLE001 - state.py convention
                if not fallback("lora", exc):
                    raise
            else:
                RAN["lora"] += 1
                return y
        FELL_BACK["lora"] += 1
        return original(self, x, *args, **kwargs)

    forward._solution_lora = True
    forward._original = original
    LoraLinear.forward = forward
    return True
