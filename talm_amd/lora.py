"""The 4-bit projections that carry a LoRA adapter (q_proj, v_proj) as one autograd node.

Mirrors solution/lora.py: `LoraProjectionTorch` runs PEFT's LoRA arithmetic op for op — the base
GEMM on the layer group's dequantized weight, dropout, the two fp16 adapter GEMMs, `* scaling`
folded into the add when it is a power of two >= 1 (exact), the fp16 add onto the base output —
but keeps only the layer input x for the backward and replays the dropout there from the saved
generator state (:151-231). The fp16 copies of the fp32 adapter weights come from
`adapters.COPIES` (one launch per optimizer step for every adapter, :57-114).

PEFT is not available here, so `LoraLinear` stands in for PEFT's LoRA wrapper of a 4-bit layer:
the attributes the reference reads (`base_layer`, `lora_A`/`lora_B`/`lora_dropout` keyed by the
adapter name, `scaling`, `active_adapters`, `disable_adapters`, `merged`) and PEFT's forward
under fp16 autocast as its own forward.
"""

import math

import torch
import torch.nn as nn
import torch.nn.functional as F

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
    """A power of two >= 1: branch * value is exact in fp16, so one rounding of
    out + value * branch equals PEFT's rounded product then rounded add (:140-148)."""
    mantissa, _ = math.frexp(value)
    return value >= 1 and mantissa == 0.5


class LoraProjectionTorch(torch.autograd.Function):
    """y = x W^T + bias + scaling * B(A(dropout(x))) on a packed 4-bit base (solution/lora.py:
    151-231): PEFT's ops, keeping only x (and the generator state for the dropout replay)."""

    @staticmethod
    def forward(ctx, x, x_base, lora_a, lora_b, group, idx, scaling, p):
        ctx.rng_state = None
        fetched = False
        try:
            x2 = x.reshape(-1, x.shape[-1])
            weight = group.weight("fwd", idx)
            fetched = True
            out = F.linear(x2, weight, group.biases[idx])
            a16, b16 = _to_half(lora_a, lora_b)
            if p > 0:
                ctx.rng_state = torch.cuda.get_rng_state(x.device)
                xd = torch.native_dropout(x2, p, True)[0]
            else:
                xd = x2
            t = torch.mm(xd, a16.t())
            del xd
            branch = torch.mm(t, b16.t())
            if _power_of_two(scaling):
                out.add_(branch, alpha=scaling)
            else:
                out.add_(branch.mul_(scaling))
        except Exception:
            if fetched:
                group.refund("fwd")
            if ctx.rng_state is not None:
                torch.cuda.set_rng_state(ctx.rng_state, x.device)
            raise
        ctx.save_for_backward(x2, t, a16, b16)
        ctx.group, ctx.idx, ctx.scaling, ctx.p = group, idx, scaling, p
        ctx.x_shape = x.shape
        return out.view(*x.shape[:-1], out.shape[1])

    @staticmethod
    def backward(ctx, grad_out):
        x2, t, a16, b16 = ctx.saved_tensors
        dy = grad_out.reshape(-1, grad_out.shape[-1])
        if dy.dtype != torch.float16:
            dy = dy.to(torch.float16)
        mask = None
        xd = x2
        if ctx.rng_state is not None:
            device = x2.device
            current = torch.cuda.get_rng_state(device)
            torch.cuda.set_rng_state(ctx.rng_state, device)
            try:
                xd, mask = torch.native_dropout(x2, ctx.p, True)
            finally:
                torch.cuda.set_rng_state(current, device)
        g = dy * ctx.scaling
        u = torch.mm(g, b16)
        dx_lora = dx_base = None
        if ctx.needs_input_grad[0]:
            dx_lora = torch.mm(u, a16)
            if mask is not None:
                dx_lora = torch.ops.aten.native_dropout_backward(dx_lora, mask, 1.0 / (1.0 - ctx.p))
            dx_lora = dx_lora.view(ctx.x_shape)
        if ctx.needs_input_grad[1]:
            dx_base = torch.mm(dy, ctx.group.weight("bwd", ctx.idx)).view(ctx.x_shape)
        da = torch.mm(u.t(), xd).float() if ctx.needs_input_grad[2] else None
        db = torch.mm(g.t(), t).float() if ctx.needs_input_grad[3] else None
        return dx_lora, dx_base, da, db, None, None, None, None


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


def _autocast_fp16():
    return torch.is_autocast_enabled("cuda") and torch.get_autocast_dtype("cuda") == torch.float16


def lora_plan(module, x):
    """(group, idx, A, B, scaling, p) when this LoRA layer can take the node, else None
    (solution/lora.py:241-281)."""
    if not (x.is_cuda and x.dtype == torch.float16 and x.dim() >= 2):
        return None
    if getattr(module, "disable_adapters", True) or getattr(module, "merged", True):
        return None
    adapters = module.active_adapters
    if len(adapters) != 1:
        return None
    name = adapters[0]
    if name not in module.lora_A or name in getattr(module, "lora_variant", {}) \
            or getattr(module, "lora_bias", {}).get(name, False):
        return None
    tag = getattr(module.base_layer, "_solution_group", None)
    if tag is None or "qgroup" in DISABLED or not _autocast_fp16():
        return None
    lin_a, lin_b = module.lora_A[name], module.lora_B[name]
    if not isinstance(lin_a, nn.Linear) or not isinstance(lin_b, nn.Linear) \
            or lin_a.bias is not None or lin_b.bias is not None:
        return None
    lora_a, lora_b = lin_a.weight, lin_b.weight
    rank, n_in = lora_a.shape
    if lora_b.shape[1] != rank or n_in != x.shape[-1] or lora_a.dtype != torch.float32 \
            or lora_b.dtype != torch.float32 or not lora_a.is_cuda:
        return None
    group, idx = tag
    if tuple(group.shapes[idx]) != (lora_b.shape[0], n_in):
        return None
    dropout = module.lora_dropout[name]
    if isinstance(dropout, nn.Dropout):
        p = float(dropout.p) if dropout.training else 0.0
    elif isinstance(dropout, nn.Identity):
        p = 0.0
    else:
        return None
    if not 0.0 <= p < 1.0:
        return None
    return group, idx, lora_a, lora_b, float(module.scaling[name]), p


def patch_lora():
    """Route LoraLinear.forward through `LoraProjectionTorch` in the plain case
    (solution/lora.py:284-321)."""
    install_cast_cache()
    ON.add("lora")
    if getattr(LoraLinear.forward, "_solution_lora", False):
        return True
    original = LoraLinear.forward

    def forward(self, x, *args, **kwargs):
        plan = None if (args or kwargs or "lora" in DISABLED) else lora_plan(self, x)
        if plan is not None:
            group, idx, lora_a, lora_b, scaling, p = plan
            try:
                out = LoraProjectionTorch.apply(x, x, lora_a, lora_b, group, idx, scaling, p)
            except Exception as exc:  # noqa: BLE001 - state.py convention
                if not fallback("lora", exc):
                    raise
            else:
                if torch.is_grad_enabled() and x.requires_grad:
                    group.expected_bwd += 1
                RAN["lora"] += 1
                return out
        FELL_BACK["lora"] += 1
        return original(self, x, *args, **kwargs)

    forward._solution_lora = True
    forward._original = original
    LoraLinear.forward = forward
    return True
