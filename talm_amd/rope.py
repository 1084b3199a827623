"""Fused rotary position embedding of q and k on the HIP kernel (talm_rope), forward and backward.

Mirrors solution/rope.py: one launch rotates q (12 heads) and k (2 heads),
    forward:  y1 = x1 c1 - x2 s1,  y2 = x2 c2 + x1 s2
    backward: dx1 = dy1 c1 + dy2 s2,  dx2 = dy2 c2 - dy1 s1
in fp32, writing fp16 (:9-15, :64-108). `_launch(q, k, cos, sin, backward)` keeps the
reference's launch-site signature and layouts (:111-134): new tensors, head-major forward
([1, H, N, D], what the attention reads) and token-major backward (free to view back as the
projection output's gradient). `rope_(q, k, cos, sin, backward)` rotates IN PLACE: the kernel
reads every pair before writing it, so q and k may be column views of the q|k|v projection
output (the fused projections node rotates there and keeps nothing, fused_proj.py).

Graceful degradation (state.py): an error in the forward launch turns "rope" off and the call
runs through transformers' `apply_rotary_pos_emb`; an error in the backward launch computes the
same rotation with PyTorch ops (`_reference`).
"""

import torch

from . import _ops  # noqa: F401 - registers torch.ops.talm.*
from .engaged import FELL_BACK, ON, RAN
from .state import DISABLED, fallback

TOKEN_MAJOR_GRAD = True


def _tokens(x):
    """[1, H, N, D] -> [N, H, D] view (no copy)."""
    return x[0].transpose(0, 1)


def rope_(q, k, cos, sin, backward=False):
    """Rotate q [N, Hq, D] and k [N, Hk, D] fp16 views in place (cos / sin float32 [N, D])."""
    torch.ops.talm.rope(q, k, cos, sin, q, k, int(backward))
    return q, k


def _launch(q, k, cos, sin, backward):
    """q [1, Hq, N, D], k [1, Hk, N, D] (last dim contiguous), cos/sin [1, N, D] fp32. Returns
    new fp16 tensors of the same shapes: head-major, or token-major for the backward."""
    _, hq, n, dim = q.shape
    hk = k.shape[1]
    if backward and TOKEN_MAJOR_GRAD:
        out_q = torch.empty((1, n, hq, dim), dtype=torch.float16, device=q.device).transpose(1, 2)
        out_k = torch.empty((1, n, hk, dim), dtype=torch.float16, device=q.device).transpose(1, 2)
    else:
        out_q = torch.empty((1, hq, n, dim), dtype=torch.float16, device=q.device)
        out_k = torch.empty((1, hk, n, dim), dtype=torch.float16, device=q.device)
    torch.ops.talm.rope(_tokens(q), _tokens(k), cos[0], sin[0], _tokens(out_q), _tokens(out_k),
                        int(backward))
    return out_q, out_k


def _reference(x, cos, sin, backward):
    """The kernel's rotation of x [1, H, N, D] in PyTorch ops (fp32, written as fp16)."""
    half = x.shape[-1] // 2
    x, c, s = x.float(), cos[:, None].float(), sin[:, None].float()
    x1, x2 = x[..., :half], x[..., half:]
    c1, c2, s1, s2 = c[..., :half], c[..., half:], s[..., :half], s[..., half:]
    if backward:
        y1, y2 = x1 * c1 + x2 * s2, x2 * c2 - x1 * s1
    else:
        y1, y2 = x1 * c1 - x2 * s1, x2 * c2 + x1 * s2
    return torch.cat((y1, y2), -1).to(torch.float16)


def _unit_cols(t):
    return t if t.stride(-1) == 1 else t.contiguous()


class RoPE(torch.autograd.Function):
    @staticmethod
    def forward(ctx, q, k, cos, sin):
        cos = _unit_cols(cos)
        sin = _unit_cols(sin)
        ctx.save_for_backward(cos, sin)
        RAN["rope"] += 1
        return _launch(q, k, cos, sin, backward=0)

    @staticmethod
    def backward(ctx, dq, dk):
        cos, sin = ctx.saved_tensors
        dq = _unit_cols(dq).to(torch.float16)
        dk = _unit_cols(dk).to(torch.float16)
        if "rope" not in DISABLED:
            try:
                gq, gk = _launch(dq, dk, cos, sin, backward=1)
                RAN["rope"] += 1
                return gq, gk, None, None
            except Exception as exc:  # noqa: BLE001 - state.py convention
                if not fallback("rope", exc):
                    raise
        FELL_BACK["rope"] += 1
        return _reference(dq, cos, sin, True), _reference(dk, cos, sin, True), None, None


def _applies(q, k, cos, sin, unsqueeze_dim):
    return (unsqueeze_dim == 1 and q.is_cuda and q.dtype == torch.float16
            and k.dtype == torch.float16 and q.dim() == 4 and k.dim() == 4 and q.shape[0] == 1
            and k.shape[0] == 1 and cos.dim() == 3 and cos.shape[0] == 1
            and cos.dtype == torch.float32 and sin.dtype == torch.float32
            and cos.shape == sin.shape and cos.shape[1] == q.shape[2] == k.shape[2]
            and cos.shape[2] == q.shape[3] == k.shape[3] and q.shape[3] % 2 == 0
            and q.shape[3] <= 512 and q.stride(-1) == 1 and k.stride(-1) == 1)


def patch_qwen2_rope():
    """Route `modeling_qwen2.apply_rotary_pos_emb` through the fused kernel for the fp16
    flat-batch case; anything else takes the original (solution/rope.py:202-224)."""
    from transformers.models.qwen2 import modeling_qwen2

    original = modeling_qwen2.apply_rotary_pos_emb
    ON.add("rope")
    if getattr(original, "_solution_rope", False):
        return

    def apply_rotary_pos_emb(q, k, cos, sin, unsqueeze_dim=1, **kwargs):
        if not kwargs and "rope" not in DISABLED and _applies(q, k, cos, sin, unsqueeze_dim):
            try:
                return RoPE.apply(q, k, cos, sin)
            except Exception as exc:  # noqa: BLE001 - state.py convention
                if not fallback("rope", exc):
                    raise
        FELL_BACK["rope"] += 1
        return original(q, k, cos, sin, unsqueeze_dim=unsqueeze_dim, **kwargs)

    apply_rotary_pos_emb._solution_rope = True
    apply_rotary_pos_emb._original = original
    modeling_qwen2.apply_rotary_pos_emb = apply_rotary_pos_emb


def _table_applies(module, x, position_ids):
    """transformers' rotary embedding of a default or statically scaled type (its inverse
    frequencies fixed: no dynamic update) on fp32 inputs with int64 positions on one GPU."""
    rope_type = getattr(module, "rope_type", "default")
    inv_freq = getattr(module, "inv_freq", None)
    return (isinstance(rope_type, str) and "dynamic" not in rope_type and rope_type != "longrope"
            and torch.is_tensor(inv_freq) and inv_freq.is_cuda and inv_freq.dim() == 1
            and inv_freq.dtype == torch.float32 and x.is_cuda and x.dtype == torch.float32
            and torch.is_tensor(position_ids) and position_ids.dtype == torch.int64
            and position_ids.dim() == 2 and position_ids.device == inv_freq.device
            and x.device == inv_freq.device)


def rope_tables(module, position_ids):
    """(cos, sin) float32 [B, T, 2 half] of the rotary embedding in one launch
    (talm_rope_table): the same products, libm calls and scaling as its forward."""
    inv_freq = module.inv_freq.contiguous()
    half = inv_freq.numel()
    b, t = position_ids.shape
    cos = torch.empty(b, t, 2 * half, dtype=torch.float32, device=inv_freq.device)
    sin = torch.empty_like(cos)
    torch.ops.talm.rope_table(position_ids.contiguous(), inv_freq,
                              float(getattr(module, "attention_scaling", 1.0)), cos, sin)
    return cos, sin


def patch_qwen2_rotary_tables():
    """`Qwen2RotaryEmbedding.forward` through `rope_tables` when `_table_applies`; the original
    forward otherwise."""
    from transformers.models.qwen2 import modeling_qwen2

    from .patches import _in_chain

    cls = modeling_qwen2.Qwen2RotaryEmbedding
    original = cls.forward
    ON.add("rope_table")
    if _in_chain(original, "_solution_rope_table"):
        return

    @torch.no_grad()
    def forward(self, x, position_ids):
        if "rope_table" not in DISABLED and _table_applies(self, x, position_ids):
            try:
                out = rope_tables(self, position_ids)
                RAN["rope_table"] += 1
                return out
            except Exception as exc:  # noqa: BLE001 - state.py convention
                if not fallback("rope_table", exc):
                    raise
        FELL_BACK["rope_table"] += 1
        return original(self, x, position_ids)

    forward._solution_rope_table = True
    forward._original = original
    cls.forward = forward
