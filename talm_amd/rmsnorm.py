"""Fused RMSNorm and residual-add + RMSNorm for Qwen2 on the HIP kernel (talm_rmsnorm).

Mirrors solution/rmsnorm.py: one kernel does the whole norm per row, forward and backward, with
runtime `backward` and `add` flags (:58-118), writing the autocast dtype directly. Saved for
backward: xhat in the output dtype and rstd [N]. The norm weight is frozen, so the backward
computes the input gradient only: dx = rstd * (g - xhat * mean(g * xhat)), g = dy * w
(`_reference_dx`, :121-127). `AddRMSNorm` folds the residual add that produces the norm's input
into the same launch (:163-203): the forward writes the sum (the residual stream) with the norm,
the backward adds the sum's gradient and writes the branch's gradient.

MI355X kernel: one 64-lane wavefront per row, the row held in registers, wave64 butterfly
reductions (talm_amd/csrc/rmsnorm.hip).

Graceful degradation (state.py): an error in a forward launch turns the component off and the
call runs through transformers' norm (or the plain add and the norm); an error in a backward
launch computes the same formula with PyTorch ops from the saved xhat and rstd.
"""

import torch

from . import _ops  # noqa: F401 - registers torch.ops.talm.*
from .engaged import FELL_BACK, ON, RAN
from .state import DISABLED, fallback

BLOCK = 1 << 24  # widest row the kernel takes (rows of any width; <= 4096 columns stay in registers)


def _rows(t):
    """[N, H] view of `t` with contiguous rows, copying only if it is not."""
    t2 = t.reshape(-1, t.shape[-1])
    return t2 if t2.is_contiguous() else t2.contiguous()


def launch(a, weight, h, xhat, rstd, eps, backward, p=None, q=None):
    """The one launch site of the kernel (solution/rmsnorm.py:103-118): a, h, xhat (and p, q)
    are contiguous [N, H]; forward reads a (+ p) and writes h, xhat, rstd (and q = a + p);
    backward reads h (= dy), xhat, rstd (and q = ds) and writes a (= dx) (and p = dx)."""
    torch.ops.talm.rmsnorm(a, q, h, xhat, p, weight, rstd, float(eps), int(backward))


def _reference_dx(dy, xhat, weight, rstd):
    """The kernel's backward in PyTorch ops, fp32 (for a backward launch that failed)."""
    g = dy.float() * weight.float()
    xh = xhat.float()
    c = (g * xh).sum(-1, keepdim=True) / xh.shape[-1]
    return rstd[:, None] * (g - xh * c)


class RMSNorm(torch.autograd.Function):
    @staticmethod
    def forward(ctx, x, weight, eps, out_dtype):
        x2 = _rows(x)
        n_rows, n_cols = x2.shape
        y = torch.empty((n_rows, n_cols), dtype=out_dtype, device=x.device)
        xhat = torch.empty_like(y)
        rstd = torch.empty(n_rows, dtype=torch.float32, device=x.device)
        launch(x2, weight, y, xhat, rstd, eps, backward=0)
        RAN["rmsnorm"] += 1
        ctx.save_for_backward(xhat, weight, rstd)
        ctx.x_dtype = x.dtype
        ctx.eps = eps
        return y.view(x.shape)

    @staticmethod
    def backward(ctx, dy):
        xhat, weight, rstd = ctx.saved_tensors
        dy2 = _rows(dy)
        if dy2.dtype != xhat.dtype:
            dy2 = dy2.to(xhat.dtype)
        if "rmsnorm" not in DISABLED:
            try:
                dx = torch.empty(xhat.shape, dtype=ctx.x_dtype, device=dy.device)
                launch(dx, weight, dy2, xhat, rstd, ctx.eps, backward=1)
                RAN["rmsnorm"] += 1
                return dx.view(dy.shape), None, None, None
            except Exception as exc:  # noqa: BLE001 - state.py convention
                if not fallback("rmsnorm", exc):
                    raise
        FELL_BACK["rmsnorm"] += 1
        dx = _reference_dx(dy2, xhat, weight, rstd).to(ctx.x_dtype)
        return dx.view(dy.shape), None, None, None


class AddRMSNorm(torch.autograd.Function):
    """(s, y) = (x + branch, rmsnorm(x + branch)) in one launch each way. The branch has the
    norm output's dtype (the caller checks)."""

    @staticmethod
    def forward(ctx, x, branch, weight, eps, out_dtype):
        x2, b2 = _rows(x), _rows(branch)
        n_rows, n_cols = x2.shape
        total = torch.empty((n_rows, n_cols), dtype=x.dtype, device=x.device)
        y = torch.empty((n_rows, n_cols), dtype=out_dtype, device=x.device)
        xhat = torch.empty_like(y)
        rstd = torch.empty(n_rows, dtype=torch.float32, device=x.device)
        launch(x2, weight, y, xhat, rstd, eps, backward=0, p=b2, q=total)
        RAN["addnorm"] += 1
        ctx.save_for_backward(xhat, weight, rstd)
        ctx.x_dtype, ctx.branch_dtype, ctx.eps = x.dtype, branch.dtype, eps
        return total.view(x.shape), y.view(x.shape)

    @staticmethod
    def backward(ctx, ds, dy):
        xhat, weight, rstd = ctx.saved_tensors
        if dy is None:
            return ds, ds.to(ctx.branch_dtype), None, None, None
        shape = dy.shape
        if ds is None:
            ds = torch.zeros(shape, dtype=ctx.x_dtype, device=dy.device)
        dy2 = _rows(dy)
        if dy2.dtype != xhat.dtype:
            dy2 = dy2.to(xhat.dtype)
        ds2 = _rows(ds)
        if ds2.dtype != ctx.x_dtype:
            ds2 = ds2.to(ctx.x_dtype)
        if "addnorm" not in DISABLED:
            try:
                dx = torch.empty(xhat.shape, dtype=ctx.x_dtype, device=dy.device)
                db = torch.empty(xhat.shape, dtype=ctx.branch_dtype, device=dy.device)
                launch(dx, weight, dy2, xhat, rstd, ctx.eps, backward=1, p=db, q=ds2)
                RAN["addnorm"] += 1
                return dx.view(shape), db.view(shape), None, None, None
            except Exception as exc:  # noqa: BLE001 - state.py convention
                if not fallback("addnorm", exc):
                    raise
        FELL_BACK["addnorm"] += 1
        total = _reference_dx(dy2, xhat, weight, rstd) + ds2.float()
        return (total.to(ctx.x_dtype).view(shape), total.to(ctx.branch_dtype).view(shape), None,
                None, None)


def _autocast_dtype():
    if torch.is_autocast_enabled("cuda"):
        return torch.get_autocast_dtype("cuda")
    return None


def rmsnorm(x, weight, eps, out_dtype=None):
    """RMSNorm of `x` with the frozen `weight`; output in `out_dtype` (default: x's dtype)."""
    return RMSNorm.apply(x, weight, eps, out_dtype or x.dtype)


def add_rmsnorm(x, branch, weight, eps, out_dtype=None):
    """(x + branch, RMSNorm(x + branch)) in one launch."""
    return AddRMSNorm.apply(x, branch, weight, eps, out_dtype or branch.dtype)


def _norm_applies(norm, hidden_states):
    weight = norm.weight
    return not (not hidden_states.is_cuda or weight.requires_grad or hidden_states.dim() < 2
                or hidden_states.shape[-1] != weight.numel()
                or hidden_states.dtype not in (torch.float32, torch.float16)
                or weight.dtype not in (torch.float32, torch.float16))


def _out_dtype(hidden_states):
    if hidden_states.dtype == torch.float32:
        return _autocast_dtype() or torch.float32
    return hidden_states.dtype


def patch_qwen2_rmsnorm():
    """`Qwen2RMSNorm.forward` through the fused kernel on the GPU when the weight is frozen;
    under autocast the output is written in the autocast dtype (solution/rmsnorm.py:235-265)."""
    from transformers.models.qwen2 import modeling_qwen2

    from .patches import _in_chain

    cls = modeling_qwen2.Qwen2RMSNorm
    original = cls.forward
    if _in_chain(original, "_solution_rmsnorm"):
        return

    def forward(self, hidden_states):
        normed = _take_normed(hidden_states, self)
        if normed is not None:
            return normed
        if "rmsnorm" not in DISABLED and _norm_applies(self, hidden_states):
            try:
                return RMSNorm.apply(hidden_states, self.weight, self.variance_epsilon,
                                     _out_dtype(hidden_states))
            except Exception as exc:  # noqa: BLE001 - state.py convention
                if not fallback("rmsnorm", exc):
                    raise
        FELL_BACK["rmsnorm"] += 1
        return original(self, hidden_states)

    forward._solution_rmsnorm = True
    forward._original = original
    cls.forward = forward
    ON.add("rmsnorm")


def _take_normed(hidden_states, norm):
    """The output of `norm` on `hidden_states` if the residual add that produced this tensor
    already computed it (AddRMSNorm at the end of the previous decoder layer), else None."""
    pending = getattr(hidden_states, "_solution_normed", None)
    if pending is None or pending[0] is not norm:
        return None
    del hidden_states._solution_normed
    return pending[1]


LAYER_FORWARDS = {}


def link_next_norms(model):
    """Tell every decoder layer which norm reads its output: the next layer's input_layernorm,
    the final norm for the last layer (solution/rmsnorm.py:278-290)."""
    if not LAYER_FORWARDS:
        return
    layers = list(getattr(model, "layers", []))
    final = getattr(model, "norm", None)
    if not layers or getattr(model, "_solution_norms_linked", None) == len(layers):
        return
    for layer, nxt in zip(layers, layers[1:] + [None]):
        layer._solution_next_norm = nxt.input_layernorm if nxt is not None else final
    model._solution_norms_linked = len(layers)


def _link_norms_in_model_forward(model_cls):
    import functools

    forward = model_cls.forward
    if getattr(forward, "_solution_link_norms", False):
        return

    @functools.wraps(forward)
    def forward_linked(self, *args, **kwargs):
        link_next_norms(self)
        return forward(self, *args, **kwargs)

    forward_linked._solution_link_norms = True
    model_cls.forward = forward_linked


def _add_ok(branch, residual, norm):
    return (residual.dtype in (torch.float32, torch.float16) and branch.shape == residual.shape
            and branch.is_cuda and branch.dtype == _out_dtype(residual)
            and _norm_applies(norm, residual))


def _add_norm(residual, branch, norm):
    if "addnorm" in DISABLED or not _add_ok(branch, residual, norm):
        return None
    try:
        return AddRMSNorm.apply(residual, branch, norm.weight, norm.variance_epsilon,
                                _out_dtype(residual))
    except Exception as exc:  # noqa: BLE001 - state.py convention
        if not fallback("addnorm", exc):
            raise
    return None


def patch_qwen2_add_norm():
    """`Qwen2DecoderLayer.forward` with the residual adds folded into the norms that read them
    (solution/rmsnorm.py:335-404): the attention's add into post_attention_layernorm and, once
    `link_next_norms` ran on the model, the MLP's add into the next layer's input_layernorm (or
    the final norm); that norm's output rides on the returned sum and is taken by that norm."""
    from transformers.models.qwen2 import modeling_qwen2

    from .patches import _in_chain

    _link_norms_in_model_forward(modeling_qwen2.Qwen2Model)
    cls = modeling_qwen2.Qwen2DecoderLayer
    original = cls.forward
    if _in_chain(original, "_solution_add_norm"):
        return

    def forward(self, hidden_states, attention_mask=None, position_ids=None,
                past_key_values=None, use_cache=False, position_embeddings=None, **kwargs):
        checkpointed = self.training and getattr(self, "gradient_checkpointing", False)
        if checkpointed:
            _take_normed(hidden_states, self.input_layernorm)
        post = self.post_attention_layernorm
        if "addnorm" in DISABLED or not (hidden_states.dtype in (torch.float32, torch.float16)
                                         and _norm_applies(post, hidden_states)):
            FELL_BACK["addnorm"] += 1
            return original(self, hidden_states, attention_mask=attention_mask,
                            position_ids=position_ids, past_key_values=past_key_values,
                            use_cache=use_cache, position_embeddings=position_embeddings,
                            **kwargs)
        if getattr(original, "_solution_group", False):
            from .qgroup import enter_layer

            enter_layer(self)
        residual = hidden_states
        hidden_states = self.input_layernorm(hidden_states)
        hidden_states, _ = self.self_attn(
            hidden_states=hidden_states, attention_mask=attention_mask,
            position_ids=position_ids, past_key_values=past_key_values, use_cache=use_cache,
            position_embeddings=position_embeddings, **kwargs)
        fused = _add_norm(residual, hidden_states, post)
        if fused is not None:
            residual, hidden_states = fused
        else:
            FELL_BACK["addnorm"] += 1
            residual = residual + hidden_states
            hidden_states = post(residual)
        hidden_states = self.mlp(hidden_states)
        nxt = None if checkpointed else getattr(self, "_solution_next_norm", None)
        fused = None if nxt is None else _add_norm(residual, hidden_states, nxt)
        if fused is not None:
            total, normed = fused
            total._solution_normed = (nxt, normed)
            return total
        FELL_BACK["addnorm"] += 1
        return residual + hidden_states

    forward._solution_add_norm = True
    forward._original = original
    LAYER_FORWARDS.update(original=original, add_norm=forward)
    cls.forward = forward
    ON.add("addnorm")
