"""RMSNorm and the residual adds of the Qwen2 decoder on one HIP kernel (talm_rmsnorm).

One launch per norm and direction computes a whole row (one wave64 per row, the row held in
registers: talm_amd/csrc/rmsnorm.hip), writes the autocast dtype directly and can take the
residual add that produces the norm's input (solution/rmsnorm.py:58-127):

    forward   s = x (+ branch);  rstd = rsqrt(mean(s^2) + eps);  xhat = s rstd;  y = w xhat
    backward  g = dy w;  dx = rstd (g - xhat mean(g xhat))  (+ ds: the sum's own gradient)

The norm weight is frozen (QLoRA), so there is no weight gradient; the node keeps xhat (output
dtype) and rstd.

Where the adds go. Every residual add of the decoder feeds a norm: the attention's add feeds the
layer's post-attention norm, the MLP's add feeds the NEXT layer's input norm (the final norm
after the last layer). The reference folds both (AddRMSNorm, solution/rmsnorm.py:335-404); so
does this module, with its own plumbing: `_layer_forward` runs the decoder layer as three stages
(attention, MLP, hand-over). The first add joins the post-attention norm inside the layer; for
the second the layer computes the next norm's output together with the sum and hands it over on
the sum (`_HANDOVER` attribute), and that norm's patched forward takes it instead of launching.
Which norm follows which layer is recorded once per model (`link_next_norms`).

Graceful degradation (state.py): a failed forward launch turns "rmsnorm" / "addnorm" off and
the call runs transformers' norm (or the plain add, then the norm); a failed backward launch
computes the same formula with PyTorch ops from the saved xhat and rstd.
"""

import functools
import weakref

import torch

from . import _ops  # noqa: F401 - registers torch.ops.talm.*
from .engaged import FELL_BACK, ON, RAN
from .state import DISABLED, fallback

_HANDOVER = "_talm_next_normed"  # attribute of a residual sum: (norm module, its output)


def launch(a, weight, h, xhat, rstd, eps, backward, p=None, q=None):
    """The one launch site of the kernel (solution/rmsnorm.py:103-118): a, h, xhat (and p, q)
    are contiguous [N, H]; forward reads a (+ p) and writes h, xhat, rstd (and q = a + p);
    backward reads h (= dy), xhat, rstd (and q = ds; None: ds = 0) and writes a (= dx) (and
    p = dx)."""
    torch.ops.talm.rmsnorm(a, q, h, xhat, p, weight, rstd, float(eps), int(backward))


def _flat(t, dtype=None):
    """t as a contiguous [rows, H] tensor (of `dtype`), copying only when it must."""
    t2 = t.reshape(-1, t.shape[-1])
    if dtype is not None and t2.dtype != dtype:
        t2 = t2.to(dtype)
    return t2 if t2.is_contiguous() else t2.contiguous()


def _dx_torch(dy, xhat, weight, rstd):
    """The backward formula with PyTorch ops in fp32 (for a backward launch that failed)."""
    g = dy.float() * weight.float()
    xh = xhat.float()
    mean_gx = (g * xh).mean(-1, keepdim=True)
    return rstd[:, None] * (g - xh * mean_gx)


class NormNode(torch.autograd.Function):
    """y = RMSNorm(x), or (x + branch, RMSNorm(x + branch)) when `branch` is given: one kernel
    launch each way. The branch has the norm output's dtype (the caller checks)."""

    @staticmethod
    def forward(ctx, x, branch, weight, eps, out_dtype):
        ctx.set_materialize_grads(False)  # an unused output: no made-up zero gradient
        xs = _flat(x)
        n_rows, width = xs.shape
        y = torch.empty((n_rows, width), dtype=out_dtype, device=x.device)
        xhat = torch.empty_like(y)
        rstd = torch.empty(n_rows, dtype=torch.float32, device=x.device)
        if branch is None:
            launch(xs, weight, y, xhat, rstd, eps, backward=0)
            total = None
        else:
            total = torch.empty((n_rows, width), dtype=x.dtype, device=x.device)
            launch(xs, weight, y, xhat, rstd, eps, backward=0, p=_flat(branch), q=total)
        RAN["rmsnorm" if branch is None else "addnorm"] += 1
        ctx.save_for_backward(xhat, weight, rstd)
        ctx.eps, ctx.x_dtype, ctx.shape = eps, x.dtype, x.shape
        ctx.branch_dtype = None if branch is None else branch.dtype
        y = y.view(x.shape)
        return y if total is None else (total.view(x.shape), y)

    @staticmethod
    def backward(ctx, *grads):
        xhat, weight, rstd = ctx.saved_tensors
        add = ctx.branch_dtype is not None
        ds, dy = grads if add else (None, grads[0])
        if dy is None:  # only the sum was used
            return ds, ds.to(ctx.branch_dtype), None, None, None
        component = "addnorm" if add else "rmsnorm"
        dys = _flat(dy, xhat.dtype)
        # no gradient of the sum (the final norm: only its output is used): the kernel takes
        # ds = 0 without a zero-filled operand
        dss = _flat(ds, ctx.x_dtype) if add and ds is not None else None
        if component not in DISABLED:
            try:
                dx = torch.empty(xhat.shape, dtype=ctx.x_dtype, device=dy.device)
                if add:
                    dbranch = torch.empty(xhat.shape, dtype=ctx.branch_dtype, device=dy.device)
                    launch(dx, weight, dys, xhat, rstd, ctx.eps, backward=1, p=dbranch, q=dss)
                else:
                    dbranch = None
                    launch(dx, weight, dys, xhat, rstd, ctx.eps, backward=1)
            except Exception as exc:  # noqa: BLE001 - state.py convention
                if not fallback(component, exc):
                    raise
            else:
                RAN[component] += 1
                return NormNode._grads(ctx, dx, dbranch)
        FELL_BACK[component] += 1
        dx32 = _dx_torch(dys, xhat, weight, rstd)
        if not add:
            return NormNode._grads(ctx, dx32.to(ctx.x_dtype), None)
        if dss is not None:
            dx32 = dx32 + dss.float()
        return NormNode._grads(ctx, dx32.to(ctx.x_dtype), dx32.to(ctx.branch_dtype))

    @staticmethod
    def _grads(ctx, dx, dbranch):
        return (dx.view(ctx.shape), None if dbranch is None else dbranch.view(ctx.shape), None,
                None, None)


def rmsnorm(x, weight, eps, out_dtype=None):
    """RMSNorm of `x` with the frozen `weight`; output in `out_dtype` (default: x's dtype)."""
    return NormNode.apply(x, None, weight, eps, out_dtype or x.dtype)


def add_rmsnorm(x, branch, weight, eps, out_dtype=None):
    """(x + branch, RMSNorm(x + branch)) in one launch."""
    return NormNode.apply(x, branch, weight, eps, out_dtype or branch.dtype)


# -- when the kernel takes a norm ------------------------------------------------------------------

_DTYPES = (torch.float32, torch.float16)


def _target_dtype(x):
    """The dtype transformers' norm would return under the current autocast: fp32 input under
    fp16/bf16 autocast gives the autocast dtype (its final cast), anything else keeps x's."""
    if x.dtype == torch.float32 and torch.is_autocast_enabled("cuda"):
        return torch.get_autocast_dtype("cuda")
    return x.dtype


def _kernel_takes(norm, x):
    """A frozen fp32/fp16 weight of x's width on the GPU, x fp32/fp16 with rows of it, an
    fp32/fp16 output (bf16 autocast takes transformers' norm)."""
    w = norm.weight
    return (x.is_cuda and x.dim() >= 2 and not w.requires_grad and x.shape[-1] == w.numel()
            and x.dtype in _DTYPES and w.dtype in _DTYPES and _target_dtype(x) in _DTYPES)


def _norm_via_kernel(norm, x):
    """norm(x) on the kernel, or None (not applicable, or the component is off / just failed)."""
    if "rmsnorm" in DISABLED or not _kernel_takes(norm, x):
        return None
    try:
        return NormNode.apply(x, None, norm.weight, norm.variance_epsilon, _target_dtype(x))
    except Exception as exc:  # noqa: BLE001 - state.py convention
        if not fallback("rmsnorm", exc):
            raise
    return None


def _sum_and_norm(residual, branch, norm):
    """(residual + branch, norm(residual + branch)) in one launch, or None."""
    if "addnorm" in DISABLED or not _kernel_takes(norm, residual) \
            or branch.shape != residual.shape or not branch.is_cuda \
            or branch.dtype != _target_dtype(residual):
        return None
    try:
        return NormNode.apply(residual, branch, norm.weight, norm.variance_epsilon,
                              _target_dtype(residual))
    except Exception as exc:  # noqa: BLE001 - state.py convention
        if not fallback("addnorm", exc):
            raise
    return None


def _take_handover(x, norm):
    """The output of `norm` on x if the add that produced x computed it already, else None."""
    held = getattr(x, _HANDOVER, None)
    if held is None or held[0] is not norm:
        return None
    delattr(x, _HANDOVER)
    return held[1]


def patch_qwen2_rmsnorm():
    """`Qwen2RMSNorm.forward`: a handed-over output, else the kernel, else transformers' norm
    (solution/rmsnorm.py:235-265)."""
    from transformers.models.qwen2 import modeling_qwen2

    from .patches import _in_chain

    cls = modeling_qwen2.Qwen2RMSNorm
    original = cls.forward
    if _in_chain(original, "_solution_rmsnorm"):
        return

    def forward(self, hidden_states):
        y = _take_handover(hidden_states, self)
        if y is None:
            y = _norm_via_kernel(self, hidden_states)
        if y is not None:
            return y
        FELL_BACK["rmsnorm"] += 1
        return original(self, hidden_states)

    forward._solution_rmsnorm = True
    forward._original = original
    cls.forward = forward
    ON.add("rmsnorm")


# -- the residual adds inside the decoder layers ---------------------------------------------------

LAYER_FORWARDS = {}


def link_next_norms(model):
    """Record on every decoder layer of `model` (a Qwen2Model) the norm that reads its output:
    the next layer's input norm, the final norm after the last layer. Once per model (again
    when its layer count changes)."""
    if not LAYER_FORWARDS:
        return
    layers = list(getattr(model, "layers", ()))
    if not layers or model.__dict__.get("_talm_linked") == len(layers):
        return
    followers = [layer.input_layernorm for layer in layers[1:]] + [getattr(model, "norm", None)]
    for layer, follower in zip(layers, followers):
        # straight into the instance dict: nn.Module's setattr would register the norm as a
        # submodule of the layer (a second owner in state_dict and the module tree)
        layer.__dict__["_talm_next_norm"] = None if follower is None else weakref.ref(follower)
    model._talm_linked = len(layers)


def _link_in_model_forward(model_cls):
    forward = model_cls.forward
    if getattr(forward, "_solution_link_norms", False):
        return

    @functools.wraps(forward)
    def forward_linked(self, *args, **kwargs):
        link_next_norms(self)
        return forward(self, *args, **kwargs)

    forward_linked._solution_link_norms = True
    model_cls.forward = forward_linked


def _layer_forward(layer, x, attn_kwargs):
    """The decoder layer with both residual adds on the norm kernel. Returns the residual sum,
    carrying the next norm's output when that norm is known and the add went to the kernel."""
    # stage 1: input norm (handed over by the previous layer when it could), attention, and the
    # attention's residual add with the post-attention norm in one launch
    h, _ = layer.self_attn(hidden_states=layer.input_layernorm(x), **attn_kwargs)
    link = layer.__dict__.get("_talm_next_norm")
    follower = None if link is None else link()
    if follower is not None:
        # stages 1 (the add and norm) to 3 as one node (mlp_block.py) when it applies
        from .mlp_block import mlp_block

        block = mlp_block(layer, x, h, follower)
        if block is not None:
            total, normed_next = block
            setattr(total, _HANDOVER, (follower, normed_next))
            return total
    fused = _sum_and_norm(x, h, layer.post_attention_layernorm)
    if fused is None:
        FELL_BACK["addnorm"] += 1
        stream = x + h
        normed = layer.post_attention_layernorm(stream)
    else:
        stream, normed = fused
    # stage 2: the MLP
    h = layer.mlp(normed)
    # stage 3: the MLP's residual add, with the next norm when there is one to hand over to
    fused = None if follower is None else _sum_and_norm(stream, h, follower)
    if fused is None:
        FELL_BACK["addnorm"] += 1
        return stream + h
    total, normed_next = fused
    setattr(total, _HANDOVER, (follower, normed_next))
    return total


def patch_qwen2_add_norm():
    """`Qwen2DecoderLayer.forward` through `_layer_forward` (solution/rmsnorm.py:335-404);
    transformers' layer forward when the post-attention norm cannot take the kernel, and in a
    gradient-checkpointed layer, whose recomputation must not hand a result to a norm outside
    it."""
    from transformers.models.qwen2 import modeling_qwen2

    from .patches import _in_chain

    _link_in_model_forward(modeling_qwen2.Qwen2Model)
    cls = modeling_qwen2.Qwen2DecoderLayer
    original = cls.forward
    if _in_chain(original, "_solution_add_norm"):
        return
    enters_group = getattr(original, "_solution_group", False)

    def forward(self, hidden_states, attention_mask=None, position_ids=None,
                past_key_values=None, use_cache=False, position_embeddings=None, **kwargs):
        checkpointed = self.training and getattr(self, "gradient_checkpointing", False)
        if checkpointed or "addnorm" in DISABLED \
                or not _kernel_takes(self.post_attention_layernorm, hidden_states):
            if checkpointed:
                _take_handover(hidden_states, self.input_layernorm)
            FELL_BACK["addnorm"] += 1
            return original(self, hidden_states, attention_mask=attention_mask,
                            position_ids=position_ids, past_key_values=past_key_values,
                            use_cache=use_cache, position_embeddings=position_embeddings,
                            **kwargs)
        if enters_group:  # the layer-group patch below this one would have done it
            from .qgroup import enter_layer

            enter_layer(self)
        return _layer_forward(self, hidden_states, dict(
            attention_mask=attention_mask, position_ids=position_ids,
            past_key_values=past_key_values, use_cache=use_cache,
            position_embeddings=position_embeddings, **kwargs))

    forward._solution_add_norm = True
    forward._original = original
    LAYER_FORWARDS.update(original=original, add_norm=forward)
    cls.forward = forward
    ON.add("addnorm")
