"""The MLP half of a Qwen2 decoder layer as ONE autograd node on this package's kernels.

After the attention's output h, the decoder layer computes (the residual adds folded into the
norms as in solution/rmsnorm.py:335-404, the MLP as solution/fused_proj.py:241-287's FusedMLP):
    s1 = x + h;   n1 = post_attention_norm(s1)              add + norm        (talm_rmsnorm)
    y  = down(silu(gate(n1)) * up(n1))                      the MLP           (hipBLASLt, SwiGLU)
    s2 = s1 + y;  n2 = next_norm(s2)                        add + the next layer's input norm
`MlpBlock` runs them as one node. The down projection runs on hipBLASLt with one fp16 output
that the next norm's add reads: at the step's ~1300 tokens that measured 0.07 ms per step faster
(same box, three runs each) than this package's split-K GEMM with its seven fp32 K-part partials
(56 MB written and read back) summed inside the next norm's launch. In the backward the gate|up
input gradient's partials (on the NF4 codes, talm_nf4_gemm_partials, or the split-K GEMM on the
transposed weight) are summed inside the post-attention norm's backward
(talm_splitk_rmsnorm_bwd): one launch fewer, and the same bits as the separate nodes (the
partials are summed in the same order and rounded to fp16 before the norm reads them, as the
product's own reduction does).

Graceful degradation (state.py): a launch failing in the forward turns its component off and the
layer runs the separate nodes; in the backward each failed launch falls back as those nodes do
(the NF4 product to the transposed weight, the norm kernels to the PyTorch formula).
"""

import os

import torch

from . import _ops, fused_mlp
from . import rmsnorm as _rms
from .engaged import FELL_BACK, ON, RAN
from .fused_mlp import DOWN, GATE
from .state import DISABLED, fallback

ENABLED = os.environ.get("SOLUTION_DISABLE_MLP_BLOCK") != "1"
MAX_WIDTH = 2048  # the fused norm launches hold a row of at most this many columns per wavefront


def _flat(t, dtype):
    t2 = t.reshape(-1, t.shape[-1])
    if t2.dtype != dtype:
        t2 = t2.to(dtype)
    return t2 if t2.is_contiguous() else t2.contiguous()


def _norm_bwd_torch(dy, xhat, weight, rstd, ds, dx, dbranch):
    """The add-norm backward with PyTorch ops (a failed launch): dx (fp32) and dbranch (fp16)."""
    dx32 = _rms._dx_torch(dy, xhat, weight, rstd)
    if ds is not None:
        dx32 = dx32 + ds.float()
    dx.copy_(dx32)
    dbranch.copy_(dx32)


def _norm_bwd(dy, xhat, weight, rstd, ds, dx, dbranch):
    """talm_rmsnorm's add backward into dx / dbranch (fp32 / fp16), else the PyTorch formula."""
    if "addnorm" not in DISABLED:
        try:
            _rms.launch(dx, weight, dy, xhat, rstd, 0.0, backward=1, p=dbranch, q=ds)
            return
        except Exception as exc:  # noqa: BLE001 - state.py convention
            if not fallback("addnorm", exc):
                raise
    FELL_BACK["addnorm"] += 1
    _norm_bwd_torch(dy, xhat, weight, rstd, ds, dx, dbranch)


def _input_grad_partials(group, gu, n_tok, hidden):
    """The K-part partials of dn1 = [dgate | dup] [W_gate; W_up] (fp32 [parts, N, H]): on the
    NF4 codes while the layer group serves gate|up that way, else on the split-K GEMM over the
    transposed weight; None when neither runs (the caller takes FusedMLP's products)."""
    if (GATE, fused_mlp.UP) in group.w4_blocks():
        try:
            part = torch.empty(group.nf4_gemm_parts(n_tok, GATE, DOWN, True), n_tok, hidden,
                               dtype=torch.float32, device=gu.device)
            group.nf4_gemm(gu, GATE, DOWN, True, None, partials=part)
            RAN["w4a16"] += 1
            return part
        except Exception as exc:  # noqa: BLE001 - state.py convention
            if not fallback("w4a16", exc):
                raise
    if not fused_mlp.SPLITK or "splitk" in DISABLED:
        return None
    w_gu_t = group.span_t(GATE, DOWN)
    if w_gu_t is None:
        return None
    try:
        part = torch.empty(_ops.gemm_splitk_parts(n_tok, hidden, gu.shape[1]), n_tok, hidden,
                           dtype=torch.float32, device=gu.device)
        torch.ops.talm.gemm_splitk_partials(gu, w_gu_t, part)
        RAN["splitk"] += 1
        return part
    except Exception as exc:  # noqa: BLE001 - state.py convention
        if not fallback("splitk", exc):
            raise
    return None


class MlpBlock(torch.autograd.Function):
    """(s2, n2) from the residual stream x (fp32) and the attention's output h (fp16); see the
    module docstring. `stage` (a one-item list) names the component of the launch in flight, for
    the caller's fallback."""

    @staticmethod
    def forward(ctx, x, h, group, norm1, norm2, stage):
        # an unused output (the last layer's sum) gets no made-up zero gradient
        ctx.set_materialize_grads(False)
        shape, hidden = x.shape, x.shape[-1]
        x2, h2 = _flat(x, torch.float32), _flat(h, torch.float16)
        n_tok, dev = x2.shape[0], x.device
        inter = group.shapes[GATE][0]
        half = dict(dtype=torch.float16, device=dev)
        # s1 = x + h, n1 = norm1(s1)
        stage[0] = "addnorm"
        s1 = torch.empty_like(x2)
        n1 = torch.empty(n_tok, hidden, **half)
        xhat1 = torch.empty_like(n1)
        rstd1 = torch.empty(n_tok, dtype=torch.float32, device=dev)
        _rms.launch(x2, norm1.weight, n1, xhat1, rstd1, norm1.variance_epsilon, backward=0, p=h2,
                    q=s1)
        # [gate | up] = n1 [W_gate; W_up]^T, act = silu(gate) * up
        stage[0] = "fused_mlp"
        w_gu = group.span(GATE, DOWN)
        if w_gu is None:
            raise RuntimeError("mlp_block: gate and up are not one span of the layer")
        gu = torch.empty(n_tok, 2 * inter, **half)
        torch.ops.talm.gemm(n1, w_gu, None, 1, gu)
        del w_gu
        act = torch.empty(n_tok, inter, **half)
        torch.ops.talm.swiglu_fwd_rows(gu[:, :inter], gu[:, inter:], act)
        # y = act W_down^T as K-part partials, summed inside the next norm's launch
        # y = act W_down^T (fp16), then s2 = s1 + y, n2 = norm2(s2)
        w_down = group.weight(DOWN)
        y = torch.empty(n_tok, hidden, **half)
        torch.ops.talm.gemm(act, w_down, None, 1, y)
        del act, w_down
        stage[0] = "addnorm"
        s2 = torch.empty_like(x2)
        n2 = torch.empty(n_tok, hidden, **half)
        xhat2 = torch.empty_like(n2)
        rstd2 = torch.empty(n_tok, dtype=torch.float32, device=dev)
        _rms.launch(s1, norm2.weight, n2, xhat2, rstd2, norm2.variance_epsilon, backward=0, p=y,
                    q=s2)
        del y
        ctx.save_for_backward(xhat1, rstd1, gu, xhat2, rstd2, norm1.weight, norm2.weight)
        ctx.group, ctx.shape, ctx.h_dtype = group, shape, h.dtype
        return s2.view(shape), n2.view(shape)

    @staticmethod
    def backward(ctx, d_s2, d_n2):
        xhat1, rstd1, gu, xhat2, rstd2, w1, w2 = ctx.saved_tensors
        group = ctx.group
        n_tok, hidden = xhat1.shape
        inter = gu.shape[1] // 2
        dev = gu.device
        ds2 = None if d_s2 is None else _flat(d_s2, torch.float32)
        dy2 = torch.zeros(n_tok, hidden, dtype=torch.float16, device=dev) if d_n2 is None \
            else _flat(d_n2, torch.float16)
        # the next norm's backward: d s1 through the add (fp32) and dy of the MLP's output (fp16)
        ds1 = torch.empty(n_tok, hidden, dtype=torch.float32, device=dev)
        dy = torch.empty(n_tok, hidden, dtype=torch.float16, device=dev)
        _norm_bwd(dy2, xhat2, w2, rstd2, ds2, ds1, dy)
        del dy2, ds2
        # the MLP's backward down to [dgate | dup], written over gu (FusedMLP's products)
        dact = torch.empty(n_tok, inter, dtype=torch.float16, device=dev)
        w_down_t = group.span_t(DOWN, DOWN + 1)
        if w_down_t is not None:
            torch.ops.talm.gemm(dy, w_down_t, None, 1, dact)
        else:
            torch.ops.talm.gemm(dy, group.weight(DOWN), None, 0, dact)
        del w_down_t, dy
        gate, up = gu[:, :inter], gu[:, inter:]
        torch.ops.talm.swiglu_bwd_rows(dact, gate, up, gate, up)
        del dact
        # dn1 = [dgate | dup] [W_gate; W_up], summed inside the post-attention norm's backward
        dx = torch.empty(n_tok, hidden, dtype=torch.float32, device=dev)
        dh = torch.empty(n_tok, hidden, dtype=torch.float16, device=dev)
        part = _input_grad_partials(group, gu, n_tok, hidden)
        if part is not None and "addnorm" not in DISABLED:
            try:
                torch.ops.talm.splitk_rmsnorm_bwd(part, xhat1, rstd1, w1, ds1, dx, dh)
                RAN["addnorm"] += 1
                return dx.view(ctx.shape), dh.view(ctx.shape).to(ctx.h_dtype), None, None, None, None
            except Exception as exc:  # noqa: BLE001 - state.py convention
                if not fallback("addnorm", exc):
                    raise
        if part is not None:  # the partials summed in part order, then the norm's backward
            dn1 = part[0].clone()
            for k in range(1, part.shape[0]):
                dn1 += part[k]
            dn1 = dn1.to(torch.float16)
        else:
            dn1 = torch.empty(n_tok, hidden, dtype=torch.float16, device=dev)
            fused_mlp.input_grad(group, gu, dn1)
        del part, gu
        _norm_bwd(dn1, xhat1, w1, rstd1, ds1, dx, dh)
        return dx.view(ctx.shape), dh.view(ctx.shape).to(ctx.h_dtype), None, None, None, None


def mlp_block(layer, x, h, follower):
    """(s2, n2) of the layer's MLP half as one `MlpBlock` node when it applies: x the fp32
    residual stream, h the attention's fp16 output of x's shape, both norms on the kernel with
    fp16 outputs, rows of at most MAX_WIDTH columns, the MLP a packed layer group in FusedMLP's
    default mode (`fused_mlp.mlp_plan`) whose gate|up input gradient can be left as K-part
    partials (the NF4 dequant-GEMM, or the split-K GEMM); else None (the caller runs the separate
    nodes)."""
    if not ENABLED or "mlp_block" in DISABLED or "addnorm" in DISABLED or "splitk" in DISABLED \
            or not fused_mlp.SPLITK:
        return None
    norm1 = layer.post_attention_layernorm
    if not (x.is_cuda and h.is_cuda and x.dtype == torch.float32 and h.dtype == torch.float16
            and h.shape == x.shape and x.shape[-1] % 8 == 0 and x.shape[-1] <= MAX_WIDTH
            and _rms._kernel_takes(norm1, x) and _rms._kernel_takes(follower, x)
            and _rms._target_dtype(x) == torch.float16):
        return None
    if "swiglu_inplace" not in ON or ("mlp_save_up" in ON and "mlp_save_up" not in DISABLED):
        return None
    group = fused_mlp.mlp_plan(layer.mlp, h)
    if group is None:
        return None
    inter = group.shapes[GATE][0]
    if inter < fused_mlp.SPLITK_MIN_K or inter % 8:
        return None
    stage = ["addnorm"]
    try:
        out = MlpBlock.apply(x, h, group, norm1, follower, stage)
    except Exception as exc:  # noqa: BLE001 - state.py convention
        if not fallback(stage[0], exc):
            raise
        FELL_BACK["mlp_block"] += 1
        return None
    RAN["mlp_block"] += 1
    RAN["fused_mlp"] += 1
    RAN["addnorm"] += 2
    return out
