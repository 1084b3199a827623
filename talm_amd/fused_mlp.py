"""The decoder MLP down(silu(gate(x)) * up(x)) on a packed layer group as ONE autograd node
(the reference's FusedMLP, solution/fused_proj.py:241-287).

gate and up are adjacent projections of the layer buffer, so [W_gate; W_up] is one [2I, H]
view, and their outputs are the two halves of one [N, 2I] buffer:
  forward   gu = x [W_gate; W_up]^T            (one GEMM: gu[:, :I] = gate, gu[:, I:] = up)
            act = silu(gu[:, :I]) * gu[:, I:]  (talm_swiglu_fwd_rows)
            y = act W_down^T                   (hipBLASLt)
  backward  dact = dy W_down
            dgate, dup over gu's halves        (talm_swiglu_bwd_rows, in place)
            dx = [dgate | dup] [W_gate; W_up]  (one GEMM reducing over 2I)
One node instead of four (three GroupLinear nodes and the SwiGLU node), no separate add of the
gate and up input gradients.

Save-up mode (`save_up=True`, the opt-in node of mlp_save_up.py): the node keeps x [N, H] and up
[N, I] for its backward instead of gate|up [N, 2I] (at H = 1536, I = 8960: 10496 instead of 17920
fp16 values per token and layer). The forward computes gate and up as two products into two
buffers, writes the activation over gate (which is then freed with the forward) and keeps up.
The backward recomputes gate into the left half of a fresh [N, 2I] buffer, x W_gate^T on the
layer's NF4 codes (talm_nf4_gemm: the backward's transposed buffer leaves gate|up out, so no
fp16 gate weight exists then), runs the SwiGLU backward from that gate and the kept up into the
buffer's two halves (dgate | dup), and continues exactly as the default mode: one input-gradient
product over both halves. The backward's dx product reads [W_gate; W_up] as NF4 codes
(talm_nf4_gemm, dequantized inside the GEMM) while the layer group serves that block that way
(qgroup.W4_BLOCKS). hipBLASLt's heuristic choice for the 2I-deep input gradient is
about twice as slow as two I-deep products; the measured solution table (gemm_tuning.py) names
one about 15% faster than the two products together. Same products with fp32 accumulation as
the per-projection path. Once "qgroup" is off (the weights come projection by projection) the
backward takes two products.
"""

import os

import torch

from . import _ops
from .engaged import FELL_BACK, ON, RAN
from .state import DISABLED, fallback

GATE, UP, DOWN = 4, 5, 6
ENABLED = os.environ.get("SOLUTION_DISABLE_FUSED_MLP") != "1"
# the long-reduction input gradient on the transposed gate|up weight (K >= SPLITK_MIN_K), when it
# does not run on the NF4 codes, on this package's split-K MFMA GEMM instead of hipBLASLt
SPLITK = os.environ.get("SOLUTION_DISABLE_SPLITK") != "1"
SPLITK_MIN_K = 4096


def _linear(a, w, out):
    """out = a w^T (fp16, both k-contiguous): split-K MFMA GEMM for long reductions, else
    hipBLASLt."""
    if SPLITK and a.shape[1] >= SPLITK_MIN_K and "splitk" not in DISABLED:
        try:
            ws = torch.empty(_ops.gemm_splitk_workspace_bytes(a.shape[0], w.shape[0], a.shape[1]),
                             dtype=torch.uint8, device=a.device)
            torch.ops.talm.gemm_splitk(a, w, out, ws)
            RAN["splitk"] += 1
            return
        except Exception as exc:  # noqa: BLE001 - state.py convention
            if not fallback("splitk", exc):
                raise
    torch.ops.talm.gemm(a, w, None, 1, out)


class FusedMLP(torch.autograd.Function):
    @staticmethod
    def forward(ctx, x, group, save_up=False):
        hidden = x.shape[-1]
        x2 = x.reshape(-1, hidden)
        if x2.stride(1) != 1:
            x2 = x2.contiguous()
        n_tok = x2.shape[0]
        inter = group.shapes[GATE][0]
        if save_up:
            # gate and up in two buffers: the backward keeps x and up, gate dies with the forward
            gate = torch.empty(n_tok, inter, dtype=torch.float16, device=x.device)
            up = torch.empty(n_tok, inter, dtype=torch.float16, device=x.device)
            torch.ops.talm.gemm(x2, group.weight(GATE), None, 1, gate)
            torch.ops.talm.gemm(x2, group.weight(UP), None, 1, up)
            act = gate  # the activation is written over gate (each element read before written)
            torch.ops.talm.swiglu_fwd_rows(gate, up, act)
            ctx.save_for_backward(x2, up)
        else:
            w_gu = group.span(GATE, DOWN)
            if w_gu is None:
                raise RuntimeError("fused_mlp: gate and up are not one span of the layer")
            # [gate | up] = x [W_gate; W_up]^T: one GEMM into the two halves of one buffer
            gu = torch.empty(n_tok, 2 * inter, dtype=torch.float16, device=x.device)
            torch.ops.talm.gemm(x2, w_gu, None, 1, gu)
            del w_gu
            act = torch.empty(n_tok, inter, dtype=torch.float16, device=x.device)
            torch.ops.talm.swiglu_fwd_rows(gu[:, :inter], gu[:, inter:], act)
            ctx.save_for_backward(gu)
        # the down projection on hipBLASLt: at ~1300 tokens its one fp16 output beats the split-K
        # GEMM's seven fp32 K-part partials (56 MB written and read back)
        w_down = group.weight(DOWN)
        y = torch.empty(n_tok, hidden, dtype=torch.float16, device=x.device)
        torch.ops.talm.gemm(act, w_down, None, 1, y)
        del act, w_down
        ctx.group, ctx.x_shape, ctx.save_up = group, x.shape, bool(save_up)
        return y.view(*x.shape[:-1], hidden)

    @staticmethod
    def backward(ctx, grad_out):
        group = ctx.group
        if ctx.save_up:
            x2, up_kept = ctx.saved_tensors
            n_tok, inter = up_kept.shape
        else:
            (gu,) = ctx.saved_tensors
            n_tok, inter = gu.shape[0], gu.shape[1] // 2
        hidden = ctx.x_shape[-1]
        dy = grad_out.reshape(n_tok, hidden)
        if dy.dtype != torch.float16:
            dy = dy.to(torch.float16)
        if dy.stride(1) != 1:
            dy = dy.contiguous()
        # the input gradients multiply by W; the group's W^T blocks [in, out] let them run in the
        # forward's product form (x W^T), which hipBLASLt runs faster at these shapes
        dact = torch.empty(n_tok, inter, dtype=torch.float16, device=dy.device)
        w_down_t = group.span_t(DOWN, DOWN + 1)
        if w_down_t is not None:
            torch.ops.talm.gemm(dy, w_down_t, None, 1, dact)
        else:
            torch.ops.talm.gemm(dy, group.weight(DOWN), None, 0, dact)
        del w_down_t
        if ctx.save_up:
            # gate recomputed into the left half of the buffer the input-gradient product reads
            gu = torch.empty(n_tok, 2 * inter, dtype=torch.float16, device=dy.device)
            gate, up = gu[:, :inter], gu[:, inter:]
            _recompute_gate(group, x2, gate)
            torch.ops.talm.swiglu_bwd_rows(dact, gate, up_kept, gate, up)
            del up_kept
        else:
            gate, up = gu[:, :inter], gu[:, inter:]
            torch.ops.talm.swiglu_bwd_rows(dact, gate, up, gate, up)
        del dact
        dx = torch.empty(n_tok, hidden, dtype=torch.float16, device=dy.device)
        input_grad(group, gu, dx)
        return dx.view(ctx.x_shape), None, None


def input_grad(group, gu, dx):
    """dx = [dgate | dup] [W_gate; W_up] (fp16 [N, H]) from gu holding dgate | dup: on the NF4
    codes while the layer group serves gate|up that way (the transposed buffer leaves them out),
    else one GEMM on the transposed or the row-major weight, else ("qgroup" off) the
    projections' own weights."""
    n_tok, hidden, inter = gu.shape[0], dx.shape[1], gu.shape[1] // 2
    if (GATE, UP) in group.w4_blocks():
        try:
            group.nf4_gemm(gu, GATE, DOWN, True, dx)
            RAN["w4a16"] += 1
            return
        except Exception as exc:  # noqa: BLE001 - state.py convention
            if not fallback("w4a16", exc):
                raise
    w_gu_t = group.span_t(GATE, DOWN)
    w_gu = None if w_gu_t is not None else group.span(GATE, DOWN)
    if w_gu_t is not None:
        # dx = [dgate | dup] [W_gate; W_up] = gu ([W_gate; W_up]^T)^T: one GEMM
        _linear(gu, w_gu_t, dx)
    elif w_gu is not None:
        # dx = [dgate | dup] [W_gate; W_up]: one GEMM with the reduction over both halves
        torch.ops.talm.gemm(gu, w_gu, None, 0, dx)
    else:  # "qgroup" is off: the projections' own weights
        gate, up = gu[:, :inter], gu[:, inter:]
        w_gate, w_up = group.weight(GATE), group.weight(UP)
        torch.ops.talm.gemm(gate, w_gate, None, 0, dx)
        # dx += dup W_up in the column-major BLAS form: dx^T [H x N] += W_up^T [H x I] dup^T
        torch.ops.talm.gemm_ex(w_up, 0, up, 0, dx, hidden, n_tok, inter, hidden, 2 * inter,
                               hidden, 1)


def _recompute_gate(group, x2, gate):
    """gate = x W_gate^T into `gate` (a row-strided view) in the backward: on the NF4 codes while
    the transposed buffer leaves gate|up out (no fp16 gate weight exists then), else on gate's
    weights dequantized alone (one launch; the transposed buffer stays resident)."""
    if (GATE, UP) in group.w4_blocks():
        try:
            group.nf4_gemm(x2, GATE, UP, False, gate)
            RAN["w4a16"] += 1
            return
        except Exception as exc:  # noqa: BLE001 - state.py convention
            if not fallback("w4a16", exc):
                raise
    if "qgroup" in DISABLED:
        w_gate = group.weight(GATE)
    else:
        w_gate = group.dequantize(GATE, UP).view(group.shapes[GATE])
    torch.ops.talm.gemm(x2, w_gate, None, 1, gate)


def mlp_plan(mlp, x, component="fused_mlp"):
    """The layer group when gate_proj, up_proj and down_proj are projections 4, 5, 6 of one
    packed group (no LoRA, no bias, no hooks) and `component` ("fused_mlp", or "mlp_save_up" for
    the save-up node) is on."""
    from .fused_proj import _no_hooks, _packed

    if component == "fused_mlp" and not ENABLED:
        return None
    if not (x.is_cuda and x.dtype == torch.float16 and x.dim() >= 2) \
            or component in DISABLED or "qgroup" in DISABLED or "swiglu" in DISABLED:
        return None
    mods = [getattr(mlp, name, None) for name in ("gate_proj", "up_proj", "down_proj")]
    if any(m is None for m in mods):
        return None
    tags = [_packed(m) for m in mods]
    if any(t is None for t in tags) or tags[0][1] != GATE or tags[1][1] != UP or tags[2][1] != DOWN:
        return None
    group = tags[0][0]
    if tags[1][0] is not group or tags[2][0] is not group or group.shapes[GATE][1] != x.shape[-1]:
        return None
    if any(group.biases[i] is not None for i in (GATE, UP, DOWN)):
        return None
    if not _no_hooks(mods + [mlp]):
        return None
    return group


def fused_mlp_forward(mlp, x):
    """FusedMLP when `mlp_plan` takes the layer, else None (the caller's own path runs). The
    node runs in save-up mode when the save-up MLP is installed (mlp_save_up.py) and the call
    records autograd; otherwise in its default mode, which belongs to the in-place MLP patch
    (swiglu_inplace.py)."""
    save_up = ("mlp_save_up" in ON and "mlp_save_up" not in DISABLED
               and torch.is_grad_enabled() and x.requires_grad)
    if not save_up and "swiglu_inplace" not in ON:
        return None
    component = "mlp_save_up" if save_up else "fused_mlp"
    group = mlp_plan(mlp, x, component)
    if group is None:
        FELL_BACK[component] += 1
        return None
    try:
        y = FusedMLP.apply(x, group, save_up)
    except Exception as exc:  # noqa: BLE001 - state.py convention
        if not fallback(component, exc):
            raise
        FELL_BACK[component] += 1
        return None
    RAN[component] += 1
    return y
