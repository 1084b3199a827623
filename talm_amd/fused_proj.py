"""q|k|v of a decoder layer as one projection node on the packed 4-bit weights (qgroup.py).

Mirrors solution/fused_proj.py:88-218: the layer group dequantizes q, k, v, o, gate, up, down
into one buffer per pass, so [Wq; Wk; Wv] ([1536 + 256 + 256, 1536]) is one row-major matrix:
[q|k|v] = x [Wq; Wk; Wv]^T + [bq|bk|bv] is ONE GEMM, the LoRA adapters of q_proj and v_proj are
added with PEFT's ops in PEFT's order (lora.py), v is returned as a fresh tensor and q, k as column
views. Backward: dX = [dq|dk|dv] [Wq; Wk; Wv] in one GEMM (K = 2048) plus the adapters' input
gradients, and the adapters' weight gradients.

On MI355X the forward runs as one launch when it can (`_mfma_ok`): talm_qkv_lora_fwd_down, an
fp16 MFMA GEMM x W^T + b whose adapter tiles also accumulate t = x A^T during the product and add
s t B^T after it, and which rotates q and k in its epilogue (qkv.hip); with
SOLUTION_QKV_SEPARATE_DOWN=1 the two launches it replaces, talm_lora_down (t) and
talm_qkv_lora_fwd ([x | s t] [W | B]^T + b); otherwise the ops below.
SOLUTION_DISABLE_QKV_MFMA=1 keeps the ops.

MI355X addition: with `rope=(cos, sin)` the node also applies the rotary embedding to q and k IN
PLACE on its own output (the rope kernel reads each rotation pair before writing it), and in the
backward rotates dq and dk back in place inside the concatenated gradient it builds for the dX
GEMM anyway: no RoPE node, no new q/k tensors, no strided gradient copies. This is safe because
the node keeps only x for its backward (the reference notes this: q and k are views of the
node's output that nothing else reads before the attention).
"""

import os

import torch
import torch.nn.functional as F

from .engaged import FELL_BACK, ON, RAN
from .lora import _power_of_two, _to_half, adapters_t, lora_plan
from .rope import rope_
from .state import DISABLED, fallback

Q, K, V, O, GATE, UP, DOWN = range(7)
QKV_MFMA = os.environ.get("SOLUTION_DISABLE_QKV_MFMA") != "1"
QKV_FUSED_DOWN = os.environ.get("SOLUTION_QKV_SEPARATE_DOWN") != "1"
COUNTS = {"attn": 0, "attn_fallback": 0}

# Adapter weight gradients written straight into buffers that a caller owns (the graphed step):
# id(parameter) -> (parameter, fp32 buffer of its shape). A q|k|v node then writes the weight's
# gradient into its buffer, overwriting it (every adapter weight gets exactly one contribution
# per backward), and returns None for that input, so autograd adds nothing into .grad and the
# buffer needs no clearing first. GRAD_WRITTEN collects the ids written, for the caller to check;
# GRAD_TWICE the ids written more than once (two nodes feeding one weight: the second write would
# drop the first contribution, so the caller must not rely on direct delivery).
GRAD_INTO = {}
GRAD_WRITTEN = set()
GRAD_TWICE = set()


def _grad_targets(params):
    """The registered buffer of each parameter (None where there is none)."""
    if not GRAD_INTO:
        return [None] * len(params)
    out = []
    for p in params:
        hit = GRAD_INTO.get(id(p))
        out.append(hit[1] if hit is not None and hit[0] is p else None)
    return out


def _deliver(lora_grads, params):
    """Gradients for the node's adapter inputs: those with a registered buffer go into it
    (None is returned for them), the others to autograd."""
    if not GRAD_INTO:
        return lora_grads
    out = list(lora_grads)
    for i, (g, buf) in enumerate(zip(lora_grads, _grad_targets(params))):
        if g is None or buf is None:
            continue
        if id(params[i]) in GRAD_WRITTEN:
            GRAD_TWICE.add(id(params[i]))
        if g is not buf:
            buf.copy_(g)
        GRAD_WRITTEN.add(id(params[i]))
        out[i] = None
    return out


class FusedProjections(torch.autograd.Function):
    """y_i = x W_i^T + b_i (+ scaling_i * B_i(A_i(dropout_i(x)))) for the adjacent packed
    projections first .. last - 1 of a LayerGroup, the base part as one GEMM; optionally the
    rotary embedding of the first two outputs (q, k) in place."""

    @staticmethod
    def forward(ctx, x, group, first, last, adapters, compact, rope, head_dim, *lora_weights):
        states = []
        try:
            return FusedProjections._forward(ctx, x, group, first, last, adapters, compact, rope,
                                             head_dim, lora_weights, states)
        except Exception:
            drawn = [state for state in states if state is not None]
            if drawn:
                torch.cuda.set_rng_state(drawn[0], x.device)
            raise

    @staticmethod
    def _forward(ctx, x, group, first, last, adapters, compact, rope, head_dim, lora_weights,
                 states):
        ctx.lora_params = tuple(lora_weights)
        x2 = x.reshape(-1, x.shape[-1])
        n_tok = x2.shape[0]
        sizes = [group.shapes[i][0] for i in range(first, last)]
        bounds = [0]
        for size in sizes:
            bounds.append(bounds[-1] + size)
        weight = group.span(first, last)
        bias = group.span_bias(first, last)
        halves = [_to_half(lora_weights[2 * k], lora_weights[2 * k + 1])
                  for k in range(len(adapters))]
        mfma = None
        if _mfma_ok(x2, weight, bias, bounds, adapters, halves, rope, head_dim):
            try:
                mfma = _mfma_forward(x2, weight, bias, bounds, adapters, halves, rope)
            except Exception as exc:  # noqa: BLE001 - state.py convention
                if not fallback("qkv_mfma", exc):
                    raise
        if mfma is not None:
            out, t = mfma
            del weight
            saved = [x2]
            for k in range(len(adapters)):
                states.append(None)
                saved += [t[:, 16 * k:16 * (k + 1)], halves[k][0], halves[k][1]]
            if rope is not None:
                saved += list(rope)
                RAN["rope"] += 1
            RAN["qkv_mfma"] += 1
            ctx.mfma = True
            # for the backward's dX (forward runs with grad mode off: ask the node's inputs)
            ctx.a_t = adapters_t([lora_weights[2 * k] for k in range(len(adapters))]) \
                if adapters and ctx.needs_input_grad[0] else None
            return FusedProjections._finish(ctx, x, out, sizes, bounds, compact, saved, group,
                                            first, last, adapters, states, rope, head_dim)
        ctx.mfma = False
        if weight is None:  # "qgroup" is off: the projections' own dequantization, stacked
            weight = torch.cat([group.weight(i) for i in range(first, last)], 0)
        out = F.linear(x2, weight, bias)
        del weight
        saved = [x2]
        for k, (seg, scaling, p) in enumerate(adapters):
            a16, b16 = halves[k]
            state = None
            if p > 0:
                state = torch.cuda.get_rng_state(x.device)
                xd = torch.native_dropout(x2, p, True)[0]
            else:
                xd = x2
            t = torch.mm(xd, a16.t())
            del xd
            branch = torch.mm(t, b16.t())
            base = out[:, bounds[seg]:bounds[seg + 1]]
            alpha = scaling
            if not _power_of_two(scaling):
                branch.mul_(scaling)
                alpha = 1
            base.add_(branch, alpha=alpha)
            states.append(state)
            saved += [t, a16, b16]
        if rope is not None:
            cos, sin = rope
            q = out[:, bounds[0]:bounds[1]].view(n_tok, -1, head_dim)
            k = out[:, bounds[1]:bounds[2]].view(n_tok, -1, head_dim)
            rope_(q, k, cos, sin, backward=False)
            RAN["rope"] += 1
            saved += [cos, sin]
        return FusedProjections._finish(ctx, x, out, sizes, bounds, compact, saved, group, first,
                                        last, adapters, states, rope, head_dim)

    @staticmethod
    def _finish(ctx, x, out, sizes, bounds, compact, saved, group, first, last, adapters, states,
                rope, head_dim):
        results = [None] * len(sizes)
        for seg in range(len(sizes)):
            base = out[:, bounds[seg]:bounds[seg + 1]]
            results[seg] = base.contiguous() if seg in compact else base
        ctx.save_for_backward(*saved)
        ctx.group, ctx.first, ctx.last = group, first, last
        ctx.adapters, ctx.states, ctx.sizes = adapters, states, sizes
        ctx.has_rope, ctx.head_dim = rope is not None, head_dim
        ctx.x_shape = x.shape
        lead = x.shape[:-1]
        return tuple(r.view(*lead, r.shape[1]) for r in results)

    @staticmethod
    def backward(ctx, *grads):
        if ctx.mfma and _mfma_bwd_ok(ctx, grads):
            try:
                result = _mfma_backward(ctx, grads)
            except Exception as exc:  # noqa: BLE001 - state.py convention
                if not fallback("qkv_mfma", exc):
                    raise
            else:
                if result is not None:
                    RAN["qkv_mfma_bwd"] += 1
                    return result
        x2, *rest = ctx.saved_tensors
        n_tok = x2.shape[0]
        group = ctx.group
        if ctx.has_rope:
            cos, sin = rest[-2:]
            rest = rest[:-2]
        bounds = [0]
        for size in ctx.sizes:
            bounds.append(bounds[-1] + size)
        # one [N, sum of out] fp16 gradient: the dX GEMM's operand and the adapters' dy
        dcat = torch.empty(n_tok, bounds[-1], dtype=torch.float16, device=x2.device)
        for i, grad in enumerate(grads):
            part = dcat[:, bounds[i]:bounds[i + 1]]
            if grad is None:
                part.zero_()
            else:
                part.copy_(grad.reshape(n_tok, -1))
        if ctx.has_rope:
            dq = dcat[:, bounds[0]:bounds[1]].view(n_tok, -1, ctx.head_dim)
            dk = dcat[:, bounds[1]:bounds[2]].view(n_tok, -1, ctx.head_dim)
            rope_(dq, dk, cos, sin, backward=True)
            RAN["rope"] += 1
        dys = [dcat[:, bounds[i]:bounds[i + 1]] for i in range(len(ctx.sizes))]
        dx = None
        if ctx.needs_input_grad[0]:
            weight = group.span(ctx.first, ctx.last)
            if weight is not None:
                dx = torch.mm(dcat, weight)
                del weight
            else:
                for i, dy in enumerate(dys):
                    weight = group.weight(ctx.first + i)
                    if dx is None:
                        dx = torch.mm(dy, weight)
                    else:
                        dx.addmm_(dy, weight)
                    del weight
        lora_grads = []
        for k, (seg, scaling, p) in enumerate(ctx.adapters):
            t, a16, b16 = rest[3 * k:3 * k + 3]
            dy = dys[seg]
            state = ctx.states[k]
            mask = None
            xd = x2
            if state is not None:
                device = x2.device
                current = torch.cuda.get_rng_state(device)
                torch.cuda.set_rng_state(state, device)
                xd, mask = torch.native_dropout(x2, p, True)
                torch.cuda.set_rng_state(current, device)
            g = dy * scaling
            u = torch.mm(g, b16)
            if dx is not None:
                dx_lora = torch.mm(u, a16)
                if mask is not None:
                    dx_lora = torch.ops.aten.native_dropout_backward(dx_lora, mask, 1.0 / (1.0 - p))
                dx.add_(dx_lora)
                del dx_lora
            index = 8 + 2 * k
            lora_grads.append(torch.mm(u.t(), xd).float() if ctx.needs_input_grad[index] else None)
            lora_grads.append(torch.mm(g.t(), t).float() if ctx.needs_input_grad[index + 1]
                              else None)
            del xd, mask
        dx = None if dx is None else dx.view(ctx.x_shape)
        return (dx, None, None, None, None, None, None, None,
                *_deliver(lora_grads, ctx.lora_params))


def _mfma_ok(x2, weight, bias, bounds, adapters, halves, rope, head_dim):
    """Whether the q|k|v node's forward can run as talm_lora_down + talm_qkv_lora_fwd: fp16
    operands with unit column strides and 16-byte rows, at most two adapters of rank 16 without
    dropout on whole 128-column tiles, the rotary embedding (if any) on 128-wide heads."""
    if not QKV_MFMA or "qkv_mfma" in DISABLED or weight is None or len(adapters) > 2:
        return False
    n_out, size = bounds[-1], x2.shape[1]
    if not (x2.dtype == weight.dtype == torch.float16 and x2.stride(1) == 1
            and weight.stride(1) == 1 and x2.stride(0) % 8 == 0 and weight.stride(0) % 8 == 0
            and x2.data_ptr() % 16 == 0 and weight.data_ptr() % 16 == 0
            and tuple(weight.shape) == (n_out, size) and size % 8 == 0):
        return False
    if bias is not None and not (bias.dtype == torch.float16 and bias.is_contiguous()):
        return False
    if adapters and size % 32:
        return False
    for (seg, _scaling, p), (a16, b16) in zip(adapters, halves):
        lo, hi = bounds[seg], bounds[seg + 1]
        if p > 0 or tuple(a16.shape) != (16, size) or tuple(b16.shape) != (hi - lo, 16) \
                or not (a16.is_contiguous() and b16.is_contiguous()) \
                or lo % 128 or (hi % 128 and hi != n_out):
            return False
    if rope is not None and (head_dim != 128 or len(bounds) < 3 or bounds[2] % 128):
        return False
    return True


def _mfma_forward(x2, weight, bias, bounds, adapters, halves, rope):
    """[q|k|v] (+ LoRA, + RoPE on q and k) on MFMA: returns the [N, n_out] output and the
    adapters' t = x A^T ([N, 16 per adapter], what the backward keeps)."""
    n, n_out = x2.shape[0], bounds[-1]
    t = ts = None
    a1 = halves[1][0] if len(adapters) > 1 else None
    s1 = adapters[1][1] if len(adapters) > 1 else 0.0
    if adapters:
        t = torch.empty(n, 16 * len(adapters), dtype=torch.float16, device=x2.device)
    segs = [(bounds[seg], bounds[seg + 1]) for seg, _s, _p in adapters] + [(0, 0)] * 2
    bs = [b16 for _a, b16 in halves] + [None] * 2
    cos, sin = rope if rope is not None else (None, None)
    out = torch.empty(n, n_out, dtype=torch.float16, device=x2.device)
    rope_cols = bounds[2] if rope is not None else 0
    if QKV_FUSED_DOWN:
        a0 = halves[0][0] if adapters else None
        s0 = adapters[0][1] if adapters else 0.0
        torch.ops.talm.qkv_lora_fwd_down(x2, weight, bias, a0, a1, s0, s1, bs[0], segs[0][0],
                                         segs[0][1], bs[1], segs[1][0], segs[1][1], cos, sin,
                                         rope_cols, t, out)
        return out, t
    if adapters:
        ts = torch.empty_like(t)
        size = x2.shape[1]
        torch.ops.talm.lora_down(x2, halves[0][0], a1, size, size, 0, 0, 0, adapters[0][1], s1,
                                 t, ts)
    torch.ops.talm.qkv_lora_fwd(x2, weight, bias, ts, bs[0], segs[0][0], segs[0][1], bs[1],
                                segs[1][0], segs[1][1], cos, sin, rope_cols, out)
    return out, t


def _mfma_bwd_ok(ctx, grads):
    """The MFMA backward takes the q|k|v node whose forward ran on MFMA (its saved tensors have
    that layout) when every output has an fp16 gradient with unit column stride."""
    if not QKV_MFMA or "qkv_mfma" in DISABLED or len(grads) != len(ctx.sizes):
        return False
    for grad, size in zip(grads, ctx.sizes):
        if grad is None or grad.dtype != torch.float16 or grad.shape[-1] != size \
                or grad.stride(-1) != 1 or grad.data_ptr() % 16 or size % 8:
            return False
    if any(ctx.sizes[seg] % 32 for seg, _s, _p in ctx.adapters):
        return False
    # q|k|v (three outputs, RoPE-back in the concatenation), or one projection without RoPE
    # whose gradient is the GEMM operand as it is
    return len(ctx.sizes) == 3 or (len(ctx.sizes) == 1 and not ctx.has_rope)


def _mfma_backward(ctx, grads):
    """dX = [dq|dk|dv] W + u A in one MFMA GEMM (talm_qkv_lora_bwd_dx) after talm_qkv_bwd_prep
    (RoPE-back, concatenation) and talm_lora_down (u = (scaling dy) B per adapter); the
    adapters' dA = u^T x and dB = g^T t as in the reference (solution/fused_proj.py:160-216).
    Returns None (the caller runs the ops) when the layer's weight is not in the group's buffer."""
    x2, *rest = ctx.saved_tensors
    group = ctx.group
    cos = sin = None
    if ctx.has_rope:
        cos, sin = rest[-2:]
        rest = rest[:-2]
    weight = weight_t = None
    if ctx.needs_input_grad[0]:
        weight_t = group.span_t(ctx.first, ctx.last)
        weight = None if weight_t is not None else group.span(ctx.first, ctx.last)
        if weight is None and weight_t is None:
            return None
    return _mfma_backward_ops(ctx, grads, x2, rest, cos, sin, weight, weight_t)


def _mfma_backward_ops(ctx, grads, x2, rest, cos, sin, weight, weight_t=None):
    wanted = [ctx.needs_input_grad[8 + i] for i in range(2 * len(ctx.adapters))]
    dx, lora_grads = _mfma_backward_core(grads, x2, rest, cos, sin, weight, ctx.sizes,
                                         ctx.adapters, ctx.has_rope, wanted,
                                         getattr(ctx, "a_t", None),
                                         _grad_targets(ctx.lora_params), weight_t)
    dx = None if dx is None else dx.view(ctx.x_shape)
    return (dx, None, None, None, None, None, None, None, *_deliver(lora_grads, ctx.lora_params))


def _mfma_backward_core(grads, x2, rest, cos, sin, weight, sizes, adapters, has_rope, wanted,
                        a_t=None, outs=None, weight_t=None):
    """dX [N, H] (None without `weight`) and the adapters' [dA, dB, ...] of the q|k|v node from
    the gradients of its q, k, v outputs (fp16, unit column stride); `rest` holds (t, A16, B16)
    per adapter, `wanted` which adapter gradients to form, `a_t` the adapters' A^T side by side
    ([H, 16 per adapter] fp16; formed here when None); `outs` optional fp32 buffers for the
    adapter gradients (written in place and returned as themselves); `weight_t` the layer
    group's W^T [H, >= sum of out] when it holds one (then `weight` is not needed)."""
    n_tok, size = x2.shape
    bounds = [0]
    for s_ in sizes:
        bounds.append(bounds[-1] + s_)
    dys = [g.reshape(n_tok, -1) for g in grads]
    if len(dys) == 1:
        dcat = dys[0]
        if dcat.stride(0) % 8 or dcat.data_ptr() % 16:
            dcat = dcat.contiguous()
    else:
        dcat = torch.empty(n_tok, bounds[-1], dtype=torch.float16, device=x2.device)
        torch.ops.talm.qkv_bwd_prep(dys[0], dys[1], dys[2], cos, sin, dcat)
    if has_rope:
        RAN["rope"] += 1
    halves = [rest[3 * k:3 * k + 3] for k in range(len(adapters))]  # (t, a16, b16)
    u = None
    if adapters:
        # u_g = (scaling_g dy_g) B_g, B_g read as stored ([segment, 16], k-major)
        t_tmp = torch.empty(n_tok, 16 * len(adapters), dtype=torch.float16, device=x2.device)
        u = torch.empty_like(t_tmp)
        lo = [bounds[seg] for seg, _s, _p in adapters] + [0]
        ks = [bounds[seg + 1] - bounds[seg] for seg, _s, _p in adapters] + [0]
        scal = [s_ for _seg, s_, _p in adapters] + [0.0]
        b1 = halves[1][2] if len(adapters) > 1 else None
        torch.ops.talm.lora_down(dcat, halves[0][2], b1, ks[0], ks[1], lo[0], lo[1], 1, scal[0],
                                 scal[1], t_tmp, u)
    dx = None
    if weight_t is None and weight is not None:
        from .fused_head import transpose_weight_exact

        weight_t = transpose_weight_exact(weight)
        del weight
    if weight_t is not None:
        if a_t is None and adapters:
            a_t = torch.cat([a16 for _t, a16, _b in halves], 0).t().contiguous()
        dx = torch.empty(n_tok, size, dtype=torch.float16, device=x2.device)
        torch.ops.talm.qkv_lora_bwd_dx(dcat, weight_t, u, a_t, dx)
        del weight_t
    lora_grads = [None] * (2 * len(adapters))
    if adapters and any(wanted):
        # all adapters' dA, dB in fp32 in one call (t of each adapter is a column view of one
        # [N, 16 * adapters] buffer when the forward ran on MFMA)
        t_all = halves[0][0]
        if len(adapters) > 1 and (halves[1][0].data_ptr() != t_all.data_ptr() + 32
                                  or halves[1][0].stride() != t_all.stride()):
            return dx, _weight_grads_ops(dcat, u, x2, halves, bounds, adapters, wanted)
        t_cat = torch.as_strided(t_all, (n_tok, 16 * len(adapters)), (t_all.stride(0), 1))
        segs = [(bounds[seg], bounds[seg + 1] - bounds[seg], s_) for seg, s_, _p in adapters]
        shapes = [(16, size) if i % 2 == 0 else (segs[i // 2][1], 16)
                  for i in range(2 * len(adapters))]
        outs = outs or [None] * len(shapes)
        grads_ = [o if o is not None and tuple(o.shape) == shp and o.dtype == torch.float32
                  and o.is_contiguous() else torch.empty(shp, dtype=torch.float32, device=x2.device)
                  for o, shp in zip(outs, shapes)]
        pad = segs + [(0, 0, 0.0)]
        ws = torch.empty(_ops_ws(n_tok, size, pad[0][1], pad[1][1]), dtype=torch.uint8,
                         device=x2.device)
        torch.ops.talm.lora_wgrad(x2, dcat, u, t_cat, pad[0][0], pad[0][1], pad[0][2], grads_[0],
                                  grads_[1], pad[1][0], pad[1][1], pad[1][2],
                                  grads_[2] if len(adapters) > 1 else None,
                                  grads_[3] if len(adapters) > 1 else None, ws)
        lora_grads = [g if w else None for g, w in zip(grads_, wanted)]
    return dx, lora_grads


def _ops_ws(n_tok, size, seg0, seg1):
    from . import _ops

    return _ops.lora_wgrad_workspace_bytes(n_tok, size, seg0, seg1)


def _weight_grads_ops(dcat, u, x2, halves, bounds, adapters, wanted):
    """The adapters' dA / dB with the reference's ops (when their t are not one buffer)."""
    lora_grads = []
    for k, (seg, scaling, _p) in enumerate(adapters):
        t, _a16, _b16 = halves[k]
        uk = u[:, 16 * k:16 * (k + 1)]
        lora_grads.append(torch.mm(uk.t(), x2).float() if wanted[2 * k] else None)
        dy = dcat[:, bounds[seg]:bounds[seg + 1]]
        lora_grads.append(torch.mm((dy * scaling).t(), t).float() if wanted[2 * k + 1] else None)
    return lora_grads


class _NotApplicable(Exception):
    """The one-node attention block does not take this call (nothing was consumed)."""


class AttentionBlock(torch.autograd.Function):
    """The whole attention half of a decoder layer as ONE node on MFMA: q|k|v (+ LoRA, + RoPE)
    as in FusedProjections, the variable-length causal GQA attention of the packed rows
    (torch.ops.talm.attn_fwd / attn_bwd) and o_proj on the layer group's weight
    (solution/fused_proj.py:88-218 and :382-445, solution/unpad.py:199-294, solution/qgroup.py:
    346-355). One node instead of FusedProjections + VarlenAttention + GroupLinear and the view
    nodes between them: the step is bound by the host's launch rate. Same kernels, same values,
    except that the backward rotates dq / dk back inside the attention backward
    (torch.ops.talm.attn_bwd_rope) from the fp32 sums, one fp16 rounding instead of two, and
    hands the projections' backward that output as it is (no separate rotary pass)."""

    @staticmethod
    def forward(ctx, x, group, adapters, rope, head_dim, n_heads, n_kv, cu, max_len, scale,
                *lora_weights):
        x2 = x.reshape(-1, x.shape[-1])
        n_tok = x2.shape[0]
        sizes = [group.shapes[i][0] for i in (Q, K, V)]
        bounds = [0, sizes[0], sizes[0] + sizes[1], sizes[0] + sizes[1] + sizes[2]]
        weight = group.span(Q, V + 1)
        if weight is None:
            raise _NotApplicable()
        halves = [_to_half(lora_weights[2 * k], lora_weights[2 * k + 1])
                  for k in range(len(adapters))]
        bias = group.span_bias(Q, V + 1)
        if not (_mfma_ok(x2, weight, bias, bounds, adapters, halves, rope, head_dim)
                and sizes[0] == n_heads * head_dim and sizes[1] == sizes[2] == n_kv * head_dim):
            raise _NotApplicable()
        out, t = _mfma_forward(x2, weight, bias, bounds, adapters, halves, rope)
        del weight
        w_o = group.weight(O)
        q = out[:, :bounds[1]].view(n_tok, n_heads, head_dim)
        k = out[:, bounds[1]:bounds[2]].view(n_tok, n_kv, head_dim)
        v = out[:, bounds[2]:].view(n_tok, n_kv, head_dim)
        o = torch.empty(n_tok, n_heads, head_dim, dtype=torch.float16, device=x.device)
        lse = torch.empty(n_heads, n_tok, dtype=torch.float32, device=x.device)
        torch.ops.talm.attn_fwd(q, k, v, cu, max_len, scale, o, lse)
        y = torch.empty(n_tok, w_o.shape[0], dtype=torch.float16, device=x.device)
        torch.ops.talm.gemm(o.view(n_tok, -1), w_o, group.biases[O], 1, y)
        del w_o
        saved = [x2, out, o, lse, cu]
        for k_ in range(len(adapters)):
            saved += [t[:, 16 * k_:16 * (k_ + 1)], halves[k_][0], halves[k_][1]]
        saved += list(rope)
        ctx.save_for_backward(*saved)
        ctx.group, ctx.adapters, ctx.sizes, ctx.bounds = group, adapters, sizes, bounds
        ctx.head_dim, ctx.n_heads, ctx.n_kv = head_dim, n_heads, n_kv
        ctx.max_len, ctx.scale, ctx.x_shape = max_len, scale, x.shape
        ctx.lora_params = tuple(lora_weights)
        # for the backward's dX (forward runs with grad mode off: ask the node's inputs)
        ctx.a_t = adapters_t([lora_weights[2 * k] for k in range(len(adapters))]) \
            if adapters and ctx.needs_input_grad[0] else None
        RAN["qkv_mfma"] += 1
        RAN["rope"] += 1
        RAN["attn_kernel"] += 1
        return y.view(*x.shape[:-1], y.shape[1])

    @staticmethod
    def backward(ctx, grad):
        from . import _ops

        x2, out, o, lse, cu, *rest = ctx.saved_tensors
        cos, sin = rest[-2:]
        rest = rest[:-2]
        group, bounds = ctx.group, ctx.bounds
        n_tok = x2.shape[0]
        dy = grad.reshape(n_tok, -1)
        if dy.dtype != torch.float16:
            dy = dy.to(torch.float16)
        if dy.stride(1) != 1:
            dy = dy.contiguous()
        # d_o = dy W_o: with the group's W_o^T [in, out], in the product form of the forward
        w_o_t = group.span_t(O, O + 1)
        if w_o_t is not None:
            d_o = torch.empty(n_tok, w_o_t.shape[0], dtype=torch.float16, device=x2.device)
            torch.ops.talm.gemm(dy, w_o_t, None, 1, d_o)
        else:
            w_o = group.weight(O)
            d_o = torch.empty(n_tok, w_o.shape[1], dtype=torch.float16, device=x2.device)
            torch.ops.talm.gemm(dy, w_o, None, 0, d_o)
        del w_o_t
        hd, nh, nkv = ctx.head_dim, ctx.n_heads, ctx.n_kv
        q = out[:, :bounds[1]].view(n_tok, nh, hd)
        k = out[:, bounds[1]:bounds[2]].view(n_tok, nkv, hd)
        v = out[:, bounds[2]:].view(n_tok, nkv, hd)
        dqkv = torch.empty(n_tok, bounds[3], dtype=torch.float16, device=x2.device)
        dq = dqkv[:, :bounds[1]]
        dk = dqkv[:, bounds[1]:bounds[2]]
        dv = dqkv[:, bounds[2]:]
        ws = torch.empty(_ops.attn_bwd_workspace_bytes(n_tok, nh), dtype=torch.uint8,
                         device=x2.device)
        views = (dq.view(n_tok, nh, hd), dk.view(n_tok, nkv, hd), dv.view(n_tok, nkv, hd), ws)
        if _rope_rows(cos, sin):
            # the rotary backward in the attention backward's epilogues: dqkv is the q|k|v
            # gradient before the rotation, the operand of the projections' backward as it is
            torch.ops.talm.attn_bwd_rope(q, k, v, o, d_o.view(n_tok, nh, hd), lse, cu,
                                         ctx.max_len, ctx.scale, cos, sin, *views)
            grads = (dqkv,)
        else:
            torch.ops.talm.attn_bwd(q, k, v, o, d_o.view(n_tok, nh, hd), lse, cu, ctx.max_len,
                                    ctx.scale, *views)
            grads = (dq, dk, dv)
        del ws, d_o, views
        weight = weight_t = None
        if ctx.needs_input_grad[0]:
            weight_t = group.span_t(Q, V + 1)
            if weight_t is None:
                weight = group.span(Q, V + 1)
                if weight is None:
                    weight = torch.cat([group.weight(i) for i in (Q, K, V)], 0)
        wanted = [ctx.needs_input_grad[10 + i] for i in range(2 * len(ctx.adapters))]
        dx, lora_grads = _mfma_backward_core(grads, x2, rest, cos, sin, weight,
                                             ctx.sizes, ctx.adapters, True, wanted, ctx.a_t,
                                             _grad_targets(ctx.lora_params), weight_t)
        RAN["attn_kernel_bwd"] += 1
        RAN["qkv_mfma_bwd"] += 1
        dx = None if dx is None else dx.view(ctx.x_shape)
        return (dx, None, None, None, None, None, None, None, None, None,
                *_deliver(lora_grads, ctx.lora_params))


def _rope_rows(cos, sin):
    """cos / sin in the row layout the attention backward's fused rotation reads: fp32 [N, >= 128]
    of one row stride, a multiple of 4 elements, 16-byte aligned."""
    return all(t.dim() == 2 and t.dtype == torch.float32 and t.stride(1) == 1
               and t.shape[1] >= 128 and t.stride(0) >= 128 and t.stride(0) % 4 == 0
               and t.data_ptr() % 16 == 0
               for t in (cos, sin)) and cos.stride(0) == sin.stride(0)


_HOOK_DICTS = ("_forward_hooks", "_forward_pre_hooks", "_backward_hooks", "_backward_pre_hooks")


def _no_hooks(modules):
    from torch.nn.modules import module as nn_module

    for name in ("_global_forward_hooks", "_global_forward_pre_hooks", "_global_backward_hooks",
                 "_global_backward_pre_hooks"):
        if getattr(nn_module, name, None):
            return False
    return all(not getattr(m, attr, None) for m in modules for attr in _HOOK_DICTS)


def _packed(module):
    return getattr(module, "_solution_group", None)


def _lora_state(attn):
    """What can change between calls in the LoRA wrappers of q / k / v: adapter switches,
    merging, the active adapter and its dropout's training flag and rate."""
    from .lora import LoraLinear

    state = []
    for name in ("q_proj", "k_proj", "v_proj"):
        module = getattr(attn, name, None)
        if isinstance(module, LoraLinear):
            adapters = tuple(module.active_adapters)
            drop = module.lora_dropout[adapters[0]] if len(adapters) == 1 \
                and adapters[0] in module.lora_dropout else None
            state.append((module.disable_adapters, module.merged, adapters,
                          getattr(drop, "training", None), getattr(drop, "p", None)))
        else:
            state.append(module)
    return tuple(state)


def qkv_plan(attn, x):
    """`qkv_plan_uncached` kept on the attention module for inputs of the same kind (device,
    dtype, width, autocast, the set of disabled components and the LoRA wrappers' mutable state);
    the per-call condition (no module hooks) is checked every time."""
    key = (x.is_cuda, x.dtype, x.dim() >= 2, x.shape[-1], torch.is_autocast_enabled("cuda"),
           torch.get_autocast_dtype("cuda"), tuple(sorted(DISABLED)), _lora_state(attn))
    cached = attn.__dict__.get("_talm_qkv_plan")
    if cached is None or cached[0] != key:
        plan = qkv_plan_uncached(attn, x)
        modules = plan[3] if plan is not None else None
        cached = (key, None if plan is None else plan[:3], modules)
        attn.__dict__["_talm_qkv_plan"] = cached
    plan, modules = cached[1], cached[2]
    if plan is None or not _no_hooks(modules):
        return None
    return plan


def qkv_plan_uncached(attn, x):
    """(group, adapters, lora weights, modules) when q_proj, k_proj and v_proj are projections
    0, 1, 2 of one packed layer group, each plain or a LoRA layer `lora_plan` takes; else None
    (solution/fused_proj.py:318-353). Hooks are the caller's."""
    from .lora import LoraLinear

    if not (x.is_cuda and x.dtype == torch.float16 and x.dim() >= 2) \
            or "fused_proj" in DISABLED or "qgroup" in DISABLED:
        return None
    group, adapters, weights, modules = None, [], [], []
    for seg, name in enumerate(("q_proj", "k_proj", "v_proj")):
        module = getattr(attn, name, None)
        if module is None:
            return None
        tag = _packed(module)
        modules.append(module)
        if tag is None:
            if not isinstance(module, LoraLinear) or "lora" in DISABLED:
                return None
            plan = lora_plan(module, x)
            if plan is None:
                return None
            tag = plan[:2]
            name_ = module.active_adapters[0]
            modules += [module.base_layer, module.lora_A[name_], module.lora_B[name_],
                        module.lora_dropout[name_]]
            adapters.append((seg, plan[4], plan[5]))
            weights += [plan[2], plan[3]]
        if group is None:
            group = tag[0]
        if tag[0] is not group or tag[1] != seg:
            return None
    if any(group.shapes[i][1] != x.shape[-1] for i in (Q, K, V)):
        return None
    return group, tuple(adapters), weights, modules


def _rope_ok(cos, sin, n_tok, head_dim):
    return (cos is not None and cos.dim() == 3 and cos.shape[0] == 1 and cos.shape[1] == n_tok
            and cos.shape[2] == head_dim and cos.dtype == torch.float32 and cos.shape == sin.shape
            and cos.stride(-1) == 1 and sin.stride(-1) == 1 and "rope" not in DISABLED)


ATTN_BLOCK = os.environ.get("SOLUTION_DISABLE_ATTN_BLOCK") != "1"


def _rows_attention(cfg):
    """The model's attention is the registered "sdpa" interface wrapped for packed rows (the
    semantics the block restates)."""
    from transformers.modeling_utils import ALL_ATTENTION_FUNCTIONS

    if getattr(cfg, "_attn_implementation", None) != "sdpa":
        return False
    try:
        return bool(getattr(ALL_ATTENTION_FUNCTIONS["sdpa"], "_solution_rows", False))
    except KeyError:
        return False


def _attention_block(attn, x, group, adapters, weights, rope, n_tok):
    """The layer's attention as one AttentionBlock node when the packed-rows context provides
    cu_seqlens, the rotary embedding goes in place, o_proj is the group's plain projection and
    the heads suit the attention kernel; else None (the per-node path runs)."""
    from . import unpad
    from .qgroup import _linear4bit

    if not ATTN_BLOCK or "attn_block" in DISABLED or rope is None or not unpad._cu \
            or unpad._cu[-1] is None or "varlen_attention" in DISABLED:
        return None
    cu, max_len, total = unpad._cu[-1]
    dropout = 0.0 if not attn.training else attn.attention_dropout
    o_proj = getattr(attn, "o_proj", None)
    tag = _packed(o_proj) if o_proj is not None else None
    cfg = attn.config
    n_heads = getattr(cfg, "num_attention_heads", None)
    n_kv = getattr(cfg, "num_key_value_heads", None)
    if total != n_tok or dropout != 0.0 or attn.sliding_window is not None or tag is None \
            or tag[0] is not group or tag[1] != O or _linear4bit(o_proj) is not o_proj \
            or attn.head_dim != 128 or not n_heads or not n_kv or n_heads % n_kv \
            or not _no_hooks([o_proj]) or not _rows_attention(cfg):
        return None
    try:
        y = AttentionBlock.apply(x, group, adapters, rope, attn.head_dim, n_heads, n_kv, cu,
                                 max_len, attn.scaling, *weights)
    except _NotApplicable:
        return None
    except Exception as exc:  # noqa: BLE001 - state.py convention
        if not fallback("attn_block", exc):
            raise
        return None
    COUNTS["attn"] += 1
    RAN["fused_proj"] += 1
    RAN["varlen_attn"] += 1
    RAN["attn_block"] += 1
    return y


def patch_qwen2_attention():
    """`Qwen2Attention.forward` with q|k|v (+ LoRA, + RoPE in place) as one FusedProjections
    node when `qkv_plan` takes the layer; transformers' own forward otherwise
    (solution/fused_proj.py:382-445)."""
    from transformers.modeling_utils import ALL_ATTENTION_FUNCTIONS
    from transformers.models.qwen2 import modeling_qwen2

    cls = modeling_qwen2.Qwen2Attention
    original = cls.forward
    ON.add("fused_proj")
    if getattr(original, "_solution_fused", False):
        return

    def forward(self, hidden_states, position_embeddings=None, attention_mask=None,
                past_key_values=None, **kwargs):
        plan = None
        if position_embeddings is not None and past_key_values is None:
            plan = qkv_plan(self, hidden_states)
        if plan is None:
            COUNTS["attn_fallback"] += 1
            FELL_BACK["fused_proj"] += 1
            return original(self, hidden_states, position_embeddings, attention_mask,
                            past_key_values=past_key_values, **kwargs)
        group, adapters, weights = plan
        cos, sin = position_embeddings
        input_shape = hidden_states.shape[:-1]
        n_tok = hidden_states.numel() // hidden_states.shape[-1]
        rope = (cos[0] if cos.dim() == 3 else cos, sin[0] if sin.dim() == 3 else sin) \
            if hidden_states.shape[0] == 1 and _rope_ok(cos, sin, n_tok, self.head_dim) else None
        y = _attention_block(self, hidden_states, group, adapters, weights, rope, n_tok)
        if y is not None:
            return y, None
        try:
            q, k, v = FusedProjections.apply(hidden_states, group, Q, V + 1, adapters, (),
                                             rope, self.head_dim, *weights)
        except Exception as exc:  # noqa: BLE001 - state.py convention
            if not fallback("fused_proj", exc):
                raise
            COUNTS["attn_fallback"] += 1
            FELL_BACK["fused_proj"] += 1
            return original(self, hidden_states, position_embeddings, attention_mask,
                            past_key_values=past_key_values, **kwargs)
        COUNTS["attn"] += 1
        RAN["fused_proj"] += 1
        hidden_shape = (*input_shape, -1, self.head_dim)
        query_states = q.view(hidden_shape).transpose(1, 2)
        key_states = k.view(hidden_shape).transpose(1, 2)
        value_states = v.view(hidden_shape).transpose(1, 2)
        del q, k, v
        if rope is None:
            query_states, key_states = modeling_qwen2.apply_rotary_pos_emb(
                query_states, key_states, cos, sin)
        attention_interface = ALL_ATTENTION_FUNCTIONS.get_interface(
            self.config._attn_implementation, modeling_qwen2.eager_attention_forward)
        attn_output, attn_weights = attention_interface(
            self, query_states, key_states, value_states, attention_mask,
            dropout=0.0 if not self.training else self.attention_dropout,
            scaling=self.scaling, sliding_window=self.sliding_window, **kwargs)
        attn_output = attn_output.reshape(*input_shape, -1).contiguous()
        attn_output = self.o_proj(attn_output)
        return attn_output, attn_weights

    forward._solution_fused = True
    forward._original = original
    cls.forward = forward
