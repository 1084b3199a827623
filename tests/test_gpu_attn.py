"""Variable-length causal GQA attention (torch.ops.talm.attn_fwd / attn_bwd / attn_bwd_rope)
against per-row causal SDPA in fp32 on the CPU (solution/unpad.py:121-134): output, log-sum-exp
and the gradients of q, k, v. fp16 operands, fp32 statistics, fp16 P and dS in the MFMA products: the
tolerances are stated per tensor relative to its largest reference magnitude."""

import math

import pytest
import torch

pytestmark = pytest.mark.gpu

HQ, HKV, D = 12, 2, 128


def _reference(q, k, v, lengths, scale, dout):
    """fp32 CPU: per sequence, causal softmax(scale q k^T) v with KV heads shared by groups of
    query heads; returns out, lse [Hq, N] and (dq, dk, dv) for the upstream gradient dout."""
    q, k, v = (t.detach().float().cpu().requires_grad_(True) for t in (q, k, v))
    outs, lses = [], []
    s0 = 0
    group = q.shape[1] // k.shape[1]
    for n in lengths:
        qs = q[s0:s0 + n].transpose(0, 1)                                  # [Hq, n, D]
        ks = k[s0:s0 + n].transpose(0, 1).repeat_interleave(group, 0)      # [Hq, n, D]
        vs = v[s0:s0 + n].transpose(0, 1).repeat_interleave(group, 0)
        scores = scale * qs @ ks.transpose(1, 2)
        mask = torch.ones(n, n, dtype=torch.bool).triu(1)
        scores = scores.masked_fill(mask, float("-inf"))
        lses.append(torch.logsumexp(scores, -1))                           # [Hq, n]
        outs.append((torch.softmax(scores, -1) @ vs).transpose(0, 1))     # [n, Hq, D]
        s0 += n
    out = torch.cat(outs)
    out.backward(dout.float().cpu())
    return out.detach(), torch.cat(lses, 1).detach(), q.grad, k.grad, v.grad


def _close(name, got, ref, rel):
    got = got.float().cpu()
    scale = ref.abs().max().item()
    err = (got - ref).abs().max().item()
    print(f"[attn] {name}: max err {err:.3e} (max |ref| {scale:.3e})", flush=True)
    assert err <= rel * scale + 1e-6, f"{name}: max error {err} > {rel} x {scale}"


def _run(lengths, strided, seed):
    import talm_amd._ops  # noqa: F401
    from talm_amd import _ops

    g = torch.Generator("cpu").manual_seed(seed)
    n = sum(lengths)
    if strided:  # the q|k|v node's layout: q and k column views of one [N, 2048] buffer
        qkv = torch.randn(n, (HQ + HKV) * D, generator=g).half().cuda()
        q = qkv[:, :HQ * D].view(n, HQ, D)
        k = qkv[:, HQ * D:].view(n, HKV, D)
    else:
        q = torch.randn(n, HQ, D, generator=g).half().cuda()
        k = torch.randn(n, HKV, D, generator=g).half().cuda()
    v = torch.randn(n, HKV, D, generator=g).half().cuda()
    dout = torch.randn(n, HQ, D, generator=g).half().cuda()
    cu = torch.tensor([0] + list(torch.tensor(lengths).cumsum(0)), dtype=torch.int32).cuda()
    scale = 1.0 / math.sqrt(D)
    out = torch.empty(n, HQ, D, dtype=torch.float16, device="cuda")
    lse = torch.empty(HQ, n, dtype=torch.float32, device="cuda")
    torch.ops.talm.attn_fwd(q, k, v, cu, max(lengths), scale, out, lse)
    dq = torch.empty_like(out)
    dk = torch.empty(n, HKV, D, dtype=torch.float16, device="cuda")
    dv = torch.empty_like(dk)
    ws = torch.empty(_ops.attn_bwd_workspace_bytes(n, HQ), dtype=torch.uint8, device="cuda")
    torch.ops.talm.attn_bwd(q, k, v, out, dout, lse, cu, max(lengths), scale, dq, dk, dv, ws)
    torch.cuda.synchronize()
    r_out, r_lse, r_dq, r_dk, r_dv = _reference(q, k, v, lengths, scale, dout)
    _close("out", out, r_out, 2e-3)
    _close("lse", lse, r_lse, 1e-4)
    _close("dq", dq, r_dq, 4e-3)
    _close("dk", dk, r_dk, 4e-3)
    _close("dv", dv, r_dv, 4e-3)


@pytest.mark.parametrize("lengths,strided,seed", [
    ([300, 128, 512, 257], True, 1),    # config-5-like packed batch, the q|k|v buffer's views
    ([1, 17, 64, 65, 129], False, 2),   # single-token and tile-boundary sequences
    ([512], False, 3),
])
def test_attention_matches_per_row_causal_sdpa(lengths, strided, seed):
    print(f"[case] attention lengths={lengths} strided={strided} seed={seed}", flush=True)
    _run(lengths, strided, seed)


def _rotate_back(dy, cos, sin):
    """The gradient of x -> x cos + rotate_half(x) sin (transformers' apply_rotary_pos_emb on one
    [N, H, 128] tensor, fp32 CPU) at dy, by autograd: the rotary backward the fused kernel folds
    in, derived from the forward rather than restated."""
    x = torch.zeros_like(dy, requires_grad=True)
    half = x.shape[-1] // 2
    rotated = torch.cat((-x[..., half:], x[..., :half]), -1)
    (x * cos[:, None, :] + rotated * sin[:, None, :]).backward(dy)
    return x.grad


@pytest.mark.parametrize("lengths,seed", [
    ([300, 128, 512, 257], 4),          # config-5-like packed batch
    ([1, 17, 64, 65, 129], 5),          # single-token and tile-boundary sequences
])
def test_attention_backward_with_the_rotary_backward_folded_in(lengths, seed):
    """attn_bwd_rope: dq / dk rotated back in the kernel's epilogues equal the reference's
    attention gradients pushed through the rotary embedding's backward. cos / sin are independent
    random rows (not the model's tables, whose two halves are equal) so that a swapped half or
    a cos read in place of a sin fails, and their rows are strided (160 of which 128 are read).
    The outputs are column views of one [N, q + k + v] buffer, as in the attention block."""
    import talm_amd._ops  # noqa: F401
    from talm_amd import _ops

    print(f"[case] attention+rope backward lengths={lengths} seed={seed}", flush=True)
    g = torch.Generator("cpu").manual_seed(seed)
    n = sum(lengths)
    qkv = torch.randn(n, (HQ + 2 * HKV) * D, generator=g).half().cuda()
    q = qkv[:, :HQ * D].view(n, HQ, D)
    k = qkv[:, HQ * D:(HQ + HKV) * D].view(n, HKV, D)
    v = qkv[:, (HQ + HKV) * D:].view(n, HKV, D)
    dout = torch.randn(n, HQ, D, generator=g).half().cuda()
    cs = torch.rand(2, n, 160, generator=g) * 2 - 1
    cos, sin = cs[0].cuda()[:, :D], cs[1].cuda()[:, :D]
    cu = torch.tensor([0] + list(torch.tensor(lengths).cumsum(0)), dtype=torch.int32).cuda()
    scale = 1.0 / math.sqrt(D)
    out = torch.empty(n, HQ, D, dtype=torch.float16, device="cuda")
    lse = torch.empty(HQ, n, dtype=torch.float32, device="cuda")
    torch.ops.talm.attn_fwd(q, k, v, cu, max(lengths), scale, out, lse)
    grads = torch.full_like(qkv, float("nan"))
    dq = grads[:, :HQ * D].view(n, HQ, D)
    dk = grads[:, HQ * D:(HQ + HKV) * D].view(n, HKV, D)
    dv = grads[:, (HQ + HKV) * D:].view(n, HKV, D)
    ws = torch.empty(_ops.attn_bwd_workspace_bytes(n, HQ), dtype=torch.uint8, device="cuda")
    torch.ops.talm.attn_bwd_rope(q, k, v, out, dout, lse, cu, max(lengths), scale, cos, sin, dq,
                                 dk, dv, ws)
    torch.cuda.synchronize()
    _r_out, _r_lse, r_dq, r_dk, r_dv = _reference(q, k, v, lengths, scale, dout)
    c, s_ = cos.cpu(), sin.cpu()
    assert not grads.isnan().any(), "a gradient element was not written"
    _close("dq (rotated back)", dq, _rotate_back(r_dq, c, s_), 4e-3)
    _close("dk (rotated back)", dk, _rotate_back(r_dk, c, s_), 4e-3)
    _close("dv", dv, r_dv, 4e-3)


def test_attention_rope_backward_rejects_bad_tables():
    import talm_amd._ops  # noqa: F401
    from talm_amd import _ops

    n = 8
    q = torch.zeros(n, HQ, D, dtype=torch.float16, device="cuda")
    k = torch.zeros(n, HKV, D, dtype=torch.float16, device="cuda")
    cu = torch.tensor([0, n], dtype=torch.int32, device="cuda")
    lse = torch.zeros(HQ, n, device="cuda")
    ws = torch.empty(_ops.attn_bwd_workspace_bytes(n, HQ), dtype=torch.uint8, device="cuda")
    narrow = torch.zeros(n, 64, device="cuda")                    # fewer than 128 columns
    with pytest.raises(ValueError):
        torch.ops.talm.attn_bwd_rope(q, k, k, q, q, lse, cu, n, 0.125, narrow, narrow, q, k, k, ws)
    odd = torch.zeros(n, 131, device="cuda")[:, :128]             # row stride not a multiple of 4
    with pytest.raises(ValueError):
        torch.ops.talm.attn_bwd_rope(q, k, k, q, q, lse, cu, n, 0.125, odd, odd, q, k, k, ws)


def test_attention_rejects_bad_shapes():
    import talm_amd._ops  # noqa: F401

    n = 8
    q = torch.zeros(n, HQ, 64, dtype=torch.float16, device="cuda")  # head_dim 64: not supported
    k = torch.zeros(n, HKV, 64, dtype=torch.float16, device="cuda")
    cu = torch.tensor([0, n], dtype=torch.int32, device="cuda")
    with pytest.raises(ValueError):
        torch.ops.talm.attn_fwd(q, k, k, cu, n, 0.125, q, torch.empty(HQ, n, device="cuda"))
