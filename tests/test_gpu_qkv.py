"""Parity of the q|k|v projection on MFMA (talm_lora_down, talm_qkv_lora_fwd) with float32
references of the same arithmetic: the reference's node is x W^T + b, per adapter
t = x A^T, + scaling * t B^T on its columns, then the rotary embedding of q and k
(solution/fused_proj.py:88-218, solution/lora.py:151-231, solution/rope.py:145-157).

Bars: t within one fp16 rounding of fp16(x A^T) (fp32 sums in another order); the projection
within 2e-3 relative + 2e-3 x the output's scale (fp16 operands, one rounding of an fp32 sum, the
reference rounds the adapter branch separately: solution/test_fused_proj.py:27-31 compares to
GEMM rounding); whole-model use is covered by tests/test_gpu_step.py."""

import pytest
import torch

import talm_amd._ops  # noqa: F401  (registers torch.ops.talm.*)

pytestmark = pytest.mark.gpu
DEV = "cuda"


def _case(msg):
    print(f"[case] {msg}", flush=True)


def _rope_tables(n, dim=128, theta=1e6, seed=0):
    g = torch.Generator().manual_seed(seed)
    pos = torch.randint(0, 512, (n,), generator=g).double()
    inv = 1.0 / theta ** (torch.arange(0, dim, 2).double() / dim)
    ang = pos[:, None] * inv[None]
    ang = torch.cat((ang, ang), -1)
    return ang.cos().float().to(DEV), ang.sin().float().to(DEV)


def _rotate(y, cos, sin, cols):
    y = y.clone()
    n = y.shape[0]
    heads = y[:, :cols].view(n, -1, 128)
    x1, x2 = heads[..., :64].clone(), heads[..., 64:].clone()
    c, s = cos[:, None], sin[:, None]
    heads[..., :64] = x1 * c[..., :64] - x2 * s[..., :64]
    heads[..., 64:] = x2 * c[..., 64:] + x1 * s[..., 64:]
    return y


def _inputs(n, size, n_out, segs, seed):
    g = torch.Generator().manual_seed(seed)
    x = torch.randn(n, size, generator=g).half().to(DEV)
    w = (torch.randn(n_out, size, generator=g) * size ** -0.5).half().to(DEV)
    bias = (torch.randn(n_out, generator=g) * 0.1).half().to(DEV)
    a = [(torch.rand(16, size, generator=g) * 2 - 1).mul(size ** -0.5).half().to(DEV) for _ in segs]
    b = [(torch.randn(hi - lo, 16, generator=g) * 0.05).half().to(DEV) for lo, hi in segs]
    return x, w, bias, a, b


@pytest.mark.parametrize("n,size,adapters", [(1130, 1536, 2), (37, 64, 1), (1, 32, 2),
                                             (300, 1536, 1)])
def test_lora_down_matches_fp32(n, size, adapters):
    _case(f"lora_down n={n} H={size} adapters={adapters}")
    segs = [(0, 128), (128, 256)][:adapters]
    x, _w, _b, a, _bb = _inputs(n, size, 256, segs, seed=n + size)
    t = torch.empty(n, 16 * adapters, dtype=torch.float16, device=DEV)
    ts = torch.empty_like(t)
    scalings = [2.0, 0.75][:adapters] + [0.0]
    torch.ops.talm.lora_down(x, a[0], a[1] if adapters > 1 else None, size, size, 0, 0, 0,
                             scalings[0], scalings[1], t, ts)
    for g in range(adapters):
        ref = x.float() @ a[g].float().t()
        got = t[:, 16 * g:16 * (g + 1)].float()
        assert torch.all((got - ref).abs() <= 2.0 ** -10 * ref.abs() + 1e-6 * size), g
        got_s = ts[:, 16 * g:16 * (g + 1)].float()
        ref_s = ref * scalings[g]
        assert torch.all((got_s - ref_s).abs() <= 2.0 ** -10 * ref_s.abs() + 1e-6 * size), g


@pytest.mark.parametrize("n,size,n_out,segs,rope_cols,with_bias", [
    (1130, 1536, 2048, [(0, 1536), (1792, 2048)], 1792, True),   # Qwen2.5-1.5B q|k|v
    (1130, 1536, 2048, [], 1792, True),                          # no adapters
    (257, 512, 1024, [(0, 512), (768, 1024)], 768, False),       # test_gpu_step's layer, no bias
    (37, 256, 1000, [(0, 256), (896, 1000)], 0, True),           # ragged n_out, no rotation
    (1, 64, 384, [(128, 256)], 256, True),                       # one token, one adapter
])
def test_qkv_lora_fwd_matches_fp32(n, size, n_out, segs, rope_cols, with_bias):
    _case(f"qkv_lora_fwd n={n} H={size} n_out={n_out} segs={segs} rope={rope_cols}")
    x, w, bias, a, b = _inputs(n, size, n_out, segs, seed=n + n_out)
    bias = bias if with_bias else None
    scalings = [2.0, 2.0]
    ts = t = None
    if segs:
        t = torch.empty(n, 16 * len(segs), dtype=torch.float16, device=DEV)
        ts = torch.empty_like(t)
        torch.ops.talm.lora_down(x, a[0], a[1] if len(segs) > 1 else None, size, size, 0, 0, 0,
                                 scalings[0], scalings[1], t, ts)
    cos, sin = _rope_tables(n) if rope_cols else (None, None)
    out = torch.empty(n, n_out, dtype=torch.float16, device=DEV)
    pad = segs + [(0, 0)] * 2
    bs = b + [None] * 2
    torch.ops.talm.qkv_lora_fwd(x, w, bias, ts, bs[0], pad[0][0], pad[0][1], bs[1], pad[1][0],
                                pad[1][1], cos, sin, rope_cols, out)
    ref = x.float() @ w.float().t()
    if bias is not None:
        ref += bias.float()
    for g, (lo, hi) in enumerate(segs):
        tg = t[:, 16 * g:16 * (g + 1)].float()
        ref[:, lo:hi] += scalings[g] * (tg @ b[g].float().t())
    ref = ref.half().float()
    if rope_cols:
        ref = _rotate(ref, cos, sin, rope_cols)
    got = out.float()
    scale = ref.abs().max()
    err = (got - ref).abs()
    assert torch.all(err <= 2e-3 * ref.abs() + 2e-3 * scale), float(err.max())


@pytest.mark.parametrize("n,size,n_out,segs,rope_cols,with_bias", [
    (1130, 1536, 2048, [(0, 1536), (1792, 2048)], 1792, True),   # Qwen2.5-1.5B q|k|v
    (1312, 1536, 2048, [(0, 1536), (1792, 2048)], 1792, True),   # a config-5 token count
    (1130, 1536, 2048, [], 1792, True),                          # no adapters
    (257, 512, 1024, [(0, 512), (768, 1024)], 768, False),       # test_gpu_step's layer, no bias
    (37, 256, 1000, [(0, 256), (896, 1000)], 0, True),           # ragged n_out, no rotation
    (1, 64, 384, [(128, 256)], 256, True),                       # one token, one adapter
    (65, 96, 256, [(128, 256), (0, 128)], 128, True),            # H not a multiple of 64
])
def test_qkv_lora_fwd_down_matches_fp32(n, size, n_out, segs, rope_cols, with_bias):
    """The one-launch forward (talm_qkv_lora_fwd_down): t = x A^T from the tiles' own product
    within one fp16 rounding of the fp32 sum, and the projection against the same fp32 reference
    as the two-launch forward."""
    _case(f"qkv_lora_fwd_down n={n} H={size} n_out={n_out} segs={segs} rope={rope_cols}")
    x, w, bias, a, b = _inputs(n, size, n_out, segs, seed=n + n_out + 7)
    bias = bias if with_bias else None
    scalings = [2.0, 0.75]
    t = torch.full((n, 16 * len(segs)), float("nan"), dtype=torch.float16,
                   device=DEV) if segs else None
    cos, sin = _rope_tables(n) if rope_cols else (None, None)
    out = torch.empty(n, n_out, dtype=torch.float16, device=DEV)
    pad = segs + [(0, 0)] * 2
    bs = b + [None] * 2
    as_ = a + [None] * 2
    torch.ops.talm.qkv_lora_fwd_down(x, w, bias, as_[0], as_[1], scalings[0], scalings[1], bs[0],
                                     pad[0][0], pad[0][1], bs[1], pad[1][0], pad[1][1], cos, sin,
                                     rope_cols, t, out)
    ref = x.float() @ w.float().t()
    if bias is not None:
        ref += bias.float()
    for g, (lo, hi) in enumerate(segs):
        t_ref = x.float() @ a[g].float().t()
        tg = t[:, 16 * g:16 * (g + 1)].float()
        assert torch.all((tg - t_ref).abs() <= 2.0 ** -10 * t_ref.abs() + 1e-6 * size), g
        ref[:, lo:hi] += scalings[g] * (t_ref @ b[g].float().t())
    ref = ref.half().float()
    if rope_cols:
        ref = _rotate(ref, cos, sin, rope_cols)
    got = out.float()
    scale = ref.abs().max()
    err = (got - ref).abs()
    assert torch.all(err <= 2e-3 * ref.abs() + 2e-3 * scale), float(err.max())
    if segs:  # the two-launch forward on the same inputs: the same values up to t's rounding
        t2 = torch.empty(n, 16 * len(segs), dtype=torch.float16, device=DEV)
        ts2 = torch.empty_like(t2)
        torch.ops.talm.lora_down(x, a[0], a[1] if len(segs) > 1 else None, size, size, 0, 0, 0,
                                 scalings[0], scalings[1], t2, ts2)
        out2 = torch.empty_like(out)
        torch.ops.talm.qkv_lora_fwd(x, w, bias, ts2, bs[0], pad[0][0], pad[0][1], bs[1],
                                    pad[1][0], pad[1][1], cos, sin, rope_cols, out2)
        assert torch.all((out.float() - out2.float()).abs() <= 2e-3 * out2.float().abs() + 1e-3 * scale)


def test_qkv_lora_fwd_rejects_misaligned_adapter_columns():
    _case("qkv_lora_fwd rejects")
    x, w, bias, a, b = _inputs(8, 64, 512, [(64, 192)], seed=1)
    t = torch.empty(8, 16, dtype=torch.float16, device=DEV)
    out = torch.empty(8, 512, dtype=torch.float16, device=DEV)
    with pytest.raises(ValueError, match="whole 128-column tiles"):
        torch.ops.talm.qkv_lora_fwd(x, w, bias, t, b[0], 64, 192, None, 0, 0, None, None, 0, out)


def _rotate_back(y, cos, sin, cols):
    y = y.clone()
    n = y.shape[0]
    heads = y[:, :cols].view(n, -1, 128)
    x1, x2 = heads[..., :64].clone(), heads[..., 64:].clone()
    c, s = cos[:, None], sin[:, None]
    heads[..., :64] = x1 * c[..., :64] + x2 * s[..., 64:]
    heads[..., 64:] = x2 * c[..., 64:] - x1 * s[..., :64]
    return y


@pytest.mark.parametrize("n,q,k,v,rope", [(1130, 1536, 256, 256, True), (37, 512, 256, 256, True),
                                          (5, 128, 0, 64, False)])
def test_qkv_bwd_prep_matches_rope_backward(n, q, k, v, rope):
    """dcat = [rope_back(dq) | rope_back(dk) | dv] from strided gradient views: one fp16
    rounding of the fp32 rotation (solution/rope.py:145-157), dv copied bit for bit."""
    _case(f"qkv_bwd_prep n={n} q={q} k={k} v={v} rope={rope}")
    g = torch.Generator().manual_seed(n + q)
    big = torch.randn(n, q + k + v + 24, generator=g).half().to(DEV)  # strided row views
    dq, dk, dv = big[:, :q], big[:, q:q + k], big[:, q + k:q + k + v]
    cos, sin = _rope_tables(n, seed=3) if rope else (None, None)
    dcat = torch.empty(n, q + k + v, dtype=torch.float16, device=DEV)
    torch.ops.talm.qkv_bwd_prep(dq, dk, dv, cos, sin, dcat)
    ref = torch.cat([dq, dk, dv], 1).float()
    if rope:
        ref = _rotate_back(ref, cos, sin, q + k)
    got = dcat.float()
    assert torch.equal(got[:, q + k:], ref[:, q + k:])
    err = (got - ref.half().float()).abs()
    assert torch.all(err <= 2.0 ** -10 * ref.abs() + 2.0 ** -24), float(err.max())


@pytest.mark.parametrize("n,width,segs", [
    (700, 2048, [(0, 1536), (1792, 2048)]),   # Qwen2.5-1.5B q|k|v: 48 + 8 k-steps of 32
    (333, 2800, [(0, 2560), (2688, 2784)]),   # 80 + 3 k-steps: two passes, a mid-pass switch
])
def test_lora_down_backward_form_matches_fp32(n, width, segs):
    """u = (scaling dy) B per adapter over its own output columns: adapter 0 reduces columns
    [lo0, hi0), adapter 1 columns [lo1, hi1) of one [N, width] gradient."""
    _case(f"lora_down backward form n={n} segs={segs}")
    g = torch.Generator().manual_seed(11 + n)
    dcat = torch.randn(n, width, generator=g).half().to(DEV)
    b = [(torch.randn(hi - lo, 16, generator=g) * 0.05).half().to(DEV) for lo, hi in segs]
    t = torch.empty(n, 32, dtype=torch.float16, device=DEV)
    u = torch.empty_like(t)
    (lo0, hi0), (lo1, hi1) = segs
    for kmajor in (0, 1):  # B_g transposed to [16, seg], or read as stored [seg, 16]
        bs = [bb.t().contiguous() for bb in b] if not kmajor else b
        torch.ops.talm.lora_down(dcat, bs[0], bs[1], hi0 - lo0, hi1 - lo1, lo0, lo1, kmajor, 2.0,
                                 2.0, t, u)
        for k, (lo, hi) in enumerate(segs):
            ref = 2.0 * (dcat[:, lo:hi].float() @ b[k].float())
            got = u[:, 16 * k:16 * (k + 1)].float()
            assert torch.all((got - ref).abs() <= 2.0 ** -10 * ref.abs() + 1e-5 * (hi - lo)), k


@pytest.mark.parametrize("n,size,n_out,rank", [(1130, 1536, 2048, 32), (257, 512, 1024, 32),
                                               (37, 256, 1024, 0), (1, 64, 384, 16)])
def test_qkv_lora_bwd_dx_matches_fp32(n, size, n_out, rank):
    _case(f"qkv_lora_bwd_dx n={n} H={size} n_out={n_out} r={rank}")
    g = torch.Generator().manual_seed(n + rank)
    dcat = torch.randn(n, n_out, generator=g).half().to(DEV)
    w = (torch.randn(n_out, size, generator=g) * n_out ** -0.5).half().to(DEV)
    u = a_t = None
    ref = dcat.float() @ w.float()
    if rank:
        u = torch.randn(n, rank, generator=g).half().to(DEV)
        a = (torch.rand(rank, size, generator=g) * 2 - 1).half().to(DEV) * 0.05
        a_t = a.t().contiguous()
        ref += u.float() @ a.float()
    wt = torch.empty(size, n_out, dtype=torch.float16, device=DEV)
    torch.ops.talm.head_weight_t(w, wt)
    dx = torch.empty(n, size, dtype=torch.float16, device=DEV)
    torch.ops.talm.qkv_lora_bwd_dx(dcat, wt, u, a_t, dx)
    err = (dx.float() - ref).abs()
    assert torch.all(err <= 2e-3 * ref.abs() + 2e-3 * ref.abs().max()), float(err.max())


@pytest.mark.parametrize("n,size,segs", [(1130, 1536, [(0, 1536), (1792, 256)]),
                                         (65, 512, [(0, 512), (768, 256)]), (1, 64, [(64, 128)]),
                                         (300, 96, [(0, 96), (128, 32)]),
                                         (70, 40, [(0, 40), (48, 24)])])
def test_lora_wgrad_matches_fp32(n, size, segs):
    """dA_g = u_g^T x and dB_g = scaling_g dy_g^T t_g in fp32 (the reference rounds the fp16
    GEMM output before its fp32 cast: within one fp16 rounding of the fp32 sums). The MFMA
    kernel takes the 32-aligned hidden sizes (a workgroup of the 96 case holds both dA columns
    and dB rows, and a wavefront's dB rows span both adapters); hidden 40 takes the VALU one."""
    from talm_amd import _ops

    _case(f"lora_wgrad n={n} H={size} segs={segs}")
    g = torch.Generator().manual_seed(n)
    n_out = max(lo + k for lo, k in segs)
    x = torch.randn(n, size, generator=g).half().to(DEV)
    dy = torch.randn(n, n_out, generator=g).half().to(DEV)
    u = torch.randn(n, 16 * len(segs), generator=g).half().to(DEV)
    t = torch.randn(n, 16 * len(segs), generator=g).half().to(DEV)
    scal = [2.0, 0.5]
    da = [torch.empty(16, size, device=DEV) for _ in segs]
    db = [torch.empty(k, 16, device=DEV) for _lo, k in segs]
    pad = segs + [(0, 0)]
    ws = torch.empty(_ops.lora_wgrad_workspace_bytes(n, size, pad[0][1], pad[1][1]),
                     dtype=torch.uint8, device=DEV)
    two = len(segs) > 1
    torch.ops.talm.lora_wgrad(x, dy, u, t, pad[0][0], pad[0][1], scal[0], da[0], db[0], pad[1][0],
                              pad[1][1], scal[1], da[1] if two else None, db[1] if two else None,
                              ws)
    for k, (lo, seg) in enumerate(segs):
        ref_a = u[:, 16 * k:16 * (k + 1)].float().t() @ x.float()
        ref_b = scal[k] * (dy[:, lo:lo + seg].float().t() @ t[:, 16 * k:16 * (k + 1)].float())
        for got, ref in ((da[k], ref_a), (db[k], ref_b)):
            err = (got - ref).abs()
            assert torch.all(err <= 1e-5 * ref.abs() + 1e-6 * n), float(err.max())
