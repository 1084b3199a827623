"""Parity of the HIP bandwidth kernels with the CPU oracle, on the BASELINE configurations'
seeded inputs (identical bytes on both sides), through the torch.ops.talm custom ops and the
C-ABI. NF4: bit-exact. RMSNorm / RoPE / SwiGLU: within 1e-3 relative of the float64 oracle
(tolerance written in each test via helpers.assert_rel)."""

import numpy as np
import pytest
import torch

from oracle import nf4 as nf4_oracle
from oracle import norm as norm_oracle
from oracle import rope as rope_oracle
from oracle import swiglu as swiglu_oracle
from talm_amd import qgroup, rmsnorm, rope, swiglu, workloads
from talm_amd.engaged import RAN
from talm_amd.nf4_dequant import nf4_dequantize
from tests.helpers import assert_rel, f16_bits, to_np

pytestmark = pytest.mark.gpu
DEV = "cuda"


def _case(msg):
    print(f"[case] {msg}", flush=True)


# ----------------------------------------------------------------------------------- NF4 -----

@pytest.mark.parametrize("streaming", [False, True], ids=["cached", "streaming"])
def test_nf4_group_dequant_config1_bit_exact(streaming):
    """Config 1: one Qwen2.5-1.5B layer (46,792,704 weights) in one launch, bit for bit the
    oracle (solution/qgroup.py:72-91); every projection slice launched alone too. Both store
    kinds (the step's ordinary stores and the streaming entry point's non-temporal ones); the
    persistent grid walks about two tiles per wavefront here."""
    _case(f"nf4 group config1 streaming={streaming}")
    d = workloads.nf4_layer()
    ref = nf4_oracle.group_dequant(d["packed"].numpy(), d["absmax8"].numpy(), d["code"].numpy(),
                                   d["absmax2"].numpy(), d["offset2"].numpy())
    t = {k: d[k].to(DEV) for k in ("packed", "absmax8", "code", "absmax2", "offset2")}
    n_rows = d["absmax8"].numel()
    out = torch.full((d["n"],), float("nan"), dtype=torch.float16, device=DEV)
    qgroup.launch(t["packed"], t["absmax8"], t["code"], t["absmax2"], t["offset2"], None, out,
                  n_rows, 64, 256, streaming=streaming)
    got = f16_bits(out)
    assert got.shape == ref.shape
    bad = np.flatnonzero(got != ref)
    assert bad.size == 0, f"{bad.size} weights differ, first {bad[:5]}"
    start = 0
    for rows, cols in d["shapes"]:
        n = rows * cols
        r0, b0 = start // 64, start // (64 * 256)
        one = torch.empty(n, dtype=torch.float16, device=DEV)
        qgroup.launch(t["packed"][start // 2:], t["absmax8"][r0:], t["code"], t["absmax2"][b0:],
                      t["offset2"][b0:], None, one, n // 64, 64, 256, streaming=streaming)
        assert np.array_equal(f16_bits(one), ref[start:start + n]), (rows, cols)
        start += n


def test_nf4_group_dequant_transposed_config1_bit_exact():
    """The backward's transposed layer (talm_nf4_group_dequant_t): every projection of the
    config-1 layer written as W^T into the four blocks q|k|v, o, gate|up, down, bit for bit the
    oracle's W transposed; the bytes around each block stay untouched."""
    _case("nf4 group transposed config1")
    d = workloads.nf4_layer()
    ref = nf4_oracle.group_dequant(d["packed"].numpy(), d["absmax8"].numpy(), d["code"].numpy(),
                                   d["absmax2"].numpy(), d["offset2"].numpy())
    t = {k: d[k].to(DEV) for k in ("packed", "absmax8", "code", "absmax2", "offset2")}
    blocks = ((0, 1, 2), (3,), (4, 5), (6,))
    segs, placed, start, off = [], [], 0, 0
    starts = np.cumsum([0] + [r * c for r, c in d["shapes"]])
    for members in blocks:
        cols = d["shapes"][members[0]][1]
        width = sum(d["shapes"][i][0] for i in members)
        o_off = 0
        for i in members:
            rows = d["shapes"][i][0]
            segs += [int(starts[i]), rows, cols, off + o_off, width]
            placed.append((i, off, cols, width, o_off))
            o_off += rows
        off += cols * width
    pad = 64
    out = torch.full((d["n"] + 2 * pad,), float("nan"), dtype=torch.float16, device=DEV)
    torch.ops.talm.nf4_group_dequant_t(t["packed"], t["absmax8"], t["code"], t["absmax2"],
                                       t["offset2"], segs, out[pad:pad + d["n"]], 64, 256)
    got = f16_bits(out)
    assert np.all(np.isnan(out[:pad].float().cpu().numpy()))
    assert np.all(np.isnan(out[pad + d["n"]:].float().cpu().numpy()))
    for i, blk, cols, width, o_off in placed:
        rows = d["shapes"][i][0]
        w = ref[starts[i]:starts[i] + rows * cols].reshape(rows, cols)
        wt = got[pad + blk:pad + blk + cols * width].reshape(cols, width)[:, o_off:o_off + rows]
        assert np.array_equal(wt, w.T), (i, rows, cols)


@pytest.mark.parametrize("rows,cols", [(8, 64), (136, 192), (264, 128)])
def test_nf4_group_dequant_transposed_partial_tiles(rows, cols):
    """Row counts that leave a partial 128-row tile (8-row chunks past the end are not
    written), into a W^T with a wider row stride whose other columns stay untouched."""
    _case(f"nf4 group transposed {rows}x{cols}")
    g = torch.Generator().manual_seed(rows * cols)
    n = rows * cols
    n_rows = n // 64
    n2 = -(-n_rows // 4)
    packed = torch.randint(0, 256, (n // 2,), generator=g, dtype=torch.int32).to(torch.uint8)
    absmax8 = torch.randint(0, 256, (n_rows,), generator=g, dtype=torch.int32).to(torch.uint8)
    code = workloads.dynamic_map()
    absmax2 = torch.rand(n2, generator=g) * 0.045 + 0.005
    offset2 = torch.full((n2,), 0.01)
    ref = nf4_oracle.group_dequant(packed.numpy(), absmax8.numpy(), code.numpy(),
                                   absmax2.numpy(), offset2.numpy(), 64, 4).reshape(rows, cols)
    ld, o_off = rows + 24, 8
    out = torch.full((cols * ld,), float("nan"), dtype=torch.float16, device=DEV)
    torch.ops.talm.nf4_group_dequant_t(packed.to(DEV), absmax8.to(DEV), code.to(DEV),
                                       absmax2.to(DEV), offset2.to(DEV), [0, rows, cols, o_off, ld],
                                       out, 64, 4)
    got = f16_bits(out).reshape(cols, ld)
    assert np.array_equal(got[:, o_off:o_off + rows], ref.T)
    rest = out.view(cols, ld).float().cpu().numpy()
    assert np.all(np.isnan(rest[:, :o_off])) and np.all(np.isnan(rest[:, o_off + rows:]))


@pytest.mark.parametrize("streaming", [False, True], ids=["cached", "streaming"])
@pytest.mark.parametrize("n_rows,qblock,qblock2,shift", [
    (256, 64, 256, 0), (1, 8, 1, 0), (37, 128, 5, 0), (1000, 64, 3, 0), (2, 4096, 1, 0),
    (33, 32, 7, 0), (1000, 64, 256, 4), (77, 16, 3, 0), (400001, 64, 256, 0)])
def test_nf4_group_dequant_edge_shapes(n_rows, qblock, qblock2, shift, streaming):
    """Partial last workgroup and wavefront, odd second-level blocks, blocks of 8 to 4096
    weights (16-byte chunks of codes from 32 up, 8-weight words below), codes that start 4
    bytes past a 16-byte boundary (`shift`: the word path); subnormal-producing scales; 400001
    blocks: more tiles than the persistent grid's wavefronts, the last tile holding 2 chunks."""
    _case(f"nf4 group rows={n_rows} qblock={qblock} qblock2={qblock2} shift={shift} "
          f"streaming={streaming}")
    g = torch.Generator().manual_seed(n_rows + qblock)
    n = n_rows * qblock
    n2 = -(-n_rows // qblock2)
    packed = torch.randint(0, 256, (n // 2,), generator=g, dtype=torch.int32).to(torch.uint8)
    absmax8 = torch.randint(0, 256, (n_rows,), generator=g, dtype=torch.int32).to(torch.uint8)
    code = workloads.dynamic_map()
    absmax2 = torch.rand(n2, generator=g) * 0.045 + 0.005
    offset2 = torch.full((n2,), 0.01)
    ref = nf4_oracle.group_dequant(packed.numpy(), absmax8.numpy(), code.numpy(), absmax2.numpy(),
                                   offset2.numpy(), qblock, qblock2)
    out = torch.empty(n, dtype=torch.float16, device=DEV)
    dev_packed = torch.empty(n // 2 + shift, dtype=torch.uint8, device=DEV)[shift:]
    dev_packed.copy_(packed)
    op = torch.ops.talm.nf4_group_dequant_streaming if streaming \
        else torch.ops.talm.nf4_group_dequant
    op(dev_packed, absmax8.to(DEV), code.to(DEV), absmax2.to(DEV), offset2.to(DEV), out, qblock,
       qblock2)
    assert np.array_equal(f16_bits(out), ref)


@pytest.mark.parametrize("rows,cols,blocksize", [(8960, 1536, 64), (256, 1536, 64),
                                                 (64, 4094, 64), (3, 10, 2), (33, 6, 128),
                                                 (100, 100, 4096)])
def test_nf4_per_projection_bit_exact(rows, cols, blocksize):
    """solution/nf4_dequant.py:38-91 on word and byte paths (n not a multiple of 8, blocks of 2)."""
    _case(f"nf4 per-projection {rows}x{cols} bs={blocksize}")
    n = rows * cols
    g = torch.Generator().manual_seed(n)
    packed = torch.randint(0, 256, (n // 2,), generator=g, dtype=torch.int32).to(torch.uint8)
    absmax = torch.rand(-(-n // blocksize), generator=g) * 0.1
    ref = nf4_oracle.dequant(packed.numpy(), absmax.numpy(), blocksize, n)
    out = torch.empty(rows, cols, dtype=torch.float16, device=DEV)
    nf4_dequantize(packed.to(DEV).view(-1, 1), absmax.to(DEV), blocksize, out)
    assert np.array_equal(f16_bits(out).reshape(-1), ref)


def test_layer_group_packs_and_keeps_one_resident_layer():
    """The packed layer group on 4-bit layers quantized by this package: one grouped launch
    serves the seven projections, bit-identical to each layer's own per-projection
    dequantization; the weights stay resident until another group's request displaces them,
    after which a request dequantizes again (never a stale buffer)."""
    _case("layer group")
    from types import SimpleNamespace

    from talm_amd.nf4_dequant import dequantize_4bit
    from talm_amd.nf4_linear import Linear4bit

    g = torch.Generator().manual_seed(7)
    shapes = [(256, 512), (64, 512), (64, 512), (512, 512), (1024, 512), (1024, 512), (512, 1024)]

    def layer_of(scale):
        mods = [Linear4bit.from_weight((torch.randn(o, i, generator=g) * scale).to(DEV),
                                       bias=torch.randn(o, generator=g).to(DEV) if k < 3 else None)
                for k, (o, i) in enumerate(shapes)]
        return mods, SimpleNamespace(
            self_attn=SimpleNamespace(q_proj=mods[0], k_proj=mods[1], v_proj=mods[2],
                                      o_proj=mods[3]),
            mlp=SimpleNamespace(gate_proj=mods[4], up_proj=mods[5], down_proj=mods[6]))

    mods, layer = layer_of(0.05)
    refs = [dequantize_4bit(m.weight.data, m.weight.quant_state) for m in mods]
    group = qgroup._pack(layer)
    assert group is not None
    other = qgroup._pack(layer_of(0.02)[1])
    qgroup.release()
    before = RAN["group"]
    group.begin_forward()
    for idx, ref in enumerate(refs):
        assert torch.equal(group.weight(idx), ref), idx
    assert RAN["group"] == before + 1  # one launch for the seven projections
    q_k_v = group.span(0, 3)
    assert q_k_v.shape == (384, 512) and torch.equal(q_k_v, torch.cat(refs[:3]))
    assert torch.equal(group.span_bias(0, 3), torch.cat([m.bias.half() for m in mods[:3]]))
    other.begin_forward()                  # another layer displaces it
    assert RAN["group"] == before + 2
    for idx, ref in enumerate(refs):       # dequantized again, once, on the first request
        assert torch.equal(group.weight(idx), ref), idx
    assert RAN["group"] == before + 3
    for m, ref in zip(mods, refs):  # the parameters became views of the packed buffers
        assert torch.equal(dequantize_4bit(m.weight.data, m.weight.quant_state), ref)
    for idx, ref in enumerate(refs):
        assert torch.equal(group.dequantize_one(idx), ref)
    # the backward's transposed blocks: one launch for the layer, the row-major buffer dropped;
    # a block the NF4 dequant-GEMM serves is left out of it and costs a second launch when asked
    # for (after a fallback)
    before_t = RAN["group_t"]
    w4 = group.w4_blocks()
    for members in [b for b in qgroup.T_BLOCKS if b not in w4] + list(w4):
        wt = group.span_t(members[0], members[-1] + 1)
        assert torch.equal(wt, torch.cat([refs[i] for i in members]).t()), members
    assert RAN["group_t"] == before_t + 1 + (1 if w4 else 0)
    assert group.span_t(0, 2) is None and group.span_t(3, 5) is None  # not one block
    assert qgroup._RESIDENT.get(group.device) is None
    group.begin_forward()  # a forward drops the transposed buffer again
    assert qgroup._RESIDENT_T.get(group.device) is None
    qgroup.release()


# ------------------------------------------------------------------------------- RMSNorm -----

@pytest.mark.parametrize("x_dtype", [torch.float16, torch.float32])
def test_add_rmsnorm_config2_forward_backward(x_dtype):
    """Config 2: fused residual add + RMSNorm forward and backward (fp16 residual as the config
    states, fp32 residual stream as the reference's model has it)."""
    _case(f"add+rmsnorm config2 x={x_dtype}")
    d = workloads.norm_rope()
    x, br, w = d["residual"].to(x_dtype), d["x"], d["weight"]
    xd, bd, wd = x.to(DEV), br.to(DEV), w.to(DEV)
    total, y = rmsnorm.NormNode.apply(xd.clone().requires_grad_(), bd.clone().requires_grad_(),
                                      wd, d["eps"], torch.float16)
    np_x = to_np(x).astype(np.float64)
    q, y_ref, xhat_ref, rstd_ref = norm_oracle.forward(np_x, to_np(w), d["eps"], p=to_np(br),
                                                       x_dtype=np.float64, out_dtype=np.float64,
                                                       dtype=np.float64)
    assert_rel(total, q, rtol=1e-3, what="sum")
    assert_rel(y, y_ref, rtol=1e-3, what="y")
    # backward through the same node: ds (sum's gradient) and dy
    xs = xd.clone().requires_grad_()
    bs = bd.clone().requires_grad_()
    total, y = rmsnorm.NormNode.apply(xs, bs, wd, d["eps"], torch.float16)
    ds = d["ds"].to(x_dtype).to(DEV)
    torch.autograd.backward([total, y], [ds, d["dy"].to(DEV)])
    dx_ref, db_ref = norm_oracle.backward(to_np(d["dy"]), xhat_ref, to_np(w), rstd_ref,
                                          ds=to_np(ds), x_dtype=np.float64,
                                          out_dtype=np.float64, dtype=np.float64)
    assert_rel(xs.grad, dx_ref, rtol=1e-3, floor=1e-4, what="dx")
    assert_rel(bs.grad, db_ref, rtol=1e-3, floor=1e-4, what="dbranch")
    assert xs.grad.dtype == x_dtype and bs.grad.dtype == torch.float16


@pytest.mark.parametrize("shape,out_dtype", [((1130, 1536), torch.float16), ((3, 77, 1536),
                                              torch.float32), ((1, 1536), torch.float16),
                                             ((5, 1000), torch.float16), ((4, 13), torch.float32),
                                             ((2, 6000), torch.float16)])
def test_rmsnorm_forward_backward(shape, out_dtype):
    """Plain RMSNorm (no add), fp32 input (the residual stream), vector and generic paths."""
    _case(f"rmsnorm {shape} out={out_dtype}")
    g = torch.Generator().manual_seed(shape[-1])
    x = torch.randn(shape, generator=g) * 3
    w = 1 + 0.1 * torch.randn(shape[-1], generator=g)
    dy = torch.randn(shape, generator=g).to(out_dtype)
    xd = x.to(DEV).requires_grad_()
    y = rmsnorm.rmsnorm(xd, w.to(DEV), 1e-6, out_dtype)
    y.backward(dy.to(DEV))
    _, y_ref, xhat_ref, rstd_ref = norm_oracle.forward(to_np(x).astype(np.float64), to_np(w),
                                                       1e-6, out_dtype=np.float64,
                                                       dtype=np.float64)
    assert y.dtype == out_dtype and y.shape == x.shape
    assert_rel(y, y_ref, rtol=1e-3, what="y")
    dx_ref, _ = norm_oracle.backward(to_np(dy), xhat_ref, to_np(w), rstd_ref,
                                     x_dtype=np.float64, out_dtype=np.float64, dtype=np.float64)
    assert_rel(xd.grad, dx_ref, rtol=1e-3, floor=1e-4, what="dx")


# ---------------------------------------------------------------------------------- RoPE -----

def _qkv_views(d):
    """q, k as column views of one [N, 2048] q|k|v projection output (the fused layout)."""
    n = d["n"]
    qkv = torch.zeros(n, 2048, dtype=torch.float16, device=DEV)
    qkv[:, :1536] = d["q"].reshape(n, 1536).to(DEV)
    qkv[:, 1536:1792] = d["k"].reshape(n, 256).to(DEV)
    q = qkv[:, :1536].view(n, 12, 128)
    k = qkv[:, 1536:1792].view(n, 2, 128)
    return qkv, q, k


@pytest.mark.parametrize("backward", [False, True])
def test_rope_in_place_config2(backward):
    """Config 2 RoPE in place on column views of the q|k|v output: every element rotated, v
    untouched, within 1e-3 of the oracle."""
    _case(f"rope in place config2 backward={backward}")
    d = workloads.norm_rope()
    qkv, q, k = _qkv_views(d)
    v_before = qkv[:, 1792:].clone()
    cos, sin = d["cos"].to(DEV), d["sin"].to(DEV)
    rope.rope_(q, k, cos, sin, backward=backward)
    ref_q = rope_oracle.rotate(to_np(d["q"]), to_np(d["cos"]), to_np(d["sin"]), backward,
                               np.float64, np.float64)
    ref_k = rope_oracle.rotate(to_np(d["k"]), to_np(d["cos"]), to_np(d["sin"]), backward,
                               np.float64, np.float64)
    assert_rel(q, ref_q, rtol=1e-3, floor=1e-4, what="q")
    assert_rel(k, ref_k, rtol=1e-3, floor=1e-4, what="k")
    assert torch.equal(qkv[:, 1792:], v_before)


@pytest.mark.parametrize("n_tokens", [1, 37, 700, 2048])
def test_rope_autograd_matches_transformers(n_tokens):
    """The reference's RoPE node (solution/rope.py:160-189) against transformers'
    apply_rotary_pos_emb: head-major forward output, token-major backward, 1e-3 relative."""
    _case(f"rope autograd n={n_tokens}")
    from transformers.models.qwen2.modeling_qwen2 import apply_rotary_pos_emb

    g = torch.Generator().manual_seed(n_tokens)
    hq, hk, dim = 12, 2, 128
    q_flat = torch.randn(1, n_tokens, hq * dim, generator=g).half().to(DEV).requires_grad_()
    k_flat = torch.randn(1, n_tokens, hk * dim, generator=g).half().to(DEV).requires_grad_()
    cos, sin = workloads.rope_cos_sin(torch.arange(n_tokens))
    cos, sin = cos[None].to(DEV), sin[None].to(DEV)
    gq = torch.randn(1, hq, n_tokens, dim, generator=g).half().to(DEV)
    gk = torch.randn(1, hk, n_tokens, dim, generator=g).half().to(DEV)
    q = q_flat.view(1, n_tokens, hq, dim).transpose(1, 2)
    k = k_flat.view(1, n_tokens, hk, dim).transpose(1, 2)
    oq, ok = rope.RoPE.apply(q, k, cos, sin)
    assert oq.is_contiguous() and oq.shape == (1, hq, n_tokens, dim)
    (oq.float() * gq.float()).sum().add((ok.float() * gk.float()).sum()).backward()
    rq, rk = apply_rotary_pos_emb(q.detach().double(), k.detach().double(), cos.double(),
                                  sin.double())
    assert_rel(oq, rq, rtol=1e-3, floor=1e-4, what="q")
    assert_rel(ok, rk, rtol=1e-3, floor=1e-4, what="k")
    qd = q_flat.detach().double().requires_grad_()
    kd = k_flat.detach().double().requires_grad_()
    r1, r2 = apply_rotary_pos_emb(qd.view(1, n_tokens, hq, dim).transpose(1, 2),
                                  kd.view(1, n_tokens, hk, dim).transpose(1, 2), cos.double(),
                                  sin.double())
    ((r1 * gq.double()).sum() + (r2 * gk.double()).sum()).backward()
    assert_rel(q_flat.grad, qd.grad, rtol=1e-3, floor=1e-4, what="dq")
    assert_rel(k_flat.grad, kd.grad, rtol=1e-3, floor=1e-4, what="dk")


def test_rope_generic_path_odd_head_dim():
    _case("rope generic head_dim=6")
    g = torch.Generator().manual_seed(3)
    n, dim = 5, 6
    q = torch.randn(n, 3, dim, generator=g).half()
    k = torch.randn(n, 1, dim, generator=g).half()
    cos, sin = workloads.rope_cos_sin(torch.arange(n), dim)
    qd, kd = q.to(DEV), k.to(DEV)
    rope.rope_(qd, kd, cos.to(DEV), sin.to(DEV))
    assert_rel(qd, rope_oracle.rotate(to_np(q), to_np(cos), to_np(sin), False, np.float64,
                                      np.float64), rtol=1e-3, floor=1e-4, what="q")


# -------------------------------------------------------------------------------- SwiGLU -----

def test_swiglu_config3_forward_backward_and_in_place():
    """Config 3: [2048, 8960] forward, backward into fresh buffers and in place (dgate over
    gate, dup over up): the in-place results equal the fresh ones bit for bit."""
    _case("swiglu config3")
    d = workloads.swiglu_inputs()
    gate, up, grad = (d[k].to(DEV) for k in ("gate", "up", "grad"))
    out = torch.empty_like(gate)
    swiglu.swiglu_fwd(gate, up, out)
    ref = swiglu_oracle.forward(to_np(d["gate"]), to_np(d["up"]), np.float64, np.float64)
    assert_rel(out, ref, rtol=1e-3, what="out")
    dgate, dup = torch.empty_like(gate), torch.empty_like(up)
    swiglu.swiglu_bwd(grad, gate, up, dgate, dup)
    rdg, rdu = swiglu_oracle.backward(to_np(d["grad"]), to_np(d["gate"]), to_np(d["up"]),
                                      np.float64, np.float64)
    assert_rel(dgate, rdg, rtol=1e-3, what="dgate")
    assert_rel(dup, rdu, rtol=1e-3, what="dup")
    g2, u2 = gate.clone(), up.clone()
    swiglu.swiglu_bwd(grad, g2, u2, g2, u2)
    assert torch.equal(g2, dgate) and torch.equal(u2, dup)
    g3 = gate.clone()
    swiglu.swiglu_fwd(g3, up, g3)  # save-up forward: act written over gate
    assert torch.equal(g3, out)


def test_swiglu_rows_on_halves_equal_flat():
    """The row-strided SwiGLU passes on the two halves of one [N, 2I] buffer (the fused MLP's
    layout) give exactly the flat kernels' results (same arithmetic per element), in place too."""
    _case("swiglu rows")
    d = workloads.swiglu_inputs()
    gate, up, grad = (d[k][:333].to(DEV) for k in ("gate", "up", "grad"))
    inter = gate.shape[1]
    gu = torch.cat([gate, up], 1)
    out_flat = torch.empty_like(gate)
    swiglu.swiglu_fwd(gate, up, out_flat)
    out = torch.empty_like(gate)
    torch.ops.talm.swiglu_fwd_rows(gu[:, :inter], gu[:, inter:], out)
    assert torch.equal(out, out_flat)
    dg, du = torch.empty_like(gate), torch.empty_like(up)
    swiglu.swiglu_bwd(grad, gate, up, dg, du)
    torch.ops.talm.swiglu_bwd_rows(grad, gu[:, :inter], gu[:, inter:], gu[:, :inter], gu[:, inter:])
    assert torch.equal(gu[:, :inter], dg) and torch.equal(gu[:, inter:], du)
    with pytest.raises(ValueError):  # columns must be whole 16-byte vectors
        torch.ops.talm.swiglu_fwd_rows(gate[:, :12], up[:, :12], out[:, :12])


@pytest.mark.parametrize("n", [1, 7, 8, 9, 1001, 4096 * 3 + 5])
def test_swiglu_tails(n):
    _case(f"swiglu tail n={n}")
    g = torch.Generator().manual_seed(n)
    gate = torch.randn(n, generator=g).half()
    up = torch.randn(n, generator=g).half()
    grad = torch.randn(n, generator=g).half()
    node_gate = gate.to(DEV).requires_grad_()
    node_up = up.to(DEV).requires_grad_()
    out = swiglu.swiglu(node_gate, node_up)
    out.backward(grad.to(DEV))
    assert_rel(out, swiglu_oracle.forward(to_np(gate), to_np(up), np.float64, np.float64),
               rtol=1e-3, what="out")
    rdg, rdu = swiglu_oracle.backward(to_np(grad), to_np(gate), to_np(up), np.float64, np.float64)
    assert_rel(node_gate.grad, rdg, rtol=1e-3, what="dgate")
    assert_rel(node_up.grad, rdu, rtol=1e-3, what="dup")
    # an unaligned view (offset by one element) takes the scalar path
    big = torch.randn(n + 1, generator=g).half().to(DEV)
    o2 = torch.empty(n, dtype=torch.float16, device=DEV)
    swiglu.swiglu_fwd(big[1:], big[1:], o2)
    b = to_np(big[1:])
    assert_rel(o2, swiglu_oracle.forward(b, b, np.float64, np.float64), rtol=1e-3, what="view")


@pytest.mark.parametrize("theta,layout", [(1e6, "packed"), (10000.0, "rows")])
def test_rotary_tables_equal_transformers(theta, layout):
    """talm_rope_table: cos / sin of transformers' Qwen2RotaryEmbedding.forward (default type)
    for packed positions (rows restarting at 0, a pad sequence) and for padded rows, bit for bit
    (the same fp32 products, the same libm cos / sin, the same scaling)."""
    from transformers.models.qwen2 import modeling_qwen2

    from talm_amd import patches, qlora_model, rope

    print(f"[case] rotary tables theta={theta} {layout}", flush=True)
    config = qlora_model.qwen2_config(rope_theta=theta)
    module = modeling_qwen2.Qwen2RotaryEmbedding(config).cuda()
    if layout == "packed":
        pos = torch.cat([torch.arange(n) for n in (300, 128, 512, 257, 16)])[None]
    else:
        pos = torch.arange(512).repeat(4, 1)
    pos = pos.cuda()
    x = torch.empty(1, dtype=torch.float32, device="cuda")
    original = patches._root(modeling_qwen2.Qwen2RotaryEmbedding.forward)
    want_cos, want_sin = original(module, x, pos)
    got_cos, got_sin = rope.rope_tables(module, pos)
    assert got_cos.shape == want_cos.shape and got_cos.dtype == want_cos.dtype
    assert torch.equal(got_cos, want_cos) and torch.equal(got_sin, want_sin)
