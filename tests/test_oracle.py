"""Pins of the CPU oracle (oracle/): each restatement is checked against something that a plausible
mistake (a dropped term, a swapped nibble, a fused multiply-add, a wrong sign or index) would
fail — closed forms, invariants, finite differences, the reference tests' known-answer
constructions — never against a retyped copy of its own formula."""

import numpy as np
import pytest
import torch

from oracle import codebook, head, nf4, norm, pack, rope, swiglu
from talm_amd import quant


# ----------------------------------------------------------------------------------- NF4 -----

def test_nf4_levels_are_the_qlora_normal_quantiles():
    """The reference's hard-coded table (solution/qgroup.py:60-63) is QLoRA's construction to
    float32 precision; the product's table is the same numbers."""
    built = codebook.nf4_levels_from_quantiles()
    assert np.abs(codebook.NF4_LEVELS.astype(np.float64) - built).max() < 2e-7
    assert np.array_equal(np.array(quant.NF4_LEVELS, np.float32), codebook.NF4_LEVELS)
    assert codebook.NF4_LEVELS[0] == -1.0 and codebook.NF4_LEVELS[7] == 0.0
    assert codebook.NF4_LEVELS[15] == 1.0 and np.all(np.diff(codebook.NF4_LEVELS) > 0)


def _f16_cases():
    rng = np.random.default_rng(0)
    bits = rng.integers(0, 2 ** 32, 400_000, dtype=np.uint64).astype(np.uint32)
    finite = bits.view(np.float32)
    h = np.arange(0, 0x7c00, dtype=np.uint16).view(np.float16).astype(np.float32)
    nxt = np.nextafter(h, np.float32(np.inf))
    mid = ((h.astype(np.float64)[:-1] + h.astype(np.float64)[1:]) / 2).astype(np.float32)
    special = np.array([0.0, -0.0, 65504, 65519.99, 65520, 65536, 1e30, np.inf, -np.inf,
                        2.0 ** -24, 2.0 ** -25, 2.0 ** -25 * 1.0000001, 2.0 ** -26, 2.0 ** -14,
                        2.0 ** -14 * 0.99999, 6.0e-8, 5.9e-8], np.float32)
    return np.concatenate([finite, h, -h, nxt, mid, -mid, special])


def test_f32_to_f16_is_ieee_round_to_nearest_even():
    """The C oracle's conversion against numpy's IEEE cast on random bit patterns, every fp16
    value, its successor, every midpoint (ties to even), subnormals and overflow."""
    x = _f16_cases()
    ours = nf4.f32_to_f16_bits(x)
    with np.errstate(over="ignore"):
        ref = x.astype(np.float16)
    nan = np.isnan(ref)
    assert np.array_equal(ours[~nan], ref[~nan].view(np.uint16))
    assert np.all(np.isnan(ours[nan].view(np.float16)))


def test_group_scale_is_rounded_twice_not_fused():
    """Blocks whose fp16 output differs between fl(fl(code*absmax2) + offset) and a fused
    fl(code*absmax2 + offset): the oracle gives the twice-rounded value
    (solution/qgroup.py:19-21, :99 enable_fp_fusion=False)."""
    rng = np.random.default_rng(1)
    n = 2_000_000
    code = rng.uniform(-1, 1, n).astype(np.float32)
    a2 = rng.uniform(0.005, 0.05, n).astype(np.float32)
    off = rng.uniform(0.005, 0.02, n).astype(np.float32)
    twice = (code * a2 + off).astype(np.float32)  # numpy rounds the product, then the sum
    fused = (code.astype(np.float64) * a2 + off).astype(np.float32)  # exact product, one rounding
    differs = (twice.astype(np.float16) != fused.astype(np.float16))
    idx = np.nonzero(differs)[0][:16]
    assert len(idx) >= 4
    for i in idx:
        table = np.zeros(256, np.float32)
        table[7] = code[i]
        packed = np.full(32, 0xFF, np.uint8)  # level 15 = 1.0: out = fp16(scale)
        out = nf4.group_dequant(packed, np.array([7], np.uint8), table, a2[i:i + 1], off[i:i + 1],
                                64, 256)
        assert np.all(out == twice[i:i + 1].astype(np.float16).view(np.uint16))
        assert np.all(out != fused[i:i + 1].astype(np.float16).view(np.uint16))


def test_nibble_order_high_first():
    """solution/test_fuzz.py:860-868: element 2i is levels[byte >> 4], element 2i+1 levels[byte
    & 15]. Byte 0x0F with scale 1 gives (-1, 1); 0xF0 gives (1, -1)."""
    absmax = np.ones(1, np.float32)
    out = nf4.dequant(np.array([0x0F, 0xF0, 0x78], np.uint8), absmax, 64, 6).view(np.float16)
    assert out.tolist() == [-1.0, 1.0, 1.0, -1.0, 0.0, np.float16(0.07958029955625534)]


def test_group_oracle_c_equals_numpy_and_per_projection():
    """C and numpy twins agree bit for bit; the grouped form equals the per-projection form fed
    with the fp32 absmax that bitsandbytes' dequantize_blockwise + offset returns (the identity
    the reference asserts between its group kernel and bitsandbytes)."""
    rng = np.random.default_rng(2)
    n_rows = 3 * 256 + 256
    packed = rng.integers(0, 256, n_rows * 32, dtype=np.uint8)
    absmax8 = rng.integers(0, 256, n_rows, dtype=np.uint8)
    code = quant.dynamic_map().numpy()
    absmax2 = rng.uniform(0.005, 0.05, n_rows // 256).astype(np.float32)
    offset2 = np.array([0.01, 0.02, 0.03, -0.004], np.float32)
    c_out = nf4.group_dequant(packed, absmax8, code, absmax2, offset2)
    np_out = nf4.group_dequant_np(packed, absmax8, code, absmax2, offset2)
    assert np.array_equal(c_out, np_out)
    blk2 = np.arange(n_rows) // 256
    absmax32 = (code[absmax8] * absmax2[blk2] + offset2[blk2]).astype(np.float32)
    assert np.array_equal(nf4.dequant(packed, absmax32, 64, n_rows * 64), c_out)
    assert np.array_equal(nf4.dequant_np(packed, absmax32, 64, n_rows * 64), c_out)


def test_group_oracle_subnormal_outputs():
    """Scales near zero give fp16 subnormal weights: kept, not flushed."""
    table = np.zeros(256, np.float32)
    table[1] = -0.2
    packed = np.arange(32, dtype=np.uint8) * 8
    out = nf4.group_dequant(packed, np.array([1], np.uint8), table,
                            np.array([0.05], np.float32), np.array([0.0100001], np.float32))
    vals = out.view(np.float16).astype(np.float32)
    sub = (np.abs(vals) > 0) & (np.abs(vals) < 2.0 ** -14)
    assert sub.any()


# ------------------------------------------------------------------------------- RMSNorm -----

def test_rmsnorm_forward_closed_form_and_invariant():
    rng = np.random.default_rng(3)
    x = rng.standard_normal((7, 1536)).astype(np.float16)
    p = rng.standard_normal((7, 1536)).astype(np.float16)
    w = (1 + 0.1 * rng.standard_normal(1536)).astype(np.float32)
    q, y, xhat, rstd = norm.forward(x, w, 1e-6, p=p, x_dtype=np.float32, out_dtype=np.float32)
    s = x.astype(np.float64) + p.astype(np.float64)
    assert np.array_equal(q, s.astype(np.float32))
    r64 = 1 / np.sqrt((s * s).mean(-1) + 1e-6)
    np.testing.assert_allclose(rstd, r64, rtol=2e-6)
    np.testing.assert_allclose(y, w * s * r64[:, None], rtol=2e-5, atol=1e-6)
    # mean(xhat^2) = var / (var + eps)
    var = (s * s).mean(-1)
    np.testing.assert_allclose((xhat.astype(np.float64) ** 2).mean(-1), var / (var + 1e-6),
                               rtol=2e-5)
    # scale invariance (eps = 0): rmsnorm(c x) = rmsnorm(x)
    _, y2, _, _ = norm.forward(3.0 * s, w, 0.0, out_dtype=np.float64, dtype=np.float64)
    _, y1, _, _ = norm.forward(s, w, 0.0, out_dtype=np.float64, dtype=np.float64)
    np.testing.assert_allclose(y2, y1, rtol=1e-12)


def test_rmsnorm_backward_matches_finite_differences():
    rng = np.random.default_rng(4)
    h, eps = 24, 1e-3
    x = rng.standard_normal((3, h))
    w = 1 + 0.1 * rng.standard_normal(h)
    dy = rng.standard_normal((3, h))
    ds = rng.standard_normal((3, h))

    def loss(xv):
        _, y, _, _ = norm.forward(xv, w, eps, out_dtype=np.float64, dtype=np.float64)
        return (dy * y).sum() + (ds * xv).sum()

    fd = np.zeros_like(x)
    step = 1e-6
    for idx in np.ndindex(x.shape):
        e = np.zeros_like(x)
        e[idx] = step
        fd[idx] = (loss(x + e) - loss(x - e)) / (2 * step)
    _, _, xhat, rstd = norm.forward(x, w, eps, out_dtype=np.float64, dtype=np.float64)
    dx, db = norm.backward(dy, xhat, w, rstd.astype(np.float64), ds=ds, x_dtype=np.float64,
                           out_dtype=np.float64, dtype=np.float64)
    np.testing.assert_allclose(dx, fd, rtol=1e-5, atol=1e-7)
    assert np.array_equal(dx, db)


# ---------------------------------------------------------------------------------- RoPE -----

def _cos_sin(n, d, theta=1e6, seed=5):
    from talm_amd.workloads import rope_cos_sin

    pos = torch.from_numpy(np.random.default_rng(seed).integers(0, 512, n))
    c, s = rope_cos_sin(pos, d, theta)
    return c.numpy(), s.numpy()


def test_rope_forward_is_complex_rotation_and_transformers_form():
    rng = np.random.default_rng(6)
    n, heads, d = 9, 3, 16
    x = rng.standard_normal((n, heads, d))
    c, s = _cos_sin(n, d)
    y = rope.rotate(x, c, s, out_dtype=np.float64, dtype=np.float64)
    half = d // 2
    z = (x[..., :half] + 1j * x[..., half:]) * np.exp(1j * np.arctan2(s[:, None, :half],
                                                                      c[:, None, :half]))
    np.testing.assert_allclose(y, np.concatenate([z.real, z.imag], -1), rtol=1e-6, atol=1e-6)
    # transformers' apply_rotary_pos_emb: q * cos + rotate_half(q) * sin (what the patch replaces)
    from transformers.models.qwen2.modeling_qwen2 import apply_rotary_pos_emb

    q = torch.from_numpy(x).permute(1, 0, 2)[None]  # [1, H, N, D]
    ref, _ = apply_rotary_pos_emb(q, q, torch.from_numpy(c)[None].double(),
                                  torch.from_numpy(s)[None].double())
    np.testing.assert_allclose(y, ref[0].permute(1, 0, 2).numpy(), rtol=1e-12, atol=1e-12)


def test_rope_identity_at_position_zero_and_backward_is_adjoint():
    rng = np.random.default_rng(7)
    n, heads, d = 5, 2, 8
    x = rng.standard_normal((n, heads, d))
    ones, zeros = np.ones((n, d)), np.zeros((n, d))
    assert np.array_equal(rope.rotate(x, ones, zeros, out_dtype=np.float64, dtype=np.float64), x)
    # general (c1 != c2) tables: <R x, g> = <x, R^T g>
    c = rng.standard_normal((n, d))
    s = rng.standard_normal((n, d))
    g = rng.standard_normal((n, heads, d))
    fwd = rope.rotate(x, c, s, False, np.float64, np.float64)
    bwd = rope.rotate(g, c, s, True, np.float64, np.float64)
    assert abs((fwd * g).sum() - (x * bwd).sum()) < 1e-10


# -------------------------------------------------------------------------------- SwiGLU -----

def test_swiglu_forward_closed_form_and_backward_finite_differences():
    rng = np.random.default_rng(8)
    gate = rng.standard_normal(64) * 3
    up = rng.standard_normal(64)
    grad = rng.standard_normal(64)
    out = swiglu.forward(gate, up, np.float64, np.float64)
    silu = torch.nn.functional.silu(torch.from_numpy(gate)).numpy()
    np.testing.assert_allclose(out, silu * up, rtol=1e-12)
    dgate, dup = swiglu.backward(grad, gate, up, np.float64, np.float64)
    step = 1e-6
    fd_g = ((swiglu.forward(gate + step, up, np.float64, np.float64)
             - swiglu.forward(gate - step, up, np.float64, np.float64)) / (2 * step)) * grad
    fd_u = ((swiglu.forward(gate, up + step, np.float64, np.float64)
             - swiglu.forward(gate, up - step, np.float64, np.float64)) / (2 * step)) * grad
    np.testing.assert_allclose(dgate, fd_g, rtol=1e-6, atol=1e-9)
    np.testing.assert_allclose(dup, fd_u, rtol=1e-6, atol=1e-9)
    z_dg, z_du = swiglu.backward(np.ones(1), np.zeros(1), np.full(1, 2.0), np.float64, np.float64)
    assert z_dg[0] == 1.0 and z_du[0] == 0.0  # gate = 0: dgate = g * up / 2, dup = 0


# ---------------------------------------------------------------------------------- head -----

def exact_head_case(n, hidden, vocab, seed, lab_frac=0.6, peak=2):
    """Exact-style inputs (solution/test_fuzz.py:225-256): {-1, 0, 1} times a power of two per
    row, so every logit is exact in fp16 whatever the summation order."""
    rng = np.random.default_rng(seed)
    a = rng.integers(-3, 1 + peak, (n, 1)).astype(np.float64)
    b = rng.integers(-6, -1, (vocab, 1)).astype(np.float64)
    h = rng.integers(-1, 2, (n, hidden)) * np.exp2(a)
    w = rng.integers(-1, 2, (vocab, hidden)) * np.exp2(b)
    targets = rng.integers(0, vocab, n)
    targets[rng.random(n) > lab_frac] = -100
    sure = (targets >= 0) & (rng.random(n) < 0.4)
    h[sure] = np.sign(w[targets[sure]]) * np.exp2(a[sure])
    return h.astype(np.float16), w.astype(np.float16), targets


def test_head_online_statistics_match_closed_form():
    """The vocabulary-sliced online algorithm (any slice / block width) gives the closed-form
    loss, entropy and first argmax over the same fp16 logits, and its gradient."""
    h, w, t = exact_head_case(37, 64, 4097, seed=9)
    ref = head.head_direct(h, w, t)
    for vchunk, block, slack in ((8192, 4096, 1), (4096, 4096, 1), (1000, 7, 4), (5, 3, 4)):
        out = head.head_ce(h, w, t, vchunk=vchunk, block=block)
        # the reference's fuzz bounds for fp32 statistics (solution/test_fuzz.py:293-297); the
        # degenerate widths (over a thousand online merges per row) get `slack` times them
        tol_loss = slack * (2e-5 + 2e-6 * ref["zmax"])
        tol_ent = slack * (2e-5 + 1e-5 * ref["zmax"])
        assert np.all(np.abs(out["token_loss"] - ref["token_loss"]) <= tol_loss)
        assert np.all(np.abs(out["entropy"] - ref["entropy"]) <= tol_ent)
        assert np.array_equal(out["best_idx"], ref["best_idx"])
        assert np.array_equal(out["correct"], ref["correct"])
        tol = 2e-3 * np.abs(ref["grad"]).max()
        np.testing.assert_allclose(out["grad"].astype(np.float64), ref["grad"], atol=tol)
        assert (out["grad"][t < 0] == 0).all() and (out["token_loss"][t < 0] == 0).all()


def test_head_gradient_matches_finite_differences():
    """d/dh of sum over labelled rows of (lse(h W^T) - h . W[y]) (no fp16 rounding) equals
    (softmax - onehot) W, the closed form the oracle's gradient follows."""
    rng = np.random.default_rng(10)
    n, hidden, vocab = 3, 5, 11
    h = rng.standard_normal((n, hidden))
    w = rng.standard_normal((vocab, hidden)) * 0.5
    t = np.array([2, -100, 10])

    def loss(hv):
        z = hv @ w.T
        lse = np.log(np.exp(z).sum(1))
        lab = t >= 0
        return (lse[lab] - z[lab, t[lab]]).sum()

    fd = np.zeros_like(h)
    for idx in np.ndindex(h.shape):
        e = np.zeros_like(h)
        e[idx] = 1e-6
        fd[idx] = (loss(h + e) - loss(h - e)) / 2e-6
    z = h @ w.T
    p = np.exp(z - z.max(1, keepdims=True))
    p /= p.sum(1, keepdims=True)
    p[np.arange(n), np.maximum(t, 0)] -= t >= 0
    p[t < 0] = 0
    np.testing.assert_allclose(p @ w, fd, rtol=1e-6, atol=1e-8)
    # head_direct computes that same gradient when its logits are exact in fp16
    hh, ww, tt = exact_head_case(4, 16, 50, seed=11)
    z = hh.astype(np.float64) @ ww.astype(np.float64).T
    p = np.exp(z - z.max(1, keepdims=True))
    p /= p.sum(1, keepdims=True)
    p[np.arange(4), np.maximum(tt, 0)] -= tt >= 0
    p[tt < 0] = 0
    np.testing.assert_allclose(head.head_direct(hh, ww, tt)["grad"], p @ ww.astype(np.float64),
                               rtol=1e-12, atol=1e-14)


def test_head_argmax_ties_report_the_first_column():
    """solution/test_kernels.py:250-282: two equal largest logits (exactly 64) inside one block,
    across blocks and across slices: the first column wins (torch.argmax's rule)."""
    rng = np.random.default_rng(12)
    vocab, hidden = 9000, 256
    pairs = [(4106, 4116), (1000, 5096), (100, 8242), (vocab - 4000, vocab - 1)]
    w = (rng.standard_normal((vocab, hidden)) * 0.05).astype(np.float16)
    h = (rng.standard_normal((2 * len(pairs), hidden)) * 2).astype(np.float16)
    t = np.zeros(2 * len(pairs), np.int64)
    for i, (a, b) in enumerate(pairs):
        signs = rng.integers(0, 2, hidden) * 2 - 1
        w[a] = w[b] = (signs / 16).astype(np.float16)
        h[2 * i] = h[2 * i + 1] = (signs * 4).astype(np.float16)
        t[2 * i], t[2 * i + 1] = a, b
    z = head.logits16(h, w).astype(np.float32)
    for i, (a, b) in enumerate(pairs):
        assert z[2 * i, a] == z[2 * i, b] == z[2 * i].max() == 64
    out = head.head_ce(h, w, t, vchunk=8192, block=4096, need_grad=False)
    assert out["correct"].tolist() == [True, False] * len(pairs)
    assert out["best_idx"].tolist() == [a for a, _ in pairs for _ in range(2)]


def test_head_planted_hits_and_label_shift():
    """solution/test_kernels.py:104-131 (boundary columns, planted hits) and :497-519 (labels
    shifted by one, the last position and ignored labels score 0)."""
    rng = np.random.default_rng(13)
    vocab, hidden, vchunk, block = 4097, 64, 4096, 4096
    w = (rng.standard_normal((vocab, hidden)) * 0.05).astype(np.float16)
    columns = [0, block - 1, vchunk - 1, vchunk, vocab - 1]
    batch, seq = 2, len(columns) + 2
    labels = rng.integers(0, vocab, (batch, seq))
    h = (rng.standard_normal((batch * seq, hidden))).astype(np.float16)
    labels[1, 4:] = -100
    shift = np.concatenate([labels[:, 1:], np.full((batch, 1), -100)], 1).reshape(-1)
    for i, col in enumerate(columns):  # row i predicts `col` and is labelled with it
        h[i] = (w[col].astype(np.float32) * 40).astype(np.float16)
        shift[i] = col
    out = head.head_ce(h, w, shift, vchunk=vchunk, block=block)
    assert out["correct"][:len(columns)].all()
    tl = out["token_loss"].reshape(batch, seq)
    assert (tl[:, -1] == 0).all() and (tl[1, 3:] == 0).all() and (tl[0, :-1] > 0).all()
    loss, denom = head.loss(out["token_loss"], shift)
    assert denom == (shift >= 0).sum()
    loss7, denom7 = head.loss(out["token_loss"], shift, num_items=7)
    assert denom7 == 7.0 and abs(loss7 * 7 - loss * denom) < 1e-9


@pytest.mark.parametrize("n_lab", [0, 1])
def test_head_no_labels_and_single_label(n_lab):
    h, w, _ = exact_head_case(6, 32, 300, seed=14)
    t = np.full(6, -100)
    t[:n_lab] = 17
    out = head.head_ce(h, w, t, vchunk=128, block=64)
    assert (out["grad"][n_lab:] == 0).all() and (out["token_loss"][n_lab:] == 0).all()
    ref = head.head_direct(h, w, t)
    assert np.all(np.abs(out["entropy"] - ref["entropy"]) <= 2e-5 + 1e-5 * ref["zmax"])


def test_torch_cpu_dequant_equals_the_group_oracle():
    """The PyTorch CPU restatement bench.py's CPU baseline runs equals the C oracle bit for bit
    on a quantized projection (bitsandbytes' QuantState layout of nf4_linear.Linear4bit)."""
    from talm_amd.nf4_linear import Linear4bit

    g = torch.Generator().manual_seed(5)
    layer = Linear4bit.from_weight(torch.randn(256, 128, generator=g) * 0.05)
    state = layer.weight.quant_state
    ours = nf4.dequant_state_torch(layer.weight.data, state)
    n_blk2 = state.absmax.numel() // state.state2.blocksize
    ref = nf4.group_dequant(layer.weight.data.numpy(), state.absmax.numpy(),
                            state.state2.code.numpy(), state.state2.absmax.numpy(),
                            np.full(n_blk2, float(state.offset), np.float32))
    assert np.array_equal(ours.view(torch.int16).numpy().view(np.uint16).reshape(-1), ref)


# ---------------------------------------------------------------------------- batch packing -----

def _batch(seed, batch, seq, lengths=None, vocab=1000):
    rng = np.random.default_rng(seed)
    if lengths is None:
        lengths = rng.integers(0, seq + 1, batch)
    mask = (np.arange(seq)[None] < np.asarray(lengths)[:, None]).astype(np.int64)
    ids = rng.integers(0, vocab, (batch, seq))
    labels = np.where(mask == 1, ids, -100)
    labels[rng.random((batch, seq)) < 0.2] = -100  # some real tokens unlabelled
    return ids, mask, labels


def test_pack_rows_known_answer():
    """A 3 x 4 batch worked by hand: rows of 2, 0 and 3 tokens packed into 7 rows."""
    ids = np.array([[11, 12, 0, 0], [21, 22, 23, 24], [31, 32, 33, 0]])
    mask = np.array([[1, 1, 0, 0], [0, 0, 0, 0], [1, 1, 1, 0]])
    labels = np.array([[11, 12, -100, -100], [-100] * 4, [31, -100, 33, -100]])
    got = pack.pack_rows(ids, mask, labels, 7)
    expect = ([11, 12, 31, 32, 33, 0, 0],          # ids (0 in the pad sequence)
              [0, 1, 0, 1, 2, 0, 1],               # positions (the pad sequence restarts)
              [0, 2, 2, 5, 7],                     # cu_seqlens (row 1 empty)
              [12, -100, -100, 33, -100, -100, -100],  # labels[b][p + 1], -100 at the row end
              [0, 1, 8, 9, 10, 12, 12])            # src (the pad slot is 3 * 4)
    for g, e in zip(got, expect):
        assert g.tolist() == e
    assert pack.row_stats(mask, labels).tolist() == [2, 0, 3, 2, 2]


@pytest.mark.parametrize("batch,seq,seed", [(4, 512, 0), (1, 1, 1), (7, 33, 2), (3, 64, 3)])
def test_pack_rows_equals_the_reference_packing_and_the_torch_form(batch, seq, seed):
    """The fixed-shape packing's real rows are the reference's `unpad_batch` gather (ids, labels
    shifted then gathered, positions); its offsets, pad sequence and truncation equal
    unpad.unpad_static's matrix-and-search formulation run on the CPU, at n_tokens above, at and
    below the real token count."""
    from talm_amd import unpad

    ids, mask, labels = _batch(seed, batch, seq)
    idx, positions, lengths, _counts = pack.unpad_batch(mask, labels)
    total = len(idx)
    shift = pack.shift_labels(labels)
    for n_tokens in sorted({max(total, 1), total + 5, max(total // 2, 1), total + 16}):
        got_ids, got_pos, cu, targets, src = pack.pack_rows(ids, mask, labels, n_tokens)
        keep = min(total, n_tokens)
        assert np.array_equal(src[:keep], idx[:keep])
        assert np.array_equal(got_pos[:keep], positions[:keep])
        assert np.array_equal(got_ids[:keep], ids.reshape(-1)[idx[:keep]])
        assert np.array_equal(targets[:keep], shift[idx[:keep]])
        assert np.all(src[keep:] == batch * seq) and np.all(targets[keep:] == -100)
        t_src, t_pos, t_cu, t_targets = unpad.unpad_static(
            torch.from_numpy(mask), torch.from_numpy(shift), n_tokens)
        assert np.array_equal(t_src.numpy(), src) and np.array_equal(t_cu.numpy(), cu)
        assert np.array_equal(t_pos[0].numpy(), got_pos)
        assert np.array_equal(t_targets.numpy(), targets)
        assert cu[-1] == n_tokens and np.all(np.diff(cu) >= 0)


def test_row_stats_and_scatter_equal_the_torch_forms():
    from talm_amd import unpad

    ids, mask, labels = _batch(5, 6, 40)
    shift = pack.shift_labels(labels)
    expect = unpad._row_values(torch.from_numpy(mask), torch.from_numpy(shift))
    assert pack.row_stats(mask, labels).tolist() == expect.tolist()
    idx, _pos, _l, _c = pack.unpad_batch(mask, labels)
    values = np.random.default_rng(6).standard_normal(len(idx)).astype(np.float32)
    full = torch.zeros(6 * 40).index_copy_(0, torch.from_numpy(idx), torch.from_numpy(values))
    assert np.array_equal(pack.scatter(values, idx, 6 * 40), full.numpy())
