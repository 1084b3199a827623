"""talm_nf4_gemm (products on the NF4 form of a weight W [rows, cols], dequantized inside the
GEMM from its codes and its blocks' absmax decoded by talm_nf4_block_scales) on the config-1
layer's packed buffers, in both forms: the forward x W^T and the input gradient dy W.

The expected weights are the C oracle's (oracle.nf4.group_dequant, solution/qgroup.py:72-91),
computed on the CPU from the same bytes. With x the identity the output is W^T (forward) or W
(input gradient), which must equal the oracle's fp16 weights bit for bit; on random x the output
is within one fp16 rounding of the fp32 product of those weights, for the q|k|v, o, gate|up and
down slices of the layer, ragged token counts and the K-split shapes (down forward, gate|up input
gradient). Two more weights cover the tiles the config-1 layer never reaches: W [520, 2048]
(x W^T with 520 output columns: a 256-row weight tile cut at 8 rows) and W [512, 2112] (dy W
with 2112 output columns: a 256-column tile cut at 64). A second call on the same buffers is
bit-identical (the split-K partials are summed in a fixed order)."""

import functools

import numpy as np
import pytest
import torch

from talm_amd import _ops, workloads

pytestmark = pytest.mark.gpu

# (name, first projection, projections): slices of the packed layer (q, k, v, o, gate, up, down)
SLICES = [("q|k|v", 0, 3), ("o", 3, 1), ("gate|up", 4, 2), ("down", 6, 1)]
# weights whose row / column counts are not multiples of the 256-wide tiles (whole 16384-weight
# groups each): (520 rows, 2048 columns) for x W^T, (512, 2112) for dy W
RAGGED_SHAPES = ((520, 2048), (512, 2112))
RAGGED = [("rows520", 0, 1, False), ("cols2112", 1, 1, True)]


@functools.lru_cache(maxsize=2)
def _layer(shapes=workloads.LAYER_SHAPES):
    """(host buffers, device buffers, expected fp16 weights on the device): the weights are the C
    oracle's, bit patterns computed on the CPU from the bytes the GPU receives."""
    from oracle import nf4 as onf4

    _ops.load()
    d = workloads.nf4_layer(shapes=shapes)
    dev = {k: v.cuda() for k, v in d.items() if torch.is_tensor(v)}
    n = d["n"]
    bits = onf4.group_dequant(d["packed"].numpy(), d["absmax8"].numpy(), d["code"].numpy(),
                              d["absmax2"].numpy(), d["offset2"].numpy(), 64, 256)
    w16 = torch.from_numpy(np.ascontiguousarray(bits).view(np.int16)).view(torch.float16).cuda()
    assert w16.numel() == n
    dev["scale"] = torch.empty(n // 64, dtype=torch.float32, device="cuda")
    torch.ops.talm.nf4_block_scales(dev["absmax8"], dev["code"], dev["absmax2"], dev["offset2"],
                                    256, dev["scale"])
    return d, dev, w16


def _slice(d, dev, w16, first, count):
    shapes = d["shapes"]
    e0 = sum(a * b for a, b in shapes[:first])
    rows = sum(shapes[i][0] for i in range(first, first + count))
    cols = shapes[first][1]
    assert e0 % 16384 == 0
    parts = dict(packed=dev["packed"][e0 // 2:], scale=dev["scale"][e0 // 64:])
    return parts, w16[e0:e0 + rows * cols].view(rows, cols), rows, cols


def _gemm(x, parts, rows, cols, transpose, out=None):
    n_out = cols if transpose else rows
    if out is None:
        out = torch.full((x.shape[0], n_out), float("nan"), dtype=torch.float16, device="cuda")
    ws = torch.empty(_ops.nf4_gemm_workspace_bytes(x.shape[0], rows, cols, transpose),
                     dtype=torch.uint8, device="cuda")
    torch.ops.talm.nf4_gemm(x, parts["packed"], parts["scale"], rows, cols, transpose, 64, out, ws)
    return out


def test_block_scales_match_the_oracle():
    """talm_nf4_block_scales: every block's decoded absmax of the config-1 layer, bit for bit the
    oracle's (the scale the group dequant multiplies the levels by)."""
    from oracle import nf4 as onf4

    print("[case] nf4_block_scales config-1 layer", flush=True)
    d, dev, _w16 = _layer()
    want = onf4.block_scales_np(d["absmax8"].numpy(), d["code"].numpy(), d["absmax2"].numpy(),
                                d["offset2"].numpy())
    got = dev["scale"].cpu().numpy()
    assert got.shape == want.shape
    assert (got.view("uint32") == want.view("uint32")).all()


@pytest.mark.parametrize("transpose", [False, True], ids=["xWt", "dyW"])
@pytest.mark.parametrize("name,first,count", SLICES)
def test_identity_input_gives_the_dequantized_weights(name, first, count, transpose):
    print(f"[case] nf4_gemm identity {name} transpose={transpose}", flush=True)
    d, dev, w16 = _layer()
    _check_identity(*_slice(d, dev, w16, first, count), transpose)


def _check_identity(parts, w, rows, cols, transpose):
    k = rows if transpose else cols
    eye = torch.eye(k, dtype=torch.float16, device="cuda")
    out = _gemm(eye, parts, rows, cols, transpose)
    # every output is 1 * w plus exact zeros: the weight's value exactly (a weight of -0, from a
    # negative block scale times the 0 level, sums to +0 with the other zero products)
    want = w if transpose else w.t().contiguous()
    same = out.view(torch.int16) == want.view(torch.int16)
    assert bool((same | ((out == 0) & (want == 0))).all()), int((~same).sum())


@pytest.mark.parametrize("transpose", [False, True], ids=["xWt", "dyW"])
@pytest.mark.parametrize("name,first,count", SLICES)
@pytest.mark.parametrize("n_tok", [1, 37, 333, 1367])
def test_matches_fp32_product_of_dequantized_weights(name, first, count, n_tok, transpose):
    print(f"[case] nf4_gemm {name} tokens={n_tok} transpose={transpose}", flush=True)
    d, dev, w16 = _layer()
    _check_product(*_slice(d, dev, w16, first, count), transpose, n_tok)


def _check_product(parts, w, rows, cols, transpose, n_tok):
    g = torch.Generator().manual_seed(n_tok)
    k = rows if transpose else cols
    x = torch.randn(n_tok, k, generator=g).half().cuda()
    out = _gemm(x, parts, rows, cols, transpose)
    ref = x.float() @ (w.float() if transpose else w.float().t())
    torch.testing.assert_close(out.float(), ref, rtol=2 ** -10,
                               atol=2 ** -11 * float(ref.abs().max()))
    again = _gemm(x, parts, rows, cols, transpose)
    assert torch.equal(again.view(torch.int16), out.view(torch.int16))


@pytest.mark.parametrize("name,first,count,transpose", RAGGED)
def test_ragged_weight_tiles_identity(name, first, count, transpose):
    print(f"[case] nf4_gemm identity ragged {name} transpose={transpose}", flush=True)
    d, dev, w16 = _layer(RAGGED_SHAPES)
    _check_identity(*_slice(d, dev, w16, first, count), transpose)


@pytest.mark.parametrize("n_tok", [5, 300, 1301])
@pytest.mark.parametrize("name,first,count,transpose", RAGGED)
def test_ragged_weight_tiles_product(name, first, count, transpose, n_tok):
    print(f"[case] nf4_gemm ragged {name} tokens={n_tok} transpose={transpose}", flush=True)
    d, dev, w16 = _layer(RAGGED_SHAPES)
    _check_product(*_slice(d, dev, w16, first, count), transpose, n_tok)


def test_row_stride_and_rejects_bad_shapes():
    print("[case] nf4_gemm strides and errors", flush=True)
    d, dev, w16 = _layer()
    parts, w, rows, cols = _slice(d, dev, w16, 4, 2)
    base = torch.randn(300, cols + 64).half().cuda()
    x = base[:, 32:32 + cols]  # row stride cols + 64
    out = torch.empty(300, 2 * rows, dtype=torch.float16, device="cuda")[:, rows:]
    _gemm(x, parts, rows, cols, False, out=out)
    ref = x.float() @ w.float().t()
    torch.testing.assert_close(out.float(), ref, rtol=2 ** -10,
                               atol=2 ** -11 * float(ref.abs().max()))
    ws = torch.empty(0, dtype=torch.uint8, device="cuda")
    with pytest.raises(ValueError):  # block size
        torch.ops.talm.nf4_gemm(x, parts["packed"], parts["scale"], rows, cols, False, 128, out, ws)
    dy = torch.randn(300, rows).half().cuda()
    dx = torch.empty(300, cols, dtype=torch.float16, device="cuda")
    with pytest.raises(ValueError):  # the gate|up input gradient splits K: no workspace given
        torch.ops.talm.nf4_gemm(dy, parts["packed"], parts["scale"], rows, cols, True, 64, dx, ws)



@pytest.mark.parametrize("name,first,count,transpose,n_tok", [
    ("gate|up dy W", 4, 2, True, 1312),   # the MLP block's backward form (7 parts)
    ("down x W^T", 6, 1, False, 1312),
    ("o x W^T", 3, 1, False, 300),        # one part: partials written all the same
])
def test_partials_sum_to_the_product(name, first, count, transpose, n_tok):
    """talm_nf4_gemm_partials: its fp32 partials, summed in part order and rounded, are the
    product talm_nf4_gemm writes, bit for bit."""
    print(f"[case] nf4_gemm_partials {name} tokens={n_tok}", flush=True)
    d, dev, w16 = _layer()
    parts, _w, rows, cols = _slice(d, dev, w16, first, count)
    k = rows if transpose else cols
    x = (torch.randn(n_tok, k, generator=torch.Generator().manual_seed(n_tok)) * 0.5).half().cuda()
    want = _gemm(x, parts, rows, cols, transpose)
    n_parts = _ops.nf4_gemm_parts(n_tok, rows, cols, transpose)
    part = torch.full((n_parts, n_tok, cols if transpose else rows), float("nan"),
                      device="cuda")
    torch.ops.talm.nf4_gemm_partials(x, parts["packed"], parts["scale"], rows, cols, transpose,
                                     64, part)
    total = part[0].clone()
    for p in range(1, n_parts):
        total += part[p]
    assert torch.equal(total.half().view(torch.int16), want.view(torch.int16))
