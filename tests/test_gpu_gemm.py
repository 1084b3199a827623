"""torch.ops.talm.gemm: the layer group's plain fp16 GEMMs on hipBLASLt with cached plans
(y = x W^T + b forward, dx = dy W backward; solution/qgroup.py:346-355), against an fp32 torch
reference of the same product. fp16 output of an fp32-accumulated product: the tolerance is a
few fp16 ulps of the output magnitude plus the accumulation-order term of K products."""

import pytest
import torch

pytestmark = pytest.mark.gpu


def _ref(a, b, bias, b_t):
    r = a.float() @ (b.float().t() if b_t else b.float())
    return r + bias.float() if bias is not None else r


def _close(out, ref, k):
    tol = 4e-3 * ref.abs().amax().item() + 1e-3 * k ** 0.5 * 2 ** -10
    err = (out.float() - ref).abs().max().item()
    assert err <= tol, f"max error {err} > {tol}"


@pytest.mark.parametrize("m,n,k,b_t,with_bias", [
    (1167, 1536, 1536, 1, False),   # o_proj forward at a config-5 token count
    (1167, 17920, 1536, 1, False),  # gate|up forward
    (1167, 1536, 8960, 1, True),    # down forward, with a bias
    (1167, 1536, 8960, 0, False),   # gate backward: dy [M, 8960] W [8960, 1536]
    (1, 256, 64, 1, True),
    (33, 40, 24, 0, False),
])
def test_gemm_matches_fp32_reference(m, n, k, b_t, with_bias):
    import talm_amd._ops  # noqa: F401

    g = torch.Generator("cpu").manual_seed(m * 7 + n + k)
    a = torch.randn(m, k, generator=g).half().cuda()
    b = (torch.randn(n, k, generator=g) * 0.05).half().cuda() if b_t else \
        (torch.randn(k, n, generator=g) * 0.05).half().cuda()
    bias = torch.randn(n, generator=g).half().cuda() if with_bias else None
    out = torch.empty(m, n, dtype=torch.float16, device="cuda")
    torch.ops.talm.gemm(a, b, bias, b_t, out)
    torch.cuda.synchronize()
    _close(out, _ref(a, b, bias, b_t), k)


def test_gemm_strided_rows_and_plan_reuse():
    """Row strides wider than the row (views of a wider buffer), and three calls in a row with
    token counts that change, one repeated (the cached plan of an earlier shape is reused)."""
    import talm_amd._ops  # noqa: F401

    g = torch.Generator("cpu").manual_seed(5)
    w = (torch.randn(384, 512, generator=g) * 0.05).half().cuda()
    for m in (700, 1024, 700):
        big = torch.randn(m, 640, generator=g).half().cuda()
        a = big[:, 64:576]                       # [m, 512], row stride 640
        out_big = torch.zeros(m, 400, dtype=torch.float16, device="cuda")
        out = out_big[:, :384]                   # [m, 384], row stride 400
        torch.ops.talm.gemm(a, w, None, 1, out)
        torch.cuda.synchronize()
        _close(out, _ref(a, w, None, 1), 512)
        assert torch.all(out_big[:, 384:] == 0)  # nothing written past the view


def test_gemm_rejects_bad_shapes():
    import talm_amd._ops  # noqa: F401

    a = torch.zeros(8, 16, dtype=torch.float16, device="cuda")
    b = torch.zeros(4, 16, dtype=torch.float16, device="cuda")
    with pytest.raises(ValueError):
        torch.ops.talm.gemm(a, b, None, 1, torch.empty(8, 5, dtype=torch.float16, device="cuda"))
    with pytest.raises(ValueError):
        torch.ops.talm.gemm(a.float(), b, None, 1,
                            torch.empty(8, 4, dtype=torch.float16, device="cuda"))


def _colmajor(buf, rows, cols, ld):
    """The column-major rows x cols matrix with leading dimension ld at the start of buf."""
    return buf[:cols * ld].view(cols, ld)[:, :rows].t()


def test_measured_table_products_match_reference():
    """Each product form of the measured hipBLASLt table (gemm_tuning.product_forms) through
    gemm_ex with the table installed, then with hipBLASLt's heuristic (empty table): both within
    the fp32-reference tolerance, at a bucket's middle and at an odd token count. The table is
    the one committed for this hipBLASLt and architecture, so load() installs rows."""
    import talm_amd._ops  # noqa: F401
    from talm_amd import gemm_tuning

    try:
        assert gemm_tuning.load() > 0, "the committed table does not match this hipBLASLt"
        for name, ta, tb, m, k, lda, ldb, ldd in gemm_tuning.product_forms():
            for n in (1216, 1167):
                g = torch.Generator("cpu").manual_seed(n + m + k + ta)
                a = (torch.randn((m if ta else k) * lda, generator=g) * 0.05).half().cuda()
                b = torch.randn((k if tb else n) * ldb, generator=g).half().cuda()
                ma = _colmajor(a, k if ta else m, m if ta else k, lda).float()
                mb = _colmajor(b, n if tb else k, k if tb else n, ldb).float()
                ref = (ma.t() if ta else ma) @ (mb.t() if tb else mb)
                for installed in (True, False):
                    if not installed:
                        torch.ops.talm.gemm_algo_table(torch.empty(0, 7, dtype=torch.int64))
                    d = torch.zeros(n * ldd, dtype=torch.float16, device="cuda")
                    torch.ops.talm.gemm_ex(a, ta, b, tb, d, m, n, k, lda, ldb, ldd, 0)
                    torch.cuda.synchronize()
                    _close(_colmajor(d, m, n, ldd), ref, k)
                    assert torch.all(d.view(n, ldd)[:, m:] == 0), name
                gemm_tuning.load()
    finally:
        torch.ops.talm.gemm_algo_table(torch.empty(0, 7, dtype=torch.int64))


@pytest.mark.parametrize("m,n,k,lda_pad,ldo_pad", [
    (1312, 1536, 8960, 0, 0),     # the MLP's down projection at a config-5 token count
    (1312, 1536, 17920, 0, 0),    # its input gradient on the transposed gate|up weight
    (2048, 1536, 17920, 8, 16),   # the largest bucket, strided operands
    (37, 24, 136, 0, 8),          # one partial tile, one K part
    (513, 1000, 4096, 24, 0),     # partial row and column tiles, several parts
    (1, 8, 8, 0, 0),
])
def test_gemm_splitk_matches_fp32_reference(m, n, k, lda_pad, ldo_pad):
    """talm_gemm_splitk (K parts on the MFMA tile core, fp32 partials summed in part order)
    against the fp32 product; a second call gives the same bits (no atomics, fixed order)."""
    from talm_amd import _ops

    g = torch.Generator("cpu").manual_seed(m + 3 * n + k)
    a_full = torch.randn(m, k + lda_pad, generator=g).half().cuda()
    a = a_full[:, :k]
    b = (torch.randn(n, k, generator=g) * 0.05).half().cuda()
    out_full = torch.full((m, n + ldo_pad), float("nan"), dtype=torch.float16, device="cuda")
    out = out_full[:, :n]
    ws = torch.empty(_ops.gemm_splitk_workspace_bytes(m, n, k), dtype=torch.uint8, device="cuda")
    torch.ops.talm.gemm_splitk(a, b, out, ws)
    ref = a.float() @ b.float().t()
    _close(out, ref, k)
    again = torch.empty_like(out)
    torch.ops.talm.gemm_splitk(a, b, again, ws)
    assert torch.equal(again, out)
    if ldo_pad:
        assert torch.isnan(out_full[:, n:].float()).all(), "columns past n were written"


def test_gemm_splitk_rejects_bad_shapes():
    from talm_amd import _ops

    a = torch.zeros(4, 12, dtype=torch.float16, device="cuda")  # k not a multiple of 8
    b = torch.zeros(8, 12, dtype=torch.float16, device="cuda")
    out = torch.empty(4, 8, dtype=torch.float16, device="cuda")
    with pytest.raises(ValueError):
        _ops.gemm_splitk_workspace_bytes(4, 8, 12)
    with pytest.raises(ValueError):
        torch.ops.talm.gemm_splitk(a, b, out, torch.empty(1 << 16, dtype=torch.uint8,
                                                          device="cuda"))
