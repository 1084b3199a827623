"""The packed step's glue kernels (talm_amd/csrc/pack.hip) against the packing oracle
(oracle/pack.py) and the head oracle's loss: bit-exact for the integer work (packing, row
statistics, scatter, counts), the loss within fp32 summation-order rounding, the head backward's
scaling bit-exact against the same fp32 arithmetic in PyTorch (solution/fused_head.py:280-287)."""

import numpy as np
import pytest
import torch

from oracle import head as head_oracle
from oracle import pack

pytestmark = pytest.mark.gpu


def _batch(seed, batch, seq, lengths=None):
    rng = np.random.default_rng(seed)
    if lengths is None:
        lengths = rng.integers(0, seq + 1, batch)
    mask = (np.arange(seq)[None] < np.asarray(lengths)[:, None]).astype(np.int64)
    ids = rng.integers(0, 151936, (batch, seq))
    labels = np.where(mask == 1, ids, -100)
    labels[rng.random((batch, seq)) < 0.2] = -100
    return ids, mask, labels


def _cuda(*arrays):
    return [torch.from_numpy(np.ascontiguousarray(a)).cuda() for a in arrays]


CASES = [  # (seed, batch, seq, lengths or None)
    (0, 4, 512, None),             # config-5 shape
    (1, 4, 512, [512, 512, 512, 512]),  # no padding
    (2, 5, 17, [0, 17, 1, 0, 5]),  # empty rows, a one-token row
    (3, 1, 1, [1]),
    (4, 16, 200, None),
]


@pytest.mark.parametrize("seed,batch,seq,lengths", CASES)
def test_pack_rows_equals_the_oracle(seed, batch, seq, lengths):
    import talm_amd._ops  # noqa: F401

    ids, mask, labels = _batch(seed, batch, seq, lengths)
    total = int(mask.sum())
    print(f"[case] pack_rows seed={seed} batch={batch} seq={seq} tokens={total}", flush=True)
    t_ids, t_mask, t_labels = _cuda(ids, mask, labels)
    for n_tokens in sorted({max(total, 1), total + 16, max(total // 3, 1)}):
        out = [torch.full((n_tokens,), -7, dtype=torch.int64, device="cuda") for _ in range(4)]
        cu = torch.full((batch + 2,), -7, dtype=torch.int32, device="cuda")
        torch.ops.talm.pack_rows(t_ids, t_mask, t_labels, n_tokens, out[0], out[1], cu, out[2],
                                 out[3])
        expect = pack.pack_rows(ids, mask, labels, n_tokens)
        got = (out[0], out[1], cu, out[2], out[3])
        for name, g, e in zip(("ids", "positions", "cu", "targets", "src"), got, expect):
            assert np.array_equal(g.cpu().numpy(), e), (name, n_tokens)


@pytest.mark.parametrize("seed,batch,seq,lengths", CASES)
def test_row_stats_equal_the_oracle(seed, batch, seq, lengths):
    import talm_amd._ops  # noqa: F401

    ids, mask, labels = _batch(seed, batch, seq, lengths)
    t_mask, t_labels = _cuda(mask, labels)
    stats = torch.full((batch + 2,), -7, dtype=torch.int64, device="cuda")
    torch.ops.talm.row_stats(t_mask, t_labels, stats)
    assert stats.cpu().tolist() == pack.row_stats(mask, labels).tolist()


@pytest.mark.parametrize("n,mode", [(1367, 0), (2048, 1), (5, 2), (0, 0), (3000, 0)])
def test_head_loss_and_scatter_equal_the_oracle(n, mode):
    import talm_amd._ops  # noqa: F401

    print(f"[case] head_loss n={n} mode={mode}", flush=True)
    rng = np.random.default_rng(n + mode)
    targets = rng.integers(-1, 3, n) * rng.integers(0, 1000, n)  # about a third negative
    targets = np.where(targets < 0, -100, targets).astype(np.int64)
    token_loss = np.where(targets >= 0, rng.random(n) * 12, 0).astype(np.float32)
    entropy = (rng.random(n) * 11).astype(np.float32)
    correct = (rng.random(n) < 0.1).astype(np.int32) * (targets >= 0)
    num_items = {0: None, 1: 777.0, 2: 1234.5}[mode]
    t_loss, t_ent, t_corr, t_tgt = _cuda(token_loss, entropy, correct.astype(np.int32), targets)
    items = torch.tensor(num_items, dtype=torch.float32, device="cuda") if mode == 1 else None
    loss = torch.empty((), dtype=torch.float32, device="cuda")
    denom = torch.empty_like(loss)
    correct_bool = torch.empty(n, dtype=torch.bool, device="cuda")
    torch.ops.talm.head_loss(t_loss, t_corr, t_tgt, items, num_items or 0.0, mode, loss, denom,
                             correct_bool)
    ref_loss, ref_denom = head_oracle.loss(token_loss, targets, num_items)
    assert float(denom) == np.float32(ref_denom)
    # fp32 tree sum of non-negative terms (a few per thread, then 6 + 16 levels): its rounding
    # stays below 30 x 2^-24 of the sum; the float64 oracle sum is exact to that bar
    assert abs(float(loss) - ref_loss) <= 2e-6 * abs(ref_loss) + 1e-30
    assert np.array_equal(correct_bool.cpu().numpy(), correct != 0)
    # the metrics back to a batch of n + 37 slots (row i -> a distinct slot, 37 left at zero)
    out_len = n + 37
    src = rng.permutation(out_len)[:n].astype(np.int64)
    full_loss = torch.full((out_len,), float("nan"), device="cuda")
    full_ent = torch.full((out_len,), float("nan"), device="cuda")
    stats = torch.empty(2, dtype=torch.int64, device="cuda")
    torch.ops.talm.scatter_rows(t_loss, t_ent, correct_bool, t_tgt, *_cuda(src), full_loss,
                                full_ent, stats)
    assert np.array_equal(full_loss.cpu().numpy(), pack.scatter(token_loss, src, out_len))
    assert np.array_equal(full_ent.cpu().numpy(), pack.scatter(entropy, src, out_len))
    assert stats.cpu().tolist() == [int((correct != 0).sum()), int((targets >= 0).sum())]


@pytest.mark.parametrize("n,denom_value", [(1367 * 1536, 1024.0), (8 * 1536 + 5, 3.0),
                                           (7, 0.0)])
def test_scale_rows_is_the_reference_arithmetic(n, denom_value):
    import talm_amd._ops  # noqa: F401

    g = (torch.randn(n, generator=torch.Generator().manual_seed(n)) * 3).half().cuda()
    grad_loss = torch.tensor(65536.0, device="cuda")
    denom = torch.tensor(denom_value, device="cuda")
    out = torch.empty_like(g)
    torch.ops.talm.scale_rows(g, grad_loss, denom, out)
    scale = torch.where(denom != 0, grad_loss / denom, 0.0)
    expect = (g.float() * scale).half()
    assert torch.equal(out.view(torch.int16), expect.view(torch.int16))


def test_rmsnorm_backward_without_a_sum_gradient_equals_a_zero_one():
    """The add-norm backward with no gradient of the sum (the final norm) reads no ds operand:
    the same bits as the launch with a zero-filled one."""
    import talm_amd._ops  # noqa: F401

    g = torch.Generator().manual_seed(9)
    n, h = 300, 1536
    dy = torch.randn(n, h, generator=g).half().cuda()
    xhat = torch.randn(n, h, generator=g).half().cuda()
    w = (torch.rand(h, generator=g) + 0.5).cuda()
    rstd = (torch.rand(n, generator=g) + 0.5).cuda()
    outs = []
    for ds in (torch.zeros(n, h, device="cuda"), None):
        dx = torch.empty(n, h, device="cuda")
        dbranch = torch.empty(n, h, dtype=torch.float16, device="cuda")
        torch.ops.talm.rmsnorm(dx, ds, dy, xhat, dbranch, w, rstd, 1e-6, 1)
        outs.append((dx, dbranch))
    assert torch.equal(outs[0][0], outs[1][0]) and torch.equal(outs[0][1], outs[1][1])
