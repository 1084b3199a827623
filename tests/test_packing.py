"""Fixed-shape packing (unpad.unpad_static, device ops only) against the host-list packing of
the reference's unpad_batch restatement (solution/unpad.py:66-92), on the CPU: the real tokens
come first with the same flat indices, positions and row offsets; the pad rows form one more
sequence, labelled -100, gathering the pad slot."""

import pytest
import torch

from talm_amd import unpad


@pytest.mark.parametrize("lengths,n_tokens", [((5, 3, 7), 16), ((4, 4), 8), ((1, 8, 2), 64),
                                              ((8, 8, 8), 24), ((3,), 3)])
def test_static_packing_matches_host_packing(lengths, n_tokens):
    seq = 8
    batch = len(lengths)
    g = torch.Generator().manual_seed(sum(lengths) * 31 + n_tokens)
    mask = (torch.arange(seq)[None, :] < torch.tensor(lengths)[:, None]).to(torch.int64)
    labels = torch.randint(0, 50, (batch * seq,), generator=g)
    labels[torch.rand(batch * seq, generator=g) < 0.2] = -100
    idx, positions, bounds, got_lengths = unpad.unpad_batch(mask, values=list(lengths))
    src, pos, cu, targets = unpad.unpad_static(mask, labels, n_tokens)
    n = sum(lengths)
    assert got_lengths == list(lengths)
    assert src.shape == (n_tokens,) and pos.shape == (1, n_tokens)
    assert torch.equal(src[:n], idx)
    assert torch.equal(pos[:, :n], positions)
    assert cu.dtype == torch.int32
    assert cu.tolist() == [0] + [e for _, e in bounds] + [n_tokens]
    assert torch.equal(targets[:n], labels[idx])
    # the pad rows: their own sequence, positions 0.., the pad slot, ignored
    assert torch.all(src[n:] == batch * seq)
    assert pos[0, n:].tolist() == list(range(n_tokens - n))
    assert torch.all(targets[n:] == -100)


def test_static_tokens_context_nests():
    assert unpad.static_n_tokens() is None
    with unpad.static_tokens(128):
        with unpad.static_tokens(64):
            assert unpad.static_n_tokens() == 64
        assert unpad.static_n_tokens() == 128
    assert unpad.static_n_tokens() is None
