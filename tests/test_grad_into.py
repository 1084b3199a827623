"""Adapter weight gradients delivered into caller-owned buffers (`fused_proj.GRAD_INTO`), on the
CPU: a registered parameter's gradient is written into its buffer and withheld from autograd;
an unregistered one, or an entry left by another tensor at a reused id, passes through."""

import torch

from talm_amd import fused_proj


def test_registered_gradient_goes_into_its_buffer(monkeypatch):
    p, q = torch.zeros(4, 3), torch.zeros(2, 3)
    buf = torch.full((4, 3), 7.0)
    monkeypatch.setattr(fused_proj, "GRAD_INTO", {id(p): (p, buf)})
    monkeypatch.setattr(fused_proj, "GRAD_WRITTEN", set())
    g_p, g_q = torch.arange(12.0).view(4, 3), torch.ones(2, 3)
    assert fused_proj._grad_targets([p, q]) == [buf, None]
    out = fused_proj._deliver([g_p, g_q], [p, q])
    assert out[0] is None and out[1] is g_q
    assert torch.equal(buf, g_p)
    assert fused_proj.GRAD_WRITTEN == {id(p)}
    # a gradient computed in the buffer itself is not copied again
    buf.fill_(3.0)
    assert fused_proj._deliver([buf, None], [p, q]) == [None, None]
    assert torch.equal(buf, torch.full((4, 3), 3.0))


def test_stale_entry_at_a_reused_id_is_ignored(monkeypatch):
    p, other = torch.zeros(2), torch.zeros(2)
    buf = torch.zeros(2)
    monkeypatch.setattr(fused_proj, "GRAD_INTO", {id(p): (other, buf)})
    monkeypatch.setattr(fused_proj, "GRAD_WRITTEN", set())
    g = torch.ones(2)
    assert fused_proj._deliver([g], [p]) == [g]
    assert torch.equal(buf, torch.zeros(2)) and not fused_proj.GRAD_WRITTEN


def test_second_write_of_one_weight_is_flagged(monkeypatch):
    """Two nodes feeding one weight: the second direct write would drop the first contribution,
    so the weight lands in GRAD_TWICE (the graphed step then captures the general way)."""
    p = torch.zeros(3)
    buf = torch.zeros(3)
    monkeypatch.setattr(fused_proj, "GRAD_INTO", {id(p): (p, buf)})
    monkeypatch.setattr(fused_proj, "GRAD_WRITTEN", set())
    monkeypatch.setattr(fused_proj, "GRAD_TWICE", set())
    fused_proj._deliver([torch.ones(3)], [p])
    assert not fused_proj.GRAD_TWICE
    fused_proj._deliver([torch.full((3,), 2.0)], [p])
    assert fused_proj.GRAD_TWICE == {id(p)}
