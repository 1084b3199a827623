"""LayerGroup's call forms on the CPU: `span` / `weight` take the projection indices alone or
after the reference's pass name ("fwd" / "bwd", solution/qgroup.py:213, :310), anything else is a
TypeError; `expected_bwd` exists for callers that add to it (:536)."""

import pytest

from talm_amd import qgroup


def test_pass_name_is_optional():
    assert qgroup._pass_args((4, 6), 2, "span") == (4, 6)
    assert qgroup._pass_args(("fwd", 4, 6), 2, "span") == (4, 6)
    assert qgroup._pass_args(("bwd", 3), 1, "weight") == (3,)
    assert qgroup._pass_args((3,), 1, "weight") == (3,)


@pytest.mark.parametrize("args", [(), ("fwd",), ("up", 4, 6), (4,), (4, 5, 6), ("fwd", 4.0, 6)])
def test_bad_call_forms_raise(args):
    with pytest.raises(TypeError):
        qgroup._pass_args(args, 2, "span")


def test_reference_call_forms_on_a_cpu_group(monkeypatch):
    """A group of small CPU projections (nothing launched): the reference's counter can be added
    to, and span / weight in both forms reach the same view of the resident buffer (its
    dequantization stubbed by a buffer whose values are their own indices)."""
    import torch

    from talm_amd.nf4_linear import Linear4bit

    shapes = [(128, 128)] * 4 + [(256, 128), (256, 128), (128, 256)]
    group = qgroup.LayerGroup([Linear4bit.from_weight(torch.randn(o, i) * 0.02, None)
                               for o, i in shapes])
    group.expected_bwd += 1
    buf = torch.arange(group.numel, dtype=torch.float32)
    monkeypatch.setattr(group, "resident", lambda: buf)
    assert torch.equal(group.span("fwd", 4, 6), group.span(4, 6))
    assert group.span(4, 6).shape == (512, 128)
    assert torch.equal(group.weight("bwd", 6), group.weight(6))
    assert int(group.weight(6)[0, 0]) == group.segments[6].start
    with pytest.raises(TypeError):
        group.span("fwd", 4)
