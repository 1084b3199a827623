"""Graceful degradation and the part switches, on the CPU (no kernel runs).

The convention (talm_amd/state.py after solution/state.py:83-112): an unexpected error in a fast
path turns that component off with one `[solution] fallback:` line and the caller runs the
original code; out-of-memory, a missing kernel library, PyTorch's checkpoint control flow,
non-Exception signals and strict mode propagate. `apply()` installs each part under
`state.installing` and leaves a part out when SOLUTION_DISABLE_<PART>=1
(solution/__init__.py:51-84). The same convention on the GPU, around real launches, is
tests/test_gpu_fallback.py."""

import pytest
import torch

from talm_amd import engaged, patches, state
from talm_amd._lib import LibraryMissing

PREFIX = "[solution] fallback: "


@pytest.fixture
def lenient(monkeypatch):
    """Strict mode off (the suite runs strict) and a clean DISABLED table, restored after."""
    monkeypatch.setattr(state, "STRICT", False)
    saved = dict(state.DISABLED)
    state.DISABLED.clear()
    yield state.DISABLED
    state.DISABLED.clear()
    state.DISABLED.update(saved)


def _fallback_lines(capsys):
    return [line for line in capsys.readouterr().out.splitlines() if line.startswith(PREFIX)]


def test_unexpected_error_turns_the_component_off_once(lenient, capsys):
    assert state.fallback("rope", RuntimeError("bad launch\n  on two lines"))
    assert state.fallback("rope", ValueError("second failure"))  # still absorbed, no new line
    assert lenient == {"rope": "RuntimeError: bad launch on two lines"}
    assert _fallback_lines(capsys) == [f"{PREFIX}rope: RuntimeError: bad launch on two lines"]


class _StopRecomputationError(Exception):
    """Named as torch.utils.checkpoint's early-stop signal."""


@pytest.mark.parametrize("exc", [
    torch.cuda.OutOfMemoryError("HIP out of memory. Tried to allocate 2.00 GiB"),
    RuntimeError("HIP error: out of memory"),
    LibraryMissing("libtalm.so is not built"),
    _StopRecomputationError(),
    KeyboardInterrupt(),
])
def test_signals_and_missing_kernels_propagate(lenient, capsys, exc):
    assert not state.fallback("rmsnorm", exc)
    assert lenient == {}
    assert _fallback_lines(capsys) == []


def test_strict_mode_absorbs_nothing(monkeypatch, capsys):
    monkeypatch.setattr(state, "STRICT", True)
    assert not state.fallback("swiglu", RuntimeError("x"))
    assert "swiglu" not in state.DISABLED
    assert _fallback_lines(capsys) == []


def test_a_long_or_broken_message_is_one_bounded_line(lenient, capsys):
    class Unprintable(Exception):
        def __str__(self):
            raise TypeError("no str")

    assert state.fallback("lora", Unprintable())
    assert state.fallback("unpad", RuntimeError("x" * 2000))
    assert lenient["lora"] == "Unprintable: <message unavailable>"
    assert len(lenient["unpad"]) < 600 and lenient["unpad"].endswith("...")
    assert len(_fallback_lines(capsys)) == 2


def test_installing_absorbs_a_failed_installer_and_reraises_signals(lenient, capsys):
    with state.installing("fused_head"):
        raise RuntimeError("installer failed")
    assert lenient == {"fused_head": "RuntimeError: installer failed"}
    with pytest.raises(torch.cuda.OutOfMemoryError):
        with state.installing("rope"):
            raise torch.cuda.OutOfMemoryError("out of memory")
    assert "rope" not in lenient


# -- apply() and the switches --------------------------------------------------------------------

SWITCHES = {
    # switch -> (components apply() no longer lists, components that stay)
    "ROPE": ({"rope"}, {"rmsnorm", "group", "head"}),
    "RMSNORM": ({"rmsnorm", "addnorm"}, {"rope", "group"}),
    "ADDNORM": ({"addnorm"}, {"rmsnorm"}),
    "GROUP": ({"group", "lora", "fused_proj"}, {"rmsnorm", "head"}),
    "LORA": ({"lora"}, {"group", "fused_proj"}),
    "FUSED_PROJ": ({"fused_proj"}, {"group", "lora"}),
    "FUSED_HEAD": ({"head", "rows_attn"}, {"group"}),
    "SWIGLU_INPLACE": ({"swiglu_inplace"}, {"group"}),
}


@pytest.fixture
def clean_apply(monkeypatch):
    """apply() without the GPU: the hipBLASLt table (which queries the device) is switched off;
    every patch is removed again afterwards."""
    monkeypatch.setenv("SOLUTION_DISABLE_GEMM_TABLE", "1")
    patches.unapply()
    yield
    patches.unapply()
    engaged.ON.clear()


def test_apply_installs_every_part_and_is_idempotent(clean_apply):
    from transformers.models.qwen2 import modeling_qwen2

    first = patches.apply()
    forwards = (modeling_qwen2.Qwen2RMSNorm.forward, modeling_qwen2.Qwen2ForCausalLM.forward,
                modeling_qwen2.apply_rotary_pos_emb)
    assert set(first) >= {"rmsnorm", "addnorm", "rope", "group", "lora", "fused_proj", "head",
                          "rows_attn", "swiglu_inplace"}
    assert patches.apply() == first
    # the second apply() wrapped nothing twice
    assert (modeling_qwen2.Qwen2RMSNorm.forward, modeling_qwen2.Qwen2ForCausalLM.forward,
            modeling_qwen2.apply_rotary_pos_emb) == forwards
    patches.unapply()
    assert not hasattr(modeling_qwen2.Qwen2RMSNorm.forward, "_solution_rmsnorm")
    assert not hasattr(modeling_qwen2.apply_rotary_pos_emb, "_original")


@pytest.mark.parametrize("switch", sorted(SWITCHES))
def test_switch_leaves_its_part_out(clean_apply, monkeypatch, switch):
    gone, kept = SWITCHES[switch]
    monkeypatch.setenv(f"SOLUTION_DISABLE_{switch}", "1")
    on = set(patches.apply())
    assert not (on & gone), (switch, on)
    assert kept <= on, (switch, on)


def test_save_up_mode_shares_the_one_mlp_wrapper(clean_apply, monkeypatch):
    """SOLUTION_MLP_SAVE_UP=1 switches the MLP node's save-up mode on without a second wrapper of
    Qwen2MLP.forward, also when the in-place MLP patch itself is switched off."""
    from transformers.models.qwen2 import modeling_qwen2

    from talm_amd import mlp_save_up

    original = modeling_qwen2.Qwen2MLP.forward
    monkeypatch.setenv("SOLUTION_MLP_SAVE_UP", "1")
    on = set(patches.apply())
    assert {"mlp_save_up", "swiglu_inplace"} <= on
    forward = modeling_qwen2.Qwen2MLP.forward
    assert forward._previous is original
    patches.unapply()
    assert modeling_qwen2.Qwen2MLP.forward is original and "mlp_save_up" not in engaged.ON
    monkeypatch.setenv("SOLUTION_DISABLE_SWIGLU_INPLACE", "1")
    on = set(patches.apply())
    assert "mlp_save_up" in on and "swiglu_inplace" not in on
    assert modeling_qwen2.Qwen2MLP.forward._previous is original
    # a call that records no autograd is not the save-up mode's
    import torch

    x = torch.zeros(2, 8)
    assert mlp_save_up.save_up_group(object(), x) is None


def test_solution_package_is_the_drop_in_name():
    import solution
    import solution.patches
    import talm_amd.patches
    import talm_amd.qgroup

    assert solution.apply is talm_amd.patches.apply
    assert solution.patches.apply is talm_amd.patches.apply
    assert solution.qgroup is talm_amd.qgroup
    from solution import fused_head, rmsnorm, rope, state as sstate

    assert callable(rmsnorm.launch) and callable(rope._launch)
    assert callable(fused_head.fused_head_loss)
    assert sstate.DISABLED is state.DISABLED
    for name in solution.patches.__all__:
        assert hasattr(solution.patches, name), name


def test_linking_the_next_norms_adds_no_submodule(clean_apply):
    """link_next_norms records each decoder layer's follower norm without making it a submodule
    of the layer (the module tree and state_dict keep their keys)."""
    from talm_amd import qlora_model, rmsnorm

    patches.apply()
    config = qlora_model.qwen2_config(vocab_size=64, hidden_size=64, intermediate_size=128,
                                      num_hidden_layers=3, num_attention_heads=2,
                                      num_key_value_heads=1, head_dim=32)
    from transformers import Qwen2Model

    model = Qwen2Model(config)
    keys = list(model.state_dict())
    rmsnorm.link_next_norms(model)
    assert list(model.state_dict()) == keys
    layers = model.layers
    assert layers[0].__dict__["_talm_next_norm"]() is layers[1].input_layernorm
    assert layers[2].__dict__["_talm_next_norm"]() is model.norm
