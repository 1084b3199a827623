"""TRL's SFTTrainer.compute_loss on the fused head (talm_amd/sft_loss.py), on the CPU.

TRL is not installed: tests/sft_fake.py stands in for `trl` with SFTTrainer's own
compute_loss restated (the loss through transformers' Trainer.compute_loss, the entropy,
num_tokens and mean_token_accuracy metrics from the full logits). The causal LM here is a tiny
module whose forward carries the fused forward's marker and, like the fused forward, leaves its
per-token entropy and correct / labelled counts in patches.LAST_STEP, computed by other routines
than the stand-in's (torch.distributions' entropy, a loop for the accuracy). The wrapped
compute_loss must log what SFTTrainer's own code logs from the logits, and hand every call the
fused path does not serve to the original.
"""

from types import SimpleNamespace

import pytest
import torch
from transformers.modeling_outputs import CausalLMOutputWithPast

import sft_fake
from talm_amd import engaged, patches, sft_loss, state

VOCAB, HIDDEN = 37, 16


class TinyLM(torch.nn.Module):
    """A causal LM standing in for the patched Qwen2ForCausalLM: full logits and the loss, and
    the fused forward's per-token record in patches.LAST_STEP. `fail` calls raise first."""

    def __init__(self, fail=0):
        super().__init__()
        gen = torch.Generator().manual_seed(3)
        self.embed = torch.nn.Parameter(torch.randn(VOCAB, HIDDEN, generator=gen))
        self.lm_head = torch.nn.Linear(HIDDEN, VOCAB, bias=False)
        with torch.no_grad():
            self.lm_head.weight.copy_(torch.randn(VOCAB, HIDDEN, generator=gen))
        self.fail = fail
        self.calls = 0

    def forward(self, input_ids=None, attention_mask=None, labels=None, use_cache=None,
                num_items_in_batch=None, **kwargs):
        self.calls += 1
        if self.fail:
            self.fail -= 1
            raise RuntimeError("planted failure of the fused forward")
        logits = self.lm_head(self.embed[input_ids])
        shift = torch.nn.functional.pad(labels, (0, 1), value=-100)[:, 1:]
        loss = torch.nn.functional.cross_entropy(logits.reshape(-1, VOCAB), shift.reshape(-1),
                                                 ignore_index=-100)
        entropy = torch.distributions.Categorical(logits=logits.detach()).entropy()
        correct = 0
        for b in range(labels.shape[0]):
            for t in range(labels.shape[1] - 1):
                y = int(labels[b, t + 1])
                correct += int(y != -100 and int(logits[b, t].argmax()) == y)
        patches.LAST_STEP.clear()
        patches.LAST_STEP.append(SimpleNamespace(
            token_entropy=entropy, correct=torch.tensor(correct),
            labelled=(shift >= 0).sum()))
        return CausalLMOutputWithPast(loss=loss, logits=logits)

    forward._solution_fused_lm = True


class PeftLike(torch.nn.Module):
    def __init__(self, inner):
        super().__init__()
        self.base = inner

    def get_base_model(self):
        return self.base

    def forward(self, **kwargs):
        return self.base(**kwargs)


def _inputs(seed=0):
    gen = torch.Generator().manual_seed(seed)
    ids = torch.randint(0, VOCAB, (3, 9), generator=gen)
    mask = torch.ones(3, 9, dtype=torch.long)
    mask[1, 6:] = 0
    mask[2, 3:] = 0
    labels = ids.clone()
    labels[:, :2] = -100
    labels[mask == 0] = -100
    return {"input_ids": ids, "attention_mask": mask, "labels": labels}


@pytest.fixture
def sft(monkeypatch):
    """The stand-in trl with the wrapper installed; the fused forward "applies" whenever the call
    has labels (its GPU conditions cannot hold here); a CPU generator state."""
    cls = sft_fake.install(monkeypatch)
    monkeypatch.setattr(patches, "_fused_forward_applies",
                        lambda lm, labels, logits_to_keep, kwargs: labels is not None)
    monkeypatch.setattr(torch.cuda, "get_rng_state", lambda device=None: torch.get_rng_state())
    monkeypatch.setattr(patches, "_restart", lambda device, rng: torch.set_rng_state(rng))
    saved = dict(state.DISABLED)
    state.DISABLED.clear()
    sft_loss.patch_sft_compute_loss()
    yield cls
    state.DISABLED.clear()
    state.DISABLED.update(saved)
    patches.LAST_STEP.clear()


def _run(cls, model, inputs, wrapped=True):
    trainer = cls(model)
    fn = cls.compute_loss if wrapped else sft_fake.SFTTrainer.compute_loss
    loss = fn(trainer, model, dict(inputs))
    return trainer, loss


def test_metrics_match_sftrainer_on_the_full_logits(sft):
    model = PeftLike(TinyLM())
    inputs = _inputs()
    ours, loss = _run(sft, model, inputs)
    assert ours.original_calls == 0, "the fused path must not run SFTTrainer's own code"
    assert getattr(ours, sft_loss.STEP_ATTR) is patches.LAST_STEP[-1]
    ref, ref_loss = _run(sft, model, inputs, wrapped=False)
    assert ref.original_calls == 1
    torch.testing.assert_close(loss, ref_loss)
    for key in ("entropy", "mean_token_accuracy"):
        assert ours._metrics["train"][key] == pytest.approx(ref._metrics["train"][key],
                                                            rel=1e-6), key
    assert ours._metrics["train"]["num_tokens"] == ref._metrics["train"]["num_tokens"] == [18]
    # a second call: entropy and accuracy append, num_tokens keeps the running count
    sft.compute_loss(ours, model, _inputs(seed=1))
    assert len(ours._metrics["train"]["entropy"]) == 2
    assert ours._metrics["train"]["num_tokens"] == [36]


def test_eval_mode_and_no_labelled_token(sft):
    model = TinyLM().eval()
    inputs = _inputs()
    inputs["labels"] = torch.full_like(inputs["labels"], -100)
    trainer = sft(model)
    sft.compute_loss(trainer, model, dict(inputs))
    assert trainer._metrics["eval"]["mean_token_accuracy"] == [0.0]
    assert trainer._metrics["eval"]["num_tokens"] == [0], "eval adds no tokens to the count"


@pytest.mark.parametrize("change", ["no labels", "label smoother", "custom loss", "liger",
                                    "no fused forward inside", "fused head off"])
def test_calls_the_fused_path_does_not_serve_run_sftrainer(sft, change):
    model = TinyLM()
    inputs = _inputs()
    trainer = sft(model)
    if change == "no labels":
        del inputs["labels"]
    elif change == "label smoother":
        trainer.label_smoother = object()
    elif change == "custom loss":
        trainer.compute_loss_func = object()
    elif change == "liger":
        trainer.args.use_liger_kernel = True
    elif change == "no fused forward inside":
        model = torch.nn.Linear(2, 2)
    elif change == "fused head off":
        state.DISABLED["fused_head"] = "switched off"
    assert sft_loss.fused_lm_for(trainer, model, inputs) is None
    if change in ("no labels", "label smoother", "custom loss", "no fused forward inside"):
        return  # SFTTrainer's own code cannot run on these stand-ins; the decision is the test
    sft.compute_loss(trainer, model, dict(inputs))
    assert trainer.original_calls == 1
    assert not hasattr(trainer, sft_loss.STEP_ATTR)


def test_a_failing_fused_path_falls_back_to_sftrainer(sft, monkeypatch, capsys):
    monkeypatch.setattr(state, "STRICT", False)
    model = TinyLM(fail=1)
    trainer = sft(model)
    loss = sft.compute_loss(trainer, model, dict(_inputs()))
    assert "fused_head" in state.DISABLED
    assert "[solution] fallback: fused_head: RuntimeError" in capsys.readouterr().out
    assert trainer.original_calls == 1 and model.calls == 2
    assert torch.isfinite(loss)
    # from then on the original runs directly
    sft.compute_loss(trainer, model, dict(_inputs()))
    assert trainer.original_calls == 2 and model.calls == 3


def test_strict_mode_propagates_the_failure(sft):
    model = TinyLM(fail=1)
    with pytest.raises(RuntimeError, match="planted failure"):
        sft.compute_loss(sft(model), model, dict(_inputs()))


def test_installed_once_and_removed_by_unapply(sft):
    wrapper = sft.compute_loss
    sft_loss.patch_sft_compute_loss()
    assert sft.compute_loss is wrapper and wrapper._original is sft_fake.SFTTrainer.compute_loss
    patches.unapply()
    engaged.ON.clear()
    assert sft.compute_loss is sft_fake.SFTTrainer.compute_loss


def test_apply_installs_it_when_trl_imports(monkeypatch):
    cls = sft_fake.install(monkeypatch)
    monkeypatch.setenv("SOLUTION_DISABLE_GEMM_TABLE", "1")
    patches.unapply()
    try:
        on = patches.apply()
        assert "sft_loss" in on
        assert getattr(cls.compute_loss, "_talm_sft_loss", False)
    finally:
        patches.unapply()
        engaged.ON.clear()
    assert cls.compute_loss is sft_fake.SFTTrainer.compute_loss
