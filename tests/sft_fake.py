"""A stand-in `trl` module for the tests (TRL is not installed in this image or on the GPU box).

`SFTTrainer.compute_loss` restates what trl 0.29.1's does (sft_trainer.py:1238-1320, as the
reference's solution/patches.py:282-320 describes the metrics it replaces): the loss from
transformers' `Trainer.compute_loss`, then, from the full logits,
  - `entropy`: the softmax entropy per position, averaged over the attention mask;
  - `num_tokens`: the running count of attended tokens (training only);
  - `mean_token_accuracy`: argmax of the logits at position t == label at t + 1, over the
    labelled positions.
The trainer carries just the attributes `Trainer.compute_loss` and the metrics read.
"""

import sys
import types
from collections import defaultdict
from types import SimpleNamespace

import torch


class SFTTrainer:
    def __init__(self, model):
        self.model = model
        self.args = SimpleNamespace(average_tokens_across_devices=False, use_liger_kernel=False,
                                    n_gpu=1)
        self.accelerator = SimpleNamespace(parallelism_config=None, num_processes=1,
                                           gather_for_metrics=lambda t: t,
                                           unwrap_model=lambda m: m)
        self.label_smoother = None
        self.compute_loss_func = None
        self.model_accepts_loss_kwargs = True
        self._metrics = {"train": defaultdict(list), "eval": defaultdict(list)}
        self._total_train_tokens = 0
        self.original_calls = 0

    def compute_loss(self, model, inputs, return_outputs=False, num_items_in_batch=None):
        import transformers

        self.original_calls += 1
        mode = "train" if self.model.training else "eval"
        inputs["use_cache"] = False
        loss, outputs = transformers.Trainer.compute_loss(
            self, model, inputs, return_outputs=True, num_items_in_batch=num_items_in_batch)
        with torch.no_grad():
            z = outputs.logits.float()
            entropy = torch.logsumexp(z, -1) - (torch.softmax(z, -1) * z).sum(-1)
            mask = inputs["attention_mask"]
            self._metrics[mode]["entropy"].append(
                ((entropy * mask).sum() / mask.sum()).item())
            if mode == "train":
                self._total_train_tokens += mask.sum().item()
            self._metrics[mode]["num_tokens"] = [self._total_train_tokens]
            pred = z[:, :-1].argmax(-1)
            labels = inputs["labels"][:, 1:]
            labelled = labels != -100
            correct = ((pred == labels) & labelled).sum()
            total = labelled.sum()
            self._metrics[mode]["mean_token_accuracy"].append(
                (correct / total).item() if total > 0 else 0.0)
        return (loss, outputs) if return_outputs else loss


def install(monkeypatch):
    """Put a fresh stand-in `trl` into sys.modules for one test; returns its SFTTrainer class."""
    module = types.ModuleType("trl")
    cls = type("SFTTrainer", (SFTTrainer,), {})
    module.SFTTrainer = cls
    monkeypatch.setitem(sys.modules, "trl", module)
    return cls
