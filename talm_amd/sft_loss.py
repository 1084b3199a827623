"""TRL's `SFTTrainer.compute_loss` on the fused causal-LM forward (the reference's
`patch_sft_compute_loss`, solution/patches.py:349-408, its metrics at :282-320).

`trl.SFTTrainer.compute_loss` (trl 0.29.1, sft_trainer.py:1238-1320) takes the loss from
transformers' `Trainer.compute_loss` and then logs three metrics from `outputs.logits`, the full
[B, T, V] logits:
  - `entropy`: the per-token entropy of the softmax, averaged over the attention mask (over every
    position when the batch is packed with `position_ids` instead of a mask);
  - `num_tokens`: the running count of attended tokens (training only);
  - `mean_token_accuracy`: argmax == label over the labelled positions of the shifted labels.
The fused forward (patches.py) never forms those logits, so SFTTrainer's own code cannot run on
it. When the fused forward will run for a call, this wrapper takes the loss from
`Trainer.compute_loss` (which calls the patched forward) and logs the same metrics from the
per-token outputs the fused head leaves in `patches.LAST_STEP`: the entropy [B, T] and the
correct / labelled counts. The per-step record itself is kept on the trainer
(`trainer.talm_step`) for callers that want the per-token loss or the argmax.

Everywhere else the original `compute_loss` runs unchanged: a model without a patched Qwen2
causal LM inside, the fused head switched off or not applicable to the call (evaluation, no
labels, gradient checkpointing), liger kernels, a label smoother or a custom loss function. A
failure of the fused path turns `fused_head` off (state.py) and the call runs again through the
original, from the same generator state.

TRL is not a dependency of this package: `apply()` installs the wrapper only when `trl` imports.
"""

import torch

from . import patches
from .state import DISABLED, fallback

STEP_ATTR = "talm_step"


def causal_lm(model):
    """The Qwen2 causal LM with the fused forward inside `model`, through the wrappers a trainer
    puts around it (DistributedDataParallel / accelerate's `.module`, PEFT's `get_base_model()`),
    or None."""
    seen = set()
    while model is not None and id(model) not in seen:
        seen.add(id(model))
        if patches._in_chain(getattr(type(model), "forward", None), "_solution_fused_lm"):
            return model
        inner = getattr(model, "module", None)
        if inner is None and callable(getattr(model, "get_base_model", None)):
            inner = model.get_base_model()
        model = inner
    return None


def fused_lm_for(trainer, model, inputs):
    """The causal LM whose fused forward a compute_loss call on `inputs` takes, or None."""
    if "fused_head" in DISABLED or not isinstance(inputs, dict):
        return None
    if (getattr(getattr(trainer, "args", None), "use_liger_kernel", False)
            or getattr(trainer, "label_smoother", None) is not None
            or getattr(trainer, "compute_loss_func", None) is not None):
        return None
    lm = causal_lm(model)
    if lm is None or not patches._fused_forward_applies(lm, inputs.get("labels"), 0, inputs):
        return None
    return lm


def log_metrics(trainer, mode, inputs, step):
    """SFTTrainer's three metrics from the fused head's per-token outputs, into
    `trainer._metrics[mode]` (and `trainer._total_train_tokens`), as SFTTrainer logs them from the
    full logits. No-op for a trainer without those attributes."""
    metrics = getattr(trainer, "_metrics", None)
    accelerator = getattr(trainer, "accelerator", None)
    if metrics is None or accelerator is None:
        return
    gather = accelerator.gather_for_metrics
    mask = inputs.get("attention_mask")
    with torch.no_grad():
        entropy = step.token_entropy.float()
        if mask is not None:
            m = mask.to(entropy.dtype)
            mean_entropy = (entropy * m).sum() / m.sum()
            tokens = mask.sum()
        elif "position_ids" in inputs:
            mean_entropy = entropy.mean()
            tokens = torch.tensor(inputs["position_ids"].size(1), device=entropy.device)
        else:
            raise ValueError("Expected 'attention_mask' or 'position_ids' in inputs.")
        metrics[mode]["entropy"].append(gather(mean_entropy).mean().item())
        if mode == "train":
            trainer._total_train_tokens += gather(tokens).sum().item()
        metrics[mode]["num_tokens"] = [trainer._total_train_tokens]
        labelled = gather(torch.as_tensor(step.labelled)).sum()
        correct = gather(torch.as_tensor(step.correct)).sum()
        metrics[mode]["mean_token_accuracy"].append(
            (correct / labelled).item() if labelled > 0 else 0.0)


def _fused_compute_loss(trainer, model, inputs, return_outputs, num_items_in_batch):
    import transformers

    mode = "train" if trainer.model.training else "eval"
    inputs.pop("_prediction_loss_only", None)
    inputs["use_cache"] = False
    patches.LAST_STEP.clear()
    loss, outputs = transformers.Trainer.compute_loss(
        trainer, model, inputs, return_outputs=True, num_items_in_batch=num_items_in_batch)
    if not patches.LAST_STEP:
        raise RuntimeError("the fused causal-LM forward did not run although it applied")
    step = patches.LAST_STEP[-1]
    setattr(trainer, STEP_ATTR, step)
    log_metrics(trainer, mode, inputs, step)
    return (loss, outputs) if return_outputs else loss


def patch_sft_compute_loss():
    """Wrap `trl.SFTTrainer.compute_loss` (idempotent). Raises ImportError without TRL."""
    import trl

    cls = trl.SFTTrainer
    if patches._in_chain(cls.compute_loss, "_talm_sft_loss"):
        return
    original = cls.compute_loss

    def compute_loss(self, model, inputs, return_outputs=False, num_items_in_batch=None):
        lm = None
        try:
            lm = fused_lm_for(self, model, inputs)
        except Exception as exc:  # noqa: BLE001 - state.py convention
            if not fallback("fused_head", exc):
                raise
        if lm is not None:
            device = lm.lm_head.weight.device
            rng_state = torch.cuda.get_rng_state(device)
            try:
                return _fused_compute_loss(self, model, dict(inputs), return_outputs,
                                           num_items_in_batch)
            except Exception as exc:  # noqa: BLE001 - state.py convention
                if not fallback("fused_head", exc):
                    raise
            patches._restart(device, rng_state)
            if getattr(self, STEP_ATTR, None) is not None:
                setattr(self, STEP_ATTR, None)
        return original(self, model, inputs, return_outputs=return_outputs,
                        num_items_in_batch=num_items_in_batch)

    compute_loss._talm_sft_loss = True
    compute_loss._original = original
    cls.compute_loss = compute_loss
