"""Configuration 5: a random-init Qwen2.5-1.5B-shaped QLoRA model and its training step.

The model is transformers' Qwen2ForCausalLM built from a hand-written config (no checkpoint, no
network): 28 layers, hidden 1536, MLP 8960, 12 query / 2 KV heads of 128, vocabulary 151936,
tied embeddings, rope_theta 1e6, RMSNorm eps 1e-6, weights ~N(0, 0.02) (transformers' init).
It is then put in the state the reference's patches find after bitsandbytes + PEFT
(`from_pretrained(..., load_in_4bit)`, `prepare_model_for_kbit_training`, fp16 tied embedding,
`get_peft_model`):
- the seven projections of every decoder layer become NF4 4-bit layers with double-quantized
  absmax (nf4_linear.Linear4bit, blocksize 64 / 256, fp16 compute);
- the tied embedding / LM head weight is stored in fp16 and its lookups return fp32, so the
  residual stream is fp32 (solution/fp16_embed.py:116-138);
- norms stay fp32 and frozen;
- q_proj and v_proj carry LoRA r=16, alpha=32 (A Kaiming-uniform, B = 0), the only trainable
  parameters.
The step: fp16 autocast, GradScaler, fused AdamW (lr 2e-4, weight decay 0.01, cosine schedule
without warm-up), gradient clipping at 1.0, on right-padded batches of 4 rows of 128-512 tokens, token ids
uniform over the vocabulary, every real token labelled.
"""

import math
import os

import torch
import torch.nn as nn

from .lora import LoraLinear
from .nf4_linear import Linear4bit

QWEN25_15B = dict(vocab_size=151936, hidden_size=1536, intermediate_size=8960,
                  num_hidden_layers=28, num_attention_heads=12, num_key_value_heads=2,
                  max_position_embeddings=32768, rope_theta=1e6, rms_norm_eps=1e-6,
                  tie_word_embeddings=True, hidden_act="silu", attention_dropout=0.0,
                  initializer_range=0.02, use_sliding_window=False)

FUSED_TAIL = os.environ.get("SOLUTION_DISABLE_FUSED_TAIL") != "1"

PROJECTIONS = (("self_attn", "q_proj"), ("self_attn", "k_proj"), ("self_attn", "v_proj"),
               ("self_attn", "o_proj"), ("mlp", "gate_proj"), ("mlp", "up_proj"),
               ("mlp", "down_proj"))


def qwen2_config(**overrides):
    from transformers import Qwen2Config

    values = {**QWEN25_15B, **overrides}
    if "num_key_value_heads" not in overrides and "num_attention_heads" in overrides:
        values["num_key_value_heads"] = min(values["num_key_value_heads"],
                                            values["num_attention_heads"])
    config = Qwen2Config(**values)
    config._attn_implementation = "sdpa"
    return config


class EmbeddingFp32Out(nn.Embedding):
    """The frozen fp16 tied embedding, whose lookups return fp32 (the residual stream's dtype)."""

    def forward(self, input):  # noqa: A002 - nn.Embedding's argument name
        return super().forward(input).float()


@torch.no_grad()
def build_model(config=None, seed=1, device="cuda", lora_r=16, lora_alpha=32, lora_dropout=0.0):
    """The QLoRA model of configuration 5 (or of `config`), on `device`, in training mode."""
    from transformers import Qwen2ForCausalLM

    config = config or qwen2_config()
    torch.manual_seed(seed)
    with torch.device(device):
        model = Qwen2ForCausalLM(config)
    embed = model.model.embed_tokens
    embed.weight.data = embed.weight.data.to(torch.float16)
    embed.__class__ = EmbeddingFp32Out
    assert model.lm_head.weight is embed.weight
    for layer in model.model.layers:
        for parent_name, name in PROJECTIONS:
            parent = getattr(layer, parent_name)
            lin = getattr(parent, name)
            q4 = Linear4bit.from_weight(lin.weight, lin.bias)
            setattr(parent, name, q4)
            del lin
        torch.cuda.empty_cache() if str(device).startswith("cuda") else None
    model.requires_grad_(False)
    torch.manual_seed(seed + 1)
    for layer in model.model.layers:
        attn = layer.self_attn
        attn.q_proj = LoraLinear(attn.q_proj, lora_r, lora_alpha, lora_dropout)
        attn.v_proj = LoraLinear(attn.v_proj, lora_r, lora_alpha, lora_dropout)
    model.train()
    return model


def lora_parameters(model):
    return [p for p in model.parameters() if p.requires_grad]


def make_batch(seed, step, vocab, batch=4, seq=512, lo=128, hi=512, device="cuda"):
    """A right-padded batch: lengths uniform in [lo, hi], ids uniform over the vocabulary,
    every real token labelled, padding -100 / id 0 / mask 0. Seeded per step (CPU generator)."""
    g = torch.Generator().manual_seed(seed * 100003 + step)
    lengths = torch.randint(lo, hi + 1, (batch,), generator=g)
    ids = torch.randint(0, vocab, (batch, seq), generator=g)
    mask = torch.arange(seq)[None, :] < lengths[:, None]
    labels = torch.where(mask, ids, torch.full_like(ids, -100))
    ids = torch.where(mask, ids, torch.zeros_like(ids))
    return {"input_ids": ids.to(device), "attention_mask": mask.to(torch.int64).to(device),
            "labels": labels.to(device)}


class Trainer:
    """AdamW + fp16 GradScaler + clipping + cosine schedule over `steps` optimizer steps."""

    def __init__(self, model, steps=64, lr=2e-4, weight_decay=0.01, max_grad_norm=1.0,
                 fused_adapters=False):
        self.model = model
        self.params = lora_parameters(model)
        # both optimizers take the GradScaler's scale and inf flag as device tensors, so the step
        # needs no host synchronization (an unfused optimizer's step reads the inf flag on the
        # host). `fused_adapters`: this package's one-launch AdamW, which also writes the next
        # forward's fp16 adapter copies; else PyTorch's fused AdamW (the reference's setup).
        if fused_adapters:
            from .adapters import AdapterAdamW

            self.opt = AdapterAdamW(self.params, lr=lr, weight_decay=weight_decay)
        else:
            self.opt = torch.optim.AdamW(self.params, lr=lr, weight_decay=weight_decay,
                                         fused=True)
        self.sched = torch.optim.lr_scheduler.LambdaLR(
            self.opt, lambda i: 0.5 * (1.0 + math.cos(math.pi * min(i, steps) / steps)))
        self.scaler = torch.amp.GradScaler("cuda")
        self.max_grad_norm = max_grad_norm
        # called as grad_hook(trainer, total_norm) after unscaling and clipping (total_norm: the
        # gradients' norm before clipping), before the optimizer step (where the reference's
        # parity test records the step's LoRA gradients)
        self.grad_hook = None

    def step(self, batch, next_batch=None):
        """One optimizer step; returns the loss tensor (not synchronized). With `next_batch`, the
        packing statistics of that batch are copied to the host ahead of time (no host sync in
        the next step)."""
        if next_batch is not None:
            from .unpad import prefetch

            prefetch(next_batch["attention_mask"], next_batch["labels"])
        with torch.autocast("cuda", dtype=torch.float16):
            out = self.model(**batch)
        loss = out.loss
        self.backward(loss)
        self.optimizer_tail()
        return loss.detach()

    def backward(self, loss):
        """`scaler.scale(loss).backward()`: the backward seeded with the scale itself once the
        scaler holds it (the same gradients: d(loss * scale) / d(loss) = scale exactly), without
        the multiply, the ones seed and the multiply's backward."""
        scale = getattr(self.scaler, "_scale", None)
        if self.scaler.is_enabled() and torch.is_tensor(scale) and scale.numel() == 1 \
                and scale.device == loss.device and loss.dim() == 0:
            torch.autograd.backward(loss, scale.reshape(()).to(loss.dtype))
        else:
            self.scaler.scale(loss).backward()

    def optimizer_tail(self):
        """After the backward: unscale, clip, the optimizer step, the scale update, the
        schedule, and the gradients released. With this package's optimizer and no grad_hook
        (which reads the unscaled, clipped gradients) the first three run as
        `AdapterAdamW.fused_tail`: three launches instead of about fifteen, the same values up
        to the order in which the norm's squares are summed."""
        norm = None
        fused = getattr(self.opt, "fused_tail", None)
        if fused is not None and self.grad_hook is None and FUSED_TAIL:
            norm = fused(self.scaler, self.max_grad_norm)
        if norm is None:
            self.scaler.unscale_(self.opt)
            norm = torch.nn.utils.clip_grad_norm_(self.params, self.max_grad_norm)
            if self.grad_hook is not None:
                self.grad_hook(self, norm)
            self.scaler.step(self.opt)
        self.scaler.update()
        self.sched.step()
        self.opt.zero_grad(set_to_none=True)
