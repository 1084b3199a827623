"""`apply()`: install the MI355X kernels into transformers' Qwen2 (the reference's patch API).

Mirrors solution.apply() (solution/__init__.py:229-408): class-level patches, looked up at call
time, each installed once (`_in_chain`, :119-129) under `state.installing`, each falling back to
the original code outside the exact situation it was written for. Installed here:

- RMSNorm and the residual adds folded into the norms (rmsnorm.py);
- RoPE and its tables (rope.py);
- SwiGLU with the in-place backward (swiglu.py, swiglu_inplace.py), or the save-up MLP
  (mlp_save_up.py, opt-in SOLUTION_MLP_SAVE_UP=1);
- grouped NF4 dequantization of the 4-bit projections (qgroup.py), the LoRA node (lora.py) and
  q|k|v as one projection node with the rotary embedding in place (fused_proj.py);
- padding removal with per-row attention (unpad.py) and the fused LM head + cross-entropy of
  the causal LM (fused_head.py, `patch_qwen2_causal_lm` below);
- the measured hipBLASLt solution table of the decoder's GEMMs (gemm_tuning.py);
- when TRL is installed, `SFTTrainer.compute_loss` on the fused head, its entropy / token /
  accuracy metrics taken from the head's per-token outputs (sft_loss.py).

Switches: SOLUTION_DISABLE_<PART>=1 leaves a part out (RMSNORM, ADDNORM, ROPE, SWIGLU_INPLACE,
GROUP, LORA, FUSED_PROJ, FUSED_HEAD, UNPAD, FUSED_MLP, ATTN_BLOCK, GEMM_TABLE), as in the
reference (solution/__init__.py:51-84).
"""

import importlib.util
import os
import sys

from .engaged import ON
from .state import DISABLED, fallback, installing


def _in_chain(fn, marker):
    """Whether a wrapper carrying `marker` is in the patch chain of `fn` (each wrapper keeps the
    function it wraps in `_original` or `_previous`)."""
    seen = set()
    while fn is not None and id(fn) not in seen:
        seen.add(id(fn))
        if getattr(fn, marker, False):
            return True
        fn = getattr(fn, "_previous", None) or getattr(fn, "_original", None)
    return False


def _off(name):
    return os.environ.get(f"SOLUTION_DISABLE_{name}") == "1"


def _have_trl():
    """Whether `trl` is imported or importable (without importing it)."""
    if "trl" in sys.modules:
        return True
    try:
        return importlib.util.find_spec("trl") is not None
    except (ImportError, ValueError):
        return False


# ------------------------------------------------------------------ the fused causal LM -----

_unpad = {"enabled": os.environ.get("SOLUTION_DISABLE_UNPAD") != "1", "checked": 0}
ORIGINAL_FORWARD = {}
LAST_STEP = []  # the per-token outputs of the last fused forward (Soup's ChunkedStep fields)


def _restart(device, rng_state):
    """Before a forward that failed part-way runs again: the generator back to `rng_state`
    (the same dropout masks are drawn again) and the resident dequantized layer dropped
    (solution/patches.py:55-63)."""
    import torch

    from . import qgroup

    torch.cuda.set_rng_state(rng_state, device)
    qgroup.reset_passes()


def _head_is_fusable(lm):
    import torch

    head = getattr(lm, "lm_head", None)
    weight = getattr(head, "weight", None)
    return (isinstance(weight, torch.Tensor) and weight.is_cuda and not weight.requires_grad
            and getattr(head, "bias", None) is None and weight.dim() == 2
            and "forward" not in lm.__dict__)


def _fused_forward_applies(lm, labels, logits_to_keep, kwargs):
    import torch

    model = getattr(lm, "model", None)
    return (labels is not None and isinstance(labels, torch.Tensor) and labels.dim() == 2
            and getattr(lm, "training", False) and isinstance(logits_to_keep, int)
            and logits_to_keep == 0 and "shift_labels" not in kwargs and _head_is_fusable(lm)
            and not getattr(model, "gradient_checkpointing", False))


def _fused_forward(self, input_ids, attention_mask, position_ids, past_key_values,
                   inputs_embeds, labels, use_cache, kwargs, output_cls, stage):
    """The fused training forward of Qwen2ForCausalLM (solution/patches.py:173-260): shift the
    labels, pack the real tokens of a right-padded batch into one flat sequence (one host sync),
    run the decoder, the fused head + cross-entropy, and scatter the per-token outputs back."""
    from types import SimpleNamespace

    import torch

    from .engaged import FELL_BACK, RAN
    from .fused_head import fused_head_loss
    from .rmsnorm import link_next_norms
    from .unpad import (is_right_padded, rows_context, static_n_tokens, take_prefetched,
                        unpad_batch)

    stage.clear()
    kwargs.pop("return_dict", None)
    num_items = kwargs.pop("num_items_in_batch", None)
    batch, seq = labels.shape
    unpad = ("unpad" not in DISABLED and _unpad["enabled"] and input_ids is not None
             and inputs_embeds is None and position_ids is None and past_key_values is None
             and isinstance(attention_mask, torch.Tensor) and attention_mask.dim() == 2
             and tuple(attention_mask.shape) == (batch, seq)
             and tuple(input_ids.shape) == (batch, seq)
             and not getattr(self.model, "has_sliding_layers", True))
    counts = None
    n_static = static_n_tokens()
    if n_static is not None:
        if not unpad:
            raise ValueError("fixed-shape packing needs a right-padded [B, T] batch with a mask")
        return _static_forward(self, input_ids, attention_mask, labels, n_static, num_items,
                               kwargs, output_cls, stage)
    shift = torch.nn.functional.pad(labels, (0, 1), value=-100)[:, 1:].reshape(-1)
    if unpad:
        try:
            idx, positions, bounds, lengths, counts = unpad_batch(
                attention_mask, shift.to(attention_mask.device),
                values=take_prefetched(attention_mask, labels))
            if _unpad["checked"] < 3:
                _unpad["checked"] += 1
                if not is_right_padded(attention_mask, lengths):
                    _unpad["enabled"] = False
                    unpad = False
        except Exception as exc:  # noqa: BLE001 - state.py convention
            if not fallback("unpad", exc):
                raise
            unpad, counts = False, None
    RAN["fused_head"] += 1
    if unpad:
        RAN["unpad"] += 1
    else:
        FELL_BACK["unpad"] += 1
    link_next_norms(self.model)
    n_labelled = None if counts is None else counts[0 if unpad else 1]
    if unpad:
        stage.append("unpadded")
        shift = shift.to(idx.device)[idx]
        with rows_context(bounds, device=input_ids.device):
            outputs = self.model(input_ids=input_ids.reshape(-1)[idx][None],
                                 attention_mask={"full_attention": None},
                                 position_ids=positions, past_key_values=None,
                                 inputs_embeds=None, use_cache=False, **kwargs)
    else:
        stage.append("padded")
        outputs = self.model(input_ids=input_ids, attention_mask=attention_mask,
                             position_ids=position_ids, past_key_values=past_key_values,
                             inputs_embeds=inputs_embeds, use_cache=use_cache, **kwargs)
    stage.append("head")
    hidden = outputs.last_hidden_state
    size = hidden.shape[-1]
    shift = shift.to(hidden.device)
    loss, token_loss, token_entropy, correct, argmax = fused_head_loss(
        hidden.reshape(-1, size), self.lm_head.weight, shift, num_items, n_labelled=n_labelled,
        return_argmax=True)
    if unpad:
        token_loss, token_entropy, n_correct, n_targets = scatter_metrics(
            token_loss, token_entropy, correct, shift, idx, batch * seq)
    else:
        n_correct, n_targets = correct.sum(), (shift >= 0).sum()
    LAST_STEP.clear()
    LAST_STEP.append(SimpleNamespace(
        token_entropy=token_entropy.view(batch, seq), token_loss=token_loss.view(batch, seq),
        correct=n_correct, labelled=n_targets, argmax=argmax))
    return output_cls(loss=loss, logits=None, past_key_values=None,
                      hidden_states=outputs.hidden_states, attentions=outputs.attentions)


def scatter_metrics(token_loss, token_entropy, correct, targets, src, out_len):
    """The per-token loss and entropy of the packed rows back to `out_len` batch slots (zero
    where no row lands; row i lands on slot src[i]) and the step's metric sums: (full loss, full
    entropy, #correct, #targets >= 0) (solution/patches.py:244-253). One launch
    (talm_scatter_rows) when the operands suit it."""
    import torch

    if (token_loss.is_cuda and token_loss.dtype == torch.float32 and token_loss.is_contiguous()
            and token_entropy.dtype == torch.float32 and token_entropy.is_contiguous()
            and correct.dtype == torch.bool and correct.is_contiguous()
            and targets.dtype == torch.int64 and targets.is_contiguous()
            and src.dtype == torch.int64 and src.is_contiguous()):
        full_loss = torch.empty(out_len, dtype=torch.float32, device=token_loss.device)
        full_entropy = torch.empty_like(full_loss)
        stats = torch.empty(2, dtype=torch.int64, device=token_loss.device)
        torch.ops.talm.scatter_rows(token_loss, token_entropy, correct, targets, src, full_loss,
                                    full_entropy, stats)
        return full_loss, full_entropy, stats[0], stats[1]
    full_loss = token_loss.new_zeros(out_len)
    full_entropy = token_entropy.new_zeros(out_len)
    full_loss.index_copy_(0, src, token_loss)
    full_entropy.index_copy_(0, src, token_entropy)
    return full_loss, full_entropy, correct.sum(), (targets >= 0).sum()


def _static_forward(self, input_ids, mask, labels, n_tokens, num_items, kwargs, output_cls,
                    stage):
    """`_fused_forward` with the fixed-shape packing of `unpad.static_tokens` (a step captured in
    a HIP graph): the batch is packed into `n_tokens` rows on the device, the pad rows form their
    own sequence labelled -100, and the head takes every row as a gradient row (an ignored row's
    gradient is zero), so no shape or launch depends on a host value of the batch."""
    from types import SimpleNamespace

    from .engaged import RAN
    from .fused_head import fused_head_loss
    from .rmsnorm import link_next_norms
    from .unpad import pack_static, rows_context_static, static_max_len

    batch, seq = labels.shape
    ids, positions, cu, rows_targets, src = pack_static(input_ids.to(mask.device), mask,
                                                        labels.to(mask.device), n_tokens)
    RAN["fused_head"] += 1
    RAN["unpad"] += 1
    link_next_norms(self.model)
    stage.append("unpadded")
    with rows_context_static(cu, static_max_len(seq), n_tokens):
        outputs = self.model(input_ids=ids[None], attention_mask={"full_attention": None},
                             position_ids=positions, past_key_values=None, inputs_embeds=None,
                             use_cache=False, **kwargs)
    stage.append("head")
    hidden = outputs.last_hidden_state
    loss, token_loss, token_entropy, correct, argmax = fused_head_loss(
        hidden.reshape(-1, hidden.shape[-1]), self.lm_head.weight, rows_targets, num_items,
        return_argmax=True, grad_all_rows=True)
    # back to [B, T]: the pad rows all land on one extra slot, dropped
    full_loss, full_entropy, n_correct, n_targets = scatter_metrics(
        token_loss, token_entropy, correct, rows_targets, src, batch * seq + 1)
    LAST_STEP.clear()
    LAST_STEP.append(SimpleNamespace(
        token_entropy=full_entropy[:-1].view(batch, seq),
        token_loss=full_loss[:-1].view(batch, seq), correct=n_correct, labelled=n_targets,
        argmax=argmax))
    return output_cls(loss=loss, logits=None, past_key_values=None,
                      hidden_states=outputs.hidden_states, attentions=outputs.attentions)


def patch_qwen2_causal_lm():
    """`Qwen2ForCausalLM.forward` through `_fused_forward` in training with labels; the original
    forward otherwise (solution/patches.py:116-159)."""
    import torch
    from transformers.modeling_outputs import CausalLMOutputWithPast
    from transformers.models.qwen2 import modeling_qwen2

    from .engaged import FELL_BACK

    cls = modeling_qwen2.Qwen2ForCausalLM
    if _in_chain(cls.forward, "_solution_fused_lm"):
        return
    original = ORIGINAL_FORWARD.setdefault(cls, cls.forward)

    def forward(self, input_ids=None, attention_mask=None, position_ids=None,
                past_key_values=None, inputs_embeds=None, labels=None, use_cache=None,
                logits_to_keep=0, **kwargs):
        if "fused_head" not in DISABLED \
                and _fused_forward_applies(self, labels, logits_to_keep, kwargs):
            device = self.lm_head.weight.device
            # a step captured in a HIP graph has no fallback (it raises): no generator state
            rng_state = None if torch.cuda.is_current_stream_capturing() \
                else torch.cuda.get_rng_state(device)
            stage = []
            for _ in range(2):
                try:
                    return _fused_forward(self, input_ids, attention_mask, position_ids,
                                          past_key_values, inputs_embeds, labels, use_cache,
                                          dict(kwargs), CausalLMOutputWithPast, stage)
                except Exception as exc:  # noqa: BLE001 - state.py convention
                    component = "unpad" if stage[-1:] == ["unpadded"] else "fused_head"
                    if rng_state is None or not fallback(component, exc):
                        raise
                _restart(device, rng_state)
                if "fused_head" in DISABLED:
                    break
        FELL_BACK["head"] += 1
        return original(self, input_ids=input_ids, attention_mask=attention_mask,
                        position_ids=position_ids, past_key_values=past_key_values,
                        inputs_embeds=inputs_embeds, labels=labels, use_cache=use_cache,
                        logits_to_keep=logits_to_keep, **kwargs)

    forward._solution_fused_lm = True
    forward._original = original
    cls.forward = forward
    ON.add("head")


def apply():
    """Install every patch (idempotent). Loads libtalm.so first: without the kernels nothing is
    installed and the error propagates (there is no CPU fallback)."""
    from . import _lib

    _lib.lib()
    if not _off("GEMM_TABLE"):
        with installing("gemm_table"):
            from . import gemm_tuning

            gemm_tuning.load()
    if not _off("SWIGLU_INPLACE"):
        with installing("swiglu"):
            from .swiglu_inplace import patch_qwen2_mlp_inplace

            patch_qwen2_mlp_inplace()
    if os.environ.get("SOLUTION_MLP_SAVE_UP") == "1":
        with installing("mlp_save_up"):
            from .mlp_save_up import patch_qwen2_mlp_save_up

            patch_qwen2_mlp_save_up()
    if not _off("RMSNORM"):
        with installing("rmsnorm"):
            from .rmsnorm import patch_qwen2_add_norm, patch_qwen2_rmsnorm

            patch_qwen2_rmsnorm()
            if not _off("ADDNORM"):
                patch_qwen2_add_norm()
    if not _off("ROPE"):
        with installing("rope"):
            from .rope import patch_qwen2_rope, patch_qwen2_rotary_tables

            patch_qwen2_rope()
            patch_qwen2_rotary_tables()
    if not _off("GROUP"):
        with installing("qgroup"):
            from .qgroup import patch_group_dequant

            patch_group_dequant()
        if not _off("LORA"):
            with installing("lora"):
                from .lora import patch_lora

                patch_lora()
        if not (_off("FUSED_PROJ") or _off("FUSED_QKV")):
            with installing("fused_proj"):
                from .fused_proj import patch_qwen2_attention

                patch_qwen2_attention()
    if not _off("FUSED_HEAD"):
        with installing("fused_head"):
            from .unpad import patch_sdpa_rows

            patch_sdpa_rows()
            patch_qwen2_causal_lm()
        if _have_trl():
            with installing("fused_head"):
                from .sft_loss import patch_sft_compute_loss

                patch_sft_compute_loss()
                ON.add("sft_loss")
    return sorted(ON)


def _root(fn):
    seen = set()
    while fn is not None and id(fn) not in seen:
        seen.add(id(fn))
        nxt = getattr(fn, "_previous", None) or getattr(fn, "_original", None)
        if nxt is None:
            return fn
        fn = nxt
    return fn


def unapply():
    """Restore every original method this package patched (for A/B runs in one process)."""
    from transformers.modeling_utils import ALL_ATTENTION_FUNCTIONS
    from transformers.models.qwen2 import modeling_qwen2

    from . import qgroup, rmsnorm
    from .lora import LoraLinear
    from .nf4_linear import Linear4bit

    for cls in (modeling_qwen2.Qwen2RMSNorm, modeling_qwen2.Qwen2DecoderLayer,
                modeling_qwen2.Qwen2MLP, modeling_qwen2.Qwen2Attention,
                modeling_qwen2.Qwen2ForCausalLM, modeling_qwen2.Qwen2RotaryEmbedding,
                Linear4bit, LoraLinear):
        cls.forward = _root(cls.forward)
    forward = modeling_qwen2.Qwen2Model.forward
    if getattr(forward, "_solution_link_norms", False):
        modeling_qwen2.Qwen2Model.forward = forward.__wrapped__
    modeling_qwen2.apply_rotary_pos_emb = _root(modeling_qwen2.apply_rotary_pos_emb)
    trl = sys.modules.get("trl")
    if trl is not None and hasattr(trl, "SFTTrainer") \
            and _in_chain(trl.SFTTrainer.compute_loss, "_talm_sft_loss"):
        trl.SFTTrainer.compute_loss = _root(trl.SFTTrainer.compute_loss)
    ALL_ATTENTION_FUNCTIONS["sdpa"] = _root(ALL_ATTENTION_FUNCTIONS["sdpa"])
    rmsnorm.LAYER_FORWARDS.clear()
    qgroup.release()
    ON.clear()
