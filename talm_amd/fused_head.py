"""Fused output head + causal-LM loss on MI355X, without a [N, V] logits tensor.

Mirrors solution/fused_head.py: the head walks the VOCABULARY in slices of VOCAB_CHUNK columns
(8192), all tokens at once; per slice it computes fp16 logits, continues each row's online
log-sum-exp / entropy / argmax, rescales the row's fp32 gradient accumulator when its running
max moved and adds fp16(e^{z - m}) times the weight slice (:11-23); a last step turns the
accumulator into dH = acc / s - W16[target] (0 on unlabelled rows). The loss is
sum(token loss) / num_items (or / #labelled) (:53-58, :272-277). The backward only scales the
saved dH (:280-287).

On MI355X the whole slice loop is ONE call of talm_head_ce (talm_amd/csrc/head_ce.hip): both
GEMMs are hand-written fp16 MFMA kernels whose epilogue / prologue do the statistics and the
e^{z - m} weights, so a slice's logits are written once (fp16) and read once, and the per-slice
accumulator GEMM, which the reference leaves to cuBLAS, runs once per group of `GROUP` slices:
the reference's per-slice rescales of the accumulator telescope over a group, so the group's
columns form one reduction, cut into as many K parts as fill the chip (fp32 partials summed in
part order, then one rescale of the accumulator per group).

As in the reference (:25-35, `labelled_first` :290-299), with the gradient on the rows are put
labelled-first, so the accumulator covers the labelled rows only; the statistics of every row are
computed, and the per-row outputs and the gradient go back to the input order at the end.

Also returned (the reference computes it but keeps it internal, :342): the per-token argmax of
the fp16 logits (`fused_head_loss(..., return_argmax=True)`).
"""

import os
import weakref

import torch

from . import _ops
from .engaged import RAN

VOCAB_CHUNK = int(os.environ.get("SOLUTION_HEAD_VCHUNK", "8192"))
GROUP = int(os.environ.get("TALM_HEAD_GROUP", "5"))
COMPACT = os.environ.get("SOLUTION_DISABLE_HEAD_COMPACT") != "1"
TILE = 128  # the kernel's statistics granule: slices are a multiple of it


def _slice_width(vocab_chunk, vocab):
    """Slice width in columns: a positive multiple of TILE (rounded up; the statistics do not
    depend on the width beyond fp32 rounding), at most the vocabulary rounded up."""
    width = max(1, min(int(vocab_chunk), vocab))
    return -(-width // TILE) * TILE


def head_ce(h16, w16, targets, vocab_chunk=VOCAB_CHUNK, n_grad=None, need_grad=True,
            group=GROUP):
    """One talm_head_ce call. h16 fp16 [N, H], w16 fp16 [V, H] (unit column strides), targets
    int64 [N]. With `need_grad`, rows [0, n_grad) are the gradient rows: every labelled row must
    be among them (labelled-first order; n_grad defaults to counting them, one host sync), and an
    ignored row among them gets a zero gradient. Returns per-row token_loss, entropy, best_idx
    (int32), correct (int32) and grad (fp16 [N, H] or None)."""
    n, size = h16.shape
    vocab = w16.shape[0]
    device = h16.device
    vchunk = _slice_width(vocab_chunk, vocab)
    if need_grad and n_grad is None:
        n_grad = int((targets >= 0).sum())
    n_grad = int(n_grad) if need_grad else 0
    out = {
        "token_loss": torch.empty(n, dtype=torch.float32, device=device),
        "entropy": torch.empty(n, dtype=torch.float32, device=device),
        "best_idx": torch.empty(n, dtype=torch.int32, device=device),
        "correct": torch.empty(n, dtype=torch.int32, device=device),
        "grad": torch.empty(n, size, dtype=torch.float16, device=device) if need_grad else None,
    }
    if n == 0:
        return out
    nbytes = _ops.head_ce_workspace_bytes(n, size, vocab, vchunk, n_grad, group)
    workspace = torch.empty(nbytes, dtype=torch.uint8, device=device)
    torch.ops.talm.head_ce(h16, w16, targets, vchunk, n_grad, group, out["token_loss"], out["entropy"], out["best_idx"],
                           out["correct"], out["grad"], workspace)
    return out


def transpose_weight_exact(w):
    """w fp16 [R, C] (unit column stride, rows a multiple of 8) -> w^T [C, R] contiguous."""
    rows, cols = w.shape
    wt = torch.empty(cols, rows, dtype=torch.float16, device=w.device)
    torch.ops.talm.head_weight_t(w, wt)
    return wt


_HEAD_WEIGHTS = {}


def head_weights(weight):
    """w16, the frozen output weight's fp16 [V, H] view (or one converted copy), kept for the
    weight object at its current version (data pointer, version counter, layout) and rebuilt when
    any of these changes: the tied embedding of the QLoRA model is frozen, so a converted copy is
    made once. Both GEMMs of the head read it as it lies (no transposed copy)."""
    w = weight.detach()
    key = (w.data_ptr(), w._version, w.dtype, tuple(w.shape), tuple(w.stride()), str(w.device))
    hit = _HEAD_WEIGHTS.get("head")
    if hit is not None and hit[0]() is weight and hit[1] == key:
        return hit[2]
    w16 = _fp16_weight(weight)
    _HEAD_WEIGHTS["head"] = (weakref.ref(weight), key, w16)
    return w16


def _denominator(num_items, labelled_count):
    if num_items is None:
        return labelled_count.clamp(min=1).to(torch.float32)
    if torch.is_tensor(num_items):
        return num_items.to(device=labelled_count.device, dtype=torch.float32)
    return torch.tensor(float(num_items), device=labelled_count.device)


def _loss(token_loss, correct, targets, num_items):
    """(loss, denom, correct as bool): loss = sum(token_loss) / denom with `_denominator`'s denom
    (solution/fused_head.py:272-277, :386), one launch (talm_head_loss) when the operands suit it;
    `correct` is the head's int32 per-row flag."""
    if (token_loss.is_cuda and token_loss.dtype == torch.float32 and token_loss.is_contiguous()
            and correct.dtype == torch.int32 and correct.is_contiguous()
            and targets.dtype == torch.int64 and targets.is_contiguous()
            and (not torch.is_tensor(num_items) or num_items.numel() == 1)):
        device = token_loss.device
        mode, value, items = 0, 0.0, None
        if torch.is_tensor(num_items):
            mode, items = 1, num_items.to(device=device, dtype=torch.float32).reshape(())
        elif num_items is not None:
            mode, value = 2, float(num_items)
        loss = torch.empty((), dtype=torch.float32, device=device)
        denom = torch.empty_like(loss)
        correct_bool = torch.empty(correct.shape, dtype=torch.bool, device=device)
        torch.ops.talm.head_loss(token_loss, correct, targets, items, value, mode, loss, denom,
                                 correct_bool)
        return loss, denom, correct_bool
    denom = _denominator(num_items, (targets >= 0).sum())
    return token_loss.sum() / denom, denom, correct.to(torch.bool)


def _head_backward(ctx, grad_loss):
    """dH = grad_loss / denom * the saved gradient (0 when denom is 0), in the forward's dtype
    (solution/fused_head.py:280-287); one launch (talm_scale_rows) for fp16."""
    if grad_loss is None:  # the loss was not used (grads are not materialized)
        return None
    (grad_hidden,) = ctx.saved_tensors
    denom = ctx.denom
    if (ctx.out_dtype == torch.float16 and grad_hidden.dtype == torch.float16
            and grad_hidden.is_contiguous() and grad_hidden.data_ptr() % 16 == 0
            and grad_loss.dtype == torch.float32 and grad_loss.numel() == 1
            and denom.dtype == torch.float32 and denom.numel() == 1
            and grad_loss.device == denom.device == grad_hidden.device):
        out = torch.empty_like(grad_hidden)
        torch.ops.talm.scale_rows(grad_hidden, grad_loss.reshape(()).contiguous(), denom, out)
        return out
    scale = grad_loss.to(torch.float32) / denom
    scale = torch.where(denom != 0, scale, 0.0)
    return (grad_hidden.to(torch.float32) * scale).to(ctx.out_dtype)


def labelled_first(labelled, n_labelled):
    """(dest, src): row r of the input goes to position dest[r] of the labelled-first order and
    reordered row i is input row src[i] (solution/fused_head.py:290-299; no host sync)."""
    n = labelled.shape[0]
    pos = torch.arange(n, device=labelled.device)
    seen = torch.cumsum(labelled, 0)
    dest = torch.where(labelled, seen - 1, pos - seen + n_labelled)
    src = torch.empty_like(dest).index_copy_(0, dest, pos)
    return dest, src


def _fp16_weight(weight):
    """The weight as fp16 with unit column stride: a view when it already is one (the tied
    embedding stored in fp16), else one converted copy."""
    w = weight.detach()
    if w.dtype == torch.float16 and w.stride(1) == 1 and w.stride(0) % 8 == 0 \
            and w.data_ptr() % 16 == 0:
        return w
    return w.to(torch.float16).contiguous()


class FusedHeadLossVocab(torch.autograd.Function):
    """loss, per-token loss, entropy, correctness and argmax from hidden states and the frozen
    output weight (solution/fused_head.py:302-397). Saves only the fp16 hidden gradient."""

    @staticmethod
    def forward(ctx, hidden, weight, targets, num_items, vocab_chunk, need_grad, n_labelled):
        # the per-token outputs are not differentiable: no zero gradients made up for them
        ctx.set_materialize_grads(False)
        n_tokens = hidden.shape[0]
        h16 = hidden.detach().to(torch.float16)
        if h16.stride(1) != 1 or h16.stride(0) % 8 or h16.data_ptr() % 16:
            h16 = h16.contiguous()
        w16 = head_weights(weight)
        targets = targets.to(device=hidden.device, dtype=torch.int64).contiguous()
        n_grad, dest, rows_targets = 0, None, targets
        if need_grad and n_tokens > 0:
            if n_labelled is None:
                n_labelled = int((targets >= 0).sum())
            n_grad = int(n_labelled)
            if not COMPACT and 0 < n_grad < n_tokens:
                raise ValueError("the MI355X head accumulates labelled-first rows only")
            if 0 < n_grad < n_tokens:
                dest, src = labelled_first(targets >= 0, n_grad)
                h16 = h16.index_select(0, src)
                rows_targets = targets.index_select(0, src)
                RAN["compact"] += 1
        out = head_ce(h16, w16, rows_targets, vocab_chunk, n_grad, need_grad)
        RAN["head"] += 1
        token_loss, entropy = out["token_loss"], out["entropy"]
        correct, best_idx, grad_hidden = out["correct"], out["best_idx"], out["grad"]
        if dest is not None:
            token_loss = token_loss.index_select(0, dest)
            entropy = entropy.index_select(0, dest)
            correct = correct.index_select(0, dest)
            best_idx = best_idx.index_select(0, dest)
            grad_hidden = grad_hidden.index_select(0, dest)
        loss, denom, correct = _loss(token_loss, correct, targets, num_items)
        ctx.denom = denom
        ctx.out_dtype = hidden.dtype
        if need_grad:
            ctx.save_for_backward(grad_hidden)
        ctx.mark_non_differentiable(token_loss, entropy, correct, best_idx)
        return loss, token_loss, entropy, correct, best_idx

    @staticmethod
    def backward(ctx, grad_loss, _gl, _ge, _gc, _gb):
        return _head_backward(ctx, grad_loss), None, None, None, None, None, None


def fused_head_loss(hidden, weight, targets, num_items=None, vocab_chunk=None, *,
                    token_chunk=None, n_labelled=None, return_argmax=False, grad_all_rows=False):
    """hidden [N, H] (fp16/fp32, may require grad), weight [V, H] frozen, targets [N] int64 already
    shifted (-100 = ignore). Returns (loss, token_loss[N], token_entropy[N], correct[N]) and, with
    `return_argmax`, the per-token argmax [N] (int32) as a fifth element
    (solution/fused_head.py:447-462). `n_labelled`: the exact host count of targets >= 0 when the
    caller has it (saves a host sync). `grad_all_rows`: every row is a gradient row (no
    labelled-first reordering, no count; an ignored row's gradient is zero), so no launch depends
    on a host value of the targets (a step captured in a HIP graph). `token_chunk` (the
    reference's token-chunked path) runs the same kernel `token_chunk` rows at a time."""
    need_grad = torch.is_grad_enabled() and hidden.requires_grad
    vchunk = vocab_chunk or VOCAB_CHUNK
    if grad_all_rows:
        n_labelled = hidden.shape[0]
    if token_chunk is None or token_chunk >= hidden.shape[0]:
        loss, token_loss, entropy, correct, best_idx = FusedHeadLossVocab.apply(
            hidden, weight, targets, num_items, vchunk, need_grad, n_labelled)
    else:
        parts = [FusedHeadLossVocab.apply(hidden[s:s + token_chunk], weight,
                                          targets[s:s + token_chunk], 1.0, vchunk, need_grad, None)
                 for s in range(0, hidden.shape[0], token_chunk)]
        denom = _denominator(num_items, (targets >= 0).sum())
        loss = sum(p[0] for p in parts) / denom
        token_loss, entropy, correct, best_idx = (torch.cat([p[i] for p in parts])
                                                  for i in range(1, 5))
    if return_argmax:
        return loss, token_loss, entropy, correct, best_idx
    return loss, token_loss, entropy, correct
