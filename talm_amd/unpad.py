"""Padding removal inside a batch (solution/unpad.py:1-92).

The causal-LM patch (patches.py) gathers the real tokens of a right-padded [B, T] batch into one
flat sequence [1, N] with per-row positions, runs the decoder on it and scatters per-token
outputs back. Attention must not cross rows: while the flat forward runs (`rows_context`), the
registered "sdpa" attention interface runs causal attention per row (`rows_sdpa`), GQA heads
shared by stride, not repeated. Attention itself is not one of this package's kernels (it is
PyTorch's SDPA); its row bounds and `cu_seqlens` are the packing contract the other kernels use.
"""

import contextlib

import torch
import torch.nn.functional as F

from .engaged import FELL_BACK, ON, RAN

_rows = []
_cu = []


@contextlib.contextmanager
def rows_context(bounds, device=None):
    """Row bounds [(start, end)] of the flat sequence for the attention of this forward; with
    `device`, also cu_seqlens (int32) on it (solution/unpad.py:46-63)."""
    cu = None
    if device is not None:
        ends = [e for s, e in bounds if e > s]
        cu = torch.tensor([0] + ends, dtype=torch.int32, device=device)
    _rows.append(bounds)
    _cu.append(cu)
    try:
        yield
    finally:
        _rows.pop()
        _cu.pop()


def unpad_batch(attention_mask, targets=None):
    """From a right-padded [B, T] mask: flat indices of the real tokens, their positions inside
    their rows, the row bounds in the flat sequence and the lengths (one host sync). With
    `targets` ([B * T] shifted labels) also `counts` = [labelled among the gathered positions,
    labelled among all positions] from the same host copy (solution/unpad.py:66-92)."""
    batch, seq = attention_mask.shape
    device = attention_mask.device
    lengths_gpu = attention_mask.to(torch.int64).sum(1)
    counts = None
    if targets is None:
        lengths = lengths_gpu.tolist()
    else:
        lab = targets.reshape(batch, seq) >= 0
        prefix = torch.arange(seq, device=device)[None] < lengths_gpu[:, None]
        values = torch.cat((lengths_gpu, torch.stack(((lab & prefix).sum(), lab.sum())))).tolist()
        lengths, counts = values[:batch], values[batch:]
    idx, positions, bounds, start = [], [], [], 0
    for b, length in enumerate(lengths):
        ar = torch.arange(length, device=device)
        idx.append(ar + b * seq)
        positions.append(ar)
        bounds.append((start, start + length))
        start += length
    out = (torch.cat(idx), torch.cat(positions)[None], bounds, lengths)
    return out if targets is None else out + (counts,)


def is_right_padded(attention_mask, lengths):
    seq = attention_mask.shape[1]
    prefix = torch.arange(seq, device=attention_mask.device)[None] < \
        torch.tensor(lengths, device=attention_mask.device)[:, None]
    return bool((attention_mask.bool() == prefix).all().item())


def _autocast_half(query):
    if query.dtype != torch.float32 or not query.is_cuda or not torch.is_autocast_enabled("cuda"):
        return None
    dtype = torch.get_autocast_dtype("cuda")
    return dtype if dtype in (torch.float16, torch.bfloat16) else None


def patch_sdpa_rows():
    """Wrap transformers' registered "sdpa" attention: per-row causal attention while a flat
    forward runs, the original interface otherwise (solution/unpad.py:338-395)."""
    from transformers.modeling_utils import ALL_ATTENTION_FUNCTIONS

    original = ALL_ATTENTION_FUNCTIONS["sdpa"]
    ON.add("rows_attn")
    if getattr(original, "_solution_rows", False):
        return

    def rows_sdpa(module, query, key, value, attention_mask, dropout=0.0, scaling=None,
                  sliding_window=None, **kwargs):
        if not _rows or query.shape[0] != 1 or sliding_window is not None:
            if _rows:
                FELL_BACK["rows_attn"] += 1
            return original(module, query, key, value, attention_mask, dropout=dropout,
                            scaling=scaling, sliding_window=sliding_window, **kwargs)
        half = _autocast_half(query)
        if half is not None:
            query, key, value = query.to(half), key.to(half), value.to(half)
        gqa = query.shape[1] != key.shape[1]
        outs = [F.scaled_dot_product_attention(query[:, :, s:e], key[:, :, s:e], value[:, :, s:e],
                                               dropout_p=dropout, is_causal=True, scale=scaling,
                                               enable_gqa=gqa)
                for s, e in _rows[-1] if e > s]
        RAN["rows_attn"] += 1
        attn = outs[0] if len(outs) == 1 else torch.cat(outs, dim=2)
        return attn.transpose(1, 2).contiguous(), None

    rows_sdpa._solution_rows = True
    rows_sdpa._original = original
    ALL_ATTENTION_FUNCTIONS["sdpa"] = rows_sdpa
