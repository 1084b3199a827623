"""Padding removal inside a batch (solution/unpad.py:1-92).

The causal-LM patch (patches.py) gathers the real tokens of a right-padded [B, T] batch into one
flat sequence [1, N] with per-row positions, runs the decoder on it and scatters per-token
outputs back. Attention must not cross rows: while the flat forward runs (`rows_context`), the
registered "sdpa" attention interface runs causal attention that never crosses rows
(`rows_sdpa`): all rows in one variable-length flash-attention launch per direction with the
row offsets `cu_seqlens` and GQA heads shared, not repeated (`VarlenAttention`: this package's
HIP kernels for fp16 heads of 128, PyTorch's varlen flash attention otherwise; the reference
launches one memory-efficient attention per KV head, solution/unpad.py:199-294), else one SDPA
call per row.
"""

import contextlib
import weakref

import torch
import torch.nn.functional as F

from . import _ops  # noqa: F401 - registers torch.ops.talm.*
from .engaged import FELL_BACK, ON, RAN
from .state import DISABLED, fallback

_rows = []
_cu = []
_ahead = {}  # batch key -> (mask ref, labels ref, pinned host values, event): row statistics
             # copied ahead of time
_AHEAD_MAX = 4


@contextlib.contextmanager
def rows_context(bounds, device=None):
    """Row bounds [(start, end)] of the flat sequence for the attention of this forward; with
    `device`, also (cu_seqlens int32 on it, longest row, total tokens) (solution/unpad.py:46-63)."""
    cu = None
    if device is not None:
        ends = [e for s, e in bounds if e > s]
        if ends:
            # pinned and asynchronous: a pageable copy would wait for the stream to drain
            cu = (torch.tensor([0] + ends, dtype=torch.int32).pin_memory().to(
                      device, non_blocking=True),
                  max(e - s for s, e in bounds if e > s), ends[-1])
    _rows.append(bounds)
    _cu.append(cu)
    try:
        yield
    finally:
        _rows.pop()
        _cu.pop()


def _row_values(attention_mask, targets=None):
    """[B] row lengths of a right-padded mask, then (with `targets`, [B * T] shifted labels) the
    labelled count among the real tokens and among all positions, as one device vector."""
    batch, seq = attention_mask.shape
    lengths = attention_mask.to(torch.int64).sum(1)
    if targets is None:
        return lengths
    lab = targets.reshape(batch, seq) >= 0
    prefix = torch.arange(seq, device=attention_mask.device)[None] < lengths[:, None]
    return torch.cat((lengths, torch.stack(((lab & prefix).sum(), lab.sum()))))


def _int64_rows(*tensors):
    """The [B, T] batch tensors suit the packing kernels: contiguous int64 on one GPU."""
    first = tensors[0]
    return all(t.is_cuda and t.dtype == torch.int64 and t.is_contiguous() and t.dim() == 2
               and t.shape == first.shape and t.device == first.device for t in tensors)


def _batch_key(attention_mask, labels):
    return (attention_mask.data_ptr(), attention_mask._version, tuple(attention_mask.shape),
            labels.data_ptr(), labels._version, tuple(labels.shape))


def prefetch(attention_mask, labels):
    """Start the host copy of a coming batch's row statistics (GPU-side packing's one host
    input): queued now, read by that batch's `unpad_batch` without waiting for the stream.
    A training loop that knows its next batch calls this one step ahead, so no step stalls the
    host on the GPU's backlog (solution/unpad.py:66-92 syncs once per step)."""
    if not (attention_mask.is_cuda and attention_mask.dim() == 2 and labels.dim() == 2
            and tuple(labels.shape) == tuple(attention_mask.shape)):
        return
    if _int64_rows(attention_mask, labels):
        # one launch (talm_row_stats) for the lengths and both labelled counts
        values = torch.empty(attention_mask.shape[0] + 2, dtype=torch.int64,
                             device=attention_mask.device)
        torch.ops.talm.row_stats(attention_mask, labels, values)
    else:
        shift = torch.nn.functional.pad(labels, (0, 1), value=-100)[:, 1:].reshape(-1)
        values = _row_values(attention_mask, shift.to(attention_mask.device))
    host = torch.empty(values.shape, dtype=torch.int64, pin_memory=True)
    host.copy_(values, non_blocking=True)
    event = torch.cuda.Event()
    event.record()
    while len(_ahead) >= _AHEAD_MAX:
        _ahead.pop(next(iter(_ahead)))
    _ahead[_batch_key(attention_mask, labels)] = (
        weakref.ref(attention_mask), weakref.ref(labels), host, event)


def take_prefetched(attention_mask, labels):
    """The row statistics `prefetch` started for this batch (a host list), or None. An entry
    counts only for the very tensors it was made from: the key (address, version, shape) alone
    would also match a later batch the allocator placed at a freed batch's address, and that
    batch would get the other one's row lengths."""
    if not _ahead or labels is None:
        return None
    hit = _ahead.pop(_batch_key(attention_mask, labels), None)
    if hit is None:
        return None
    mask_ref, labels_ref, host, event = hit
    if mask_ref() is not attention_mask or labels_ref() is not labels:
        return None
    event.synchronize()  # queued a step ago: long done
    return host.tolist()


def unpad_batch(attention_mask, targets=None, values=None):
    """From a right-padded [B, T] mask: flat indices of the real tokens, their positions inside
    their rows, the row bounds in the flat sequence and the lengths (one host sync, or none when
    `values` holds what `take_prefetched` returned). With `targets` ([B * T] shifted labels) also
    `counts` = [labelled among the gathered positions, labelled among all positions] from the
    same host copy (solution/unpad.py:66-92)."""
    batch, seq = attention_mask.shape
    device = attention_mask.device
    counts = None
    if values is None:
        values = _row_values(attention_mask, targets).tolist()
    if targets is None:
        lengths = values[:batch]
    else:
        lengths, counts = values[:batch], values[batch:batch + 2]
    idx, positions, bounds, start = [], [], [], 0
    for b, length in enumerate(lengths):
        ar = torch.arange(length, device=device)
        idx.append(ar + b * seq)
        positions.append(ar)
        bounds.append((start, start + length))
        start += length
    out = (torch.cat(idx), torch.cat(positions)[None], bounds, lengths)
    return out if targets is None else out + (counts,)


_static = []  # (token count, longest pad sequence) of the fixed-shape packing in force


@contextlib.contextmanager
def static_tokens(n_tokens, max_pad=None):
    """While it is open, the causal-LM patch packs every batch into exactly `n_tokens` rows on the
    device (`unpad_static`): no host value of the batch is read, so the forward and backward can
    be captured in a HIP graph and replayed for any batch of at most `n_tokens` real tokens.
    `max_pad` bounds the pad sequence's length (n_tokens minus the real tokens) for every batch
    the packing will serve; the attention's grid must cover it (default: n_tokens)."""
    n_tokens = int(n_tokens)
    _static.append((n_tokens, n_tokens if max_pad is None else min(int(max_pad), n_tokens)))
    try:
        yield
    finally:
        _static.pop()


def static_n_tokens():
    return _static[-1][0] if _static else None


def static_max_len(seq):
    """The longest sequence of the packing in force with rows of at most `seq` tokens: a real
    row, or the pad sequence."""
    return max(int(seq), _static[-1][1]) if _static else int(seq)


def unpad_static(attention_mask, targets, n_tokens):
    """Packing into a fixed row count with device ops only. The real tokens of the right-padded
    [B, T] mask come first, in row order (as `unpad_batch`); the remaining n_tokens - N rows form
    one more sequence that attends only to itself and is labelled -100, so its loss and every
    gradient that flows through it are exactly zero (the head gives ignored rows a zero gradient,
    and no other sequence reads its keys). Returns (src, positions [1, n_tokens], cu_seqlens
    int32 [B + 2], targets [n_tokens]): src indexes the flat [B * T + 1] batch whose last element
    is the pad slot. The caller guarantees N <= n_tokens."""
    batch, seq = attention_mask.shape
    device = attention_mask.device
    # elementwise ops and single-block sums only (no library scan, no host value): every launch
    # here can be recorded in a HIP graph
    lengths = attention_mask.sum(1, dtype=torch.int32)
    k = torch.arange(batch + 2, dtype=torch.int32, device=device)
    before = k[:, None] > k[None, :batch]                       # [B + 2, B]: row b < k
    cu = torch.where(k == batch + 1, n_tokens, (before * lengths[None, :]).sum(1, dtype=torch.int32))
    # a batch with more real tokens than rows (a caller's wrong count) loses its last tokens
    # instead of sending the attention past the [n_tokens] buffers
    cu = cu.clamp(0, n_tokens).to(torch.int32)
    j = torch.arange(n_tokens, dtype=torch.int32, device=device)
    row = torch.searchsorted(cu[1:batch + 1], j, right=True)
    pos = j - cu.index_select(0, row)
    src = torch.where(row < batch, row * seq + pos, batch * seq)
    ext = torch.cat((targets.reshape(-1), targets.new_full((1,), -100)))
    return src, pos.to(torch.int64)[None], cu, ext.index_select(0, src)


def pack_static(input_ids, attention_mask, labels, n_tokens):
    """`unpad_static` from the unshifted batch, with the ids gathered: (ids [n_tokens], positions
    [1, n_tokens], cu_seqlens int32 [B + 2], targets [n_tokens], src [n_tokens]). One launch
    (talm_pack_rows) for contiguous int64 batch tensors; the same values as shifting the labels
    and composing `unpad_static` with the id gather otherwise. Row lengths are clamped to the
    row width (a mask whose row sums exceed it is not a right-padded mask)."""
    n_tokens = int(n_tokens)
    if _int64_rows(input_ids, attention_mask, labels):
        device = attention_mask.device
        ids, positions, targets, src = (torch.empty(n_tokens, dtype=torch.int64, device=device)
                                        for _ in range(4))
        cu = torch.empty(attention_mask.shape[0] + 2, dtype=torch.int32, device=device)
        torch.ops.talm.pack_rows(input_ids, attention_mask, labels, n_tokens, ids, positions, cu,
                                 targets, src)
        RAN["pack_rows"] += 1
        return ids, positions[None], cu, targets, src
    shift = torch.nn.functional.pad(labels, (0, 1), value=-100)[:, 1:].reshape(-1)
    src, positions, cu, targets = unpad_static(attention_mask, shift.to(attention_mask.device),
                                               n_tokens)
    ids = torch.cat((input_ids.reshape(-1), input_ids.new_zeros(1))).index_select(0, src)
    return ids, positions, cu, targets, src


@contextlib.contextmanager
def rows_context_static(cu, max_len, total):
    """`rows_context` for `unpad_static`'s packing: cu_seqlens already on the device, no host row
    bounds (the per-row fallback attention cannot run; the varlen kernel must)."""
    _rows.append(None)
    _cu.append((cu, max_len, total))
    try:
        yield
    finally:
        _rows.pop()
        _cu.pop()


def is_right_padded(attention_mask, lengths):
    seq = attention_mask.shape[1]
    prefix = torch.arange(seq, device=attention_mask.device)[None] < \
        torch.tensor(lengths, device=attention_mask.device)[:, None]
    return bool((attention_mask.bool() == prefix).all().item())


def _kernel_applies(q, k, v):
    """The [N, H, D] views suit torch.ops.talm.attn_*: fp16, head_dim 128, strides of whole
    16-byte chunks, 16-byte aligned."""
    return (q.dtype == torch.float16 and q.shape[-1] == 128
            and all(t.stride(0) % 8 == 0 and t.stride(1) % 8 == 0 and t.data_ptr() % 16 == 0
                    for t in (q, k, v)))


class VarlenAttention(torch.autograd.Function):
    """Causal attention of every row of the flat sequence in ONE launch each way, with the row
    offsets `cu_seqlens` and the KV heads shared by the query heads of their group (GQA, no
    repeated K/V): this package's HIP kernels (`torch.ops.talm.attn_fwd` / `attn_bwd`) for fp16
    heads of 128, else PyTorch's variable-length flash attention. Inputs are the [1, H, N, D]
    views the attention interface receives; the output is [1, N, Hq, D] as SDPA's transposed
    output is. Semantics of per-row `scaled_dot_product_attention(..., is_causal=True)`
    (solution/unpad.py:121-134, :199-294)."""

    @staticmethod
    def forward(ctx, query, key, value, cu, max_len, scale):
        q, k, v = (t[0].transpose(0, 1) for t in (query, key, value))  # [N, H, D] views
        ctx.max_len, ctx.scale = max_len, scale
        ctx.kernel = _kernel_applies(q, k, v)
        if ctx.kernel:
            n, hq = q.shape[0], q.shape[1]
            out = torch.empty(n, hq, q.shape[2], dtype=q.dtype, device=q.device)
            lse = torch.empty(hq, n, dtype=torch.float32, device=q.device)
            torch.ops.talm.attn_fwd(q, k, v, cu, max_len, scale, out, lse)
            ctx.save_for_backward(q, k, v, out, lse, cu)
            RAN["attn_kernel"] += 1
            return out[None]
        out, lse, rng, unused, _ = torch.ops.aten._flash_attention_forward(
            q, k, v, cu, cu, max_len, max_len, 0.0, True, False, scale=scale)
        ctx.save_for_backward(q, k, v, out, lse, rng, unused, cu)
        return out[None]

    @staticmethod
    def backward(ctx, grad):
        g = grad[0]
        if ctx.kernel:
            q, k, v, out, lse, cu = ctx.saved_tensors
            if g.stride(-1) != 1 or g.stride(0) % 8 or g.stride(1) % 8 or g.data_ptr() % 16:
                g = g.contiguous()
            dq = torch.empty_like(out)
            dk = torch.empty(k.shape, dtype=k.dtype, device=k.device)
            dv = torch.empty(v.shape, dtype=v.dtype, device=v.device)
            ws = torch.empty(_ops.attn_bwd_workspace_bytes(q.shape[0], q.shape[1]),
                             dtype=torch.uint8, device=q.device)
            torch.ops.talm.attn_bwd(q, k, v, out, g, lse, cu, ctx.max_len, ctx.scale, dq, dk, dv,
                                    ws)
            RAN["attn_kernel_bwd"] += 1
        else:
            q, k, v, out, lse, rng, unused, cu = ctx.saved_tensors
            if not g.is_contiguous():
                g = g.contiguous()
            dq, dk, dv = torch.ops.aten._flash_attention_backward(
                g, q, k, v, out, lse, cu, cu, ctx.max_len, ctx.max_len, 0.0, True, rng, unused,
                scale=ctx.scale)
        return (dq.transpose(0, 1)[None], dk.transpose(0, 1)[None], dv.transpose(0, 1)[None],
                None, None, None)


def _varlen_applies(query, key, value, dropout, cu):
    return (cu is not None and dropout == 0.0 and query.is_cuda and query.dim() == 4
            and query.shape[0] == 1 and query.dtype in (torch.float16, torch.bfloat16)
            and key.dtype == query.dtype and value.dtype == query.dtype
            and key.shape == value.shape and query.shape[1] % key.shape[1] == 0
            and query.shape[2] == key.shape[2] and query.shape[3] == key.shape[3]
            and query.stride(-1) == 1 and key.stride(-1) == 1 and value.stride(-1) == 1)


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
        cu = _cu[-1] if _cu else None
        if "varlen_attention" not in DISABLED and cu is not None \
                and _varlen_applies(query, key, value, dropout, cu[0]) \
                and cu[2] == query.shape[2]:
            try:
                scale = scaling if scaling is not None else query.shape[-1] ** -0.5
                out = VarlenAttention.apply(query, key, value, cu[0], cu[1], scale)
            except Exception as exc:  # noqa: BLE001 - state.py convention
                if not fallback("varlen_attention", exc):
                    raise
            else:
                RAN["varlen_attn"] += 1
                return out, None
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
