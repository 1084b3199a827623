"""Batch packing oracle of the packed causal-LM step (test infrastructure), numpy + Python loops.

Only tests/ (and `__graft_entry__.smoke()`, bench.py's CPU baseline) use this module, as the
checker of talm_amd's kernels; the product path never imports it.

- `shift_labels`: the causal-LM label shift, labels[b][t + 1] at position t and -100 at a row's
  last position (solution/patches.py:186).
- `unpad_batch`: the reference's packing of a right-padded batch (solution/unpad.py:66-92): row b
  holds len_b = sum_t mask[b][t] real tokens; the flat sequence is row 0's first len_0 tokens,
  then row 1's, ...; per token its source index b * seq + p and its position p; `counts` = the
  labelled shifted targets among the gathered positions and among all positions.
- `pack_rows`: the same packing into exactly `n_tokens` rows (a step captured in a HIP graph):
  the real tokens first (row lengths clamped to [0, seq], the running total to n_tokens), then one
  more sequence over the remaining rows that reads the pad slot batch * seq (id 0, target -100).
  Written as per-row loops, independently of the offsets-and-search form of talm_pack_rows and
  of unpad.unpad_static's matrix form.
- `row_stats`: [len_0 .. len_{B-1}, labelled among gathered, labelled among all]
  (solution/unpad.py:77-83).
- `scatter`: per-token values back to `out_len` batch slots, zero elsewhere
  (solution/patches.py:244-249).
"""

import numpy as np


def shift_labels(labels):
    labels = np.asarray(labels, np.int64)
    out = np.full_like(labels, -100)
    out[:, :-1] = labels[:, 1:]
    return out.reshape(-1)


def unpad_batch(mask, labels):
    """(idx, positions, lengths, counts) of the reference's packing."""
    mask = np.asarray(mask, np.int64)
    batch, seq = mask.shape
    lengths = [int(v) for v in mask.sum(1)]
    shift = shift_labels(labels).reshape(batch, seq)
    idx, positions = [], []
    gathered = 0
    for b, length in enumerate(lengths):
        for p in range(length):
            idx.append(b * seq + p)
            positions.append(p)
            gathered += int(shift[b, p] >= 0)
    counts = [gathered, int((shift >= 0).sum())]
    return np.array(idx, np.int64), np.array(positions, np.int64), lengths, counts


def row_stats(mask, labels):
    _idx, _pos, lengths, counts = unpad_batch(mask, labels)
    return np.array(lengths + counts, np.int64)


def pack_rows(input_ids, mask, labels, n_tokens):
    """(ids, positions, cu_seqlens, targets, src) of the fixed-shape packing."""
    input_ids = np.asarray(input_ids, np.int64)
    mask = np.asarray(mask, np.int64)
    batch, seq = mask.shape
    shift = shift_labels(labels)
    ids, positions, targets, src, cu = [], [], [], [], [0]
    for b in range(batch):
        length = min(max(int(mask[b].sum()), 0), seq)
        for p in range(length):
            if len(src) == n_tokens:
                break
            src.append(b * seq + p)
            positions.append(p)
            ids.append(int(input_ids[b, p]))
            targets.append(int(shift[b * seq + p]))
        cu.append(len(src))
    pad_start = len(src)
    for j in range(pad_start, n_tokens):
        src.append(batch * seq)
        positions.append(j - pad_start)
        ids.append(0)
        targets.append(-100)
    cu.append(n_tokens)
    return (np.array(ids, np.int64), np.array(positions, np.int64), np.array(cu, np.int32),
            np.array(targets, np.int64), np.array(src, np.int64))


def scatter(values, src, out_len):
    """full[k] = 0, then full[src[i]] = values[i] in row order (a later row wins a shared slot)."""
    full = np.zeros(out_len, np.asarray(values).dtype)
    for i, k in enumerate(np.asarray(src)):
        full[k] = values[i]
    return full
