"""Fused LM head + cross-entropy oracle (test infrastructure), numpy.

`head_ce` restates the vocabulary-sliced head of the reference step by step
(FusedHeadLossVocab.forward, solution/fused_head.py:315-393, with fused_head_vocab_kernel,
:88-182): per slice of `vchunk` columns, fp16 logits z = fp16(h16 @ W16[slice]^T) (fp32
accumulation, :364); per BLOCK_V block of the slice the online statistics m (max), s (sum of
e^{z-m}), t (sum of e^{z-m} z), the first maximum and its column (tie to the left, :147-150), and
z at the target (:151-153); then, for labelled rows, the accumulator rescale by e^{m_old - m} when
the row maximum grew (:171-177), P = fp16(e^{z - m}) (:178-182) and acc += P @ W16[slice] in fp32
(:369-371). Finally lse = m + log s, entropy = lse - t / s, token loss = log s + m - z_target
(0 unlabelled), correct = labelled & argmax == target, dH = acc / s - W16[target] (0 unlabelled,
:111-125, written in fp16). The loss is sum(token loss) / denominator (:272-277, :385-386).

`head_direct` is the closed form of the same quantities in float64 over the same fp16 logits
(transformers' cross-entropy, TRL's entropy, torch.argmax's first maximum: `reference_head`,
solution/test_kernels.py:70-83, and `_head_reference`, solution/test_fuzz.py:145-185). The
online algorithm is pinned against it (any slice / block width gives the same statistics).
"""

import numpy as np

F32 = np.float32


def logits16(h16, w16):
    """fp16 logits of an fp16 GEMM with fp32 accumulation (exact for exact-style inputs)."""
    return (np.asarray(h16, np.float32) @ np.asarray(w16, np.float32).T).astype(np.float16)


def head_ce(h16, w16, targets, vchunk=8192, block=4096, need_grad=True):
    """dict(token_loss f32, entropy f32, best_idx int64, correct bool, grad f16 or None, m, s)."""
    h16 = np.asarray(h16, np.float16)
    w16 = np.asarray(w16, np.float16)
    targets = np.asarray(targets, np.int64)
    n, hidden = h16.shape
    vocab = w16.shape[0]
    lab = targets >= 0
    m = np.full(n, -np.inf, F32)
    s = np.zeros(n, F32)
    t = np.zeros(n, F32)
    best = np.full(n, -np.inf, F32)
    best_idx = np.zeros(n, np.int64)
    zt = np.zeros(n, F32)
    acc = np.zeros((n, hidden), F32)
    rows = np.arange(n)
    for start in range(0, vocab, vchunk):
        cols = min(vchunk, vocab - start)
        w_slice = w16[start:start + cols]
        z = logits16(h16, w_slice).astype(F32)
        m_old = m.copy()
        with np.errstate(invalid="ignore", over="ignore"):
            for b0 in range(0, cols, block):
                zb = z[:, b0:b0 + block]
                bmax = zb.max(1)
                m_new = np.maximum(m, bmax)
                alpha = np.exp(m - m_new).astype(F32)
                e = np.exp(zb - m_new[:, None]).astype(F32)
                s = (s * alpha + e.sum(1, dtype=F32)).astype(F32)
                t = (t * alpha + (e * zb).sum(1, dtype=F32)).astype(F32)
                m = m_new
                bidx = zb.argmax(1)
                better = bmax > best
                best_idx = np.where(better, start + b0 + bidx, best_idx)
                best = np.maximum(best, bmax)
        rel = targets - start
        here = lab & (rel >= 0) & (rel < cols)
        zt[here] = z[rows[here], rel[here]]
        if need_grad and lab.any():
            grow = lab & (m > m_old) & (start > 0)
            acc[grow] *= np.exp(m_old[grow] - m[grow]).astype(F32)[:, None]
            p16 = np.exp(z[lab] - m[lab][:, None]).astype(np.float16)
            acc[lab] += p16.astype(F32) @ w_slice.astype(F32)
    with np.errstate(divide="ignore", invalid="ignore"):
        ls = np.log(s).astype(F32)
        lse = m + ls
        entropy = (lse - t / s).astype(F32)
        token_loss = np.where(lab, ls + (m - zt), F32(0)).astype(F32)
    correct = lab & (best_idx == targets)
    grad = None
    if need_grad:
        w_t = w16[np.maximum(targets, 0)].astype(F32)
        with np.errstate(divide="ignore", invalid="ignore"):
            g = acc / s[:, None] - w_t
        grad = np.where(lab[:, None], g, F32(0)).astype(np.float16)
    return {"token_loss": token_loss, "entropy": entropy, "best_idx": best_idx,
            "correct": correct, "grad": grad, "m": m, "s": s}


def head_direct(h16, w16, targets):
    """Closed form in float64 over the fp16 logits: token loss, entropy, first argmax, correct,
    and the gradient of sum(token loss) w.r.t. the hidden states (float64)."""
    z = logits16(h16, w16).astype(np.float64)
    targets = np.asarray(targets, np.int64)
    lab = targets >= 0
    m = z.max(1)
    lse = m + np.log(np.exp(z - m[:, None]).sum(1))
    p = np.exp(z - lse[:, None])
    entropy = lse - (p * z).sum(1)
    tc = np.maximum(targets, 0)
    token_loss = np.where(lab, lse - z[np.arange(len(z)), tc], 0.0)
    best_idx = z.argmax(1)
    correct = lab & (best_idx == targets)
    p[np.arange(len(z)), tc] -= lab
    p[~lab] = 0.0
    grad = p @ np.asarray(w16, np.float64)
    return {"token_loss": token_loss, "entropy": entropy, "best_idx": best_idx,
            "correct": correct, "grad": grad, "zmax": np.abs(z).max(1)}


def loss(token_loss, targets, num_items=None):
    """The reference's mean: sum(token loss) / (num_items or max(#labelled, 1))."""
    n_lab = int((np.asarray(targets) >= 0).sum())
    denom = float(num_items) if num_items is not None else float(max(n_lab, 1))
    return float(np.asarray(token_loss, np.float64).sum() / denom), denom
