"""Seeded synthetic inputs of the five benchmark configurations (CPU generator, then copied to
the device, so a CPU checker and the GPU see identical bytes).

1. grouped NF4 dequant of one Qwen2.5-1.5B decoder layer;
2. add+RMSNorm and Q/K RoPE on packed varlen tokens;
3. SwiGLU forward / backward on [2048, 8960];
4. the vocabulary-chunked LM head + cross-entropy;
5. (the full QLoRA step builds its own model: talm_amd.model).
"""

import torch

from .quant import dynamic_map

HIDDEN = 1536
INTERMEDIATE = 8960
VOCAB = 151936
Q_HEADS, KV_HEADS, HEAD_DIM = 12, 2, 128
ROPE_THETA = 1e6
EPS = 1e-6

# Qwen2.5-1.5B projections of one decoder layer, in the packing order of the layer group
# (q, k, v, o, gate, up, down): (out_features, in_features).
LAYER_SHAPES = ((1536, 1536), (256, 1536), (256, 1536), (1536, 1536), (8960, 1536),
                (8960, 1536), (1536, 8960))

SEEDS = {1: 1001, 2: 1002, 3: 1003, 4: 1004, 5: 1005}


def _gen(seed):
    return torch.Generator("cpu").manual_seed(seed)


def nf4_layer(seed=SEEDS[1], shapes=LAYER_SHAPES, qblock=64, qblock2=256, offset=0.01):
    """Config 1: the packed buffers of one layer group. Nibbles uniform in 0..15, absmax codes
    uniform in 0..255, second-level scales U[0.005, 0.05], one offset for every projection."""
    g = _gen(seed)
    n = sum(a * b for a, b in shapes)
    n_rows = n // qblock
    n_blk2 = n_rows // qblock2
    return {
        "packed": torch.randint(0, 256, (n // 2,), generator=g, dtype=torch.int32).to(torch.uint8),
        "absmax8": torch.randint(0, 256, (n_rows,), generator=g, dtype=torch.int32).to(torch.uint8),
        "absmax2": torch.rand(n_blk2, generator=g) * 0.045 + 0.005,
        "offset2": torch.full((n_blk2,), offset, dtype=torch.float32),
        "code": dynamic_map(),
        "qblock": qblock, "qblock2": qblock2, "n": n, "shapes": shapes,
    }


def varlen_lengths(seed, batch=4, lo=128, hi=512):
    """Per-sequence lengths uniform in [lo, hi] and the packed offsets cu_seqlens [batch + 1]."""
    lengths = torch.randint(lo, hi + 1, (batch,), generator=_gen(seed))
    cu = torch.zeros(batch + 1, dtype=torch.int32)
    cu[1:] = torch.cumsum(lengths, 0)
    return lengths, cu


def positions_from_lengths(lengths):
    """Per-sequence positions 0 .. len - 1 of the packed tokens."""
    return torch.cat([torch.arange(int(n)) for n in lengths])


def rope_cos_sin(positions, dim=HEAD_DIM, theta=ROPE_THETA):
    """cos, sin float32 [T, dim] as transformers' Qwen2RotaryEmbedding builds them
    (inv_freq = 1 / theta^(2i / dim), emb = cat(freqs, freqs))."""
    inv_freq = 1.0 / (theta ** (torch.arange(0, dim, 2, dtype=torch.int64).float() / dim))
    freqs = positions.float()[:, None] * inv_freq[None, :]
    emb = torch.cat((freqs, freqs), dim=-1)
    return emb.cos(), emb.sin()


def norm_rope(seed=SEEDS[2]):
    """Config 2: packed varlen tokens, x / residual / dy fp16 ~N(0, 1) [N, 1536], norm weight
    ~N(1, 0.1), Q [N, 12, 128], K [N, 2, 128] ~N(0, 1) and their gradients, cos / sin."""
    lengths, cu = varlen_lengths(seed)
    n = int(cu[-1])
    g = _gen(seed + 1)
    pos = positions_from_lengths(lengths)
    cos, sin = rope_cos_sin(pos)
    return {
        "lengths": lengths, "cu_seqlens": cu, "n": n, "positions": pos,
        "x": torch.randn(n, HIDDEN, generator=g).half(),
        "residual": torch.randn(n, HIDDEN, generator=g).half(),
        "weight": 1.0 + 0.1 * torch.randn(HIDDEN, generator=g),
        "dy": torch.randn(n, HIDDEN, generator=g).half(),
        "ds": torch.randn(n, HIDDEN, generator=g).half(),
        "q": torch.randn(n, Q_HEADS, HEAD_DIM, generator=g).half(),
        "k": torch.randn(n, KV_HEADS, HEAD_DIM, generator=g).half(),
        "cos": cos, "sin": sin, "eps": EPS,
    }


def swiglu_inputs(seed=SEEDS[3], rows=2048, cols=INTERMEDIATE):
    """Config 3: gate, up ~N(0, 1) and dOut ~N(0, 0.02), fp16 [rows, cols]."""
    g = _gen(seed)
    return {"gate": torch.randn(rows, cols, generator=g).half(),
            "up": torch.randn(rows, cols, generator=g).half(),
            "grad": (torch.randn(rows, cols, generator=g) * 0.02).half()}


def head_inputs(seed=SEEDS[4], n=2048, hidden=HIDDEN, vocab=VOCAB, ignore_frac=0.1):
    """Config 4: H ~N(0, 1) fp16 [n, hidden], tied W ~N(0, 0.02) fp16 [vocab, hidden], labels
    uniform over the vocabulary with `ignore_frac` of them -100."""
    g = _gen(seed)
    hid = torch.randn(n, hidden, generator=g).half()
    w = (torch.randn(vocab, hidden, generator=g) * 0.02).half()
    targets = torch.randint(0, vocab, (n,), generator=g)
    targets[torch.rand(n, generator=g) < ignore_frac] = -100
    return {"hidden": hid, "weight": w, "targets": targets}
