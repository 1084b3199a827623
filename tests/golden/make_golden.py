"""Writes the committed golden fixtures of tests/golden/ (run once, on the CPU):

    python tests/golden/make_golden.py

The reference commits no vectors (its tests draw their inputs on the CUDA RNG), so these are
built here from seeded CPU generators. Expected values come from PyTorch, not from `oracle/`:
float64 autograd for the norm, the rotary embedding and SwiGLU, PyTorch's float32 elementwise ops
for the NF4 closed form (`_nf4_manual`, solution/test_fuzz.py:860-868), and a float64 softmax
over the full fp16 logits for the head. tests/test_golden.py checks the oracle and the package
against them; tests/test_gpu_golden.py checks the HIP kernels.

Files (all plain data: numpy .npz without pickles, and text):
- dynamic_map.txt    bitsandbytes' double-quant code table, create_dynamic_map(signed=True),
                     run as its published code does (float32 torch.linspace), 256 lines
                     "<index> <float32 bits hex> <value>";
- nf4_group.npz      a 7 x 16384-weight layer group (uniform nibbles and absmax codes,
                     absmax2 U[0.005, 0.05], one offset per projection) with the sha256 of the
                     fp16 output and 704 explicit (index, fp16 bits) values;
- norm_rope_swiglu.npz  small fp16-representable inputs with float64 outputs and gradients;
- head_v4097.npz     an exact-style LM head case (solution/test_fuzz.py:249-256), V = 4097 (one
                     partial slice at any power-of-two slice width), a planted argmax tie, ignored
                     rows, float64 loss / entropy / argmax / dH.
"""

import hashlib
import sys
from pathlib import Path

import numpy as np
import torch

HERE = Path(__file__).resolve().parent
ROOT = HERE.parents[1]

NF4_LEVELS = (-1.0, -0.6961928009986877, -0.5250730514526367, -0.39491748809814453,
              -0.28444138169288635, -0.18477343022823334, -0.09105003625154495, 0.0,
              0.07958029955625534, 0.16093020141124725, 0.24611230194568634, 0.33791524171829224,
              0.44070982933044434, 0.5626170039176941, 0.7229568362236023, 1.0)


def create_dynamic_map(signed=True, max_exponent_bits=7, total_bits=8):
    """bitsandbytes.functional.create_dynamic_map as published (Dettmers et al., 8-bit
    optimizers via block-wise quantization, 2022): per exponent i, the midpoints of
    2^(i + non_sign_bits - max_exponent_bits) + 1 float32 points of torch.linspace(0.1, 1)
    times 10^(i - (max_exponent_bits - 1)), both signs when signed, then 0 and 1, padded with
    zeros to 2^total_bits and sorted."""
    data = []
    non_sign_bits = total_bits - 1
    additional_items = 2 ** (non_sign_bits - max_exponent_bits) - 1
    for i in range(max_exponent_bits):
        fraction_items = int(2 ** (i + non_sign_bits - max_exponent_bits) + 1 if signed
                             else 2 ** (i + non_sign_bits - max_exponent_bits + 1) + 1)
        boundaries = torch.linspace(0.1, 1, fraction_items, dtype=torch.float32)
        means = (boundaries[:-1] + boundaries[1:]) / 2.0
        data += ((10 ** (-(max_exponent_bits - 1) + i)) * means).tolist()
        if signed:
            data += (-(10 ** (-(max_exponent_bits - 1) + i)) * means).tolist()
    if additional_items > 0:
        boundaries = torch.linspace(0.1, 1, additional_items + 1, dtype=torch.float32)
        means = (boundaries[:-1] + boundaries[1:]) / 2.0
        data += ((10 ** (-(max_exponent_bits - 1) + i)) * means).tolist()
        if signed:
            data += (-(10 ** (-(max_exponent_bits - 1) + i)) * means).tolist()
    data.append(0)
    data.append(1.0)
    assert len(data) == 2 ** total_bits
    data += [0] * (256 - len(data))
    data.sort()
    return torch.tensor(data, dtype=torch.float32)


def write_dynamic_map():
    table = create_dynamic_map()
    bits = table.view(torch.int32).numpy().view(np.uint32)
    lines = [f"{i} {int(b):08x} {float(v)!r}" for i, (b, v) in enumerate(zip(bits, table))]
    (HERE / "dynamic_map.txt").write_text("\n".join(lines) + "\n")
    return table


def nf4_closed_form(packed, absmax8, code, absmax2, offset2, qblock=64, qblock2=256):
    """fp16 bits of the grouped NF4 dequantization with PyTorch float32 ops, one rounding per
    operation: scale = (code[absmax8] * absmax2) + offset2 per block, out = level * scale."""
    packed = torch.from_numpy(packed).to(torch.int64)
    nib = torch.stack((packed >> 4, packed & 15), 1).reshape(-1)
    levels = torch.tensor(NF4_LEVELS, dtype=torch.float32)
    blk = torch.arange(absmax8.size) // qblock2
    prod = torch.from_numpy(code)[torch.from_numpy(absmax8).long()] * torch.from_numpy(absmax2)[blk]
    scale = prod + torch.from_numpy(offset2)[blk]
    vals = levels[nib] * scale.repeat_interleave(qblock)
    return vals.to(torch.float16).view(torch.int16).numpy().view(np.uint16)


def write_nf4(table):
    g = torch.Generator().manual_seed(2024)
    n_proj, per = 7, 16384
    n = n_proj * per
    packed = torch.randint(0, 256, (n // 2,), generator=g, dtype=torch.int32).to(torch.uint8)
    packed[:4] = torch.tensor([0x0F, 0xF0, 0x77, 0x88], dtype=torch.uint8)  # level order checks
    absmax8 = torch.randint(0, 256, (n // 64,), generator=g, dtype=torch.int32).to(torch.uint8)
    absmax2 = torch.rand(n // 16384, generator=g) * 0.045 + 0.005
    offset2 = torch.tensor([0.01, 0.012, 0.009, 0.011, 0.0105, 0.0095, 0.013], dtype=torch.float32)
    arrays = {k: v.numpy() for k, v in (("packed", packed), ("absmax8", absmax8),
                                        ("absmax2", absmax2), ("offset2", offset2),
                                        ("code", table))}
    out = nf4_closed_form(**arrays)
    pick = np.unique(np.concatenate([np.arange(64), np.arange(n - 64, n),
                                     torch.randint(0, n, (576,), generator=g).numpy()]))
    np.savez_compressed(HERE / "nf4_group.npz", **arrays, sample_index=pick.astype(np.int64),
                        sample_bits=out[pick], sha256=np.frombuffer(
                            hashlib.sha256(out.tobytes()).digest(), dtype=np.uint8))


def _f16(t):
    return t.half().double()


def write_norm_rope_swiglu():
    g = torch.Generator().manual_seed(77)
    # add + RMSNorm, eps 1e-6: y = w * x * rsqrt(mean(x^2) + eps), x = a + p
    a = _f16(torch.randn(6, 64, generator=g, dtype=torch.float64))
    p = _f16(torch.randn(6, 64, generator=g, dtype=torch.float64))
    w = 1 + 0.1 * torch.randn(64, generator=g, dtype=torch.float64)
    w = w.float().double()
    dy = _f16(torch.randn(6, 64, generator=g, dtype=torch.float64))
    x = (a + p).requires_grad_()
    y = torch.nn.functional.rms_norm(x, (64,), w, eps=1e-6)
    (dx,) = torch.autograd.grad(y, x, dy)
    rstd = torch.rsqrt(x.detach().pow(2).mean(-1) + 1e-6)
    # rotary embedding, theta 1e6, positions of two rows (3 and 2 tokens), as complex products
    q = _f16(torch.randn(5, 3, 16, generator=g, dtype=torch.float64))
    dq = _f16(torch.randn(5, 3, 16, generator=g, dtype=torch.float64))
    pos = torch.tensor([0, 1, 2, 0, 1], dtype=torch.float64)
    inv = 1.0 / (1e6 ** (torch.arange(0, 16, 2, dtype=torch.float64) / 16))
    ang = pos[:, None] * inv[None, :]                               # [T, 8]
    qv = q.clone().requires_grad_()
    z = torch.complex(qv[..., :8], qv[..., 8:]) * torch.polar(torch.ones_like(ang), ang)[:, None]
    rot = torch.cat((z.real, z.imag), -1)
    (dq_back,) = torch.autograd.grad(rot, qv, dq)
    cos = torch.cat((ang, ang), -1).cos()
    sin = torch.cat((ang, ang), -1).sin()
    # SwiGLU: silu(gate) * up
    gate = _f16(3 * torch.randn(4, 40, generator=g, dtype=torch.float64))
    gate[0, :4] = torch.tensor([0.0, -20.0, 20.0, -0.5], dtype=torch.float64)
    up = _f16(torch.randn(4, 40, generator=g, dtype=torch.float64))
    dout = _f16(0.02 * torch.randn(4, 40, generator=g, dtype=torch.float64))
    gv, uv = gate.clone().requires_grad_(), up.clone().requires_grad_()
    act = torch.nn.functional.silu(gv) * uv
    dgate, dup = torch.autograd.grad(act, (gv, uv), dout)
    arrays = {
        "norm_a": a, "norm_p": p, "norm_w": w, "norm_dy": dy, "norm_sum": x.detach(),
        "norm_y": y.detach(), "norm_rstd": rstd, "norm_dx": dx,
        "rope_x": q, "rope_dy": dq, "rope_cos": cos, "rope_sin": sin, "rope_y": rot.detach(),
        "rope_dx": dq_back, "rope_positions": pos,
        "swiglu_gate": gate, "swiglu_up": up, "swiglu_grad": dout, "swiglu_out": act.detach(),
        "swiglu_dgate": dgate, "swiglu_dup": dup,
    }
    np.savez_compressed(HERE / "norm_rope_swiglu.npz",
                        **{k: v.numpy() for k, v in arrays.items()})


def write_head():
    """Exact-style inputs: every product is a power of two times a small integer, so the fp16
    logits are exact and their argmax has no rounding ambiguity; row 5's target column has a
    duplicate at a later column (an exact tie: the first one is the argmax)."""
    g = torch.Generator().manual_seed(4097)
    n, hidden, vocab = 40, 128, 4097
    a = torch.randint(-3, 3, (n, 1), generator=g).double()
    b = torch.randint(-6, -1, (vocab, 1), generator=g).double()
    h = torch.randint(-1, 2, (n, hidden), generator=g).double() * torch.exp2(a)
    w = torch.randint(-1, 2, (vocab, hidden), generator=g).double() * torch.exp2(b)
    targets = torch.randint(0, vocab, (n,), generator=g)
    targets[torch.rand(n, generator=g) < 0.2] = -100
    targets[[0, 7]] = torch.tensor([vocab - 1, 4096 - 128])  # last column, a slice boundary
    targets[5] = 100
    w[3001] = w[100]                                          # the planted tie
    sure = (targets >= 0) & (torch.rand(n, generator=g) < 0.5)
    h[sure] = torch.sign(w[targets[sure]]) * torch.exp2(a[sure])
    h[5] = torch.sign(w[100]) * 2.0
    h16, w16 = h.half(), w.half()
    assert torch.equal(h16.double(), h) and torch.equal(w16.double(), w)
    z = h @ w.T
    assert torch.equal(z.half().double(), z)  # exact in fp16
    lse = torch.logsumexp(z, 1)
    prob = torch.softmax(z, 1)
    lab = targets >= 0
    zt = z.gather(1, targets.clamp(min=0)[:, None])[:, 0]
    token_loss = torch.where(lab, lse - zt, torch.zeros_like(lse))
    entropy = lse - (prob * z).sum(1)
    argmax = z.argmax(1)
    assert int(argmax[5]) == 100
    onehot = torch.zeros_like(z)
    onehot[lab, targets[lab]] = 1.0
    dh = torch.where(lab[:, None], (prob - onehot) @ w, torch.zeros(n, hidden, dtype=torch.float64))
    np.savez_compressed(HERE / "head_v4097.npz", hidden=h16.numpy(), weight=w16.numpy(),
                        targets=targets.numpy(), token_loss=token_loss.numpy(),
                        entropy=entropy.numpy(), argmax=argmax.numpy(),
                        correct=(lab & (argmax == targets)).numpy(), grad=dh.numpy(),
                        loss=np.float64(token_loss.sum() / max(int(lab.sum()), 1)))


def main():
    table = write_dynamic_map()
    write_nf4(table)
    write_norm_rope_swiglu()
    write_head()
    print("golden fixtures written to", HERE, file=sys.stderr)


if __name__ == "__main__":
    main()
