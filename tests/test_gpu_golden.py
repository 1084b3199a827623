"""The HIP kernels against the committed golden fixtures of tests/golden/ (expected values from
PyTorch's float64 autograd, float32 ops and a float64 softmax; tests/golden/make_golden.py).
Bars as for every kernel: NF4 bit-exact; norm / RoPE / SwiGLU within 1e-3 relative (fp16
outputs); head loss 1e-4, argmax exact on these exact-style logits, dH within 2e-3."""

import hashlib

import numpy as np
import pytest
import torch

from talm_amd import fused_head, qgroup, rmsnorm, rope, swiglu
from tests.test_golden import load

pytestmark = pytest.mark.gpu
DEV = "cuda"


def _rel(ours, ref, rtol, what, floor=1e-3):
    ours = ours.detach().double().cpu().numpy() if torch.is_tensor(ours) else ours
    ref = np.asarray(ref, np.float64)
    tol = rtol * (np.abs(ref) + floor * np.abs(ref).max())
    bad = np.abs(ours - ref) > tol
    assert not bad.any(), f"{what}: {int(bad.sum())} elements off, max err {np.abs(ours - ref).max():.3g}"


def test_nf4_group_kernel_on_the_fixture():
    print("[case] golden: nf4 group (7 x 16384)", flush=True)
    d = load("nf4_group.npz")
    t = {k: torch.from_numpy(d[k]).to(DEV) for k in ("packed", "absmax8", "code", "absmax2",
                                                     "offset2")}
    n = d["packed"].size * 2
    out = torch.empty(n, dtype=torch.float16, device=DEV)
    qgroup.launch(t["packed"], t["absmax8"], t["code"], t["absmax2"], t["offset2"], None, out,
                  n // 64, 64, 256)
    bits = out.cpu().view(torch.int16).numpy().view(np.uint16)
    assert np.array_equal(bits[d["sample_index"]], d["sample_bits"])
    assert hashlib.sha256(bits.tobytes()).digest() == d["sha256"].tobytes()


def test_add_rmsnorm_kernel_on_the_fixture():
    print("[case] golden: add + rmsnorm fwd/bwd", flush=True)
    d = load("norm_rope_swiglu.npz")
    a = torch.tensor(d["norm_a"], dtype=torch.float16, device=DEV).requires_grad_()
    p = torch.tensor(d["norm_p"], dtype=torch.float16, device=DEV).requires_grad_()
    w = torch.tensor(d["norm_w"], dtype=torch.float32, device=DEV)
    total, y = rmsnorm.add_rmsnorm(a, p, w, 1e-6, torch.float16)
    _rel(total, d["norm_sum"], 1e-3, "sum")
    _rel(y, d["norm_y"], 1e-3, "y")
    dy = torch.tensor(d["norm_dy"], dtype=torch.float16, device=DEV)
    y.backward(dy)
    # the sum's gradient is zero here: dx of both inputs is the norm's input gradient
    _rel(a.grad, d["norm_dx"], 2e-3, "dx (a)", floor=1e-2)
    _rel(p.grad, d["norm_dx"], 2e-3, "dx (branch)", floor=1e-2)


@pytest.mark.parametrize("backward", [False, True])
def test_rope_kernel_on_the_fixture(backward):
    print(f"[case] golden: rope backward={backward}", flush=True)
    d = load("norm_rope_swiglu.npz")
    x = d["rope_dy"] if backward else d["rope_x"]
    q = torch.tensor(x, dtype=torch.float16, device=DEV)       # [T, 3, 16]
    k = q[:, :1].clone()
    cos = torch.tensor(d["rope_cos"], dtype=torch.float32, device=DEV)
    sin = torch.tensor(d["rope_sin"], dtype=torch.float32, device=DEV)
    rope.rope_(q, k, cos, sin, backward=backward)               # in place
    ref = d["rope_dx"] if backward else d["rope_y"]
    _rel(q, ref, 1e-3, "q")
    _rel(k, ref[:, :1], 1e-3, "k")


def test_swiglu_kernels_on_the_fixture():
    print("[case] golden: swiglu fwd/bwd", flush=True)
    d = load("norm_rope_swiglu.npz")
    gate, up, grad = (torch.tensor(d[k], dtype=torch.float16, device=DEV).reshape(-1)
                      for k in ("swiglu_gate", "swiglu_up", "swiglu_grad"))
    out = torch.empty_like(gate)
    swiglu.swiglu_fwd(gate, up, out)
    _rel(out, d["swiglu_out"].reshape(-1), 1e-3, "out")
    dgate, dup = torch.empty_like(gate), torch.empty_like(up)
    swiglu.swiglu_bwd(grad, gate, up, dgate, dup)
    _rel(dgate, d["swiglu_dgate"].reshape(-1), 1e-3, "dgate", floor=1e-2)
    _rel(dup, d["swiglu_dup"].reshape(-1), 1e-3, "dup", floor=1e-2)


@pytest.mark.parametrize("vchunk", [8192, 1024, 384])
def test_head_kernel_on_the_v4097_fixture(vchunk):
    print(f"[case] golden: head V=4097 vchunk={vchunk}", flush=True)
    d = load("head_v4097.npz")
    x = torch.from_numpy(d["hidden"]).to(DEV).requires_grad_()
    w = torch.from_numpy(d["weight"]).to(DEV)
    t = torch.from_numpy(d["targets"]).to(DEV)
    loss, token_loss, entropy, correct, argmax = fused_head.fused_head_loss(
        x, w, t, None, vchunk, return_argmax=True)
    loss.backward()
    lab = d["targets"] >= 0
    assert np.array_equal(argmax.cpu().numpy(), d["argmax"])
    assert int(argmax[5]) == 100  # the planted tie goes to the first column
    assert np.array_equal(correct.cpu().numpy().astype(bool), d["correct"])
    assert abs(float(loss) - float(d["loss"])) <= 1e-4 * abs(float(d["loss"]))
    _rel(token_loss.cpu().numpy()[lab], d["token_loss"][lab], 1e-4, "token loss", floor=1e-2)
    _rel(entropy, d["entropy"], 1e-4, "entropy", floor=1e-2)
    g_ref = d["grad"] / max(int(lab.sum()), 1)
    g = x.grad.double().cpu().numpy()
    assert np.all(np.abs(g - g_ref) <= 2e-3 * np.abs(g_ref) + 2.0 ** -7 * np.abs(g_ref).max())
    assert np.all(g[~lab] == 0)
