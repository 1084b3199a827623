"""The oracle and the package's host-side tables against the committed golden fixtures of
tests/golden/ (written by tests/golden/make_golden.py from PyTorch's float64 autograd, float32
elementwise ops and a float64 full softmax; see that script). CPU only: the HIP kernels meet the
same fixtures in tests/test_gpu_golden.py."""

import hashlib
from pathlib import Path

import numpy as np
import pytest

from oracle import head, nf4, norm, rope, swiglu
from talm_amd import quant

GOLDEN = Path(__file__).resolve().parent / "golden"


def load(name):
    with np.load(GOLDEN / name, allow_pickle=False) as data:
        return {k: data[k] for k in data.files}


def golden_code_table():
    rows = [line.split() for line in (GOLDEN / "dynamic_map.txt").read_text().splitlines()]
    assert [int(r[0]) for r in rows] == list(range(256))
    return np.array([int(r[1], 16) for r in rows], dtype=np.uint32).view(np.float32)


def test_code_table_is_the_fixture_bit_for_bit():
    """The product's double-quant table (what the synthetic model's quantizer and the config-1
    inputs use) is bitsandbytes' create_dynamic_map output, bit for bit."""
    table = golden_code_table()
    ours = quant.dynamic_map().numpy()
    assert np.array_equal(ours.view(np.uint32), table.view(np.uint32))
    # structure bitsandbytes' construction implies: sorted, 0 and 1, +-symmetric, 7 decades
    assert np.all(np.diff(table) >= 0) and table[-1] == 1.0 and (table == 0).sum() == 1
    inner = table[(table != 0) & (table != 1)]
    assert np.array_equal(np.sort(-inner), np.sort(inner))
    assert np.unique(np.floor(np.log10(np.abs(inner)))).tolist() == list(range(-7, 0))


def test_nf4_oracle_matches_the_group_fixture():
    d = load("nf4_group.npz")
    args = [d[k] for k in ("packed", "absmax8", "code", "absmax2", "offset2")]
    for fn in (nf4.group_dequant, nf4.group_dequant_np):
        out = fn(*args)
        assert hashlib.sha256(out.tobytes()).digest() == d["sha256"].tobytes()
        assert np.array_equal(out[d["sample_index"]], d["sample_bits"])
    # the first bytes 0x0F, 0xF0, 0x77, 0x88: levels -1, +1 | +1, -1 | 0, 0 | 0.0796 twice
    # (high nibble first), all times block 0's scale
    out = nf4.group_dequant(*args).view(np.float16).astype(np.float32)
    scale = out[1]
    assert scale != 0 and out[0] == -scale and out[2] == scale and out[3] == -scale
    assert out[4] == 0 and out[5] == 0
    assert out[6] == out[7] and np.sign(out[6]) == np.sign(scale)
    assert abs(out[6] / scale - 0.07958029955625534) < 1e-3


def _close(ours, ref, rtol, what, floor=1e-12):
    """|ours - ref| <= rtol * (|ref| + floor * max|ref|) elementwise: `floor` covers the values
    that cancel to (near) zero, whose relative error means nothing."""
    ours, ref = np.asarray(ours, np.float64), np.asarray(ref, np.float64)
    err = np.abs(ours - ref) / (np.abs(ref) + floor * np.abs(ref).max())
    assert err.max() <= rtol, f"{what}: max rel err {err.max():.3g}"


def test_norm_oracle_matches_float64_autograd():
    d = load("norm_rope_swiglu.npz")
    total, y, xhat, rstd = norm.forward(d["norm_a"], d["norm_w"], 1e-6, p=d["norm_p"],
                                        x_dtype=np.float64, out_dtype=np.float64,
                                        dtype=np.float64)
    _close(total, d["norm_sum"], 1e-15, "sum")
    _close(y, d["norm_y"], 1e-12, "y")
    _close(rstd, d["norm_rstd"], 1e-7, "rstd")  # rstd is returned in float32
    dx, _ = norm.backward(d["norm_dy"], xhat, d["norm_w"], d["norm_rstd"],
                          x_dtype=np.float64, out_dtype=np.float64, dtype=np.float64)
    _close(dx, d["norm_dx"], 1e-10, "dx")
    # the kernel's arithmetic (float32, fp16 outputs) stays within the fp16 bar
    _, y32, xhat32, rstd32 = norm.forward(d["norm_a"], d["norm_w"], 1e-6, p=d["norm_p"])
    _close(y32, d["norm_y"], 1e-3, "y fp16")
    dx32, _ = norm.backward(d["norm_dy"], xhat32, d["norm_w"], rstd32)
    assert np.abs(dx32 - d["norm_dx"]).max() <= 2e-3 * np.abs(d["norm_dx"]).max()


def test_rope_oracle_matches_complex_rotation_and_its_adjoint():
    d = load("norm_rope_swiglu.npz")
    y = rope.rotate(d["rope_x"], d["rope_cos"], d["rope_sin"], out_dtype=np.float64,
                    dtype=np.float64)
    _close(y, d["rope_y"], 1e-12, "rope forward")
    dx = rope.rotate(d["rope_dy"], d["rope_cos"], d["rope_sin"], backward=True,
                     out_dtype=np.float64, dtype=np.float64)
    _close(dx, d["rope_dx"], 1e-12, "rope backward")


def test_swiglu_oracle_matches_float64_autograd():
    d = load("norm_rope_swiglu.npz")
    out = swiglu.forward(d["swiglu_gate"], d["swiglu_up"], out_dtype=np.float64, dtype=np.float64)
    _close(out, d["swiglu_out"], 1e-12, "swiglu forward")
    dgate, dup = swiglu.backward(d["swiglu_grad"], d["swiglu_gate"], d["swiglu_up"],
                                 out_dtype=np.float64, dtype=np.float64)
    _close(dgate, d["swiglu_dgate"], 1e-11, "dgate")
    _close(dup, d["swiglu_dup"], 1e-11, "dup")


@pytest.mark.parametrize("vchunk,block", [(8192, 4096), (1024, 512), (384, 128)])
def test_head_oracle_matches_the_v4097_fixture(vchunk, block):
    d = load("head_v4097.npz")
    out = head.head_ce(d["hidden"], d["weight"], d["targets"], vchunk=vchunk, block=block)
    assert np.array_equal(out["best_idx"], d["argmax"])  # exact-style: the tie goes left
    assert out["best_idx"][5] == 100
    assert np.array_equal(out["correct"], d["correct"])
    lab = d["targets"] >= 0
    # fp32 statistics: rows whose target dominates have a loss near 1e-14, which fp32 gives as
    # 0, so the per-row bar has a floor of 1e-2 of the largest loss
    _close(out["token_loss"][lab], d["token_loss"][lab], 1e-4, "token loss", floor=1e-2)
    assert np.all(out["token_loss"][~lab] == 0)
    _close(out["entropy"], d["entropy"], 1e-4, "entropy", floor=1e-2)
    loss, _ = head.loss(out["token_loss"], d["targets"])
    assert abs(loss - d["loss"]) <= 1e-5 * abs(d["loss"])
    g = out["grad"].astype(np.float64)
    assert np.abs(g - d["grad"]).max() <= 2e-3 * np.abs(d["grad"]).max()
    assert np.all(g[~lab] == 0)
    direct = head.head_direct(d["hidden"], d["weight"], d["targets"])
    assert np.array_equal(direct["best_idx"], d["argmax"])
    _close(direct["token_loss"][lab], d["token_loss"][lab], 1e-12, "closed form")
