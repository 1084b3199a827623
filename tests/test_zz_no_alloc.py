"""talm_lora_wgrad_noalloc (the allocation-free LoRA weight gradients) against talm_lora_wgrad
(the same kernels with a caller-owned workspace), both called through the C-ABI with ctypes.

Two calls in a row on one GPU, the second with fewer tokens: the fixed scratch array keeps the
first call's partials, and the second call's results must not depend on them. Outputs are
compared bit for bit (same kernels, same fixed summation order)."""

import ctypes

import pytest
import torch

from talm_amd import _lib

HIDDEN, QCOLS, KCOLS, VCOLS = 1536, 1536, 256, 256
LD = QCOLS + KCOLS + VCOLS


def _ptr(t):
    return ctypes.c_void_p(t.data_ptr())


def _inputs(n_tokens, seed):
    g = torch.Generator().manual_seed(seed)
    x = torch.randn(n_tokens, HIDDEN, generator=g).half().cuda()
    dy = (0.05 * torch.randn(n_tokens, LD, generator=g)).half().cuda()
    u = (0.1 * torch.randn(n_tokens, 32, generator=g)).half().cuda()
    t = torch.randn(n_tokens, 32, generator=g).half().cuda()
    return x, dy, u, t


def _outputs():
    return [torch.full(shape, float("nan"), device="cuda")
            for shape in ((16, HIDDEN), (QCOLS, 16), (16, HIDDEN), (VCOLS, 16))]


def _call(lib, noalloc, x, dy, u, t, outs, stream):
    n = x.shape[0]
    da0, db0, da1, db1 = outs
    args = [_ptr(x), HIDDEN, _ptr(dy), LD, _ptr(u), 32, _ptr(t), 32, n, HIDDEN, 2,
            0, QCOLS, ctypes.c_float(2.0), _ptr(da0), _ptr(db0),
            QCOLS + KCOLS, VCOLS, ctypes.c_float(2.0), _ptr(da1), _ptr(db1)]
    if noalloc:
        status = lib.talm_lora_wgrad_noalloc(*args, stream)
    else:
        size = lib.talm_lora_wgrad_workspace(n, HIDDEN, QCOLS, VCOLS)
        ws = torch.empty(size, dtype=torch.uint8, device="cuda")
        status = lib.talm_lora_wgrad(*args, _ptr(ws), size, stream)
    _lib.check(status, "lora_wgrad_noalloc" if noalloc else "lora_wgrad")


@pytest.mark.gpu
def test_noalloc_matches_workspace_entry_on_two_calls():
    lib = _lib.lib()
    stream = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
    for seed, n_tokens in ((1, 1300), (2, 517)):
        print(f"wgrad noalloc vs workspace: seed {seed}, {n_tokens} tokens", flush=True)
        x, dy, u, t = _inputs(n_tokens, seed)
        ref, got = _outputs(), _outputs()
        _call(lib, False, x, dy, u, t, ref, stream)
        _call(lib, True, x, dy, u, t, got, stream)
        torch.cuda.synchronize()
        for name, r, o in zip(("dA_q", "dB_q", "dA_v", "dB_v"), ref, got):
            assert torch.isfinite(r).all(), name
            assert torch.equal(r, o), f"{name} differs at {n_tokens} tokens"
        # the result is the fp32 product the partials sum to
        xf, dyf, uf, tf = x.float(), dy.float(), u.float(), t.float()
        torch.testing.assert_close(got[0], uf[:, :16].T @ xf, rtol=1e-4, atol=1e-3)
        torch.testing.assert_close(got[3], 2.0 * dyf[:, QCOLS + KCOLS:].T @ tf[:, 16:],
                                   rtol=1e-4, atol=1e-3)


@pytest.mark.gpu
def test_noalloc_rejects_more_tokens_than_its_scratch():
    lib = _lib.lib()
    n = 6000  # 94 chunks of 64 tokens x 3328 columns x 128 B: above the 32 MiB scratch
    assert lib.talm_lora_wgrad_workspace(n, HIDDEN, QCOLS, VCOLS) > (32 << 20)
    x, dy, u, t = _inputs(8, 3)
    outs = _outputs()
    da0, db0, da1, db1 = outs
    status = lib.talm_lora_wgrad_noalloc(
        _ptr(x), HIDDEN, _ptr(dy), LD, _ptr(u), 32, _ptr(t), 32, n, HIDDEN, 2, 0, QCOLS,
        ctypes.c_float(2.0), _ptr(da0), _ptr(db0), QCOLS + KCOLS, VCOLS, ctypes.c_float(2.0),
        _ptr(da1), _ptr(db1), None)
    assert status == _lib.TALM_EINVAL
    assert b"scratch" in lib.talm_last_error()
