"""Shared checks of the parity tests."""

import numpy as np
import torch


def to_np(t):
    return t.detach().cpu().numpy()


def assert_rel(ours, ref, rtol=1e-3, floor=1e-5, what=""):
    """|ours - ref| <= rtol * |ref| + floor * max|ref|, elementwise (float64). `floor` covers
    elements that cancel to near zero and fp16 subnormals; the stated bar is `rtol` relative."""
    ours = np.asarray(to_np(ours) if torch.is_tensor(ours) else ours, np.float64)
    ref = np.asarray(to_np(ref) if torch.is_tensor(ref) else ref, np.float64)
    assert ours.shape == ref.shape, f"{what}: shape {ours.shape} != {ref.shape}"
    scale = np.abs(ref).max() if ref.size else 0.0
    tol = rtol * np.abs(ref) + floor * scale
    bad = ~(np.abs(ours - ref) <= tol)
    if bad.any():
        i = np.flatnonzero(bad)[0]
        raise AssertionError(
            f"{what}: {int(bad.sum())} of {bad.size} elements off (rtol {rtol}); first at flat "
            f"{i}: ours {ours.flat[i]!r} ref {ref.flat[i]!r} tol {tol.flat[i]:.3g}")


def f16_bits(t):
    """uint16 bit patterns of an fp16 tensor (numpy)."""
    return to_np(t.contiguous().view(torch.int16)).view(np.uint16)
