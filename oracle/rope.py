"""Rotary embedding oracle (test infrastructure), numpy.

Restates rope_kernel (solution/rope.py:64-108) and its PyTorch twin `_reference`
(solution/rope.py:145-157) in float32 (or float64):
  forward:  y1 = x1 c1 - x2 s1,  y2 = x2 c2 + x1 s2
  backward: y1 = x1 c1 + x2 s2,  y2 = x2 c2 - x1 s1
x1, x2: the first and second half of the head dimension; c, s: cos / sin of the token's
position (c1, c2 and s1, s2 their halves), broadcast over heads.
"""

import numpy as np


def rotate(x, cos, sin, backward=False, out_dtype=np.float16, dtype=np.float32):
    """x [..., T, Hd, D] or [T, H, D] with cos/sin [T, D] broadcast over the head axis."""
    x = np.asarray(x).astype(dtype)
    half = x.shape[-1] // 2
    c = np.asarray(cos).astype(dtype)[:, None, :]
    s = np.asarray(sin).astype(dtype)[:, None, :]
    x1, x2 = x[..., :half], x[..., half:]
    c1, c2, s1, s2 = c[..., :half], c[..., half:], s[..., :half], s[..., half:]
    if backward:
        y1, y2 = x1 * c1 + x2 * s2, x2 * c2 - x1 * s1
    else:
        y1, y2 = x1 * c1 - x2 * s1, x2 * c2 + x1 * s2
    return np.concatenate([y1, y2], axis=-1).astype(out_dtype)
