"""Fused (residual-add +) RMSNorm oracle (test infrastructure), numpy.

Restates rmsnorm_kernel (solution/rmsnorm.py:58-94) in float32 arithmetic:
  forward:  x = a (+ p);  q = x (x dtype);  rstd = rsqrt(sum(x * x) / H + eps);
            xhat = x * rstd;  y = w * xhat      (y, xhat in the output dtype)
  backward: g = dy * w;  c = sum(g * xhat) / H;  dx = rstd * (g - xhat * c)  (+ ds, also to p)
and the same in float64 for error bounds. The backward is `_reference_dx`
(solution/rmsnorm.py:121-127); the forward without add is transformers' Qwen2RMSNorm with a
single rounding of y (solution/test_kernels.py:524-529 rounds x * rstd first, as the model does;
the kernel and this oracle round once).
"""

import numpy as np


def forward(a, w, eps, p=None, x_dtype=np.float32, out_dtype=np.float16, dtype=np.float32):
    """(q, y, xhat, rstd): q in x_dtype (None without p), y and xhat in out_dtype, rstd float32.
    `dtype` is the arithmetic type (float32: the kernel's; float64: a reference)."""
    x = np.asarray(a).astype(dtype)
    q = None
    if p is not None:
        x = x + np.asarray(p).astype(dtype)
        q = x.astype(x_dtype)
    n = x.shape[-1]
    var = (x * x).sum(-1, dtype=dtype) / dtype(n)
    rstd = (dtype(1.0) / np.sqrt(var + dtype(eps))).astype(dtype)
    xhat = x * rstd[..., None]
    y = np.asarray(w).astype(dtype) * xhat
    return q, y.astype(out_dtype), xhat.astype(out_dtype), rstd.astype(np.float32)


def backward(dy, xhat, w, rstd, ds=None, x_dtype=np.float32, out_dtype=np.float16,
             dtype=np.float32):
    """(dx in x_dtype, dbranch in out_dtype or None)."""
    g = np.asarray(dy).astype(dtype) * np.asarray(w).astype(dtype)
    xh = np.asarray(xhat).astype(dtype)
    c = (g * xh).sum(-1, dtype=dtype) / dtype(xh.shape[-1])
    dx = np.asarray(rstd).astype(dtype)[..., None] * (g - xh * c[..., None])
    db = None
    if ds is not None:
        dx = dx + np.asarray(ds).astype(dtype)
        db = dx.astype(out_dtype)
    return dx.astype(x_dtype), db
