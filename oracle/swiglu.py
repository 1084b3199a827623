"""SwiGLU oracle (test infrastructure), numpy.

Restates example_swiglu_fwd_kernel / example_swiglu_bwd_kernel (solution/swiglu.py:23-45) and
`reference_grads` (solution/swiglu.py:48-54):
  forward:  out = gate * sigmoid(gate) * up
  backward: sig = sigmoid(gate); dup = g * gate * sig; dgate = g * up * sig * (1 + gate (1 - sig))
"""

import numpy as np


def _sigmoid(x):
    return 1.0 / (1.0 + np.exp(-x))


def forward(gate, up, out_dtype=np.float16, dtype=np.float32):
    g = np.asarray(gate).astype(dtype)
    with np.errstate(over="ignore"):
        return (g * _sigmoid(g) * np.asarray(up).astype(dtype)).astype(out_dtype)


def backward(grad, gate, up, out_dtype=np.float16, dtype=np.float32):
    """(dgate, dup)."""
    d = np.asarray(grad).astype(dtype)
    g = np.asarray(gate).astype(dtype)
    u = np.asarray(up).astype(dtype)
    with np.errstate(over="ignore"):
        sig = _sigmoid(g)
    dup = d * g * sig
    dgate = d * u * sig * (1.0 + g * (1.0 - sig))
    return dgate.astype(out_dtype), dup.astype(out_dtype)
