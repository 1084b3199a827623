"""The 4-bit linear layer of the QLoRA base model: bitsandbytes' `Linear4bit` data model.

bitsandbytes is not available on this platform, so this module stands in for what the
reference's patches find at run time (solution/qgroup.py:112-176 reads these exact fields):
- `weight`: a frozen uint8 Parameter [n / 2, 1] of packed NF4 codes, carrying `quant_state`;
- `weight.quant_state`: `quant_type` "nf4", `nested` (double quantization), `blocksize` (64),
  `shape` (out, in), `absmax` (uint8 codes), `offset`, `dtype`, and `state2` with `absmax`
  (fp32), `code` (the 256-entry table) and `blocksize` (256);
- `bias` (fp16 or None) and `compute_dtype` (fp16).
Its own forward is bitsandbytes' for fp16 inputs (`MatMul4Bit`): dequantize the weight to fp16
(on the per-projection HIP kernel, nf4_dequant.py), `F.linear`, and in the backward dequantize
again for grad_input = grad @ W16. `talm_amd.apply()` routes packed projections through the
grouped kernel instead (qgroup.GroupLinear).
"""

import torch
import torch.nn as nn
import torch.nn.functional as F

from .nf4_dequant import dequantize_4bit
from .quant import quantize_nf4


class State2:
    __slots__ = ("absmax", "code", "blocksize")

    def __init__(self, absmax, code, blocksize):
        self.absmax, self.code, self.blocksize = absmax, code, blocksize


class QuantState:
    """The fields of bitsandbytes' QuantState that the kernels read."""

    def __init__(self, absmax, shape, code, blocksize, offset, state2, dtype=torch.float16):
        self.absmax, self.shape, self.code, self.blocksize = absmax, torch.Size(shape), code, blocksize
        self.offset, self.state2, self.dtype = offset, state2, dtype
        self.quant_type = "nf4"
        self.nested = True

    def to(self, device):
        s2 = State2(self.state2.absmax.to(device), self.state2.code.to(device),
                    self.state2.blocksize)
        return QuantState(self.absmax.to(device), self.shape, self.code.to(device),
                          self.blocksize, self.offset.to(device), s2, self.dtype)


class MatMul4Bit(torch.autograd.Function):
    """y = x W^T + b with W dequantized per call (fp16) and cast to x's dtype, forward and
    backward (bitsandbytes' MatMul4Bit: dx = dy W in the input's dtype)."""

    @staticmethod
    def forward(ctx, x, packed, state, bias):
        ctx.packed, ctx.state, ctx.dtype = packed, state, x.dtype
        weight = dequantize_4bit(packed, state).to(x.dtype)
        return F.linear(x, weight, None if bias is None else bias.to(x.dtype))

    @staticmethod
    def backward(ctx, grad):
        grad_x = None
        if ctx.needs_input_grad[0]:
            weight = dequantize_4bit(ctx.packed, ctx.state).to(ctx.dtype)
            grad_x = torch.matmul(grad.to(ctx.dtype), weight)
        return grad_x, None, None, None


class Linear4bit(nn.Module):
    """Frozen NF4 linear layer (double-quantized absmax), fp16 compute."""

    def __init__(self, in_features, out_features, bias=True, compute_dtype=torch.float16,
                 device=None):
        super().__init__()
        self.in_features, self.out_features = in_features, out_features
        self.compute_dtype = compute_dtype
        n = in_features * out_features
        self.weight = nn.Parameter(torch.zeros(n // 2, 1, dtype=torch.uint8, device=device),
                                   requires_grad=False)
        self.weight.quant_state = None
        self.bias = None
        if bias:
            self.bias = nn.Parameter(torch.zeros(out_features, dtype=torch.float16, device=device),
                                     requires_grad=False)

    @classmethod
    @torch.no_grad()
    def from_weight(cls, weight, bias=None, blocksize=64, blocksize2=256):
        """Quantize a float weight [out, in] (and keep an fp16 bias)."""
        out_f, in_f = weight.shape
        layer = cls(in_f, out_f, bias=bias is not None, device=weight.device)
        q = quantize_nf4(weight, blocksize, blocksize2)
        layer.weight.data = q.packed.view(-1, 1)
        layer.weight.quant_state = QuantState(
            q.absmax8, (out_f, in_f), q.code, blocksize, q.offset.to(torch.float32),
            State2(q.absmax2, q.code, blocksize2))
        if bias is not None:
            layer.bias.data = bias.detach().to(torch.float16).clone()
        return layer

    def _apply(self, fn, recurse=True):
        # Moving the module moves the quantization state along with the packed weight.
        state = self.weight.quant_state
        out = super()._apply(fn, recurse)
        if state is not None:
            self.weight.quant_state = state.to(self.weight.device)
        return out

    def forward(self, x):
        state = self.weight.quant_state
        out = MatMul4Bit.apply(x.to(self.compute_dtype), self.weight.data, state, self.bias)
        return out
