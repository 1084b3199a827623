"""Per-projection NF4 dequantization on the HIP kernel (talm_nf4_dequant).

Mirrors solution/nf4_dequant.py:83-91 (`nf4_dequantize(packed, absmax, blocksize, out)`): each
byte holds two NF4 codes (high nibble first), each code selects one of the 16 NormalFloat levels,
and each block of `blocksize` weights is scaled by its fp32 absmax; one fp32 product and one
round-to-nearest-even to fp16 per weight (bit-identical to bitsandbytes' dequantize_4bit,
solution/test_fuzz.py:860-868).

`dequantize_4bit(packed, quant_state)` is the full per-projection dequantization of a 4-bit
weight: the double-quantized absmax is rebuilt as bitsandbytes' dequantize_blockwise + offset
does (code[absmax8] * absmax2, then + offset, each rounded in fp32), then the kernel runs. It is
what the 4-bit linear layer (nf4_linear.Linear4bit) runs when its projection is not packed in a
layer group (solution/nf4_dequant.py:110-149 routes bitsandbytes there).
"""

import torch

from . import _ops  # noqa: F401 - registers torch.ops.talm.*
from .engaged import RAN
from .quant import NF4_LEVELS

NF4_TABLE = list(NF4_LEVELS)


def nf4_dequantize(packed, absmax, blocksize, out):
    """packed: uint8 [(n+1)//2, 1] or flat; absmax: fp32 [ceil(n / blocksize)]; out: contiguous
    fp16 tensor with an even number of elements. Returns out."""
    torch.ops.talm.nf4_dequant(packed.contiguous().view(-1), absmax.contiguous(), out.view(-1),
                               int(blocksize))
    return out


def absmax32(state):
    """fp32 absmax per block of a double-quantized state: code[absmax8] * absmax2 + offset."""
    if not state.nested:
        return state.absmax
    s2 = state.state2
    a2 = s2.absmax.repeat_interleave(s2.blocksize)[:state.absmax.numel()]
    return s2.code[state.absmax.long()] * a2 + state.offset


def dequantize_4bit(packed, state, out=None):
    """fp16 [out, in] weight of one 4-bit projection on the kernel."""
    if out is None:
        out = torch.empty(state.shape, dtype=torch.float16, device=packed.device)
    nf4_dequantize(packed, absmax32(state), state.blocksize, out)
    RAN["nf4_dequant"] += 1
    return out
