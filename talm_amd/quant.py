"""NF4 storage with double quantization for the base weights of the QLoRA model.

The layout is bitsandbytes' (the one the reference's kernels read, solution/qgroup.py:121-168):
- `packed`  uint8 [n / 2]: two 4-bit codes per byte, the even element in the high nibble;
- `absmax8` uint8 [n / blocksize]: per block of `blocksize` (64) weights, an index into `code`;
- `code`    float32 [256]: the second-level table (bitsandbytes' signed dynamic map);
- `absmax2` float32 [n / (blocksize * blocksize2)]: per `blocksize2` (256) blocks, the scale;
- `offset`  float32 scalar: the mean that was subtracted before the second quantization.
The block scale is code[absmax8] * absmax2 + offset (solution/qgroup.py:12-14).

`quantize_nf4` is this package's own quantizer (nearest level, nearest code), used to build
the synthetic model: bitsandbytes is not available here, so its quantizer's exact tie-breaking
is not reproduced (the dequantization, which the kernels implement, does not depend on it).
"""

import torch

NF4_LEVELS = (-1.0, -0.6961928009986877, -0.5250730514526367, -0.39491748809814453,
              -0.28444138169288635, -0.18477343022823334, -0.09105003625154495, 0.0,
              0.07958029955625534, 0.16093020141124725, 0.24611230194568634, 0.33791524171829224,
              0.44070982933044434, 0.5626170039176941, 0.7229568362236023, 1.0)


def dynamic_map():
    """bitsandbytes' signed dynamic map (create_dynamic_map(signed=True), the code table of its
    double quantization), float32 [256] sorted. Decade e = 10^(i - 6), i = 0..6, holds the
    midpoints of the 2^i + 1 float32 points torch.linspace(0.1, 1) places on [0.1, 1], scaled by
    e, with both signs; then 0 and 1. The float32 linspace matters: its points (and so 22 of the
    256 entries) differ by one ulp from a float64 linspace rounded to float32. The committed
    fixture tests/golden/dynamic_map.txt holds the table bit for bit."""
    values = [0.0, 1.0]
    for i in range(7):
        points = torch.linspace(0.1, 1.0, 2 ** i + 1, dtype=torch.float32)
        mids = (points[1:] + points[:-1]) / 2.0
        for sign in (1.0, -1.0):
            values += (sign * 10.0 ** (i - 6) * mids).tolist()
    return torch.tensor(sorted(values), dtype=torch.float32)


class NF4Weight:
    """One NF4 double-quantized weight [out, in] (bitsandbytes' QuantState fields)."""

    __slots__ = ("packed", "absmax8", "code", "absmax2", "offset", "shape", "blocksize",
                 "blocksize2")

    def __init__(self, packed, absmax8, code, absmax2, offset, shape, blocksize=64,
                 blocksize2=256):
        self.packed, self.absmax8, self.code, self.absmax2 = packed, absmax8, code, absmax2
        self.offset, self.shape = offset, tuple(shape)
        self.blocksize, self.blocksize2 = blocksize, blocksize2

    @property
    def numel(self):
        return self.shape[0] * self.shape[1]

    def to(self, device):
        return NF4Weight(self.packed.to(device), self.absmax8.to(device), self.code.to(device),
                         self.absmax2.to(device), self.offset.to(device), self.shape,
                         self.blocksize, self.blocksize2)


@torch.no_grad()
def quantize_nf4(weight, blocksize=64, blocksize2=256, code=None):
    """NF4 with double-quantized absmax of a float weight [out, in] (numel a multiple of
    blocksize * blocksize2). Runs on the weight's device with PyTorch ops."""
    w = weight.detach().float().reshape(-1)
    n = w.numel()
    if n % (blocksize * blocksize2):
        raise ValueError(f"{n} weights are not a multiple of {blocksize} * {blocksize2}")
    device = w.device
    levels = torch.tensor(NF4_LEVELS, dtype=torch.float32, device=device)
    blocks = w.view(-1, blocksize)
    absmax = blocks.abs().amax(1)
    normed = blocks / absmax.clamp(min=torch.finfo(torch.float32).tiny)[:, None]
    codes = (normed[..., None] - levels).abs().argmin(-1).to(torch.uint8).view(-1)
    packed = (codes[0::2] << 4) | codes[1::2]
    code = (dynamic_map() if code is None else code).to(device)
    offset = absmax.mean()
    centred = (absmax - offset).view(-1, blocksize2)
    absmax2 = centred.abs().amax(1).clamp(min=torch.finfo(torch.float32).tiny)
    absmax8 = ((centred / absmax2[:, None]).reshape(-1, 1) - code).abs().argmin(-1)
    return NF4Weight(packed.contiguous(), absmax8.to(torch.uint8).contiguous(), code.contiguous(),
                     absmax2.contiguous(), offset.reshape(()), weight.shape, blocksize, blocksize2)


def block_absmax(q):
    """The fp32 absmax of every block, code[absmax8] * absmax2 + offset with each product and
    sum rounded in fp32 (what bitsandbytes' dequantize_blockwise + offset returns)."""
    a2 = q.absmax2.repeat_interleave(q.blocksize2)[:q.absmax8.numel()]
    return q.code[q.absmax8.long()] * a2 + q.offset
