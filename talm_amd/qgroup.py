"""One NF4 dequantization launch per decoder layer and pass (the HIP grouped kernel).

Mirrors solution/qgroup.py: the seven 4-bit projections of a layer (q, k, v, o, gate, up, down)
are packed into one contiguous set of buffers (the parameters become views of it, no memory is
duplicated, :148-160) and dequantized by ONE launch when the layer's first projection runs, in
the forward and in the backward; the other projections slice the cached fp16 buffer, which is
dropped after its last expected use (`_take`, :273-289). The reference dequantizes the last
layers (at the memory peak) projection by projection (`SPLIT_LAYERS`, :68-69, `dequantize_one`,
:200-211) to spare a T4's 16 GB one layer's fp16 buffer (94 MB for Qwen2.5-1.5B); with 288 GB
of HBM that trade only costs launches, so here it is opt-in (SOLUTION_SPLIT_DEQUANT=1).

The kernel (talm_nf4_group_dequant, talm_amd/csrc/nf4.hip) rebuilds each block's fp32 scale from
the double-quantized absmax exactly as the reference kernel does (:72-91) and matches it bit for
bit; `launch` keeps the reference's launch-site signature (:94-99).

Graceful degradation (state.py): an unexpected error in `weight` turns "qgroup" off and the
weight comes from the per-projection dequantization of that projection (the same values).
"""

import os
import weakref

import torch

from . import _ops  # noqa: F401 - registers torch.ops.talm.*
from .engaged import FELL_BACK, ON, RAN
from .nf4_dequant import dequantize_4bit
from .quant import NF4_LEVELS
from .state import DISABLED, fallback

ROWS = 64  # the reference kernel's tile (rows of one program); kept as the packing granule
NSEG = 7
_SPLIT_ON = os.environ.get("SOLUTION_SPLIT_DEQUANT") == "1" \
    and os.environ.get("SOLUTION_DISABLE_SPLIT_DEQUANT") != "1"
SPLIT_LAYERS = {"fwd": 1 if _SPLIT_ON else 0, "bwd": 2 if _SPLIT_ON else 0}
PROJECTIONS = ("self_attn.q_proj", "self_attn.k_proj", "self_attn.v_proj", "self_attn.o_proj",
               "mlp.gate_proj", "mlp.up_proj", "mlp.down_proj")


def launch(packed, absmax8, code, absmax2, offset2, levels, out, n_rows, qblock, qblock2):
    """The one launch site of the grouped kernel: `out` is the contiguous fp16 output of
    `n_rows` absmax blocks of `qblock` weights (solution/qgroup.py:94-99). `levels` is accepted
    for the reference's signature; the kernel holds the NF4 table itself."""
    del levels
    torch.ops.talm.nf4_group_dequant(packed[:n_rows * qblock // 2], absmax8[:n_rows], code,
                                     absmax2, offset2, out.view(-1)[:n_rows * qblock],
                                     int(qblock), int(qblock2))


def _state_ok(state, first):
    return (state is not None and state.quant_type == "nf4" and state.nested
            and state.blocksize == first.blocksize
            and state.state2.blocksize == first.state2.blocksize
            and len(state.shape) == 2 and state.absmax.dtype == torch.uint8
            and state.state2.absmax.dtype == torch.float32
            and torch.equal(state.state2.code, first.state2.code))


class LayerGroup:
    """The seven 4-bit projections of one decoder layer, packed, with per-pass caches."""

    def __init__(self, modules):
        assert len(modules) == NSEG
        states = [m.weight.quant_state for m in modules]
        first = states[0]
        if not all(_state_ok(s, first) for s in states):
            raise ValueError("unsupported quant state")
        if first.blocksize % 8 or first.blocksize & (first.blocksize - 1):
            raise ValueError("block size is not a power of two >= 8")
        double = first.blocksize * first.state2.blocksize
        for s in states:
            if (s.shape[0] * s.shape[1]) % double:
                raise ValueError("weight size not a multiple of the absmax double-block")
        device = modules[0].weight.device
        self.qblock, self.qblock2 = first.blocksize, first.state2.blocksize
        self.shapes = [tuple(s.shape) for s in states]
        self.numels = [a * b for a, b in self.shapes]
        self.elem_bounds = [0]
        for n in self.numels:
            self.elem_bounds.append(self.elem_bounds[-1] + n)
        total = self.elem_bounds[-1]
        packed = torch.cat([m.weight.data.view(-1) for m in modules])
        absmax8 = torch.cat([s.absmax.view(-1) for s in states])
        absmax2 = torch.cat([s.state2.absmax.view(-1) for s in states])
        p = a = c = 0
        for m, s in zip(modules, states):
            n = s.shape[0] * s.shape[1]
            m.weight.data = packed[p:p + n // 2].view(-1, 1)
            s.absmax = absmax8[a:a + n // self.qblock]
            s.state2.absmax = absmax2[c:c + n // double]
            p += n // 2
            a += n // self.qblock
            c += n // double
        self.packed, self.absmax8, self.absmax2 = packed, absmax8, absmax2
        self.code = first.state2.code.contiguous()
        offsets = torch.stack([s.offset.reshape(()).to(torch.float32) for s in states]).to(device)
        self.offset2 = torch.cat([offsets[i:i + 1].expand(n // double)
                                  for i, n in enumerate(self.numels)]).contiguous()
        self.n_rows = total // self.qblock
        if total >= 2 ** 40:
            raise ValueError("layer too large")
        self.levels = None
        self.biases = [None if m.bias is None else m.bias.detach().to(torch.float16)
                       for m in modules]
        self.modules = [weakref.ref(m) for m in modules]
        self._span_biases = {}
        self.cache = {"fwd": [None, 0], "bwd": [None, 0]}
        self.expected_bwd = 0
        self.split_left = 0
        self.checkpointed = False
        self.depth = None
        self.row_bounds = [e // self.qblock for e in self.elem_bounds]
        self.splittable = all(r0 % self.qblock2 == 0 for r0 in self.row_bounds[:-1])

    def dequantize_all(self):
        out = torch.empty(self.elem_bounds[-1], dtype=torch.float16, device=self.packed.device)
        launch(self.packed, self.absmax8, self.code, self.absmax2, self.offset2, self.levels, out,
               self.n_rows, self.qblock, self.qblock2)
        return out

    def dequantize_one(self, idx):
        """fp16 [out, in] of projection `idx` alone: the same kernel on that weight's slice of
        the packed buffers (it starts on an absmax2 block, so the block indices stay right)."""
        r0, r1 = self.row_bounds[idx], self.row_bounds[idx + 1]
        b0 = r0 // self.qblock2
        out = torch.empty(self.numels[idx], dtype=torch.float16, device=self.packed.device)
        launch(self.packed[r0 * (self.qblock // 2):], self.absmax8[r0:], self.code,
               self.absmax2[b0:], self.offset2[b0:], self.levels, out, r1 - r0, self.qblock,
               self.qblock2)
        return out.view(self.shapes[idx])

    def weight(self, which, idx):
        """fp16 [out, in] of projection `idx`; one dequant launch per pass per layer. Once
        "qgroup" is off, the per-projection dequantization of that projection (same values)."""
        if "qgroup" not in DISABLED:
            try:
                return self._weight(which, idx)
            except Exception as exc:  # noqa: BLE001 - state.py convention
                if not fallback("qgroup", exc):
                    raise
        return self.reference_weight(idx)

    def reference_weight(self, idx):
        if self.cache["fwd"][0] is not None or self.cache["bwd"][0] is not None:
            self.reset()
        FELL_BACK["group"] += 1
        module = self.modules[idx]()
        return dequantize_4bit(module.weight.data, module.weight.quant_state)

    def reset(self):
        self.cache = {"fwd": [None, 0], "bwd": [None, 0]}
        self.expected_bwd = 0
        self.split_left = 0

    def refund(self, which, uses=1):
        entry = self.cache[which]
        if entry[0] is not None:
            entry[1] += uses

    def start_forward(self, checkpointed=False):
        fwd, bwd = self.cache["fwd"], self.cache["bwd"]
        fwd[0] = bwd[0] = None
        fwd[1] = bwd[1] = 0
        self.expected_bwd = self.split_left = 0
        self.checkpointed = checkpointed

    def split_now(self, which):
        return (self.cache[which][0] is None and self.depth is not None
                and self.depth < SPLIT_LAYERS[which] and self.splittable) or self.checkpointed

    def _take(self, which, uses):
        entry = self.cache[which]
        if entry[0] is None:
            entry[0] = self.dequantize_all()
            RAN["group"] += 1
            if which == "fwd":
                entry[1] = NSEG
            else:
                entry[1] = max(self.expected_bwd, 1)
                self.expected_bwd = 0
        buf = entry[0]
        entry[1] -= uses
        if entry[1] <= 0:
            entry[0] = None
        return buf

    def _weight(self, which, idx):
        if self.split_now(which):
            if self.checkpointed:
                self.expected_bwd = 0
                if not self.splittable:
                    RAN["group"] += 1
                    full = self.dequantize_all()
                    return full[self.elem_bounds[idx]:self.elem_bounds[idx + 1]].view(
                        self.shapes[idx])
            elif which == "bwd":
                if self.split_left == 0:
                    self.split_left = max(self.expected_bwd, 1)
                    self.expected_bwd = 0
                self.split_left -= 1
            RAN["split"] += 1
            return self.dequantize_one(idx)
        buf = self._take(which, 1)
        return buf[self.elem_bounds[idx]:self.elem_bounds[idx + 1]].view(self.shapes[idx])

    def span(self, which, first, last):
        """fp16 [sum of out, in] of the adjacent projections first .. last - 1 as ONE view of the
        layer's buffer, counted as last - first uses; None in a split pass or once off."""
        if "qgroup" in DISABLED:
            return None
        try:
            if self.split_now(which):
                return None
            buf = self._take(which, last - first)
        except Exception as exc:  # noqa: BLE001 - state.py convention
            if not fallback("qgroup", exc):
                raise
            return None
        rows = sum(self.shapes[i][0] for i in range(first, last))
        return buf[self.elem_bounds[first]:self.elem_bounds[last]].view(rows, self.shapes[first][1])

    def span_bias(self, first, last):
        key = (first, last)
        if key not in self._span_biases:
            parts = self.biases[first:last]
            if all(b is None for b in parts):
                self._span_biases[key] = None
            else:
                ref = next(b for b in parts if b is not None)
                self._span_biases[key] = torch.cat([
                    b if b is not None else ref.new_zeros(self.shapes[first + i][0])
                    for i, b in enumerate(parts)])
        return self._span_biases[key]


def _rows(t):
    """t [..., C] as a 2-D [R, C] view (a copy only when its columns are not unit-stride)."""
    t2 = t.reshape(-1, t.shape[-1])
    return t2 if t2.stride(-1) == 1 else t2.contiguous()


def linear(x, weight, bias=None):
    """x [..., K] W^T (+ b) for fp16 x and W [N, K]: torch.ops.talm.gemm (hipBLASLt)."""
    x2 = _rows(x)
    out = torch.empty(x2.shape[0], weight.shape[0], dtype=torch.float16, device=x.device)
    torch.ops.talm.gemm(x2, weight, bias, 1, out)
    return out.view(*x.shape[:-1], weight.shape[0])


def matmul(dy, weight):
    """dy [..., N] W for fp16 dy and W [N, K]: torch.ops.talm.gemm (hipBLASLt)."""
    d2 = _rows(dy)
    out = torch.empty(d2.shape[0], weight.shape[1], dtype=torch.float16, device=dy.device)
    torch.ops.talm.gemm(d2, weight, None, 0, out)
    return out.view(*dy.shape[:-1], weight.shape[1])


class GroupLinear(torch.autograd.Function):
    """y = x W16^T + b on the layer group's dequantized weight; dx = dy W16 (solution/qgroup.py:
    346-355). Both GEMMs go to hipBLASLt through torch.ops.talm.gemm."""

    @staticmethod
    def forward(ctx, x, group, idx):
        ctx.group, ctx.idx = group, idx
        return linear(x, group.weight("fwd", idx), group.biases[idx])

    @staticmethod
    def backward(ctx, grad_out):
        weight = ctx.group.weight("bwd", ctx.idx)
        return matmul(grad_out.to(weight.dtype), weight), None, None


_GROUPS = []


def reset_passes():
    alive = []
    for ref in _GROUPS:
        group = ref()
        if group is not None:
            group.reset()
            alive.append(ref)
    _GROUPS[:] = alive


def _linear4bit(module):
    from .nf4_linear import Linear4bit

    base = getattr(module, "base_layer", module)
    return base if isinstance(base, Linear4bit) else None


def _pack(layer):
    modules = []
    for path in PROJECTIONS:
        obj = layer
        for part in path.split("."):
            obj = getattr(obj, part, None)
            if obj is None:
                return None
        base = _linear4bit(obj)
        if base is None or base.weight.requires_grad or not base.weight.is_cuda:
            return None
        if base.bias is not None and base.bias.requires_grad:
            return None
        if getattr(base, "compute_dtype", None) not in (None, torch.float16):
            return None
        modules.append(base)
    try:
        group = LayerGroup(modules)
    except ValueError:
        return None
    attn = getattr(layer, "self_attn", None)
    layer_idx = getattr(attn, "layer_idx", None)
    n_layers = getattr(getattr(attn, "config", None), "num_hidden_layers", None)
    if isinstance(layer_idx, int) and isinstance(n_layers, int) and 0 <= layer_idx < n_layers:
        group.depth = n_layers - 1 - layer_idx
    for idx, base in enumerate(modules):
        base._solution_group = (group, idx)
    _GROUPS.append(weakref.ref(group))
    return group


def setup_layer(layer):
    if getattr(layer, "_solution_group_done", False):
        return
    layer._solution_group_done = True
    layer._solution_layer_group = _pack(layer)


def enter_layer(layer):
    """The decoder layer's forward begins: pack on first use, then start its passes afresh."""
    if "qgroup" in DISABLED:
        return
    try:
        if not getattr(layer, "_solution_group_done", False):
            setup_layer(layer)
        group = getattr(layer, "_solution_layer_group", None)
        if group is not None:
            group.start_forward(bool(getattr(layer, "training", False)
                                     and getattr(layer, "gradient_checkpointing", False)))
    except Exception as exc:  # noqa: BLE001 - state.py convention
        if not fallback("qgroup", exc):
            raise


def patch_group_dequant():
    """`Qwen2DecoderLayer.forward` packs its layer on first use (enter_layer); the 4-bit linear
    layer routes packed modules through GroupLinear for fp16 inputs (solution/qgroup.py:498-545)."""
    from transformers.models.qwen2 import modeling_qwen2

    from .nf4_linear import Linear4bit
    from .patches import _in_chain

    layer_cls = modeling_qwen2.Qwen2DecoderLayer
    layer_forward = layer_cls.forward
    ON.add("group")
    if not _in_chain(layer_forward, "_solution_group"):
        def forward(self, *args, **kwargs):
            enter_layer(self)
            return layer_forward(self, *args, **kwargs)

        forward._solution_group = True
        forward._original = layer_forward
        layer_cls.forward = forward

    lin_forward = Linear4bit.forward
    if _in_chain(lin_forward, "_solution_group"):
        return True

    def linear_forward(self, x):
        tag = getattr(self, "_solution_group", None)
        if tag is not None and "qgroup" not in DISABLED and x.is_cuda \
                and x.dtype == torch.float16:
            group, idx = tag
            try:
                out = GroupLinear.apply(x, group, idx)
            except Exception as exc:  # noqa: BLE001 - state.py convention
                if not fallback("qgroup", exc):
                    raise
            else:
                if torch.is_grad_enabled() and x.requires_grad:
                    group.expected_bwd += 1
                return out
        FELL_BACK["group"] += 1
        return lin_forward(self, x)

    linear_forward._solution_group = True
    linear_forward._original = lin_forward
    Linear4bit.forward = linear_forward
    return True


def nf4_levels(device):
    return torch.tensor(NF4_LEVELS, dtype=torch.float32, device=device)
