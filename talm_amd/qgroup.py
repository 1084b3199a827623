"""The seven 4-bit projections of a decoder layer as one packed weight set, dequantized by ONE
kernel launch (talm_nf4_group_dequant, talm_amd/csrc/nf4.hip).

What stays as in the reference (solution/qgroup.py): the launch site `launch(...)` with its
signature (:94-99), the packing of q, k, v, o, gate, up, down into contiguous packed / absmax8 /
absmax2 buffers with the modules' parameters turned into views of them (no memory duplicated,
:148-160), `GroupLinear` (y = x W^T + b, dx = dy W), `span` (adjacent projections as one [sum of out, in]
view, for the q|k|v and gate|up GEMMs) and `weight` (one projection). The reference's callers
name the pass first (`span("fwd", first, last)`, `weight("bwd", idx)`, :213, :310) and report
backward uses (`expected_bwd += 1`, :536); both forms are accepted here, and the pass name and
the counter are ignored, since nothing is counted (below).

What this build does its own way is the lifetime of the fp16 weights. The reference keeps a
cache per pass and counts uses (the forward's seven, the backward's expected uses reported by
every node, refunds when a node fails, per-projection "split" passes for the last layers at a
T4's memory peak: :263-343). Here each GPU holds exactly ONE resident dequantized layer:

- a decoder layer's forward makes its group resident when it begins (`enter_layer`);
- every projection request, forward or backward, reads the resident buffer when its group is
  the resident one, and otherwise dequantizes its group (one launch) and makes it resident.

Autograd runs the decoder's backward layer by layer (each layer's input gradient needs its whole
branch), so the backward dequantizes each layer once, and the last layer's forward buffer serves
its backward with no launch at all. Correctness never depends on how often a projection is used:
a request from a group that is not resident simply dequantizes it again (a checkpointed layer's
recomputation, a fallback path, two models interleaved), so nothing is counted, refunded or reset
when a step is cut short. The price is that one fp16 layer (94 MB for Qwen2.5-1.5B) stays
allocated between steps, against 288 GB of HBM.

The backward multiplies by W^T (dX = dY W reads W as the k-contiguous operand of the product in
the form the forward uses): `resident_t` holds ONE layer's weights dequantized transposed
(talm_nf4_group_dequant_t, the same values), laid out as four row-major blocks [in, sum of out]:
q|k|v, o, gate|up, down. `span_t` hands out a block. Each layer's backward makes its group's
transposed buffer resident with one launch, as the forward does with the row-major one, and
drops the row-major buffer the forward left behind. The gate|up block is left out of it while
the NF4 dequant-GEMM serves that input gradient (`nf4_gemm`, W4_BLOCKS): its weights are then
read as 4-bit codes and never written out in fp16.

Graceful degradation (state.py): an unexpected error here turns "qgroup" off; each projection
then takes the per-projection dequantization (nf4_dequant.py, the same values) and the 4-bit
layer its own forward.
"""

import os
import weakref
from collections import namedtuple

import torch

from . import _ops  # noqa: F401 - registers torch.ops.talm.*
from .engaged import FELL_BACK, ON, RAN
from .nf4_dequant import dequantize_4bit
from .state import DISABLED, fallback

NSEG = 7
PROJECTIONS = ("self_attn.q_proj", "self_attn.k_proj", "self_attn.v_proj", "self_attn.o_proj",
               "mlp.gate_proj", "mlp.up_proj", "mlp.down_proj")

# device -> (group, fp16 buffer of all its weights): the one dequantized layer per GPU
_RESIDENT = {}
# device -> (group, fp16 buffer of its W^T blocks): the backward's one transposed layer per GPU
_RESIDENT_T = {}
# the blocks of the transposed buffer: projections used as one [in, sum of out] operand
T_BLOCKS = ((0, 1, 2), (3,), (4, 5), (6,))
# blocks whose input gradient runs on the NF4 dequant-GEMM (talm_nf4_gemm, the weights read as
# 4-bit codes and dequantized inside the GEMM): the transposed buffer leaves them out. gate|up,
# where that GEMM is faster than the split-K GEMM on the transposed weights plus their share of
# the transposed dequantization.
W4_BLOCKS = ((4, 5),) if os.environ.get("SOLUTION_DISABLE_W4A16") != "1" else ()


def launch(packed, absmax8, code, absmax2, offset2, levels, out, n_rows, qblock, qblock2,
           streaming=False):
    """The one launch site of the grouped kernel: `out` is the contiguous fp16 output of
    `n_rows` absmax blocks of `qblock` weights (solution/qgroup.py:94-99). `levels` is accepted
    for the reference's signature; the kernel holds the NF4 table itself. `streaming`: write with
    non-temporal stores (talm_nf4_group_dequant_streaming, the same values) for an output that
    is not read again soon; the layer group's own dequantization, read by the GEMMs right
    after, keeps the ordinary stores."""
    del levels
    op = torch.ops.talm.nf4_group_dequant_streaming if streaming \
        else torch.ops.talm.nf4_group_dequant
    op(packed[:n_rows * qblock // 2], absmax8[:n_rows], code, absmax2, offset2,
       out.view(-1)[:n_rows * qblock], int(qblock), int(qblock2))


def release():
    """Drop every GPU's resident layer (a forward that failed part-way is about to run again;
    the patches are being removed)."""
    _RESIDENT.clear()
    _RESIDENT_T.clear()


def reset_passes():
    """The reference's name for the step-boundary reset (solution/qgroup.py:358-366)."""
    release()


def _nf4_layout(state):
    """(blocksize, second-level blocksize) of an NF4 state with double-quantized uint8 absmax,
    else None."""
    if state is None or getattr(state, "quant_type", None) != "nf4" \
            or not getattr(state, "nested", False) or len(getattr(state, "shape", ())) != 2:
        return None
    inner = state.state2
    if state.absmax.dtype != torch.uint8 or inner.absmax.dtype != torch.float32:
        return None
    return state.blocksize, inner.blocksize


# One projection inside the group: its element range, its [out, in] shape, its fp16 bias.
Segment = namedtuple("Segment", "start stop shape bias")


class LayerGroup:
    """The seven 4-bit projections of one decoder layer, packed into one set of buffers."""

    def __init__(self, modules):
        if len(modules) != NSEG:
            raise ValueError(f"a layer group has {NSEG} projections, got {len(modules)}")
        states = [m.weight.quant_state for m in modules]
        layouts = {_nf4_layout(s) for s in states}
        if len(layouts) != 1 or None in layouts:
            raise ValueError("the projections do not share one NF4 double-quant layout")
        (qblock, qblock2), = layouts
        code = states[0].state2.code
        if any(not torch.equal(s.state2.code, code) for s in states[1:]):
            raise ValueError("the projections use different second-level code tables")
        if qblock < 8 or qblock & (qblock - 1):
            raise ValueError(f"block size {qblock} is not a power of two >= 8")
        span2 = qblock * qblock2  # weights per second-level scale
        segments, start = [], 0
        for m, s in zip(modules, states):
            n = s.shape[0] * s.shape[1]
            if n % span2:
                raise ValueError(f"{n} weights are not whole second-level blocks of {span2}")
            bias = None if m.bias is None else m.bias.detach().to(torch.float16)
            segments.append(Segment(start, start + n, tuple(s.shape), bias))
            start += n
        if start >= 2 ** 40:
            raise ValueError("layer too large")
        self.qblock, self.qblock2, self.segments = qblock, qblock2, segments
        self.numel = start
        self.device = modules[0].weight.device
        # one buffer per field, in projection order; each parameter becomes a view of its part
        self.packed = torch.cat([m.weight.data.reshape(-1) for m in modules])
        self.absmax8 = torch.cat([s.absmax.reshape(-1) for s in states])
        self.absmax2 = torch.cat([s.state2.absmax.reshape(-1) for s in states])
        for m, s, seg in zip(modules, states, segments):
            m.weight.data = self.packed[seg.start // 2:seg.stop // 2].view(-1, 1)
            s.absmax = self.absmax8[seg.start // qblock:seg.stop // qblock]
            s.state2.absmax = self.absmax2[seg.start // span2:seg.stop // span2]
        self.code = code.contiguous()
        # each projection's offset repeated over its second-level blocks: no lookup per block
        self.offset2 = torch.cat([
            s.offset.reshape(1).to(device=self.device, dtype=torch.float32)
            .expand((seg.stop - seg.start) // span2) for s, seg in zip(states, segments)])
        self.modules = [weakref.ref(m) for m in modules]
        self._bias_spans = {}
        self._scales = None
        self.t_layout = self._transposed_layout()
        # the reference's count of backward uses (solution/qgroup.py:179, :536): callers written
        # for it may add to it; nothing here reads it
        self.expected_bwd = 0

    # -- shapes ----------------------------------------------------------------------------------
    @property
    def shapes(self):
        return [seg.shape for seg in self.segments]

    @property
    def biases(self):
        return [seg.bias for seg in self.segments]

    # -- dequantization ----------------------------------------------------------------------------
    def dequantize(self, first=0, last=NSEG):
        """fp16 weights of projections first .. last - 1 (one launch): the kernel runs on their
        slice of the packed buffers, which starts on a second-level block."""
        lo, hi = self.segments[first].start, self.segments[last - 1].stop
        out = torch.empty(hi - lo, dtype=torch.float16, device=self.packed.device)
        row0 = lo // self.qblock
        launch(self.packed[lo // 2:], self.absmax8[row0:], self.code,
               self.absmax2[row0 // self.qblock2:], self.offset2[row0 // self.qblock2:], None,
               out, (hi - lo) // self.qblock, self.qblock, self.qblock2)
        return out

    def _transposed_layout(self):
        """(per projection (block, W^T element offset, row stride), per block (offset, in,
        width)) of the transposed buffer, or None when the kernel cannot write it (block sizes
        below 64, rows not multiples of 8 or columns of 64, a block's projections of different
        input sizes)."""
        if self.qblock < 64:
            return None
        per_proj, blocks, off = [None] * NSEG, [], 0
        for b, members in enumerate(T_BLOCKS):
            cols = {self.segments[i].shape[1] for i in members}
            width = sum(self.segments[i].shape[0] for i in members)
            if len(cols) != 1 or any(self.segments[i].shape[0] % 8 for i in members):
                return None
            (cin,) = cols
            if cin % 64:
                return None
            o_off = 0
            for i in members:
                per_proj[i] = (b, off + o_off, width)
                o_off += self.segments[i].shape[0]
            blocks.append((off, cin, width))
            off += cin * width
        return per_proj, blocks

    def w4_blocks(self):
        """The transposed buffer's blocks served by the NF4 dequant-GEMM now (left out of it)."""
        if "w4a16" in DISABLED:
            return ()
        return tuple(b for b in W4_BLOCKS if self.w4_ok(b[0], b[-1] + 1))

    def dequantize_all(self):
        """fp16 [numel] of all seven projections (the reference's name, :194)."""
        return self.dequantize()

    def dequantize_t(self, skip=()):
        """The layer's W^T blocks (one launch): block b at blocks[b][0], [in, width] row-major;
        the blocks in `skip` are not written."""
        per_proj, _blocks = self.t_layout
        left_out = {i for b in skip for i in b}
        segs = []
        for i, seg in enumerate(self.segments):
            if i in left_out:
                continue
            _b, dst, ld = per_proj[i]
            segs += [seg.start, seg.shape[0], seg.shape[1], dst, ld]
        out = torch.empty(self.numel, dtype=torch.float16, device=self.packed.device)
        torch.ops.talm.nf4_group_dequant_t(self.packed, self.absmax8, self.code, self.absmax2,
                                           self.offset2, segs, out, self.qblock, self.qblock2)
        return out

    def resident_t(self, need=None):
        """This layer's transposed buffer: the GPU's resident one when it is this group's and
        holds block `need`, else one launch that makes it so (the forward's row-major buffer is
        dropped: the backward has begun)."""
        held = _RESIDENT_T.get(self.device)
        if held is not None and held[0] is self and need not in held[2]:
            return held[1]
        _RESIDENT.pop(self.device, None)
        _RESIDENT_T.pop(self.device, None)
        skip = tuple(b for b in self.w4_blocks() if b != need)
        buf = self.dequantize_t(skip)
        RAN["group_t"] += 1
        _RESIDENT_T[self.device] = (self, buf, skip)
        return buf

    def span_t(self, first, last):
        """fp16 W^T [in, sum of out] of projections first .. last - 1 when they are one block of
        the transposed buffer (q|k|v, o, gate|up, down), else None, as when "qgroup" is off or
        dequantization fails (the caller then takes the row-major weight)."""
        if "qgroup" in DISABLED or self.t_layout is None:
            return None
        members = tuple(range(first, last))
        if members not in T_BLOCKS:
            return None
        try:
            buf = self.resident_t(members)
        except Exception as exc:  # noqa: BLE001 - state.py convention
            if not fallback("qgroup", exc):
                raise
            return None
        off, cin, width = self.t_layout[1][T_BLOCKS.index(members)]
        return buf[off:off + cin * width].view(cin, width)

    # -- the NF4 dequant-GEMM ------------------------------------------------------------------------
    def w4_ok(self, first, last):
        """Projections first .. last - 1 are one [sum of out, in] matrix talm_nf4_gemm takes:
        64-weight blocks in groups of 256, starting on a second-level block, one input size."""
        segs = self.segments[first:last]
        cols = {seg.shape[1] for seg in segs}
        rows = sum(seg.shape[0] for seg in segs)
        return (self.qblock == 64 and self.qblock2 == 256 and len(cols) == 1
                and segs[0].start % (64 * 256) == 0 and next(iter(cols)) % 64 == 0
                and rows % 64 == 0 and "qgroup" not in DISABLED)

    def block_scales(self):
        """Every block's decoded absmax, fp32 [numel / qblock] (one launch, made once: the base
        weights are frozen; 2.9 MB per Qwen2.5-1.5B layer)."""
        if self._scales is None:
            scales = torch.empty(self.numel // self.qblock, dtype=torch.float32,
                                 device=self.device)
            torch.ops.talm.nf4_block_scales(self.absmax8, self.code, self.absmax2, self.offset2,
                                            self.qblock2, scales)
            self._scales = scales
        return self._scales

    def nf4_gemm(self, x, first, last, transpose, out, partials=None):
        """out = x W^T (transpose False: the forward) or x W (True: the input gradient) with W the
        [sum of out, in] rows of projections first .. last - 1 read as NF4 codes and dequantized
        inside the GEMM (the same fp16 weights as `span`). With `partials` (fp32 [parts, N, n],
        `nf4_gemm_parts`) the product's K-part partials are left there instead (out unused)."""
        segs = self.segments[first:last]
        rows, cols = sum(seg.shape[0] for seg in segs), segs[0].shape[1]
        lo = segs[0].start
        scales = self.block_scales()
        if partials is not None:
            torch.ops.talm.nf4_gemm_partials(x, self.packed[lo // 2:], scales[lo // self.qblock:],
                                             rows, cols, transpose, self.qblock, partials)
            return
        ws = torch.empty(_ops.nf4_gemm_workspace_bytes(x.shape[0], rows, cols, transpose),
                         dtype=torch.uint8, device=x.device)
        torch.ops.talm.nf4_gemm(x, self.packed[lo // 2:], scales[lo // self.qblock:], rows, cols,
                                transpose, self.qblock, out, ws)

    def nf4_gemm_parts(self, n_tokens, first, last, transpose):
        """The K-part count of `nf4_gemm`'s plan for n_tokens rows of x."""
        segs = self.segments[first:last]
        rows, cols = sum(seg.shape[0] for seg in segs), segs[0].shape[1]
        return _ops.nf4_gemm_parts(n_tokens, rows, cols, transpose)

    def dequantize_one(self, idx):
        return self.dequantize(idx, idx + 1).view(self.segments[idx].shape)

    def resident(self):
        """This layer's fp16 weights [numel]: the GPU's resident buffer when it is this group's,
        else one launch that makes it so."""
        held = _RESIDENT.get(self.device)
        if held is not None and held[0] is self:
            return held[1]
        buf = self.dequantize()
        RAN["group"] += 1
        _RESIDENT[self.device] = (self, buf)
        return buf

    def begin_forward(self):
        """The layer's forward begins: its weights become resident now, with one launch."""
        held = _RESIDENT.pop(self.device, None)
        held_t = _RESIDENT_T.pop(self.device, None)  # the last backward's: not read by a forward
        del held, held_t  # the previous buffers go back to the allocator first
        self.resident()

    # -- views -------------------------------------------------------------------------------------
    def span(self, *args):
        """span(first, last) or span(which, first, last) (the reference's form; `which`, "fwd"
        or "bwd", is ignored): fp16 [sum of out, in] of the adjacent projections first .. last - 1
        as one view of the resident buffer; None once "qgroup" is off or when dequantization
        fails (state.py), and the caller then takes them one at a time with `weight`."""
        first, last = _pass_args(args, 2, "span")
        if "qgroup" in DISABLED:
            return None
        try:
            buf = self.resident()
        except Exception as exc:  # noqa: BLE001 - state.py convention
            if not fallback("qgroup", exc):
                raise
            return None
        segs = self.segments[first:last]
        rows = sum(seg.shape[0] for seg in segs)
        return buf[segs[0].start:segs[-1].stop].view(rows, segs[0].shape[1])

    def weight(self, *args):
        """weight(idx) or weight(which, idx) (the reference's form, `which` ignored): fp16
        [out, in] of projection `idx` (the per-projection dequantization once "qgroup" is off:
        the same values)."""
        (idx,) = _pass_args(args, 1, "weight")
        view = self.span(idx, idx + 1)
        return view if view is not None else self.reference_weight(idx)

    def reference_weight(self, idx):
        FELL_BACK["group"] += 1
        module = self.modules[idx]()
        return dequantize_4bit(module.weight.data, module.weight.quant_state)

    def span_bias(self, first, last):
        """The fp16 biases of projections first .. last - 1 end to end (zeros stand in for a
        projection without one: adding 0 is exact), or None when none has one; built once."""
        key = (first, last)
        if key not in self._bias_spans:
            segs = self.segments[first:last]
            if all(seg.bias is None for seg in segs):
                self._bias_spans[key] = None
            else:
                self._bias_spans[key] = torch.cat([
                    seg.bias if seg.bias is not None else
                    torch.zeros(seg.shape[0], dtype=torch.float16, device=self.device)
                    for seg in segs])
        return self._bias_spans[key]


def _pass_args(args, count, what):
    """The `count` projection indices of a call that may name the pass first ("fwd" / "bwd", the
    reference's signature)."""
    if len(args) == count + 1 and args[0] in ("fwd", "bwd"):
        args = args[1:]
    if len(args) != count or not all(isinstance(a, int) for a in args):
        raise TypeError(f"LayerGroup.{what}: expected {count} projection index(es), optionally "
                        f"after 'fwd' / 'bwd', got {args!r}")
    return args


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
        return linear(x, group.weight(idx), group.biases[idx])

    @staticmethod
    def backward(ctx, grad_out):
        weight = ctx.group.weight(ctx.idx)
        return matmul(grad_out.to(weight.dtype), weight), None, None


def _linear4bit(module):
    from .nf4_linear import Linear4bit

    base = getattr(module, "base_layer", module)
    return base if isinstance(base, Linear4bit) else None


def _find(layer, path):
    obj = layer
    for part in path.split("."):
        obj = getattr(obj, part, None)
        if obj is None:
            return None
    return obj


def _pack(layer):
    """The decoder layer's LayerGroup, or None when its projections are not seven frozen fp16
    4-bit layers of one layout (each projection then runs its own layer's forward)."""
    modules = []
    for path in PROJECTIONS:
        base = _find(layer, path)
        base = None if base is None else _linear4bit(base)
        if base is None or base.weight.requires_grad or not base.weight.is_cuda \
                or (base.bias is not None and base.bias.requires_grad) \
                or getattr(base, "compute_dtype", None) not in (None, torch.float16):
            return None
        modules.append(base)
    try:
        group = LayerGroup(modules)
    except ValueError:
        return None
    for idx, base in enumerate(modules):
        base._solution_group = (group, idx)
    return group


def setup_layer(layer):
    if not getattr(layer, "_solution_group_done", False):
        layer._solution_group_done = True
        layer._solution_layer_group = _pack(layer)


def enter_layer(layer):
    """The decoder layer's forward begins: pack on first use, then make its weights resident."""
    if "qgroup" in DISABLED:
        return
    try:
        setup_layer(layer)
        group = layer._solution_layer_group
        if group is not None:
            group.begin_forward()
    except Exception as exc:  # noqa: BLE001 - state.py convention
        if not fallback("qgroup", exc):
            raise


def patch_group_dequant():
    """`Qwen2DecoderLayer.forward` makes its layer's weights resident as it begins; the 4-bit
    linear layer routes packed modules through GroupLinear for fp16 inputs
    (solution/qgroup.py:498-545)."""
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
                return GroupLinear.apply(x, group, idx)
            except Exception as exc:  # noqa: BLE001 - state.py convention
                if not fallback("qgroup", exc):
                    raise
        FELL_BACK["group"] += 1
        return lin_forward(self, x)

    linear_forward._solution_group = True
    linear_forward._original = lin_forward
    Linear4bit.forward = linear_forward
    return True
