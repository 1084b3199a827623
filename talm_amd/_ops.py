"""`torch.ops.talm.*`: the PyTorch custom ops over the C-ABI of libtalm.so.

Each op validates device, dtype and layout, passes raw data pointers and the current HIP stream
of the tensors' device to one `extern "C"` entry point, and returns nothing (outputs are the
caller's tensors, annotated as mutated). Registered for the CUDA (= HIP on ROCm) dispatch key
only: a CPU tensor raises NotImplementedError from the dispatcher, never a CPU fallback.
"""

import torch

from . import _lib

_DEF = torch.library.Library("talm", "DEF")


def _stream(t):
    return torch._C._cuda_getCurrentRawStream(t.device.index)


def _ptr(t):
    return t.data_ptr() if t is not None else None


def _require(cond, message):
    if not cond:
        raise ValueError(message)


def _fp16(t, name):
    _require(t.is_cuda and t.dtype == torch.float16, f"{name} must be a CUDA float16 tensor")


def _op(schema):
    """Define `talm::<schema>` and register the decorated function as its CUDA kernel."""
    name = schema.split("(", 1)[0]
    _DEF.define(schema)

    def register(fn):
        _DEF.impl(name, fn, "CUDA")
        return fn

    return register


@_op("nf4_group_dequant(Tensor packed, Tensor absmax8, Tensor code, Tensor absmax2, "
     "Tensor offset2, Tensor(a!) out, int qblock, int qblock2) -> ()")
def nf4_group_dequant(packed, absmax8, code, absmax2, offset2, out, qblock, qblock2):
    _require(packed.dtype == torch.uint8 and absmax8.dtype == torch.uint8, "packed/absmax8: uint8")
    _require(code.dtype == absmax2.dtype == offset2.dtype == torch.float32,
             "code/absmax2/offset2: float32")
    _fp16(out, "out")
    for t in (packed, absmax8, code, absmax2, offset2, out):
        _require(t.is_contiguous() and t.device == out.device, "operands: contiguous, one device")
    n_rows = absmax8.numel()
    _require(code.numel() >= 256, "code: 256 entries")
    _require(packed.numel() * 2 == n_rows * qblock and out.numel() == n_rows * qblock,
             "packed / out sizes do not match n_rows * qblock")
    _require(absmax2.numel() * qblock2 >= n_rows and offset2.numel() == absmax2.numel(),
             "absmax2 / offset2 do not cover every block")
    lib = _lib.lib()
    _lib.check(lib.talm_nf4_group_dequant(packed.data_ptr(), absmax8.data_ptr(), code.data_ptr(),
                                          absmax2.data_ptr(), offset2.data_ptr(), out.data_ptr(),
                                          n_rows, qblock, qblock2, _stream(out)),
               "nf4_group_dequant")


@_op("nf4_dequant(Tensor packed, Tensor absmax, Tensor(a!) out, int blocksize) -> ()")
def nf4_dequant(packed, absmax, out, blocksize):
    _require(packed.dtype == torch.uint8 and absmax.dtype == torch.float32,
             "packed: uint8, absmax: float32")
    _fp16(out, "out")
    _require(packed.is_contiguous() and absmax.is_contiguous() and out.is_contiguous(),
             "operands must be contiguous")
    n = out.numel()
    _require(packed.numel() * 2 >= n and absmax.numel() * blocksize >= n,
             "packed / absmax do not cover out")
    lib = _lib.lib()
    _lib.check(lib.talm_nf4_dequant(packed.data_ptr(), absmax.data_ptr(), out.data_ptr(), n,
                                    blocksize, _stream(out)), "nf4_dequant")


@_op("rmsnorm(Tensor(a!) a, Tensor(b!)? q, Tensor(c!) h, Tensor(d!) xhat, Tensor(e!)? p, "
     "Tensor weight, Tensor(f!) rstd, float eps, int backward) -> ()")
def rmsnorm(a, q, h, xhat, p, weight, rstd, eps, backward):
    n_rows, n_cols = xhat.shape
    add = p is not None
    _require(not add or q is not None, "rmsnorm: p and q go together")
    for t in (a, h, xhat) + ((p, q) if add else ()):
        _require(t.is_cuda and t.is_contiguous() and tuple(t.shape) == (n_rows, n_cols),
                 "rmsnorm: [N, H] operands must be contiguous CUDA tensors of one shape")
    _require(a.dtype == (q.dtype if add else a.dtype), "rmsnorm: q has a's dtype")
    _require(h.dtype == xhat.dtype and (not add or p.dtype == h.dtype),
             "rmsnorm: h, xhat and p share the output dtype")
    _require(weight.is_contiguous() and weight.numel() == n_cols, "rmsnorm: weight [H]")
    _require(rstd.dtype == torch.float32 and rstd.numel() == n_rows, "rmsnorm: rstd float32 [N]")
    lib = _lib.lib()
    _lib.check(lib.talm_rmsnorm(a.data_ptr(), _ptr(q), h.data_ptr(), xhat.data_ptr(), _ptr(p),
                                weight.data_ptr(), rstd.data_ptr(), n_rows, n_cols,
                                _lib.dtype_code(a.dtype), _lib.dtype_code(h.dtype),
                                _lib.dtype_code(weight.dtype), float(eps), int(backward), int(add),
                                _stream(xhat)), "rmsnorm")


@_op("rope(Tensor q, Tensor k, Tensor cos, Tensor sin, Tensor(a!) out_q, Tensor(b!) out_k, "
     "int backward) -> ()")
def rope(q, k, cos, sin, out_q, out_k, backward):
    """q, out_q [T, Hq, D] and k, out_k [T, Hk, D] fp16 views (any token / head strides, unit
    column stride); cos, sin float32 [T, D] with unit column stride. out_* may be q / k."""
    n_tokens, hq, dim = q.shape
    hk = k.shape[1]
    for t, heads in ((q, hq), (k, hk), (out_q, hq), (out_k, hk)):
        _fp16(t, "q/k")
        _require(tuple(t.shape) == (n_tokens, heads, dim) and t.stride(2) == 1,
                 "rope: q/k must be [T, H, D] views with unit column stride")
    for t in (cos, sin):
        _require(t.is_cuda and t.dtype == torch.float32 and tuple(t.shape) == (n_tokens, dim)
                 and t.stride(1) == 1, "rope: cos/sin float32 [T, D]")
    _require(cos.stride(0) == sin.stride(0), "rope: cos and sin share their token stride")
    lib = _lib.lib()
    _lib.check(lib.talm_rope(q.data_ptr(), k.data_ptr(), cos.data_ptr(), sin.data_ptr(),
                             out_q.data_ptr(), out_k.data_ptr(), n_tokens, hq, hk, dim,
                             q.stride(0), q.stride(1), k.stride(0), k.stride(1),
                             out_q.stride(0), out_q.stride(1), out_k.stride(0), out_k.stride(1),
                             cos.stride(0), int(backward), _stream(q)), "rope")


@_op("swiglu_fwd(Tensor gate, Tensor up, Tensor(a!) out) -> ()")
def swiglu_fwd(gate, up, out):
    for t in (gate, up, out):
        _fp16(t, "swiglu operand")
        _require(t.is_contiguous() and t.numel() == gate.numel(), "swiglu: contiguous, one size")
    lib = _lib.lib()
    _lib.check(lib.talm_swiglu_fwd(gate.data_ptr(), up.data_ptr(), out.data_ptr(), gate.numel(),
                                   _stream(gate)), "swiglu_fwd")


@_op("swiglu_bwd(Tensor grad, Tensor gate, Tensor up, Tensor(a!) dgate, Tensor(b!) dup) -> ()")
def swiglu_bwd(grad, gate, up, dgate, dup):
    for t in (grad, gate, up, dgate, dup):
        _fp16(t, "swiglu operand")
        _require(t.is_contiguous() and t.numel() == gate.numel(), "swiglu: contiguous, one size")
    lib = _lib.lib()
    _lib.check(lib.talm_swiglu_bwd(grad.data_ptr(), gate.data_ptr(), up.data_ptr(),
                                   dgate.data_ptr(), dup.data_ptr(), gate.numel(), _stream(gate)),
               "swiglu_bwd")


def head_ce_workspace_bytes(n_rows, hidden, vocab, vchunk, n_grad, group):
    size = _lib.lib().talm_head_ce_workspace(n_rows, hidden, vocab, vchunk, n_grad, group)
    if size < 0:
        raise ValueError(f"head_ce: unsupported shape rows={n_rows} hidden={hidden} "
                         f"vocab={vocab} vchunk={vchunk} n_grad={n_grad} group={group}")
    return int(size)


@_op("head_weight_t(Tensor weight, Tensor(a!) weight_t) -> ()")
def head_weight_t(weight, weight_t):
    """weight fp16 [V, H] (unit column stride) -> weight_t fp16 [H, ldwt] (unit column stride,
    ldwt >= V): the transpose, with columns [V, ldwt) zero."""
    vocab, size = weight.shape
    _fp16(weight, "weight")
    _fp16(weight_t, "weight_t")
    _require(weight.stride(1) == 1 and weight_t.stride(1) == 1 and weight_t.shape[0] == size
             and weight_t.stride(0) >= vocab and weight_t.shape[1] >= vocab,
             "head_weight_t: weight [V, H] and weight_t [H, >= V] with unit column stride")
    lib = _lib.lib()
    _lib.check(lib.talm_head_weight_t(weight.data_ptr(), weight.stride(0), vocab, size,
                                      weight_t.data_ptr(), weight_t.stride(0), _stream(weight)),
               "head_weight_t")


@_op("head_ce(Tensor hidden, Tensor weight, Tensor? weight_t, Tensor targets, int vchunk, "
     "int n_grad, int group, Tensor(a!) token_loss, Tensor(b!) entropy, Tensor(c!) best_idx, "
     "Tensor(d!) correct, Tensor(e!)? grad_hidden, Tensor(f!) workspace) -> ()")
def head_ce(hidden, weight, weight_t, targets, vchunk, n_grad, group, token_loss, entropy,
            best_idx, correct, grad_hidden, workspace):
    """hidden fp16 [N, H] (unit column stride), weight fp16 [V, H] (unit column stride),
    weight_t its head_weight_t transpose (needed with the gradient), targets int64 [N] with rows
    [0, n_grad) exactly the labelled ones."""
    n_rows, size = hidden.shape
    vocab = weight.shape[0]
    _fp16(hidden, "hidden")
    _fp16(weight, "weight")
    _require(hidden.stride(1) == 1 and weight.stride(1) == 1 and weight.shape[1] == size,
             "head_ce: hidden [N, H] and weight [V, H] with unit column stride")
    if weight_t is not None:
        _fp16(weight_t, "weight_t")
        _require(weight_t.stride(1) == 1 and weight_t.shape[0] == size
                 and weight_t.shape[1] >= vocab, "head_ce: weight_t [H, >= V], unit column stride")
    _require(targets.dtype == torch.int64 and targets.is_contiguous() and
             targets.numel() == n_rows, "head_ce: targets int64 [N]")
    for t, dt in ((token_loss, torch.float32), (entropy, torch.float32), (best_idx, torch.int32),
                  (correct, torch.int32)):
        _require(t.dtype == dt and t.is_contiguous() and t.numel() == n_rows,
                 "head_ce: per-row outputs of N elements")
    if grad_hidden is not None:
        _fp16(grad_hidden, "grad_hidden")
        _require(grad_hidden.is_contiguous() and tuple(grad_hidden.shape) == (n_rows, size),
                 "head_ce: grad_hidden contiguous [N, H]")
    _require(workspace.is_cuda and workspace.is_contiguous(), "head_ce: workspace")
    lib = _lib.lib()
    _lib.check(lib.talm_head_ce(hidden.data_ptr(), hidden.stride(0), weight.data_ptr(),
                                weight.stride(0), _ptr(weight_t),
                                0 if weight_t is None else weight_t.stride(0), targets.data_ptr(),
                                n_rows, size, vocab, int(vchunk), int(n_grad), int(group),
                                token_loss.data_ptr(), entropy.data_ptr(), best_idx.data_ptr(),
                                correct.data_ptr(), _ptr(grad_hidden), workspace.data_ptr(),
                                workspace.numel() * workspace.element_size(), _stream(hidden)),
               "head_ce")


@_op("lora_down(Tensor x, Tensor a0, Tensor? a1, int k0, int k1, int xcol0, int xcol1, "
     "int a_kmajor, float scaling0, float scaling1, Tensor(a!) t, Tensor(b!) ts) -> ()")
def lora_down(x, a0, a1, k0, k1, xcol0, xcol1, a_kmajor, scaling0, scaling1, t, ts):
    """Adapter g: t[:, 16g:16g+16] = x[:, xcol_g:xcol_g + k_g] A_g^T, ts = scaling_g * that;
    x fp16 (unit column stride), A_g fp16 contiguous [16, k_g] (or [k_g, 16] with a_kmajor),
    t / ts fp16 with one row stride."""
    for name, v in (("x", x), ("a0", a0), ("t", t), ("ts", ts)):
        _fp16(v, name)
    n = x.shape[0]
    adapters = [(a0, k0, xcol0)] + ([(a1, k1, xcol1)] if a1 is not None else [])
    for a, k, col in adapters:
        _fp16(a, "lora A")
        shape = (k, 16) if a_kmajor else (16, k)
        _require(a.is_contiguous() and tuple(a.shape) == shape and col + k <= x.shape[1],
                 "lora_down: A [16, k] ([k, 16] k-major) inside x's columns")
    _require(x.stride(1) == 1 and t.stride(1) == 1 and ts.stride(1) == 1
             and t.stride(0) == ts.stride(0) and t.shape[0] == n and ts.shape[0] == n
             and t.shape[1] >= 16 * len(adapters) and ts.shape[1] >= 16 * len(adapters),
             "lora_down: x [N, *], t/ts [N, 16 * adapters] with one row stride")
    lib = _lib.lib()
    _lib.check(lib.talm_lora_down(x.data_ptr(), x.stride(0), n, int(k0), int(k1), int(xcol0),
                                  int(xcol1), a0.data_ptr(), _ptr(a1), len(adapters),
                                  int(a_kmajor), float(scaling0), float(scaling1), t.data_ptr(),
                                  ts.data_ptr(), t.stride(0), _stream(x)), "lora_down")


@_op("qkv_lora_fwd(Tensor x, Tensor weight, Tensor? bias, Tensor? ts, Tensor? b0, int seg0_begin, "
     "int seg0_end, Tensor? b1, int seg1_begin, int seg1_end, Tensor? cos, Tensor? sin, "
     "int rope_cols, Tensor(a!) out) -> ()")
def qkv_lora_fwd(x, weight, bias, ts, b0, seg0_begin, seg0_end, b1, seg1_begin, seg1_end, cos,
                 sin, rope_cols, out):
    """out [N, n_out] = x W^T + bias + the adapters' ts B^T on their columns, then the rotary
    embedding (cos/sin fp32 [N, >= 128]) on the 128-column heads below rope_cols."""
    _fp16(x, "x")
    _fp16(weight, "weight")
    _fp16(out, "out")
    n, size = x.shape
    n_out = weight.shape[0]
    _require(x.stride(1) == 1 and weight.stride(1) == 1 and out.stride(1) == 1
             and weight.shape[1] == size and tuple(out.shape) == (n, n_out),
             "qkv_lora_fwd: x [N, H], weight [n_out, H], out [N, n_out], unit column strides")
    if bias is not None:
        _fp16(bias, "bias")
        _require(bias.is_contiguous() and bias.numel() == n_out, "qkv_lora_fwd: bias [n_out]")
    bs = [b for b in (b0, b1) if b is not None]
    for b in bs:
        _fp16(b, "lora B")
        _require(b.is_contiguous() and b.shape[1] == 16, "qkv_lora_fwd: B [segment, 16]")
    if bs:
        _fp16(ts, "ts")
        _require(ts.stride(1) == 1 and ts.shape[0] == n and ts.shape[1] >= 16 * len(bs),
                 "qkv_lora_fwd: ts [N, 16 * adapters]")
    if cos is not None:
        for v in (cos, sin):
            _require(v is not None and v.is_cuda and v.dtype == torch.float32 and v.stride(1) == 1
                     and v.shape[0] == n and v.shape[1] >= 128 and v.stride(0) == cos.stride(0),
                     "qkv_lora_fwd: cos/sin fp32 [N, >= 128] with one row stride")
    lib = _lib.lib()
    _lib.check(lib.talm_qkv_lora_fwd(
        x.data_ptr(), x.stride(0), n, size, weight.data_ptr(), weight.stride(0), n_out,
        _ptr(bias), _ptr(ts), 0 if ts is None else ts.stride(0), len(bs), _ptr(b0), seg0_begin,
        seg0_end, _ptr(b1), seg1_begin, seg1_end, _ptr(cos), _ptr(sin),
        0 if cos is None else cos.stride(0), rope_cols, out.data_ptr(), out.stride(0),
        _stream(x)), "qkv_lora_fwd")


@_op("qkv_bwd_prep(Tensor dq, Tensor dk, Tensor dv, Tensor? cos, Tensor? sin, "
     "Tensor(a!) dcat) -> ()")
def qkv_bwd_prep(dq, dk, dv, cos, sin, dcat):
    """dcat [N, q + k + v] = [rope_back(dq) | rope_back(dk) | dv] (cos/sin fp32 [N, >= 128], or
    None for no rotation); every operand fp16 with unit column stride."""
    n = dcat.shape[0]
    for name, v in (("dq", dq), ("dk", dk), ("dv", dv), ("dcat", dcat)):
        _fp16(v, name)
        _require(v.dim() == 2 and v.stride(1) == 1 and v.shape[0] == n,
                 f"qkv_bwd_prep: {name} [N, columns] with unit column stride")
    _require(dcat.shape[1] == dq.shape[1] + dk.shape[1] + dv.shape[1],
             "qkv_bwd_prep: dcat holds q, k and v")
    if cos is not None:
        for v in (cos, sin):
            _require(v is not None and v.is_cuda and v.dtype == torch.float32 and v.stride(1) == 1
                     and v.shape[0] == n and v.shape[1] >= 128 and v.stride(0) == cos.stride(0),
                     "qkv_bwd_prep: cos/sin fp32 [N, >= 128] with one row stride")
    lib = _lib.lib()
    _lib.check(lib.talm_qkv_bwd_prep(dq.data_ptr(), dq.stride(0), dk.data_ptr(), dk.stride(0),
                                     dv.data_ptr(), dv.stride(0), n, dq.shape[1], dk.shape[1],
                                     dv.shape[1], _ptr(cos), _ptr(sin),
                                     0 if cos is None else cos.stride(0), dcat.data_ptr(),
                                     dcat.stride(0), _stream(dcat)), "qkv_bwd_prep")


@_op("qkv_lora_bwd_dx(Tensor dcat, Tensor weight_t, Tensor? u, Tensor? a_t, Tensor(a!) dx) -> ()")
def qkv_lora_bwd_dx(dcat, weight_t, u, a_t, dx):
    """dx [N, H] = dcat [N, n_out] W + u [N, r] A, from weight_t = W^T [H, >= n_out] and
    a_t = A^T [H, r] (the adapters side by side); fp16, unit column strides."""
    for name, v in (("dcat", dcat), ("weight_t", weight_t), ("dx", dx)):
        _fp16(v, name)
        _require(v.dim() == 2 and v.stride(1) == 1, f"qkv_lora_bwd_dx: {name} unit column stride")
    n, n_out = dcat.shape
    size = weight_t.shape[0]
    _require(weight_t.shape[1] >= n_out and tuple(dx.shape) == (n, size),
             "qkv_lora_bwd_dx: weight_t [H, >= n_out], dx [N, H]")
    rank = 0
    if u is not None:
        _fp16(u, "u")
        _fp16(a_t, "a_t")
        rank = u.shape[1]
        _require(u.stride(1) == 1 and a_t.stride(1) == 1 and u.shape[0] == n
                 and tuple(a_t.shape) == (size, rank), "qkv_lora_bwd_dx: u [N, r], a_t [H, r]")
    lib = _lib.lib()
    _lib.check(lib.talm_qkv_lora_bwd_dx(
        dcat.data_ptr(), dcat.stride(0), n, n_out, weight_t.data_ptr(), weight_t.stride(0), size,
        _ptr(u), 0 if u is None else u.stride(0), rank, _ptr(a_t),
        0 if a_t is None else a_t.stride(0), dx.data_ptr(), dx.stride(0), _stream(dcat)),
        "qkv_lora_bwd_dx")


def lora_wgrad_workspace_bytes(n_tokens, hidden, seg0, seg1):
    size = _lib.lib().talm_lora_wgrad_workspace(n_tokens, hidden, seg0, seg1)
    _require(size >= 0, "lora_wgrad: unsupported shape")
    return int(size)


@_op("lora_wgrad(Tensor x, Tensor dy, Tensor u, Tensor t, int lo0, int seg0, float scaling0, "
     "Tensor(a!) da0, Tensor(b!) db0, int lo1, int seg1, float scaling1, Tensor(c!)? da1, "
     "Tensor(d!)? db1, Tensor(e!) workspace) -> ()")
def lora_wgrad(x, dy, u, t, lo0, seg0, scaling0, da0, db0, lo1, seg1, scaling1, da1, db1,
               workspace):
    """fp32 dA_g [16, H] = u_g^T x, dB_g [seg_g, 16] = scaling_g dy[:, lo_g:lo_g+seg_g]^T t_g."""
    for name, v in (("x", x), ("dy", dy), ("u", u), ("t", t)):
        _fp16(v, name)
        _require(v.dim() == 2 and v.stride(1) == 1, f"lora_wgrad: {name} unit column stride")
    n, size = x.shape
    two = da1 is not None
    for da, db, seg in ((da0, db0, seg0),) + (((da1, db1, seg1),) if two else ()):
        _require(da.is_cuda and da.dtype == torch.float32 and da.is_contiguous()
                 and tuple(da.shape) == (16, size), "lora_wgrad: dA fp32 [16, H]")
        _require(db.is_cuda and db.dtype == torch.float32 and db.is_contiguous()
                 and tuple(db.shape) == (seg, 16), "lora_wgrad: dB fp32 [segment, 16]")
    _require(workspace.is_cuda and workspace.is_contiguous(), "lora_wgrad: workspace")
    if n == 0:  # no tokens: zero gradients, no launch
        for out in (da0, db0, da1, db1):
            if out is not None:
                out.zero_()
        return
    lib = _lib.lib()
    _lib.check(lib.talm_lora_wgrad(
        x.data_ptr(), x.stride(0), dy.data_ptr(), dy.stride(0), u.data_ptr(), u.stride(0),
        t.data_ptr(), t.stride(0), n, size, 2 if two else 1, int(lo0), int(seg0), float(scaling0),
        da0.data_ptr(), db0.data_ptr(), int(lo1), int(seg1), float(scaling1), _ptr(da1),
        _ptr(db1), workspace.data_ptr(), workspace.numel() * workspace.element_size(),
        _stream(x)), "lora_wgrad")
