// `torch.ops.talm.*`: the PyTorch custom ops over the C-ABI of libtalm.so (include/talm.h).
//
// Each op checks device, dtype and layout of its tensors, then passes raw data pointers, sizes
// and the current HIP stream of the tensors' device to one `extern "C"` entry point, and returns
// nothing (outputs are the caller's tensors, marked as mutated in the schema). The ops are
// registered for the CUDA (= HIP on ROCm) dispatch key only: CPU tensors raise
// NotImplementedError from the dispatcher, never a CPU fallback. A rejected shape raises
// ValueError, a failed launch RuntimeError (the message is talm_last_error()), as the reference's
// launchers raise ValueError for unsupported shapes (solution/rmsnorm.py:113-114,
// solution/qgroup.py:129-168).
//
// This layer is C++ so that a launch costs a few microseconds of host time: the QLoRA step
// issues several hundred of these ops per optimizer step.
//
// `talm::gemm` is the one op here that is not a libtalm.so kernel: the plain fp16 projection
// GEMMs of the layer group (solution/qgroup.py:346-355, cuBLAS in the reference) on hipBLASLt,
// through PyTorch's own hipBLASLt handle and workspace, with the algorithm chosen once per shape
// and kept (PyTorch's matmul asks hipBLASLt's heuristic on every call).
#include <ATen/ATen.h>
#include <ATen/hip/HIPContext.h>
#include <hipblaslt/hipblaslt-ext.hpp>
#include <hipblaslt/hipblaslt.h>
#include <torch/library.h>

#include <atomic>
#include <mutex>
#include <vector>

#include <optional>
#include <string>
#include <unordered_map>

#include "talm.h"

namespace {

using at::Tensor;
using OptTensor = std::optional<Tensor>;

void require(bool ok, const char* message) { TORCH_CHECK_VALUE(ok, message); }

void require_fp16(const Tensor& t, const char* name) {
  TORCH_CHECK_VALUE(t.is_cuda() && t.scalar_type() == at::kHalf, name,
                    " must be a CUDA float16 tensor");
}

void* stream_of(const Tensor& t) {
  return static_cast<void*>(at::hip::getCurrentHIPStream(t.device().index()).stream());
}

void* ptr(const Tensor& t) { return t.data_ptr(); }
void* ptr(const OptTensor& t) { return t.has_value() ? t->data_ptr() : nullptr; }
template <class T>
T* as(const Tensor& t) { return static_cast<T*>(t.data_ptr()); }
template <class T>
T* as(const OptTensor& t) { return t.has_value() ? static_cast<T*>(t->data_ptr()) : nullptr; }

void check(int status, const char* what) {
  if (status == TALM_OK) return;
  const char* m = talm_last_error();
  const std::string message =
      (m && *m) ? std::string(m) : std::string(what) + ": status " + std::to_string(status);
  TORCH_CHECK_VALUE(status != TALM_EINVAL, message);
  TORCH_CHECK(false, message);
}

int32_t dtype_code(at::ScalarType s) {
  if (s == at::kFloat) return TALM_F32;
  if (s == at::kHalf) return TALM_F16;
  TORCH_CHECK_VALUE(false, "libtalm: unsupported dtype ", s);
  return -1;
}

bool same_shape(const Tensor& t, int64_t rows, int64_t cols) {
  return t.dim() == 2 && t.size(0) == rows && t.size(1) == cols;
}

// ------------------------------------------------------------------------------------------

void nf4_group_dequant_impl(const Tensor& packed, const Tensor& absmax8, const Tensor& code,
                            const Tensor& absmax2, const Tensor& offset2, const Tensor& out,
                            int64_t qblock, int64_t qblock2, bool streaming) {
  require(packed.scalar_type() == at::kByte && absmax8.scalar_type() == at::kByte,
          "packed/absmax8: uint8");
  require(code.scalar_type() == at::kFloat && absmax2.scalar_type() == at::kFloat &&
              offset2.scalar_type() == at::kFloat,
          "code/absmax2/offset2: float32");
  require_fp16(out, "out");
  for (const Tensor* t : {&packed, &absmax8, &code, &absmax2, &offset2, &out})
    require(t->is_contiguous() && t->device() == out.device(), "operands: contiguous, one device");
  const int64_t n_rows = absmax8.numel();
  require(code.numel() >= 256, "code: 256 entries");
  require(packed.numel() * 2 == n_rows * qblock && out.numel() == n_rows * qblock,
          "packed / out sizes do not match n_rows * qblock");
  require(absmax2.numel() * qblock2 >= n_rows && offset2.numel() == absmax2.numel(),
          "absmax2 / offset2 do not cover every block");
  auto entry = streaming ? talm_nf4_group_dequant_streaming : talm_nf4_group_dequant;
  check(entry(as<uint8_t>(packed), as<uint8_t>(absmax8), as<float>(code), as<float>(absmax2),
              as<float>(offset2), as<uint16_t>(out), n_rows, static_cast<int32_t>(qblock),
              static_cast<int32_t>(qblock2), stream_of(out)),
        streaming ? "nf4_group_dequant_streaming" : "nf4_group_dequant");
}

void nf4_group_dequant(const Tensor& packed, const Tensor& absmax8, const Tensor& code,
                       const Tensor& absmax2, const Tensor& offset2, const Tensor& out,
                       int64_t qblock, int64_t qblock2) {
  nf4_group_dequant_impl(packed, absmax8, code, absmax2, offset2, out, qblock, qblock2, false);
}

void nf4_group_dequant_streaming(const Tensor& packed, const Tensor& absmax8, const Tensor& code,
                                 const Tensor& absmax2, const Tensor& offset2, const Tensor& out,
                                 int64_t qblock, int64_t qblock2) {
  nf4_group_dequant_impl(packed, absmax8, code, absmax2, offset2, out, qblock, qblock2, true);
}

// W^T of projections of a packed layer: segs holds (start, rows, cols, dst, ld) per projection.
void nf4_group_dequant_t(const Tensor& packed, const Tensor& absmax8, const Tensor& code,
                         const Tensor& absmax2, const Tensor& offset2, at::IntArrayRef segs,
                         const Tensor& out, int64_t qblock, int64_t qblock2) {
  require(packed.scalar_type() == at::kByte && absmax8.scalar_type() == at::kByte,
          "packed/absmax8: uint8");
  require(code.scalar_type() == at::kFloat && absmax2.scalar_type() == at::kFloat &&
              offset2.scalar_type() == at::kFloat,
          "code/absmax2/offset2: float32");
  require_fp16(out, "out");
  for (const Tensor* t : {&packed, &absmax8, &code, &absmax2, &offset2, &out})
    require(t->is_contiguous() && t->device() == out.device(), "operands: contiguous, one device");
  require(code.numel() >= 256, "code: 256 entries");
  require(segs.size() % 5 == 0, "segs: five integers per projection");
  require(qblock > 0 && qblock2 > 0, "qblock / qblock2 positive");
  for (size_t g = 0; g < segs.size(); g += 5) {
    const int64_t end = segs[g] + segs[g + 1] * segs[g + 2];  // one past the last weight
    require(segs[g] >= 0 && segs[g + 1] > 0 && segs[g + 2] > 0 && end <= packed.numel() * 2 &&
                (end + qblock - 1) / qblock <= absmax8.numel() &&
                ((end + qblock - 1) / qblock + qblock2 - 1) / qblock2 <= absmax2.numel() &&
                offset2.numel() == absmax2.numel(),
            "nf4_group_dequant_t: a projection outside the packed buffers");
  }
  check(talm_nf4_group_dequant_t(as<uint8_t>(packed), as<uint8_t>(absmax8), as<float>(code),
                                 as<float>(absmax2), as<float>(offset2), segs.data(),
                                 static_cast<int32_t>(segs.size() / 5),
                                 static_cast<int32_t>(qblock), static_cast<int32_t>(qblock2),
                                 as<uint16_t>(out), out.numel(), stream_of(out)),
        "nf4_group_dequant_t");
}

// out [m, n] = a [m, k] b [n, k]^T (fp16, fp32 accumulation) as K parts plus a reduction.
void gemm_splitk(const Tensor& a, const Tensor& b, const Tensor& out, const Tensor& workspace) {
  for (const auto& [v, name] : {std::pair<const Tensor*, const char*>{&a, "a"}, {&b, "b"},
                                {&out, "out"}}) {
    require_fp16(*v, name);
    TORCH_CHECK_VALUE(v->dim() == 2 && v->stride(1) == 1, "gemm_splitk: ", name,
                      " unit column stride");
  }
  const int64_t m = a.size(0), k = a.size(1), n = b.size(0);
  require(b.size(1) == k && same_shape(out, m, n), "gemm_splitk: a [m, k], b [n, k], out [m, n]");
  require(workspace.is_cuda() && workspace.is_contiguous() && workspace.device() == out.device(),
          "gemm_splitk: workspace");
  check(talm_gemm_splitk(as<uint16_t>(a), a.stride(0), as<uint16_t>(b), b.stride(0),
                         as<uint16_t>(out), out.stride(0), m, n, k, workspace.data_ptr(),
                         workspace.numel() * static_cast<int64_t>(workspace.element_size()),
                         stream_of(out)),
        "gemm_splitk");
}

void nf4_dequant(const Tensor& packed, const Tensor& absmax, const Tensor& out,
                 int64_t blocksize) {
  require(packed.scalar_type() == at::kByte && absmax.scalar_type() == at::kFloat,
          "packed: uint8, absmax: float32");
  require_fp16(out, "out");
  require(packed.is_contiguous() && absmax.is_contiguous() && out.is_contiguous(),
          "operands must be contiguous");
  const int64_t n = out.numel();
  require(packed.numel() * 2 >= n && absmax.numel() * blocksize >= n,
          "packed / absmax do not cover out");
  check(talm_nf4_dequant(as<uint8_t>(packed), as<float>(absmax), as<uint16_t>(out), n,
                         static_cast<int32_t>(blocksize), stream_of(out)),
        "nf4_dequant");
}

void rmsnorm(const Tensor& a, const OptTensor& q, const Tensor& h, const Tensor& xhat,
             const OptTensor& p, const Tensor& weight, const Tensor& rstd, double eps,
             int64_t backward) {
  require(xhat.dim() == 2, "rmsnorm: [N, H] operands must be contiguous CUDA tensors of one shape");
  const int64_t n_rows = xhat.size(0), n_cols = xhat.size(1);
  const bool add = p.has_value();
  require(!add || backward || q.has_value(), "rmsnorm: p and q go together in the forward");
  auto ok = [&](const Tensor& t) {
    return t.is_cuda() && t.is_contiguous() && same_shape(t, n_rows, n_cols);
  };
  require(ok(a) && ok(h) && ok(xhat) && (!add || (ok(*p) && (!q.has_value() || ok(*q)))),
          "rmsnorm: [N, H] operands must be contiguous CUDA tensors of one shape");
  require(!add || !q.has_value() || a.scalar_type() == q->scalar_type(),
          "rmsnorm: q has a's dtype");
  require(h.scalar_type() == xhat.scalar_type() && (!add || p->scalar_type() == h.scalar_type()),
          "rmsnorm: h, xhat and p share the output dtype");
  require(weight.is_contiguous() && weight.numel() == n_cols, "rmsnorm: weight [H]");
  require(rstd.scalar_type() == at::kFloat && rstd.numel() == n_rows, "rmsnorm: rstd float32 [N]");
  check(talm_rmsnorm(ptr(a), ptr(q), ptr(h), ptr(xhat), ptr(p), ptr(weight), as<float>(rstd),
                     n_rows, n_cols, dtype_code(a.scalar_type()), dtype_code(h.scalar_type()),
                     dtype_code(weight.scalar_type()), static_cast<float>(eps),
                     backward ? 1 : 0, add ? 1 : 0, stream_of(xhat)),
        "rmsnorm");
}

// q, out_q [T, Hq, D] and k, out_k [T, Hk, D] fp16 views (any token / head strides, unit column
// stride); cos, sin float32 [T, D] with unit column stride. out_* may be q / k.
void rope(const Tensor& q, const Tensor& k, const Tensor& cos, const Tensor& sin,
          const Tensor& out_q, const Tensor& out_k, int64_t backward) {
  require(q.dim() == 3 && k.dim() == 3, "rope: q/k must be [T, H, D] views with unit column stride");
  const int64_t n_tokens = q.size(0), hq = q.size(1), dim = q.size(2), hk = k.size(1);
  for (const auto& [t, heads] : {std::pair<const Tensor*, int64_t>{&q, hq}, {&k, hk},
                                 {&out_q, hq}, {&out_k, hk}}) {
    require_fp16(*t, "q/k");
    require(t->dim() == 3 && t->size(0) == n_tokens && t->size(1) == heads &&
                t->size(2) == dim && t->stride(2) == 1,
            "rope: q/k must be [T, H, D] views with unit column stride");
  }
  for (const Tensor* t : {&cos, &sin})
    require(t->is_cuda() && t->scalar_type() == at::kFloat && same_shape(*t, n_tokens, dim) &&
                t->stride(1) == 1,
            "rope: cos/sin float32 [T, D]");
  require(cos.stride(0) == sin.stride(0), "rope: cos and sin share their token stride");
  check(talm_rope(as<uint16_t>(q), as<uint16_t>(k), as<float>(cos), as<float>(sin),
                  as<uint16_t>(out_q), as<uint16_t>(out_k), n_tokens, static_cast<int32_t>(hq),
                  static_cast<int32_t>(hk), static_cast<int32_t>(dim), q.stride(0), q.stride(1),
                  k.stride(0), k.stride(1), out_q.stride(0), out_q.stride(1), out_k.stride(0),
                  out_k.stride(1), cos.stride(0), backward ? 1 : 0, stream_of(q)),
        "rope");
}

void swiglu_fwd(const Tensor& gate, const Tensor& up, const Tensor& out) {
  for (const Tensor* t : {&gate, &up, &out}) {
    require_fp16(*t, "swiglu operand");
    require(t->is_contiguous() && t->numel() == gate.numel(), "swiglu: contiguous, one size");
  }
  check(talm_swiglu_fwd(as<uint16_t>(gate), as<uint16_t>(up), as<uint16_t>(out), gate.numel(),
                        stream_of(gate)),
        "swiglu_fwd");
}

void swiglu_bwd(const Tensor& grad, const Tensor& gate, const Tensor& up, const Tensor& dgate,
                const Tensor& dup) {
  for (const Tensor* t : {&grad, &gate, &up, &dgate, &dup}) {
    require_fp16(*t, "swiglu operand");
    require(t->is_contiguous() && t->numel() == gate.numel(), "swiglu: contiguous, one size");
  }
  check(talm_swiglu_bwd(as<uint16_t>(grad), as<uint16_t>(gate), as<uint16_t>(up),
                        as<uint16_t>(dgate), as<uint16_t>(dup), gate.numel(), stream_of(gate)),
        "swiglu_bwd");
}

// [rows, cols] fp16 views with unit column stride (any row strides); outputs may alias inputs.
void swiglu_rows_view(const Tensor& t, int64_t rows, int64_t cols) {
  require_fp16(t, "swiglu operand");
  require(same_shape(t, rows, cols) && t.stride(1) == 1,
          "swiglu_rows: [rows, cols] views with unit column stride, one shape");
}

void swiglu_fwd_rows(const Tensor& gate, const Tensor& up, const Tensor& out) {
  require(gate.dim() == 2, "swiglu_rows: [rows, cols] views with unit column stride, one shape");
  const int64_t rows = gate.size(0), cols = gate.size(1);
  for (const Tensor* t : {&gate, &up, &out}) swiglu_rows_view(*t, rows, cols);
  check(talm_swiglu_fwd_rows(as<uint16_t>(gate), gate.stride(0), as<uint16_t>(up), up.stride(0),
                             as<uint16_t>(out), out.stride(0), rows, cols, stream_of(gate)),
        "swiglu_fwd_rows");
}

void swiglu_bwd_rows(const Tensor& grad, const Tensor& gate, const Tensor& up,
                     const Tensor& dgate, const Tensor& dup) {
  require(gate.dim() == 2, "swiglu_rows: [rows, cols] views with unit column stride, one shape");
  const int64_t rows = gate.size(0), cols = gate.size(1);
  for (const Tensor* t : {&grad, &gate, &up, &dgate, &dup}) swiglu_rows_view(*t, rows, cols);
  check(talm_swiglu_bwd_rows(as<uint16_t>(grad), grad.stride(0), as<uint16_t>(gate),
                             gate.stride(0), as<uint16_t>(up), up.stride(0), as<uint16_t>(dgate),
                             dgate.stride(0), as<uint16_t>(dup), dup.stride(0), rows, cols,
                             stream_of(gate)),
        "swiglu_bwd_rows");
}

// weight fp16 [V, H] (unit column stride) -> weight_t fp16 [H, ldwt] (unit column stride,
// ldwt >= V): the transpose, with columns [V, ldwt) zero.
void head_weight_t(const Tensor& weight, const Tensor& weight_t) {
  require_fp16(weight, "weight");
  require_fp16(weight_t, "weight_t");
  require(weight.dim() == 2 && weight_t.dim() == 2,
          "head_weight_t: weight [V, H] and weight_t [H, >= V] with unit column stride");
  const int64_t vocab = weight.size(0), size = weight.size(1);
  require(weight.stride(1) == 1 && weight_t.stride(1) == 1 && weight_t.size(0) == size &&
              weight_t.stride(0) >= vocab && weight_t.size(1) >= vocab,
          "head_weight_t: weight [V, H] and weight_t [H, >= V] with unit column stride");
  check(talm_head_weight_t(as<uint16_t>(weight), weight.stride(0), vocab, size,
                           as<uint16_t>(weight_t), weight_t.stride(0), stream_of(weight)),
        "head_weight_t");
}

// hidden fp16 [N, H] (unit column stride), weight fp16 [V, H] (unit column stride), targets
// int64 [N] with rows [0, n_grad) exactly the labelled ones.
void head_ce(const Tensor& hidden, const Tensor& weight, const Tensor& targets, int64_t vchunk, int64_t n_grad, int64_t group,
             const Tensor& token_loss, const Tensor& entropy, const Tensor& best_idx,
             const Tensor& correct, const OptTensor& grad_hidden, const Tensor& workspace) {
  require_fp16(hidden, "hidden");
  require_fp16(weight, "weight");
  require(hidden.dim() == 2 && weight.dim() == 2,
          "head_ce: hidden [N, H] and weight [V, H] with unit column stride");
  const int64_t n_rows = hidden.size(0), size = hidden.size(1), vocab = weight.size(0);
  require(hidden.stride(1) == 1 && weight.stride(1) == 1 && weight.size(1) == size,
          "head_ce: hidden [N, H] and weight [V, H] with unit column stride");
  require(targets.scalar_type() == at::kLong && targets.is_contiguous() &&
              targets.numel() == n_rows,
          "head_ce: targets int64 [N]");
  for (const auto& [t, dt] : {std::pair<const Tensor*, at::ScalarType>{&token_loss, at::kFloat},
                              {&entropy, at::kFloat}, {&best_idx, at::kInt}, {&correct, at::kInt}})
    require(t->scalar_type() == dt && t->is_contiguous() && t->numel() == n_rows,
            "head_ce: per-row outputs of N elements");
  if (grad_hidden.has_value()) {
    require_fp16(*grad_hidden, "grad_hidden");
    require(grad_hidden->is_contiguous() && same_shape(*grad_hidden, n_rows, size),
            "head_ce: grad_hidden contiguous [N, H]");
  }
  require(workspace.is_cuda() && workspace.is_contiguous(), "head_ce: workspace");
  check(talm_head_ce(as<uint16_t>(hidden), hidden.stride(0), as<uint16_t>(weight),
                     weight.stride(0), as<int64_t>(targets),
                     n_rows, size, vocab, vchunk, n_grad, static_cast<int32_t>(group),
                     as<float>(token_loss), as<float>(entropy), as<int32_t>(best_idx),
                     as<int32_t>(correct), as<uint16_t>(grad_hidden), workspace.data_ptr(),
                     workspace.numel() * static_cast<int64_t>(workspace.element_size()),
                     stream_of(hidden)),
        "head_ce");
}

// Adapter g: t[:, 16g:16g+16] = x[:, xcol_g:xcol_g + k_g] A_g^T, ts = scaling_g * that;
// x fp16 (unit column stride), A_g fp16 contiguous [16, k_g] (or [k_g, 16] with a_kmajor),
// t / ts fp16 with one row stride.
void lora_down(const Tensor& x, const Tensor& a0, const OptTensor& a1, int64_t k0, int64_t k1,
               int64_t xcol0, int64_t xcol1, int64_t a_kmajor, double scaling0, double scaling1,
               const Tensor& t, const Tensor& ts) {
  require_fp16(x, "x");
  require_fp16(a0, "a0");
  require_fp16(t, "t");
  require_fp16(ts, "ts");
  require(x.dim() == 2 && t.dim() == 2 && ts.dim() == 2,
          "lora_down: x [N, *], t/ts [N, 16 * adapters] with one row stride");
  const int64_t n = x.size(0);
  const int n_adapters = a1.has_value() ? 2 : 1;
  for (int g = 0; g < n_adapters; ++g) {
    const Tensor& a = g ? *a1 : a0;
    const int64_t k = g ? k1 : k0, col = g ? xcol1 : xcol0;
    require_fp16(a, "lora A");
    const bool shape_ok = a.dim() == 2 && (a_kmajor ? (a.size(0) == k && a.size(1) == 16)
                                                    : (a.size(0) == 16 && a.size(1) == k));
    require(a.is_contiguous() && shape_ok && col + k <= x.size(1),
            "lora_down: A [16, k] ([k, 16] k-major) inside x's columns");
  }
  require(x.stride(1) == 1 && t.stride(1) == 1 && ts.stride(1) == 1 && t.stride(0) == ts.stride(0) &&
              t.size(0) == n && ts.size(0) == n && t.size(1) >= 16 * n_adapters &&
              ts.size(1) >= 16 * n_adapters,
          "lora_down: x [N, *], t/ts [N, 16 * adapters] with one row stride");
  check(talm_lora_down(as<uint16_t>(x), x.stride(0), n, k0, k1, xcol0, xcol1, as<uint16_t>(a0),
                       as<uint16_t>(a1), n_adapters, a_kmajor ? 1 : 0,
                       static_cast<float>(scaling0), static_cast<float>(scaling1),
                       as<uint16_t>(t), as<uint16_t>(ts), t.stride(0), stream_of(x)),
        "lora_down");
}

void cos_sin_rows(const OptTensor& cos, const OptTensor& sin, int64_t n, const char* message) {
  if (!cos.has_value()) return;
  for (const OptTensor* v : {&cos, &sin})
    require(v->has_value() && (*v)->is_cuda() && (*v)->scalar_type() == at::kFloat &&
                (*v)->dim() == 2 && (*v)->stride(1) == 1 && (*v)->size(0) == n &&
                (*v)->size(1) >= 128 && (*v)->stride(0) == cos->stride(0),
            message);
}

// out [N, n_out] = x W^T + bias + the adapters' ts B^T on their columns, then the rotary
// embedding (cos/sin fp32 [N, >= 128]) on the 128-column heads below rope_cols.
void qkv_lora_fwd(const Tensor& x, const Tensor& weight, const OptTensor& bias,
                  const OptTensor& ts, const OptTensor& b0, int64_t seg0_begin,
                  int64_t seg0_end, const OptTensor& b1, int64_t seg1_begin, int64_t seg1_end,
                  const OptTensor& cos, const OptTensor& sin, int64_t rope_cols,
                  const Tensor& out) {
  require_fp16(x, "x");
  require_fp16(weight, "weight");
  require_fp16(out, "out");
  require(x.dim() == 2 && weight.dim() == 2,
          "qkv_lora_fwd: x [N, H], weight [n_out, H], out [N, n_out], unit column strides");
  const int64_t n = x.size(0), size = x.size(1), n_out = weight.size(0);
  require(x.stride(1) == 1 && weight.stride(1) == 1 && out.dim() == 2 && out.stride(1) == 1 &&
              weight.size(1) == size && same_shape(out, n, n_out),
          "qkv_lora_fwd: x [N, H], weight [n_out, H], out [N, n_out], unit column strides");
  if (bias.has_value()) {
    require_fp16(*bias, "bias");
    require(bias->is_contiguous() && bias->numel() == n_out, "qkv_lora_fwd: bias [n_out]");
  }
  int n_adapters = 0;
  for (const OptTensor* b : {&b0, &b1}) {
    if (!b->has_value()) continue;
    ++n_adapters;
    require_fp16(**b, "lora B");
    require((*b)->is_contiguous() && (*b)->dim() == 2 && (*b)->size(1) == 16,
            "qkv_lora_fwd: B [segment, 16]");
  }
  if (n_adapters) {
    TORCH_CHECK_VALUE(ts.has_value(), "ts must be a CUDA float16 tensor");
    require_fp16(*ts, "ts");
    require(ts->dim() == 2 && ts->stride(1) == 1 && ts->size(0) == n &&
                ts->size(1) >= 16 * n_adapters,
            "qkv_lora_fwd: ts [N, 16 * adapters]");
  }
  cos_sin_rows(cos, sin, n, "qkv_lora_fwd: cos/sin fp32 [N, >= 128] with one row stride");
  check(talm_qkv_lora_fwd(as<uint16_t>(x), x.stride(0), n, size, as<uint16_t>(weight),
                          weight.stride(0), n_out, as<uint16_t>(bias), as<uint16_t>(ts),
                          ts.has_value() ? ts->stride(0) : 0, n_adapters, as<uint16_t>(b0),
                          seg0_begin, seg0_end, as<uint16_t>(b1), seg1_begin, seg1_end,
                          as<float>(cos), as<float>(sin), cos.has_value() ? cos->stride(0) : 0,
                          rope_cols, as<uint16_t>(out), out.stride(0), stream_of(x)),
        "qkv_lora_fwd");
}

// qkv_lora_fwd with the adapters' t = x A_g^T computed inside the same GEMM: A_g fp16 [16, H]
// contiguous, t [N, 16 * adapters] written for the backward.
void qkv_lora_fwd_down(const Tensor& x, const Tensor& weight, const OptTensor& bias,
                       const OptTensor& a0, const OptTensor& a1, double scaling0, double scaling1,
                       const OptTensor& b0, int64_t seg0_begin, int64_t seg0_end,
                       const OptTensor& b1, int64_t seg1_begin, int64_t seg1_end,
                       const OptTensor& cos, const OptTensor& sin, int64_t rope_cols,
                       const OptTensor& t, const Tensor& out) {
  require_fp16(x, "x");
  require_fp16(weight, "weight");
  require_fp16(out, "out");
  require(x.dim() == 2 && weight.dim() == 2,
          "qkv_lora_fwd_down: x [N, H], weight [n_out, H], out [N, n_out], unit column strides");
  const int64_t n = x.size(0), size = x.size(1), n_out = weight.size(0);
  require(x.stride(1) == 1 && weight.stride(1) == 1 && out.dim() == 2 && out.stride(1) == 1 &&
              weight.size(1) == size && same_shape(out, n, n_out),
          "qkv_lora_fwd_down: x [N, H], weight [n_out, H], out [N, n_out], unit column strides");
  if (bias.has_value()) {
    require_fp16(*bias, "bias");
    require(bias->is_contiguous() && bias->numel() == n_out, "qkv_lora_fwd_down: bias [n_out]");
  }
  int n_adapters = 0;
  const OptTensor* as_[2] = {&a0, &a1};
  const OptTensor* bs_[2] = {&b0, &b1};
  for (int g = 0; g < 2; ++g) {
    if (!bs_[g]->has_value()) continue;
    require(g == n_adapters && as_[g]->has_value(),
            "qkv_lora_fwd_down: adapters in order, each with its A and B");
    ++n_adapters;
    require_fp16(**bs_[g], "lora B");
    require((*bs_[g])->is_contiguous() && (*bs_[g])->dim() == 2 && (*bs_[g])->size(1) == 16,
            "qkv_lora_fwd_down: B [segment, 16]");
    require_fp16(**as_[g], "lora A");
    require((*as_[g])->is_contiguous() && same_shape(**as_[g], 16, size),
            "qkv_lora_fwd_down: A [16, H] contiguous");
  }
  if (n_adapters) {
    TORCH_CHECK_VALUE(t.has_value(), "t must be a CUDA float16 tensor");
    require_fp16(*t, "t");
    require(t->dim() == 2 && t->stride(1) == 1 && t->size(0) == n && t->size(1) >= 16 * n_adapters,
            "qkv_lora_fwd_down: t [N, 16 * adapters]");
  }
  cos_sin_rows(cos, sin, n, "qkv_lora_fwd_down: cos/sin fp32 [N, >= 128] with one row stride");
  check(talm_qkv_lora_fwd_down(
            as<uint16_t>(x), x.stride(0), n, size, as<uint16_t>(weight), weight.stride(0), n_out,
            as<uint16_t>(bias), n_adapters, as<uint16_t>(a0), as<uint16_t>(a1), size,
            static_cast<float>(scaling0), static_cast<float>(scaling1), as<uint16_t>(b0),
            seg0_begin, seg0_end, as<uint16_t>(b1), seg1_begin, seg1_end, as<float>(cos),
            as<float>(sin), cos.has_value() ? cos->stride(0) : 0, rope_cols, as<uint16_t>(t),
            t.has_value() ? t->stride(0) : 0, as<uint16_t>(out), out.stride(0), stream_of(x)),
        "qkv_lora_fwd_down");
}

// dcat [N, q + k + v] = [rope_back(dq) | rope_back(dk) | dv] (cos/sin fp32 [N, >= 128], or None
// for no rotation); every operand fp16 with unit column stride.
void qkv_bwd_prep(const Tensor& dq, const Tensor& dk, const Tensor& dv, const OptTensor& cos,
                  const OptTensor& sin, const Tensor& dcat) {
  require(dcat.dim() == 2, "qkv_bwd_prep: dcat [N, columns] with unit column stride");
  const int64_t n = dcat.size(0);
  for (const auto& [v, name] : {std::pair<const Tensor*, const char*>{&dq, "dq"}, {&dk, "dk"},
                                {&dv, "dv"}, {&dcat, "dcat"}}) {
    require_fp16(*v, name);
    TORCH_CHECK_VALUE(v->dim() == 2 && v->stride(1) == 1 && v->size(0) == n, "qkv_bwd_prep: ",
                      name, " [N, columns] with unit column stride");
  }
  require(dcat.size(1) == dq.size(1) + dk.size(1) + dv.size(1),
          "qkv_bwd_prep: dcat holds q, k and v");
  cos_sin_rows(cos, sin, n, "qkv_bwd_prep: cos/sin fp32 [N, >= 128] with one row stride");
  check(talm_qkv_bwd_prep(as<uint16_t>(dq), dq.stride(0), as<uint16_t>(dk), dk.stride(0),
                          as<uint16_t>(dv), dv.stride(0), n, dq.size(1), dk.size(1), dv.size(1),
                          as<float>(cos), as<float>(sin), cos.has_value() ? cos->stride(0) : 0,
                          as<uint16_t>(dcat), dcat.stride(0), stream_of(dcat)),
        "qkv_bwd_prep");
}

// dx [N, H] = dcat [N, n_out] W + u [N, r] A, from weight_t = W^T [H, >= n_out] and a_t = A^T
// [H, r] (the adapters side by side); fp16, unit column strides.
void qkv_lora_bwd_dx(const Tensor& dcat, const Tensor& weight_t, const OptTensor& u,
                     const OptTensor& a_t, const Tensor& dx) {
  for (const auto& [v, name] : {std::pair<const Tensor*, const char*>{&dcat, "dcat"},
                                {&weight_t, "weight_t"}, {&dx, "dx"}}) {
    require_fp16(*v, name);
    TORCH_CHECK_VALUE(v->dim() == 2 && v->stride(1) == 1, "qkv_lora_bwd_dx: ", name,
                      " unit column stride");
  }
  const int64_t n = dcat.size(0), n_out = dcat.size(1), size = weight_t.size(0);
  require(weight_t.size(1) >= n_out && same_shape(dx, n, size),
          "qkv_lora_bwd_dx: weight_t [H, >= n_out], dx [N, H]");
  int64_t rank = 0;
  if (u.has_value()) {
    require_fp16(*u, "u");
    TORCH_CHECK_VALUE(a_t.has_value(), "a_t must be a CUDA float16 tensor");
    require_fp16(*a_t, "a_t");
    require(u->dim() == 2 && a_t->dim() == 2, "qkv_lora_bwd_dx: u [N, r], a_t [H, r]");
    rank = u->size(1);
    require(u->stride(1) == 1 && a_t->stride(1) == 1 && u->size(0) == n &&
                same_shape(*a_t, size, rank),
            "qkv_lora_bwd_dx: u [N, r], a_t [H, r]");
  }
  check(talm_qkv_lora_bwd_dx(as<uint16_t>(dcat), dcat.stride(0), n, n_out,
                             as<uint16_t>(weight_t), weight_t.stride(0), size, as<uint16_t>(u),
                             u.has_value() ? u->stride(0) : 0, rank, as<uint16_t>(a_t),
                             a_t.has_value() ? a_t->stride(0) : 0, as<uint16_t>(dx),
                             dx.stride(0), stream_of(dcat)),
        "qkv_lora_bwd_dx");
}

// fp32 dA_g [16, H] = u_g^T x, dB_g [seg_g, 16] = scaling_g dy[:, lo_g:lo_g+seg_g]^T t_g.
void lora_wgrad(const Tensor& x, const Tensor& dy, const Tensor& u, const Tensor& t, int64_t lo0,
                int64_t seg0, double scaling0, const Tensor& da0, const Tensor& db0, int64_t lo1,
                int64_t seg1, double scaling1, const OptTensor& da1, const OptTensor& db1,
                const Tensor& workspace) {
  for (const auto& [v, name] : {std::pair<const Tensor*, const char*>{&x, "x"}, {&dy, "dy"},
                                {&u, "u"}, {&t, "t"}}) {
    require_fp16(*v, name);
    TORCH_CHECK_VALUE(v->dim() == 2 && v->stride(1) == 1, "lora_wgrad: ", name,
                      " unit column stride");
  }
  const int64_t n = x.size(0), size = x.size(1);
  const bool two = da1.has_value();
  TORCH_CHECK_VALUE(!two || db1.has_value(), "lora_wgrad: dB fp32 [segment, 16]");
  for (int g = 0; g < (two ? 2 : 1); ++g) {
    const Tensor& da = g ? *da1 : da0;
    const Tensor& db = g ? *db1 : db0;
    const int64_t seg = g ? seg1 : seg0;
    require(da.is_cuda() && da.scalar_type() == at::kFloat && da.is_contiguous() &&
                same_shape(da, 16, size),
            "lora_wgrad: dA fp32 [16, H]");
    require(db.is_cuda() && db.scalar_type() == at::kFloat && db.is_contiguous() &&
                same_shape(db, seg, 16),
            "lora_wgrad: dB fp32 [segment, 16]");
  }
  require(workspace.is_cuda() && workspace.is_contiguous(), "lora_wgrad: workspace");
  if (n == 0) {  // no tokens: zero gradients, no launch
    da0.zero_();
    db0.zero_();
    if (two) {
      da1->zero_();
      db1->zero_();
    }
    return;
  }
  check(talm_lora_wgrad(as<uint16_t>(x), x.stride(0), as<uint16_t>(dy), dy.stride(0),
                        as<uint16_t>(u), u.stride(0), as<uint16_t>(t), t.stride(0), n, size,
                        two ? 2 : 1, lo0, seg0, static_cast<float>(scaling0), as<float>(da0),
                        as<float>(db0), lo1, seg1, static_cast<float>(scaling1), as<float>(da1),
                        as<float>(db1), workspace.data_ptr(),
                        workspace.numel() * static_cast<int64_t>(workspace.element_size()),
                        stream_of(x)),
        "lora_wgrad");
}


// ------------------------------------------------------------------------------------------
// Variable-length causal GQA attention
// ------------------------------------------------------------------------------------------
void attn_heads(const Tensor& t, const char* name, int64_t n_tokens, int64_t heads) {
  require_fp16(t, name);
  TORCH_CHECK_VALUE(t.dim() == 3 && t.size(0) == n_tokens && t.size(1) == heads &&
                        t.size(2) == 128 && t.stride(2) == 1,
                    "attn: ", name, " must be an fp16 [N, heads, 128] view with unit column stride");
}

void attn_cu(const Tensor& cu, const Tensor& q) {
  require(cu.is_cuda() && cu.scalar_type() == at::kInt && cu.dim() == 1 && cu.numel() >= 1 &&
              cu.is_contiguous() && cu.device() == q.device(),
          "attn: cu_seqlens int32 [n_seqs + 1] on the tensors' device");
}

// q [N, Hq, 128], k / v [N, Hkv, 128] fp16 views; out [N, Hq, 128]; lse f32 [Hq, N].
void attn_fwd(const Tensor& q, const Tensor& k, const Tensor& v, const Tensor& cu,
              int64_t max_seqlen, double scale, const Tensor& out, const Tensor& lse) {
  require(q.dim() == 3 && k.dim() == 3, "attn: q [N, Hq, 128], k / v [N, Hkv, 128]");
  const int64_t n = q.size(0), hq = q.size(1), hkv = k.size(1);
  attn_heads(q, "q", n, hq);
  attn_heads(k, "k", n, hkv);
  attn_heads(v, "v", n, hkv);
  attn_heads(out, "out", n, hq);
  attn_cu(cu, q);
  require(lse.is_cuda() && lse.scalar_type() == at::kFloat && lse.is_contiguous() &&
              same_shape(lse, hq, n),
          "attn_fwd: lse float32 [Hq, N]");
  check(talm_attn_fwd(as<uint16_t>(q), q.stride(0), q.stride(1), as<uint16_t>(k), k.stride(0),
                      k.stride(1), as<uint16_t>(v), v.stride(0), v.stride(1), as<int32_t>(cu),
                      static_cast<int32_t>(cu.numel() - 1), static_cast<int32_t>(max_seqlen), n,
                      static_cast<int32_t>(hq), static_cast<int32_t>(hkv), 128,
                      static_cast<float>(scale), as<uint16_t>(out), out.stride(0), out.stride(1),
                      as<float>(lse), stream_of(q)),
        "attn_fwd");
}

// The attention backward; with cos / sin (fp32 [N, >= 128], one row stride) q and k are the
// rotated projections and dq / dk come out rotated back (the rotary backward folded in).
void attn_bwd_any(const Tensor& q, const Tensor& k, const Tensor& v, const Tensor& out,
                  const Tensor& dout, const Tensor& lse, const Tensor& cu, int64_t max_seqlen,
                  double scale, const OptTensor& cos, const OptTensor& sin, const Tensor& dq,
                  const Tensor& dk, const Tensor& dv, const Tensor& workspace) {
  require(q.dim() == 3 && k.dim() == 3, "attn: q [N, Hq, 128], k / v [N, Hkv, 128]");
  const int64_t n = q.size(0), hq = q.size(1), hkv = k.size(1);
  attn_heads(q, "q", n, hq);
  attn_heads(k, "k", n, hkv);
  attn_heads(v, "v", n, hkv);
  attn_heads(out, "out", n, hq);
  attn_heads(dout, "dout", n, hq);
  attn_heads(dq, "dq", n, hq);
  attn_heads(dk, "dk", n, hkv);
  attn_heads(dv, "dv", n, hkv);
  attn_cu(cu, q);
  require(lse.is_cuda() && lse.scalar_type() == at::kFloat && lse.is_contiguous() &&
              same_shape(lse, hq, n),
          "attn_bwd: lse float32 [Hq, N]");
  require(workspace.is_cuda() && workspace.is_contiguous(), "attn_bwd: workspace");
  const int64_t ws_bytes = workspace.numel() * static_cast<int64_t>(workspace.element_size());
  if (!cos.has_value()) {
    check(talm_attn_bwd(as<uint16_t>(q), q.stride(0), q.stride(1), as<uint16_t>(k), k.stride(0),
                        k.stride(1), as<uint16_t>(v), v.stride(0), v.stride(1), as<uint16_t>(out),
                        out.stride(0), out.stride(1), as<uint16_t>(dout), dout.stride(0),
                        dout.stride(1), as<float>(lse), as<int32_t>(cu),
                        static_cast<int32_t>(cu.numel() - 1), static_cast<int32_t>(max_seqlen), n,
                        static_cast<int32_t>(hq), static_cast<int32_t>(hkv), 128,
                        static_cast<float>(scale), as<uint16_t>(dq), dq.stride(0), dq.stride(1),
                        as<uint16_t>(dk), dk.stride(0), dk.stride(1), as<uint16_t>(dv),
                        dv.stride(0), dv.stride(1), workspace.data_ptr(), ws_bytes,
                        stream_of(q)),
          "attn_bwd");
    return;
  }
  cos_sin_rows(cos, sin, n, "attn_bwd_rope: cos/sin fp32 [N, >= 128] with one row stride");
  check(talm_attn_bwd_rope(as<uint16_t>(q), q.stride(0), q.stride(1), as<uint16_t>(k),
                           k.stride(0), k.stride(1), as<uint16_t>(v), v.stride(0), v.stride(1),
                           as<uint16_t>(out), out.stride(0), out.stride(1), as<uint16_t>(dout),
                           dout.stride(0), dout.stride(1), as<float>(lse), as<int32_t>(cu),
                           static_cast<int32_t>(cu.numel() - 1),
                           static_cast<int32_t>(max_seqlen), n, static_cast<int32_t>(hq),
                           static_cast<int32_t>(hkv), 128, static_cast<float>(scale),
                           as<float>(cos), as<float>(sin), cos->stride(0), as<uint16_t>(dq),
                           dq.stride(0), dq.stride(1), as<uint16_t>(dk), dk.stride(0),
                           dk.stride(1), as<uint16_t>(dv), dv.stride(0), dv.stride(1),
                           workspace.data_ptr(), ws_bytes, stream_of(q)),
        "attn_bwd_rope");
}

void attn_bwd(const Tensor& q, const Tensor& k, const Tensor& v, const Tensor& out,
              const Tensor& dout, const Tensor& lse, const Tensor& cu, int64_t max_seqlen,
              double scale, const Tensor& dq, const Tensor& dk, const Tensor& dv,
              const Tensor& workspace) {
  attn_bwd_any(q, k, v, out, dout, lse, cu, max_seqlen, scale, std::nullopt, std::nullopt, dq,
               dk, dv, workspace);
}

void attn_bwd_rope(const Tensor& q, const Tensor& k, const Tensor& v, const Tensor& out,
                   const Tensor& dout, const Tensor& lse, const Tensor& cu, int64_t max_seqlen,
                   double scale, const Tensor& cos, const Tensor& sin, const Tensor& dq,
                   const Tensor& dk, const Tensor& dv, const Tensor& workspace) {
  attn_bwd_any(q, k, v, out, dout, lse, cu, max_seqlen, scale, cos, sin, dq, dk, dv, workspace);
}

// ------------------------------------------------------------------------------------------
// LoRA adapters: fp16 copies and the fused AdamW step over a device table (9 int64 per tensor,
// layout in include/talm.h; the addresses in it are the caller's to keep alive).
// ------------------------------------------------------------------------------------------
void adapter_table(const Tensor& table, int64_t n_tensors, const Tensor& out, const char* what) {
  TORCH_CHECK_VALUE(table.is_cuda() && table.scalar_type() == at::kLong && table.is_contiguous() &&
                        table.numel() >= 9 * n_tensors && out.device() == table.device(),
                    what, ": table int64 [n_tensors, 9] on the copies' device");
  require_fp16(out, "out");
  require(out.is_contiguous(), "lora adapters: out must be contiguous");
}

void lora_mirror(const Tensor& table, int64_t n_tensors, int64_t max_numel, const Tensor& out) {
  adapter_table(table, n_tensors, out, "lora_mirror");
  check(talm_lora_mirror(as<int64_t>(table), static_cast<int32_t>(n_tensors), max_numel,
                         as<uint16_t>(out), stream_of(out)),
        "lora_mirror");
}

void lora_adamw(const Tensor& table, int64_t n_tensors, int64_t max_numel, double lr,
                double beta1, double beta2, double eps, double weight_decay,
                const Tensor& step_in, const Tensor& step_out, const OptTensor& grad_scale,
                const OptTensor& found_inf, const Tensor& out) {
  adapter_table(table, n_tensors, out, "lora_adamw");
  for (const Tensor* t : {&step_in, &step_out})
    require(t->is_cuda() && t->scalar_type() == at::kFloat && t->numel() == 1 &&
                t->device() == out.device(),
            "lora_adamw: step counters float32 [1] on the copies' device");
  require(step_in.data_ptr() != step_out.data_ptr(), "lora_adamw: step_in and step_out alias");
  for (const OptTensor* t : {&grad_scale, &found_inf})
    if (t->has_value())
      require((*t)->is_cuda() && (*t)->scalar_type() == at::kFloat && (*t)->numel() == 1 &&
                  (*t)->device() == out.device(),
              "lora_adamw: grad_scale / found_inf float32 [1] on the copies' device");
  check(talm_lora_adamw(as<int64_t>(table), static_cast<int32_t>(n_tensors), max_numel,
                        static_cast<float>(lr), static_cast<float>(beta1),
                        static_cast<float>(beta2), static_cast<float>(eps),
                        static_cast<float>(weight_decay), as<float>(step_in),
                        as<float>(step_out), as<float>(grad_scale), as<float>(found_inf),
                        as<uint16_t>(out), stream_of(out)),
        "lora_adamw");
}

// stats float32 [4] = {found_inf, inv_scale, clip coefficient, norm} of the table's gradients.
void lora_grad_norm(const Tensor& table, int64_t n_tensors, int64_t max_numel, const Tensor& scale,
                    double max_norm, const Tensor& workspace, const Tensor& stats) {
  require(table.is_cuda() && table.scalar_type() == at::kLong && table.is_contiguous() &&
              table.numel() >= n_tensors * 9,
          "lora_grad_norm: table int64 [n_tensors, 9]");
  for (const Tensor* t : {&scale, &stats})
    require(t->is_cuda() && t->scalar_type() == at::kFloat && t->is_contiguous() &&
                t->device() == table.device(),
            "lora_grad_norm: scale and stats float32 on the table's device");
  require(scale.numel() == 1 && stats.numel() == 4, "lora_grad_norm: scale [1], stats [4]");
  require(workspace.is_cuda() && workspace.is_contiguous() && workspace.device() == table.device(),
          "lora_grad_norm: workspace");
  check(talm_lora_grad_norm(as<int64_t>(table), static_cast<int32_t>(n_tensors), max_numel,
                            as<float>(scale), static_cast<float>(max_norm), workspace.data_ptr(),
                            workspace.numel() * static_cast<int64_t>(workspace.element_size()),
                            as<float>(stats), stream_of(stats)),
        "lora_grad_norm");
}

// lora_adamw with the gradients unscaled and clipped by grad_mul = stats[1:3] and skipped on
// found_inf = stats[0:1] (lora_grad_norm's outputs).
void lora_adamw_clipped(const Tensor& table, int64_t n_tensors, int64_t max_numel, double lr,
                        double beta1, double beta2, double eps, double weight_decay,
                        const Tensor& step_in, const Tensor& step_out, const Tensor& found_inf,
                        const Tensor& grad_mul, const Tensor& out) {
  adapter_table(table, n_tensors, out, "lora_adamw_clipped");
  for (const Tensor* t : {&step_in, &step_out, &found_inf, &grad_mul})
    require(t->is_cuda() && t->scalar_type() == at::kFloat && t->is_contiguous() &&
                t->device() == out.device(),
            "lora_adamw_clipped: counters, inf flag and multipliers float32 on the copies' "
            "device");
  require(step_in.numel() == 1 && step_out.numel() == 1 && found_inf.numel() == 1 &&
              grad_mul.numel() == 2 && step_in.data_ptr() != step_out.data_ptr(),
          "lora_adamw_clipped: step counters [1] (distinct), found_inf [1], grad_mul [2]");
  check(talm_lora_adamw_clipped(as<int64_t>(table), static_cast<int32_t>(n_tensors), max_numel,
                                static_cast<float>(lr), static_cast<float>(beta1),
                                static_cast<float>(beta2), static_cast<float>(eps),
                                static_cast<float>(weight_decay), as<float>(step_in),
                                as<float>(step_out), as<float>(found_inf), as<float>(grad_mul),
                                as<uint16_t>(out), stream_of(out)),
        "lora_adamw_clipped");
}

// ------------------------------------------------------------------------------------------
// Products on the NF4 form of W [rows, cols] (dequantized inside the GEMM): out = x W^T
// (transpose false: x [N, cols], out [N, rows]) or out = x W (transpose true: x [N, rows],
// out [N, cols]); scale holds the blocks' decoded absmax (nf4_block_scales), the workspace the
// split-K partials (talm_nf4_gemm_workspace bytes).
// ------------------------------------------------------------------------------------------
void nf4_block_scales(const Tensor& absmax8, const Tensor& code, const Tensor& absmax2,
                      const Tensor& offset2, int64_t qblock2, const Tensor& out) {
  for (const Tensor* t : {&absmax8, &code, &absmax2, &offset2, &out})
    require(t->is_cuda() && t->is_contiguous() && t->device() == out.device(),
            "nf4_block_scales: operands contiguous on one device");
  require(absmax8.scalar_type() == at::kByte && code.scalar_type() == at::kFloat &&
              absmax2.scalar_type() == at::kFloat && offset2.scalar_type() == at::kFloat &&
              out.scalar_type() == at::kFloat,
          "nf4_block_scales: absmax8 uint8, code / absmax2 / offset2 / out float32");
  const int64_t n = out.numel();
  require(qblock2 > 0 && absmax8.numel() >= n && code.numel() >= 256 &&
              absmax2.numel() >= (n + qblock2 - 1) / qblock2 && offset2.numel() >= absmax2.numel(),
          "nf4_block_scales: the inputs do not cover out's blocks");
  check(talm_nf4_block_scales(as<uint8_t>(absmax8), as<float>(code), as<float>(absmax2),
                              as<float>(offset2), n, static_cast<int32_t>(qblock2),
                              as<float>(out), stream_of(out)),
        "nf4_block_scales");
}

void nf4_gemm(const Tensor& x, const Tensor& packed, const Tensor& scale, int64_t rows,
              int64_t cols, bool transpose, int64_t blocksize, const Tensor& out,
              const Tensor& workspace) {
  require_fp16(x, "x");
  require_fp16(out, "out");
  const int64_t k = transpose ? rows : cols, n_out = transpose ? cols : rows;
  require(x.dim() == 2 && out.dim() == 2 && x.stride(1) == 1 && out.stride(1) == 1 &&
              x.size(1) == k && out.size(0) == x.size(0) && out.size(1) == n_out,
          "nf4_gemm: x [N, K], out [N, n_out] with unit column stride (K, n_out = cols, rows, "
          "or rows, cols with transpose)");
  const int64_t n = x.size(0);
  for (const Tensor* t : {&packed, &scale, &workspace})
    require(t->is_cuda() && t->is_contiguous() && t->device() == x.device(),
            "nf4_gemm: packed, scale and workspace contiguous on x's device");
  require(packed.scalar_type() == at::kByte && scale.scalar_type() == at::kFloat,
          "nf4_gemm: packed uint8, scale float32");
  require(blocksize > 0 && packed.numel() >= rows * cols / 2 &&
              scale.numel() >= rows * cols / blocksize,
          "nf4_gemm: packed / scale do not cover [rows, cols]");
  check(talm_nf4_gemm(as<uint16_t>(x), x.stride(0), n, as<uint8_t>(packed), as<float>(scale),
                      rows, cols, transpose ? 1 : 0, static_cast<int32_t>(blocksize),
                      as<uint16_t>(out), out.stride(0),
                      workspace.numel() ? workspace.data_ptr() : nullptr,
                      workspace.numel() * workspace.element_size(), stream_of(x)),
        "nf4_gemm");
}

// The MLP's long products leaving their fp32 K-part partials for the fused norm launches
// below: partials float32 [parts, m, n] (parts from talm_gemm_splitk_parts / talm_nf4_gemm_parts).
void gemm_splitk_partials(const Tensor& a, const Tensor& b, const Tensor& partials) {
  require_fp16(a, "a");
  require_fp16(b, "b");
  require(a.dim() == 2 && b.dim() == 2 && a.stride(1) == 1 && b.stride(1) == 1,
          "gemm_splitk_partials: a [m, k], b [n, k] with unit column stride");
  const int64_t m = a.size(0), k = a.size(1), n = b.size(0);
  require(b.size(1) == k, "gemm_splitk_partials: a [m, k], b [n, k]");
  require(partials.is_cuda() && partials.scalar_type() == at::kFloat &&
              partials.is_contiguous() && partials.device() == a.device() &&
              partials.numel() == talm_gemm_splitk_parts(m, n, k) * m * n,
          "gemm_splitk_partials: partials float32 [parts, m, n]");
  check(talm_gemm_splitk_partials(as<uint16_t>(a), a.stride(0), as<uint16_t>(b), b.stride(0), m,
                                  n, k, as<float>(partials), partials.numel() * 4, stream_of(a)),
        "gemm_splitk_partials");
}

void nf4_gemm_partials(const Tensor& x, const Tensor& packed, const Tensor& scale, int64_t rows,
                       int64_t cols, bool transpose, int64_t blocksize, const Tensor& partials) {
  require_fp16(x, "x");
  const int64_t k = transpose ? rows : cols, n_out = transpose ? cols : rows;
  require(x.dim() == 2 && x.stride(1) == 1 && x.size(1) == k,
          "nf4_gemm_partials: x [N, K] with unit column stride");
  const int64_t n = x.size(0);
  for (const Tensor* t : {&packed, &scale})
    require(t->is_cuda() && t->is_contiguous() && t->device() == x.device(),
            "nf4_gemm_partials: packed and scale contiguous on x's device");
  require(packed.scalar_type() == at::kByte && scale.scalar_type() == at::kFloat,
          "nf4_gemm_partials: packed uint8, scale float32");
  require(blocksize > 0 && packed.numel() >= rows * cols / 2 &&
              scale.numel() >= rows * cols / blocksize,
          "nf4_gemm_partials: packed / scale do not cover [rows, cols]");
  require(partials.is_cuda() && partials.scalar_type() == at::kFloat &&
              partials.is_contiguous() && partials.device() == x.device() &&
              partials.numel() == talm_nf4_gemm_parts(n, rows, cols, transpose ? 1 : 0) * n * n_out,
          "nf4_gemm_partials: partials float32 [parts, N, n_out]");
  check(talm_nf4_gemm_partials(as<uint16_t>(x), x.stride(0), n, as<uint8_t>(packed),
                               as<float>(scale), rows, cols, transpose ? 1 : 0,
                               static_cast<int32_t>(blocksize), as<float>(partials),
                               partials.numel() * 4, stream_of(x)),
        "nf4_gemm_partials");
}

// partials float32 [parts, N, H]; resid, sum_out float32 [N, H]; h, xhat fp16 [N, H]; rstd [N].
void splitk_add_rmsnorm(const Tensor& partials, const Tensor& resid, const Tensor& weight,
                        double eps, const Tensor& sum_out, const Tensor& h, const Tensor& xhat,
                        const Tensor& rstd) {
  require(partials.is_cuda() && partials.scalar_type() == at::kFloat && partials.dim() == 3 &&
              partials.is_contiguous(),
          "splitk_add_rmsnorm: partials float32 [parts, N, H]");
  const int64_t n = partials.size(1), hd = partials.size(2);
  for (const Tensor* t : {&resid, &sum_out})
    require(t->is_cuda() && t->scalar_type() == at::kFloat && t->is_contiguous() &&
                same_shape(*t, n, hd),
            "splitk_add_rmsnorm: resid and sum_out float32 [N, H]");
  for (const Tensor* t : {&h, &xhat})
    require(t->is_cuda() && t->scalar_type() == at::kHalf && t->is_contiguous() &&
                same_shape(*t, n, hd),
            "splitk_add_rmsnorm: h and xhat float16 [N, H]");
  require(weight.is_contiguous() && weight.numel() == hd, "splitk_add_rmsnorm: weight [H]");
  require(rstd.scalar_type() == at::kFloat && rstd.is_contiguous() && rstd.numel() == n,
          "splitk_add_rmsnorm: rstd float32 [N]");
  check(talm_splitk_add_rmsnorm(as<float>(partials), static_cast<int32_t>(partials.size(0)),
                                as<float>(resid), weight.data_ptr(),
                                dtype_code(weight.scalar_type()), static_cast<float>(eps), n, hd,
                                as<float>(sum_out), as<uint16_t>(h), as<uint16_t>(xhat),
                                as<float>(rstd), stream_of(resid)),
        "splitk_add_rmsnorm");
}

// partials float32 [parts, N, H] (dy); xhat fp16 [N, H]; rstd [N]; ds float32 [N, H] or None;
// dx float32, dbranch fp16 [N, H].
void splitk_rmsnorm_bwd(const Tensor& partials, const Tensor& xhat, const Tensor& rstd,
                        const Tensor& weight, const OptTensor& ds, const Tensor& dx,
                        const Tensor& dbranch) {
  require(partials.is_cuda() && partials.scalar_type() == at::kFloat && partials.dim() == 3 &&
              partials.is_contiguous(),
          "splitk_rmsnorm_bwd: partials float32 [parts, N, H]");
  const int64_t n = partials.size(1), hd = partials.size(2);
  require(dx.is_cuda() && dx.scalar_type() == at::kFloat && dx.is_contiguous() &&
              same_shape(dx, n, hd) &&
              (!ds.has_value() || (ds->is_cuda() && ds->scalar_type() == at::kFloat &&
                                   ds->is_contiguous() && same_shape(*ds, n, hd))),
          "splitk_rmsnorm_bwd: dx (and ds) float32 [N, H]");
  for (const Tensor* t : {&xhat, &dbranch})
    require(t->is_cuda() && t->scalar_type() == at::kHalf && t->is_contiguous() &&
                same_shape(*t, n, hd),
            "splitk_rmsnorm_bwd: xhat and dbranch float16 [N, H]");
  require(weight.is_contiguous() && weight.numel() == hd, "splitk_rmsnorm_bwd: weight [H]");
  require(rstd.scalar_type() == at::kFloat && rstd.is_contiguous() && rstd.numel() == n,
          "splitk_rmsnorm_bwd: rstd float32 [N]");
  check(talm_splitk_rmsnorm_bwd(as<float>(partials), static_cast<int32_t>(partials.size(0)),
                                as<uint16_t>(xhat), as<float>(rstd), weight.data_ptr(),
                                dtype_code(weight.scalar_type()), as<float>(ds), n, hd,
                                as<float>(dx), as<uint16_t>(dbranch), stream_of(dx)),
        "splitk_rmsnorm_bwd");
}

// ------------------------------------------------------------------------------------------
// Plain fp16 GEMMs on hipBLASLt with cached plans.
// ------------------------------------------------------------------------------------------
struct GemmKey {
  int device;
  int64_t m, n, k, lda, ldb, ldd;
  int trans_a, trans_b, bias;
  bool operator==(const GemmKey& o) const {
    return device == o.device && m == o.m && n == o.n && k == o.k && lda == o.lda &&
           ldb == o.ldb && ldd == o.ldd && trans_a == o.trans_a && trans_b == o.trans_b &&
           bias == o.bias;
  }
};

struct GemmKeyHash {
  size_t operator()(const GemmKey& key) const {
    size_t h = static_cast<size_t>(key.device);
    for (int64_t v : {key.m, key.n, key.k, key.lda, key.ldb, key.ldd,
                      static_cast<int64_t>(key.trans_a * 4 + key.trans_b * 2 + key.bias)})
      h = h * 1000003u ^ static_cast<size_t>(v);
    return h;
  }
};

struct GemmPlan {
  hipblasLtMatmulDesc_t desc = nullptr;
  hipblasLtMatrixLayout_t a = nullptr, b = nullptr, d = nullptr;
  hipblasLtMatmulAlgo_t algo{};
  size_t workspace = 0;
  int generation = 0;  // of the measured table it was planned under
};

// Measured solutions (gemm_tuning.py): for products of this layout, m and k with n in
// [n_lo, n_hi), hipBLASLt's solution `index`, validated against the exact shape when planned
// (hipBLASLt's heuristic otherwise). Installing a table re-plans every shape at its next call.
struct TunedRange {
  int64_t trans_a, trans_b, m, k, n_lo, n_hi, index;
};
std::mutex tuned_mutex;
std::vector<TunedRange> tuned_table;
std::atomic<int> tuned_generation{0};

int64_t tuned_index(const GemmKey& key) {
  std::lock_guard<std::mutex> lock(tuned_mutex);
  for (const TunedRange& r : tuned_table)
    if (r.trans_a == key.trans_a && r.trans_b == key.trans_b && r.m == key.m && r.k == key.k &&
        key.n >= r.n_lo && key.n < r.n_hi)
      return r.index;
  return -1;
}

void lt_check(hipblasStatus_t status, const char* what) {
  TORCH_CHECK(status == HIPBLAS_STATUS_SUCCESS, "gemm: hipBLASLt ", what, " failed (status ",
              static_cast<int>(status), ")");
}

void destroy(GemmPlan& p) {
  if (p.a) hipblasLtMatrixLayoutDestroy(p.a);
  if (p.b) hipblasLtMatrixLayoutDestroy(p.b);
  if (p.d) hipblasLtMatrixLayoutDestroy(p.d);
  if (p.desc) hipblasLtMatmulDescDestroy(p.desc);
  p = GemmPlan{};
}

// Plans per thread (forward launches come from the main thread, backward launches from the
// autograd thread): a plan's bias pointer is set per call without a lock. Bounded: the token
// count of a packed batch changes every step, so shapes keep arriving.
struct PlanCache {
  std::unordered_map<GemmKey, GemmPlan, GemmKeyHash> plans;
  ~PlanCache() {
    for (auto& kv : plans) destroy(kv.second);
  }
};
thread_local PlanCache plan_cache;
constexpr size_t kMaxPlans = 2048;

// D [m, n] = op(A) [m, k] op(B) [k, n] in hipBLASLt's column-major terms, fp16 in and out, fp32
// accumulation; op(A) = A^T when trans_a (A stored k x m), else A (stored m x k); op(B) = B^T
// when trans_b (B stored n x k), else B (stored k x n).
// Descriptor and layouts of a plan (no algorithm yet).
void describe(const GemmKey& key, GemmPlan& p) {
  lt_check(hipblasLtMatmulDescCreate(&p.desc, HIPBLAS_COMPUTE_32F, HIP_R_32F), "descriptor");
  const hipblasOperation_t op_a = key.trans_a ? HIPBLAS_OP_T : HIPBLAS_OP_N;
  const hipblasOperation_t op_b = key.trans_b ? HIPBLAS_OP_T : HIPBLAS_OP_N;
  lt_check(hipblasLtMatmulDescSetAttribute(p.desc, HIPBLASLT_MATMUL_DESC_TRANSA, &op_a,
                                           sizeof(op_a)), "transa");
  lt_check(hipblasLtMatmulDescSetAttribute(p.desc, HIPBLASLT_MATMUL_DESC_TRANSB, &op_b,
                                           sizeof(op_b)), "transb");
  if (key.bias) {
    const hipblasLtEpilogue_t epilogue = HIPBLASLT_EPILOGUE_BIAS;
    const hipDataType bias_type = HIP_R_16F;
    lt_check(hipblasLtMatmulDescSetAttribute(p.desc, HIPBLASLT_MATMUL_DESC_EPILOGUE, &epilogue,
                                             sizeof(epilogue)), "epilogue");
    lt_check(hipblasLtMatmulDescSetAttribute(p.desc, HIPBLASLT_MATMUL_DESC_BIAS_DATA_TYPE,
                                             &bias_type, sizeof(bias_type)), "bias type");
  }
  lt_check(hipblasLtMatrixLayoutCreate(&p.a, HIP_R_16F, key.trans_a ? key.k : key.m,
                                       key.trans_a ? key.m : key.k, key.lda), "layout A");
  lt_check(hipblasLtMatrixLayoutCreate(&p.b, HIP_R_16F, key.trans_b ? key.n : key.k,
                                       key.trans_b ? key.k : key.n, key.ldb), "layout B");
  lt_check(hipblasLtMatrixLayoutCreate(&p.d, HIP_R_16F, key.m, key.n, key.ldd), "layout D");
}

// The measured table's solution for `key` when hipBLASLt confirms it supports this product.
bool tuned_algo(const GemmKey& key, hipblasLtHandle_t handle, size_t workspace_limit,
                GemmPlan& p) {
  const int64_t index = tuned_index(key);
  if (index < 0) return false;
  std::vector<int> ids{static_cast<int>(index)};
  std::vector<hipblasLtMatmulHeuristicResult_t> found;
  if (hipblaslt_ext::getAlgosFromIndex(handle, ids, found) != HIPBLAS_STATUS_SUCCESS ||
      found.empty())
    return false;
  const float alpha = 1.f, beta = 0.f;
  size_t workspace = 0;
  if (hipblaslt_ext::matmulIsAlgoSupported(handle, p.desc, &alpha, p.a, p.b, &beta, p.d, p.d,
                                           found[0].algo, workspace) != HIPBLAS_STATUS_SUCCESS ||
      workspace > workspace_limit)
    return false;
  p.algo = found[0].algo;
  p.workspace = workspace;
  return true;
}

const GemmPlan& plan_for(const GemmKey& key, hipblasLtHandle_t handle, size_t workspace_limit) {
  const int generation = tuned_generation.load();
  auto it = plan_cache.plans.find(key);
  if (it != plan_cache.plans.end()) {
    if (it->second.generation == generation) return it->second;
    destroy(it->second);
    plan_cache.plans.erase(it);
  }
  if (plan_cache.plans.size() >= kMaxPlans) {
    for (auto& kv : plan_cache.plans) destroy(kv.second);
    plan_cache.plans.clear();
  }
  GemmPlan p;
  p.generation = generation;
  try {
    describe(key, p);
    if (tuned_algo(key, handle, workspace_limit, p))
      return plan_cache.plans.emplace(key, p).first->second;
    hipblasLtMatmulPreference_t pref = nullptr;
    lt_check(hipblasLtMatmulPreferenceCreate(&pref), "preference");
    const uint64_t limit = workspace_limit;
    hipblasStatus_t st = hipblasLtMatmulPreferenceSetAttribute(
        pref, HIPBLASLT_MATMUL_PREF_MAX_WORKSPACE_BYTES, &limit, sizeof(limit));
    hipblasLtMatmulHeuristicResult_t result{};
    int found = 0;
    if (st == HIPBLAS_STATUS_SUCCESS)
      st = hipblasLtMatmulAlgoGetHeuristic(handle, p.desc, p.a, p.b, p.d, p.d, pref, 1, &result,
                                           &found);
    hipblasLtMatmulPreferenceDestroy(pref);
    lt_check(st, "heuristic");
    TORCH_CHECK(found > 0, "gemm: hipBLASLt has no algorithm for m ", key.m, " n ", key.n, " k ",
                key.k);
    p.algo = result.algo;
    p.workspace = result.workspaceSize;
  } catch (...) {
    destroy(p);
    throw;
  }
  return plan_cache.plans.emplace(key, p).first->second;
}

// D = op(A) op(B) (+ bias per row of D) (+ beta D) on the stream of `ref`.
void run_gemm(const GemmKey& key, const void* a, const void* b, const void* bias, void* d,
              float beta, const Tensor& ref) {
  hipblasLtHandle_t handle = at::cuda::getCurrentCUDABlasLtHandle();
  void* workspace = at::cuda::getCUDABlasLtWorkspace();
  const size_t workspace_size = at::cuda::getCUDABlasLtWorkspaceSize();
  const GemmPlan& p = plan_for(key, handle, workspace_size);
  if (key.bias)
    lt_check(hipblasLtMatmulDescSetAttribute(p.desc, HIPBLASLT_MATMUL_DESC_BIAS_POINTER, &bias,
                                             sizeof(bias)), "bias");
  const float alpha = 1.f;
  lt_check(hipblasLtMatmul(handle, p.desc, &alpha, a, p.a, b, p.b, &beta, d, p.d, d, p.d,
                           &p.algo, workspace, p.workspace,
                           static_cast<hipStream_t>(stream_of(ref))),
           "matmul");
}

// out [M, N] = a [M, K] b^T (+ bias [N]) with b [N, K] when b_t != 0, else a [M, K] b with
// b [K, N]; fp16 operands with unit column stride, fp32 accumulation.
void gemm(const Tensor& a, const Tensor& b, const OptTensor& bias, int64_t b_t,
          const Tensor& out) {
  require_fp16(a, "a");
  require_fp16(b, "b");
  require_fp16(out, "out");
  require(a.dim() == 2 && b.dim() == 2 && out.dim() == 2 && a.stride(1) == 1 &&
              b.stride(1) == 1 && out.stride(1) == 1,
          "gemm: 2-D operands with unit column stride");
  const int64_t m_rows = a.size(0), k = a.size(1), n_cols = out.size(1);
  require(out.size(0) == m_rows && (b_t ? (b.size(0) == n_cols && b.size(1) == k)
                                        : (b.size(0) == k && b.size(1) == n_cols)),
          "gemm: a [M, K], b [N, K] (b_t) or [K, N], out [M, N]");
  require(a.device() == b.device() && a.device() == out.device(), "gemm: one device");
  if (bias.has_value()) {
    require_fp16(*bias, "bias");
    require(bias->is_contiguous() && bias->numel() == n_cols, "gemm: bias [N]");
  }
  require(k > 0, "gemm: empty reduction");
  if (m_rows == 0 || n_cols == 0) return;
  // column-major: out^T [N, M] = op(b) [N, K] a^T [K, M]
  run_gemm(GemmKey{static_cast<int>(a.device().index()), n_cols, m_rows, k, b.stride(0),
                   a.stride(0), out.stride(0), b_t ? 1 : 0, 0, bias.has_value() ? 1 : 0},
           b.data_ptr(), a.data_ptr(), bias.has_value() ? bias->data_ptr() : nullptr,
           out.data_ptr(), 0.f, out);
}

// Elements of t's storage from its first element on.
int64_t storage_span(const Tensor& t) {
  return static_cast<int64_t>(t.storage().nbytes() / t.element_size()) - t.storage_offset();
}

// The BLAS form: D [m, n] = op(A) [m, k] op(B) [k, n] (+ D when accumulate) in column-major
// terms with leading dimensions lda, ldb, ldd (elements), each matrix starting at its tensor's
// first element; the tensors' storage must cover every element the product touches (views of a
// wider buffer are fine).
void gemm_ex(const Tensor& a, int64_t trans_a, const Tensor& b, int64_t trans_b, const Tensor& d,
             int64_t m, int64_t n, int64_t k, int64_t lda, int64_t ldb, int64_t ldd,
             int64_t accumulate) {
  require_fp16(a, "a");
  require_fp16(b, "b");
  require_fp16(d, "d");
  require(a.device() == b.device() && a.device() == d.device(), "gemm_ex: one device");
  require(m >= 0 && n >= 0 && k >= 1, "gemm_ex: m, n >= 0 and k >= 1");
  if (m == 0 || n == 0) return;
  // rows x cols of each stored (column-major) matrix
  const int64_t ar = trans_a ? k : m, ac = trans_a ? m : k;
  const int64_t br = trans_b ? n : k, bc = trans_b ? k : n;
  require(lda >= ar && ldb >= br && ldd >= m, "gemm_ex: leading dimensions below the row count");
  require((ac - 1) * lda + ar <= storage_span(a) && (bc - 1) * ldb + br <= storage_span(b) &&
              (n - 1) * ldd + m <= storage_span(d),
          "gemm_ex: an operand's storage does not cover the product");
  run_gemm(GemmKey{static_cast<int>(a.device().index()), m, n, k, lda, ldb, ldd,
                   trans_a ? 1 : 0, trans_b ? 1 : 0, 0},
           a.data_ptr(), b.data_ptr(), nullptr, d.data_ptr(), accumulate ? 1.f : 0.f, d);
}

// Installs the measured table: int64 [rows, 7] on the CPU (trans_a, trans_b, m, k, n_lo, n_hi,
// solution index); an empty table restores hipBLASLt's heuristic everywhere.
void gemm_algo_table(const Tensor& rows) {
  require(!rows.is_cuda() && rows.scalar_type() == at::kLong && rows.dim() == 2 &&
              rows.size(1) == 7 && rows.is_contiguous(),
          "gemm_algo_table: int64 [rows, 7] on the CPU");
  std::vector<TunedRange> table;
  const int64_t* v = rows.data_ptr<int64_t>();
  for (int64_t r = 0; r < rows.size(0); ++r, v += 7)
    table.push_back(TunedRange{v[0], v[1], v[2], v[3], v[4], v[5], v[6]});
  {
    std::lock_guard<std::mutex> lock(tuned_mutex);
    tuned_table.swap(table);
  }
  tuned_generation.fetch_add(1);
}

int64_t gemm_lib_version() {
  int version = 0;
  lt_check(hipblasLtGetVersion(at::cuda::getCurrentCUDABlasLtHandle(), &version), "version");
  return version;
}

// Times every hipBLASLt solution that supports D = op(A) op(B) (the BLAS form of gemm_ex, D
// overwritten) on the current stream: `reps` launches each after two warm-up launches. Returns
// [best solution index, its µs, the heuristic's first choice's index, its µs] (float64, CPU).
// For building the measured table; only D's contents change.
Tensor gemm_tune(const Tensor& a, int64_t trans_a, const Tensor& b, int64_t trans_b,
                 const Tensor& d, int64_t m, int64_t n, int64_t k, int64_t lda, int64_t ldb,
                 int64_t ldd, int64_t reps) {
  require_fp16(a, "a");
  require_fp16(b, "b");
  require_fp16(d, "d");
  require(m > 0 && n > 0 && k > 0 && reps > 0, "gemm_tune: positive sizes and reps");
  const int64_t ar = trans_a ? k : m, ac = trans_a ? m : k;
  const int64_t br = trans_b ? n : k, bc = trans_b ? k : n;
  require(lda >= ar && ldb >= br && ldd >= m &&
              (ac - 1) * lda + ar <= storage_span(a) && (bc - 1) * ldb + br <= storage_span(b) &&
              (n - 1) * ldd + m <= storage_span(d),
          "gemm_tune: operands do not cover the product");
  const GemmKey key{static_cast<int>(a.device().index()), m, n, k, lda, ldb, ldd,
                    trans_a ? 1 : 0, trans_b ? 1 : 0, 0};
  hipblasLtHandle_t handle = at::cuda::getCurrentCUDABlasLtHandle();
  void* workspace = at::cuda::getCUDABlasLtWorkspace();
  const size_t limit = at::cuda::getCUDABlasLtWorkspaceSize();
  const hipStream_t stream = static_cast<hipStream_t>(stream_of(d));
  GemmPlan p;
  std::vector<hipblasLtMatmulHeuristicResult_t> all;
  double out[4] = {-1, -1, -1, -1};
  hipEvent_t e0 = nullptr, e1 = nullptr;
  try {
    describe(key, p);
    lt_check(hipblaslt_ext::getAllAlgos(handle, hipblaslt_ext::GemmType::HIPBLASLT_GEMM,
                                        trans_a ? HIPBLAS_OP_T : HIPBLAS_OP_N,
                                        trans_b ? HIPBLAS_OP_T : HIPBLAS_OP_N, HIP_R_16F,
                                        HIP_R_16F, HIP_R_16F, HIP_R_16F, HIPBLAS_COMPUTE_32F, all),
             "getAllAlgos");
    TORCH_CHECK(hipEventCreate(&e0) == hipSuccess && hipEventCreate(&e1) == hipSuccess,
                "gemm_tune: events");
    const float alpha = 1.f, beta = 0.f;
    auto time = [&](hipblasLtMatmulAlgo_t& algo, size_t ws) -> double {
      for (int i = 0; i < 2; ++i)
        if (hipblasLtMatmul(handle, p.desc, &alpha, a.data_ptr(), p.a, b.data_ptr(), p.b, &beta,
                            d.data_ptr(), p.d, d.data_ptr(), p.d, &algo, workspace, ws,
                            stream) != HIPBLAS_STATUS_SUCCESS)
          return -1;
      TORCH_CHECK(hipEventRecord(e0, stream) == hipSuccess, "gemm_tune: event");
      for (int64_t i = 0; i < reps; ++i)
        hipblasLtMatmul(handle, p.desc, &alpha, a.data_ptr(), p.a, b.data_ptr(), p.b, &beta,
                        d.data_ptr(), p.d, d.data_ptr(), p.d, &algo, workspace, ws, stream);
      TORCH_CHECK(hipEventRecord(e1, stream) == hipSuccess &&
                      hipEventSynchronize(e1) == hipSuccess,
                  "gemm_tune: event");
      float ms = 0.f;
      TORCH_CHECK(hipEventElapsedTime(&ms, e0, e1) == hipSuccess, "gemm_tune: event");
      return 1e3 * ms / reps;
    };
    for (auto& r : all) {
      size_t ws = 0;
      if (hipblaslt_ext::matmulIsAlgoSupported(handle, p.desc, &alpha, p.a, p.b, &beta, p.d,
                                               p.d, r.algo, ws) != HIPBLAS_STATUS_SUCCESS ||
          ws > limit)
        continue;
      const double us = time(r.algo, ws);
      if (us > 0 && (out[1] < 0 || us < out[1])) {
        out[0] = hipblaslt_ext::getIndexFromAlgo(r.algo);
        out[1] = us;
      }
    }
    hipblasLtMatmulPreference_t pref = nullptr;
    lt_check(hipblasLtMatmulPreferenceCreate(&pref), "preference");
    const uint64_t lim = limit;
    hipblasLtMatmulPreferenceSetAttribute(pref, HIPBLASLT_MATMUL_PREF_MAX_WORKSPACE_BYTES, &lim,
                                          sizeof(lim));
    hipblasLtMatmulHeuristicResult_t first{};
    int found = 0;
    const hipblasStatus_t st = hipblasLtMatmulAlgoGetHeuristic(handle, p.desc, p.a, p.b, p.d, p.d,
                                                               pref, 1, &first, &found);
    hipblasLtMatmulPreferenceDestroy(pref);
    if (st == HIPBLAS_STATUS_SUCCESS && found > 0) {
      out[2] = hipblaslt_ext::getIndexFromAlgo(first.algo);
      out[3] = time(first.algo, first.workspaceSize);
    }
  } catch (...) {
    if (e0) hipEventDestroy(e0);
    if (e1) hipEventDestroy(e1);
    destroy(p);
    throw;
  }
  hipEventDestroy(e0);
  hipEventDestroy(e1);
  destroy(p);
  Tensor result = at::empty({4}, at::TensorOptions().dtype(at::kDouble));
  for (int i = 0; i < 4; ++i) result.data_ptr<double>()[i] = out[i];
  return result;
}

// positions int64 [N] (contiguous), inv_freq float32 [half] -> cos, sin float32 [N, 2 half].
void rope_table(const Tensor& positions, const Tensor& inv_freq, double scaling,
                const Tensor& cos, const Tensor& sin) {
  require(positions.is_cuda() && positions.scalar_type() == at::kLong &&
              positions.is_contiguous(),
          "rope_table: positions contiguous CUDA int64");
  require(inv_freq.is_cuda() && inv_freq.scalar_type() == at::kFloat && inv_freq.is_contiguous() &&
              inv_freq.dim() == 1,
          "rope_table: inv_freq float32 [half]");
  const int64_t n = positions.numel(), half = inv_freq.numel();
  for (const Tensor* t : {&cos, &sin})
    require(t->is_cuda() && t->scalar_type() == at::kFloat && t->is_contiguous() &&
                t->numel() == n * 2 * half,
            "rope_table: cos, sin float32 [N, 2 half]");
  check(talm_rope_table(as<int64_t>(positions), n, as<float>(inv_freq),
                        static_cast<int32_t>(half), static_cast<float>(scaling), as<float>(cos),
                        as<float>(sin), stream_of(cos)),
        "rope_table");
}

// ------------------------------------------------------------------------------------------
// The packed causal-LM step's per-step glue: batch packing, row statistics, the head's loss and
// metrics, the head backward's scaling (csrc/pack.hip).

void i64_cuda(const Tensor& t, const char* name) {
  TORCH_CHECK_VALUE(t.is_cuda() && t.scalar_type() == at::kLong && t.is_contiguous(), name,
                    " must be a contiguous CUDA int64 tensor");
}

void f32_cuda(const Tensor& t, const char* name) {
  TORCH_CHECK_VALUE(t.is_cuda() && t.scalar_type() == at::kFloat && t.is_contiguous(), name,
                    " must be a contiguous CUDA float32 tensor");
}

// input_ids, mask, labels int64 [B, T] (right-padded) -> ids, positions, targets, src int64
// [n_tokens] and cu int32 [B + 2].
void pack_rows(const Tensor& input_ids, const Tensor& mask, const Tensor& labels,
               int64_t n_tokens, const Tensor& ids, const Tensor& positions, const Tensor& cu,
               const Tensor& targets, const Tensor& src) {
  i64_cuda(input_ids, "input_ids");
  i64_cuda(mask, "mask");
  i64_cuda(labels, "labels");
  require(mask.dim() == 2 && input_ids.sizes() == mask.sizes() && labels.sizes() == mask.sizes(),
          "pack_rows: input_ids, mask and labels [B, T]");
  const int64_t b = mask.size(0), t = mask.size(1);
  for (const auto& [v, name] : {std::pair<const Tensor*, const char*>{&ids, "ids"},
                                {&positions, "positions"}, {&targets, "targets"}, {&src, "src"}}) {
    i64_cuda(*v, name);
    TORCH_CHECK_VALUE(v->numel() == n_tokens, "pack_rows: ", name, " holds n_tokens values");
  }
  require(cu.is_cuda() && cu.scalar_type() == at::kInt && cu.is_contiguous() &&
              cu.numel() == b + 2,
          "pack_rows: cu int32 [B + 2]");
  require(b <= INT32_MAX && t <= INT32_MAX, "pack_rows: batch and row length fit int32");
  check(talm_pack_rows(as<int64_t>(input_ids), as<int64_t>(mask), as<int64_t>(labels),
                       static_cast<int32_t>(b), static_cast<int32_t>(t), n_tokens, as<int64_t>(ids),
                       as<int64_t>(positions), as<int32_t>(cu), as<int64_t>(targets),
                       as<int64_t>(src), stream_of(mask)),
        "pack_rows");
}

// mask, labels int64 [B, T] -> stats int64 [B + 2].
void row_stats(const Tensor& mask, const Tensor& labels, const Tensor& stats) {
  i64_cuda(mask, "mask");
  i64_cuda(labels, "labels");
  i64_cuda(stats, "stats");
  require(mask.dim() == 2 && labels.sizes() == mask.sizes() && stats.numel() == mask.size(0) + 2,
          "row_stats: mask, labels [B, T], stats [B + 2]");
  require(mask.size(0) <= INT32_MAX && mask.size(1) <= INT32_MAX,
          "row_stats: batch and row length fit int32");
  check(talm_row_stats(as<int64_t>(mask), as<int64_t>(labels), static_cast<int32_t>(mask.size(0)),
                       static_cast<int32_t>(mask.size(1)), as<int64_t>(stats), stream_of(mask)),
        "row_stats");
}

// token_loss f32 [N], correct int32 [N], targets int64 [N] -> loss, denom f32 [] and
// correct_bool bool [N]. mode 0: denom = max(#labelled, 1); 1: num_items (f32 []); 2: value.
void head_loss(const Tensor& token_loss, const Tensor& correct, const Tensor& targets,
               const OptTensor& num_items, double num_items_value, int64_t mode,
               const Tensor& loss, const Tensor& denom, const Tensor& correct_bool) {
  f32_cuda(token_loss, "token_loss");
  i64_cuda(targets, "targets");
  const int64_t n = token_loss.numel();
  require(correct.is_cuda() && correct.scalar_type() == at::kInt && correct.is_contiguous() &&
              correct.numel() == n && targets.numel() == n,
          "head_loss: correct int32 [N], targets [N]");
  require(correct_bool.is_cuda() && correct_bool.scalar_type() == at::kBool &&
              correct_bool.is_contiguous() && correct_bool.numel() == n,
          "head_loss: correct_bool bool [N]");
  f32_cuda(loss, "loss");
  f32_cuda(denom, "denom");
  require(loss.numel() == 1 && denom.numel() == 1, "head_loss: loss and denom hold one value");
  require(mode >= 0 && mode <= 2 && (mode != 1 || num_items.has_value()), "head_loss: mode");
  if (num_items.has_value()) {
    f32_cuda(*num_items, "num_items");
    require(num_items->numel() == 1, "head_loss: num_items holds one value");
  }
  check(talm_head_loss(as<float>(token_loss), as<int32_t>(correct), as<int64_t>(targets), n,
                       as<float>(num_items), static_cast<float>(num_items_value),
                       static_cast<int32_t>(mode), as<float>(loss), as<float>(denom),
                       static_cast<uint8_t*>(correct_bool.data_ptr()), stream_of(token_loss)),
        "head_loss");
}

// token_loss, entropy f32 [N], correct bool [N], targets, src int64 [N] -> full_loss,
// full_entropy f32 [L] and stats int64 [2].
void scatter_rows(const Tensor& token_loss, const Tensor& entropy, const Tensor& correct,
                  const Tensor& targets, const Tensor& src, const Tensor& full_loss,
                  const Tensor& full_entropy, const Tensor& stats) {
  f32_cuda(token_loss, "token_loss");
  f32_cuda(entropy, "entropy");
  f32_cuda(full_loss, "full_loss");
  f32_cuda(full_entropy, "full_entropy");
  i64_cuda(targets, "targets");
  i64_cuda(src, "src");
  i64_cuda(stats, "stats");
  const int64_t n = token_loss.numel();
  require(entropy.numel() == n && targets.numel() == n && src.numel() == n &&
              correct.is_cuda() && correct.scalar_type() == at::kBool &&
              correct.is_contiguous() && correct.numel() == n,
          "scatter_rows: entropy, correct (bool), targets and src [N]");
  require(full_entropy.numel() == full_loss.numel() && stats.numel() == 2,
          "scatter_rows: full_loss, full_entropy [L], stats [2]");
  check(talm_scatter_rows(as<float>(token_loss), as<float>(entropy),
                          static_cast<const uint8_t*>(correct.data_ptr()),
                          as<int64_t>(targets), as<int64_t>(src), n, full_loss.numel(),
                          as<float>(full_loss), as<float>(full_entropy), as<int64_t>(stats),
                          stream_of(token_loss)),
        "scatter_rows");
}

// out = fp16(fp32(g) * (denom != 0 ? grad_loss / denom : 0)); g, out fp16 of one size.
void scale_rows(const Tensor& g, const Tensor& grad_loss, const Tensor& denom, const Tensor& out) {
  require_fp16(g, "g");
  require_fp16(out, "out");
  require(g.is_contiguous() && out.is_contiguous() && g.numel() == out.numel(),
          "scale_rows: g and out contiguous, of one size");
  f32_cuda(grad_loss, "grad_loss");
  f32_cuda(denom, "denom");
  require(grad_loss.numel() == 1 && denom.numel() == 1,
          "scale_rows: grad_loss and denom hold one value");
  check(talm_scale_rows(as<uint16_t>(g), g.numel(), as<float>(grad_loss), as<float>(denom),
                        as<uint16_t>(out), stream_of(g)),
        "scale_rows");
}

}  // namespace


TORCH_LIBRARY(talm, m) {
  m.def("nf4_group_dequant(Tensor packed, Tensor absmax8, Tensor code, Tensor absmax2, "
        "Tensor offset2, Tensor(a!) out, int qblock, int qblock2) -> ()");
  m.def("nf4_group_dequant_streaming(Tensor packed, Tensor absmax8, Tensor code, "
        "Tensor absmax2, Tensor offset2, Tensor(a!) out, int qblock, int qblock2) -> ()");
  m.def("nf4_group_dequant_t(Tensor packed, Tensor absmax8, Tensor code, Tensor absmax2, "
        "Tensor offset2, int[] segs, Tensor(a!) out, int qblock, int qblock2) -> ()");
  m.def("nf4_dequant(Tensor packed, Tensor absmax, Tensor(a!) out, int blocksize) -> ()");
  m.def("gemm_splitk(Tensor a, Tensor b, Tensor(a!) out, Tensor(b!) workspace) -> ()");
  m.def("rmsnorm(Tensor(a!) a, Tensor(b!)? q, Tensor(c!) h, Tensor(d!) xhat, Tensor(e!)? p, "
        "Tensor weight, Tensor(f!) rstd, float eps, int backward) -> ()");
  m.def("rope(Tensor q, Tensor k, Tensor cos, Tensor sin, Tensor(a!) out_q, Tensor(b!) out_k, "
        "int backward) -> ()");
  m.def("swiglu_fwd(Tensor gate, Tensor up, Tensor(a!) out) -> ()");
  m.def("swiglu_bwd(Tensor grad, Tensor gate, Tensor up, Tensor(a!) dgate, Tensor(b!) dup) -> ()");
  m.def("swiglu_fwd_rows(Tensor gate, Tensor up, Tensor(a!) out) -> ()");
  m.def("swiglu_bwd_rows(Tensor grad, Tensor gate, Tensor up, Tensor(a!) dgate, "
        "Tensor(b!) dup) -> ()");
  m.def("head_weight_t(Tensor weight, Tensor(a!) weight_t) -> ()");
  m.def("head_ce(Tensor hidden, Tensor weight, Tensor targets, int vchunk, "
        "int n_grad, int group, Tensor(a!) token_loss, Tensor(b!) entropy, Tensor(c!) best_idx, "
        "Tensor(d!) correct, Tensor(e!)? grad_hidden, Tensor(f!) workspace) -> ()");
  m.def("lora_down(Tensor x, Tensor a0, Tensor? a1, int k0, int k1, int xcol0, int xcol1, "
        "int a_kmajor, float scaling0, float scaling1, Tensor(a!) t, Tensor(b!) ts) -> ()");
  m.def("qkv_lora_fwd(Tensor x, Tensor weight, Tensor? bias, Tensor? ts, Tensor? b0, "
        "int seg0_begin, int seg0_end, Tensor? b1, int seg1_begin, int seg1_end, Tensor? cos, "
        "Tensor? sin, int rope_cols, Tensor(a!) out) -> ()");
  m.def("qkv_lora_fwd_down(Tensor x, Tensor weight, Tensor? bias, Tensor? a0, Tensor? a1, "
        "float scaling0, float scaling1, Tensor? b0, int seg0_begin, int seg0_end, Tensor? b1, "
        "int seg1_begin, int seg1_end, Tensor? cos, Tensor? sin, int rope_cols, Tensor(a!)? t, "
        "Tensor(b!) out) -> ()");
  m.def("qkv_bwd_prep(Tensor dq, Tensor dk, Tensor dv, Tensor? cos, Tensor? sin, "
        "Tensor(a!) dcat) -> ()");
  m.def("qkv_lora_bwd_dx(Tensor dcat, Tensor weight_t, Tensor? u, Tensor? a_t, "
        "Tensor(a!) dx) -> ()");
  m.def("lora_wgrad(Tensor x, Tensor dy, Tensor u, Tensor t, int lo0, int seg0, float scaling0, "
        "Tensor(a!) da0, Tensor(b!) db0, int lo1, int seg1, float scaling1, Tensor(c!)? da1, "
        "Tensor(d!)? db1, Tensor(e!) workspace) -> ()");
  m.def("gemm(Tensor a, Tensor b, Tensor? bias, int b_t, Tensor(a!) out) -> ()");
  m.def("gemm_ex(Tensor a, int trans_a, Tensor b, int trans_b, Tensor(a!) d, int m, int n, int k, "
        "int lda, int ldb, int ldd, int accumulate) -> ()");
  m.def("attn_fwd(Tensor q, Tensor k, Tensor v, Tensor cu_seqlens, int max_seqlen, float scale, "
        "Tensor(a!) out, Tensor(b!) lse) -> ()");
  m.def("attn_bwd(Tensor q, Tensor k, Tensor v, Tensor out, Tensor dout, Tensor lse, "
        "Tensor cu_seqlens, int max_seqlen, float scale, Tensor(a!) dq, Tensor(b!) dk, "
        "Tensor(c!) dv, Tensor(d!) workspace) -> ()");
  m.def("attn_bwd_rope(Tensor q, Tensor k, Tensor v, Tensor out, Tensor dout, Tensor lse, "
        "Tensor cu_seqlens, int max_seqlen, float scale, Tensor cos, Tensor sin, Tensor(a!) dq, "
        "Tensor(b!) dk, Tensor(c!) dv, Tensor(d!) workspace) -> ()");
  m.def("lora_mirror(Tensor table, int n_tensors, int max_numel, Tensor(a!) out) -> ()");
  m.def("pack_rows(Tensor input_ids, Tensor mask, Tensor labels, int n_tokens, Tensor(a!) ids, "
        "Tensor(b!) positions, Tensor(c!) cu, Tensor(d!) targets, Tensor(e!) src) -> ()");
  m.def("row_stats(Tensor mask, Tensor labels, Tensor(a!) stats) -> ()");
  m.def("head_loss(Tensor token_loss, Tensor correct, Tensor targets, Tensor? num_items, "
        "float num_items_value, int mode, Tensor(a!) loss, Tensor(b!) denom, "
        "Tensor(c!) correct_bool) -> ()");
  m.def("scatter_rows(Tensor token_loss, Tensor entropy, Tensor correct, Tensor targets, "
        "Tensor src, Tensor(a!) full_loss, Tensor(b!) full_entropy, Tensor(c!) stats) -> ()");
  m.def("scale_rows(Tensor g, Tensor grad_loss, Tensor denom, Tensor(a!) out) -> ()");
  m.def("lora_grad_norm(Tensor table, int n_tensors, int max_numel, Tensor scale, "
        "float max_norm, Tensor(a!) workspace, Tensor(b!) stats) -> ()");
  m.def("lora_adamw_clipped(Tensor table, int n_tensors, int max_numel, float lr, float beta1, "
        "float beta2, float eps, float weight_decay, Tensor step_in, Tensor(a!) step_out, "
        "Tensor found_inf, Tensor grad_mul, Tensor(b!) out) -> ()");
  m.def("rope_table(Tensor positions, Tensor inv_freq, float scaling, Tensor(a!) cos, "
        "Tensor(b!) sin) -> ()");
  m.def("gemm_splitk_partials(Tensor a, Tensor b, Tensor(a!) partials) -> ()");
  m.def("nf4_gemm_partials(Tensor x, Tensor packed, Tensor scale, int rows, int cols, "
        "bool transpose, int blocksize, Tensor(a!) partials) -> ()");
  m.def("splitk_add_rmsnorm(Tensor partials, Tensor resid, Tensor weight, float eps, "
        "Tensor(a!) sum_out, Tensor(b!) h, Tensor(c!) xhat, Tensor(d!) rstd) -> ()");
  m.def("splitk_rmsnorm_bwd(Tensor partials, Tensor xhat, Tensor rstd, Tensor weight, "
        "Tensor? ds, Tensor(a!) dx, Tensor(b!) dbranch) -> ()");
  m.def("gemm_algo_table(Tensor rows) -> ()", &gemm_algo_table);
  m.def("gemm_lib_version() -> int", &gemm_lib_version);
  m.def("gemm_tune(Tensor a, int trans_a, Tensor b, int trans_b, Tensor(a!) d, int m, int n, "
        "int k, int lda, int ldb, int ldd, int reps) -> Tensor");
  m.def("nf4_gemm(Tensor x, Tensor packed, Tensor scale, int rows, int cols, bool transpose, "
        "int blocksize, Tensor(a!) out, Tensor(b!) workspace) -> ()");
  m.def("nf4_block_scales(Tensor absmax8, Tensor code, Tensor absmax2, Tensor offset2, "
        "int qblock2, Tensor(a!) out) -> ()");
  m.def("lora_adamw(Tensor table, int n_tensors, int max_numel, float lr, float beta1, "
        "float beta2, float eps, float weight_decay, Tensor step_in, Tensor(a!) step_out, "
        "Tensor? grad_scale, Tensor? found_inf, Tensor(b!) out) -> ()");
}

TORCH_LIBRARY_IMPL(talm, CUDA, m) {
  m.impl("nf4_group_dequant", &nf4_group_dequant);
  m.impl("nf4_group_dequant_streaming", &nf4_group_dequant_streaming);
  m.impl("nf4_group_dequant_t", &nf4_group_dequant_t);
  m.impl("gemm_splitk", &gemm_splitk);
  m.impl("nf4_dequant", &nf4_dequant);
  m.impl("rmsnorm", &rmsnorm);
  m.impl("rope", &rope);
  m.impl("swiglu_fwd", &swiglu_fwd);
  m.impl("swiglu_bwd", &swiglu_bwd);
  m.impl("swiglu_fwd_rows", &swiglu_fwd_rows);
  m.impl("swiglu_bwd_rows", &swiglu_bwd_rows);
  m.impl("head_weight_t", &head_weight_t);
  m.impl("head_ce", &head_ce);
  m.impl("lora_down", &lora_down);
  m.impl("qkv_lora_fwd", &qkv_lora_fwd);
  m.impl("qkv_lora_fwd_down", &qkv_lora_fwd_down);
  m.impl("qkv_bwd_prep", &qkv_bwd_prep);
  m.impl("qkv_lora_bwd_dx", &qkv_lora_bwd_dx);
  m.impl("lora_wgrad", &lora_wgrad);
  m.impl("gemm", &gemm);
  m.impl("gemm_ex", &gemm_ex);
  m.impl("attn_fwd", &attn_fwd);
  m.impl("attn_bwd", &attn_bwd);
  m.impl("attn_bwd_rope", &attn_bwd_rope);
  m.impl("lora_mirror", &lora_mirror);
  m.impl("gemm_tune", &gemm_tune);
  m.impl("nf4_gemm", &nf4_gemm);
  m.impl("nf4_block_scales", &nf4_block_scales);
  m.impl("lora_adamw", &lora_adamw);
  m.impl("pack_rows", &pack_rows);
  m.impl("row_stats", &row_stats);
  m.impl("head_loss", &head_loss);
  m.impl("scatter_rows", &scatter_rows);
  m.impl("scale_rows", &scale_rows);
  m.impl("rope_table", &rope_table);
  m.impl("lora_grad_norm", &lora_grad_norm);
  m.impl("lora_adamw_clipped", &lora_adamw_clipped);
  m.impl("gemm_splitk_partials", &gemm_splitk_partials);
  m.impl("nf4_gemm_partials", &nf4_gemm_partials);
  m.impl("splitk_add_rmsnorm", &splitk_add_rmsnorm);
  m.impl("splitk_rmsnorm_bwd", &splitk_rmsnorm_bwd);
}
