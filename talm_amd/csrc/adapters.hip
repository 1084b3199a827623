// The LoRA adapters' per-step state on the device: fp16 images of the fp32 weights (the MFMA
// kernels' operands) and the AdamW update of those weights, for every adapter of the model in
// one launch each.
//
// A table in device memory describes the tensors, kTableCols int64 per tensor:
//   0 w      fp32 weight [rows, cols], row-major contiguous (updated in place by the optimizer)
//   1 numel  element count
//   2 cols   column count
//   3 h_off  element offset of its fp16 copy in `out` (same layout), or -1: no copy
//   4 t_off  element offset of its transposed fp16 copy in `out`, or -1: none;
//            out[t_off + c * ld_t + r] = fp16(w[r, c])
//   5 ld_t   row stride of the transposed copy (elements)
//   6 grad   fp32 gradient, same layout as w (optimizer only)
//   7 m      fp32 first moment (optimizer only)
//   8 v      fp32 second moment (optimizer only)
// The transposed copies of a q|k|v node's two A matrices side by side are A^T = [A_q^T | A_v^T]
// ([hidden, 32]), the B operand of the extra reduction step of its backward dX GEMM. Grid:
// (element chunks of the largest tensor, tensors); a workgroup past its tensor's end exits.
#include "common.h"

namespace talm {
namespace {

constexpr int kTableCols = 9;
constexpr int kPerThread = 4;
constexpr int kThreads = 256;

struct Entry {
  float* w;
  int64_t n, cols, h_off, t_off, ld_t;
  const float* g;
  float* m;
  float* v;
};

__device__ __forceinline__ Entry entry(const int64_t* __restrict__ table, int t) {
  const int64_t* e = table + static_cast<int64_t>(t) * kTableCols;
  Entry x;
  x.w = reinterpret_cast<float*>(e[0]);
  x.n = e[1];
  x.cols = e[2];
  x.h_off = e[3];
  x.t_off = e[4];
  x.ld_t = e[5];
  x.g = reinterpret_cast<const float*>(e[6]);
  x.m = reinterpret_cast<float*>(e[7]);
  x.v = reinterpret_cast<float*>(e[8]);
  return x;
}

__device__ __forceinline__ void write_copies(const Entry& x, int64_t i, float p, uint16_t* out) {
  const uint16_t h = f2h(p);
  if (x.h_off >= 0) out[x.h_off + i] = h;
  if (x.t_off >= 0) {
    const int64_t r = i / x.cols, c = i - r * x.cols;
    out[x.t_off + c * x.ld_t + r] = h;
  }
}

__global__ __launch_bounds__(kThreads) void lora_mirror_kernel(const int64_t* __restrict__ table,
                                                               uint16_t* __restrict__ out) {
  const Entry x = entry(table, blockIdx.y);
  const int64_t i0 = (static_cast<int64_t>(blockIdx.x) * kThreads + threadIdx.x) * kPerThread;
  if (i0 >= x.n) return;
#pragma unroll
  for (int j = 0; j < kPerThread; ++j)
    if (i0 + j < x.n) write_copies(x, i0 + j, x.w[i0 + j], out);
}

struct AdamArgs {
  float lr, beta1, beta2, eps, weight_decay;
  const float* step_in;    // completed steps before this one
  float* step_out;         // written by one thread: step_in + 1, or step_in when skipped
  const float* grad_scale; // gradients are divided by it, or null
  const float* found_inf;  // nonzero: no update (the weights' copies are still written), or null
};

// Decoupled weight decay, then Adam with bias correction (Loshchilov & Hutter, AdamW):
//   w -= lr wd w;  m = b1 m + (1 - b1) g;  v = b2 v + (1 - b2) g^2;
//   w -= (lr / (1 - b1^t)) m / (sqrt(v) / sqrt(1 - b2^t) + eps)
__global__ __launch_bounds__(kThreads) void lora_adamw_kernel(const int64_t* __restrict__ table,
                                                              AdamArgs a,
                                                              uint16_t* __restrict__ out) {
  const bool skip = a.found_inf && *a.found_inf != 0.f;
  const float done = *a.step_in;
  if (blockIdx.x == 0 && blockIdx.y == 0 && threadIdx.x == 0) *a.step_out = skip ? done : done + 1.f;
  const Entry x = entry(table, blockIdx.y);
  const int64_t i0 = (static_cast<int64_t>(blockIdx.x) * kThreads + threadIdx.x) * kPerThread;
  if (i0 >= x.n) return;
  const float t = done + 1.f;
  const float bc1 = 1.f - powf(a.beta1, t);
  const float bc2_sqrt = sqrtf(1.f - powf(a.beta2, t));
  const float step_size = a.lr / bc1;
  const float inv_scale = a.grad_scale ? 1.f / *a.grad_scale : 1.f;
#pragma unroll
  for (int j = 0; j < kPerThread; ++j) {
    const int64_t i = i0 + j;
    if (i >= x.n) break;
    float p = x.w[i];
    if (!skip) {
      const float g = a.grad_scale ? x.g[i] * inv_scale : x.g[i];
      p -= a.lr * a.weight_decay * p;
      const float m = a.beta1 * x.m[i] + (1.f - a.beta1) * g;
      const float v = a.beta2 * x.v[i] + (1.f - a.beta2) * g * g;
      p -= step_size * m / (sqrtf(v) / bc2_sqrt + a.eps);
      x.m[i] = m;
      x.v[i] = v;
      x.w[i] = p;
    }
    write_copies(x, i, p, out);
  }
}

int check_table(const char* what, const int64_t* table, int32_t n_tensors, int64_t max_numel,
                const uint16_t* out) {
  if (n_tensors < 0 || n_tensors > 65535 || max_numel < 0)
    return fail(TALM_EINVAL, "%s: %d tensors, max_numel %lld", what, n_tensors,
                (long long)max_numel);
  if (n_tensors > 0 && (!table || !out)) return fail(TALM_EINVAL, "%s: null pointer", what);
  if (!aligned(table, 8)) return fail(TALM_EINVAL, "%s: table must be 8-byte aligned", what);
  return TALM_OK;
}

dim3 grid_for(int32_t n_tensors, int64_t max_numel) {
  const int64_t per = static_cast<int64_t>(kThreads) * kPerThread;
  return dim3(static_cast<unsigned>((max_numel + per - 1) / per), static_cast<unsigned>(n_tensors));
}

}  // namespace
}  // namespace talm

using namespace talm;

TALM_API int talm_lora_mirror(const int64_t* table, int32_t n_tensors, int64_t max_numel,
                              uint16_t* out, void* stream) {
  if (check_table("lora_mirror", table, n_tensors, max_numel, out)) return TALM_EINVAL;
  if (n_tensors == 0 || max_numel == 0) return ok();
  hipLaunchKernelGGL(lora_mirror_kernel, grid_for(n_tensors, max_numel), dim3(kThreads), 0,
                     as_stream(stream), table, out);
  return check_launch("lora_mirror");
}

TALM_API int talm_lora_adamw(const int64_t* table, int32_t n_tensors, int64_t max_numel,
                             float lr, float beta1, float beta2, float eps, float weight_decay,
                             const float* step_in, float* step_out, const float* grad_scale,
                             const float* found_inf, uint16_t* out, void* stream) {
  if (check_table("lora_adamw", table, n_tensors, max_numel, out)) return TALM_EINVAL;
  if (!step_in || !step_out) return fail(TALM_EINVAL, "lora_adamw: null step counter");
  if (!(beta1 >= 0.f && beta1 < 1.f && beta2 >= 0.f && beta2 < 1.f && eps > 0.f && lr >= 0.f))
    return fail(TALM_EINVAL, "lora_adamw: betas in [0, 1), eps > 0 and lr >= 0");
  if (n_tensors == 0 || max_numel == 0) return ok();
  AdamArgs a{lr, beta1, beta2, eps, weight_decay, step_in, step_out, grad_scale, found_inf};
  hipLaunchKernelGGL(lora_adamw_kernel, grid_for(n_tensors, max_numel), dim3(kThreads), 0,
                     as_stream(stream), table, a, out);
  return check_launch("lora_adamw");
}
