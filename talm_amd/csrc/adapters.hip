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
  const float* grad_mul;   // [2]: gradients times [0] (the inverse loss scale), then times [1]
                           // (the clipping coefficient), each product rounded; or null
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
  // the multipliers in registers before any store (the stores below may alias them as far as
  // the compiler knows, which would reload them after each element)
  const float gm0 = a.grad_mul ? a.grad_mul[0] : 1.f, gm1 = a.grad_mul ? a.grad_mul[1] : 1.f;
  // every element's loads first (indices past the tensor clamped to its last element, their
  // results unused), then the updates: one memory round trip instead of one per element
  float w0[kPerThread], g0[kPerThread], m0[kPerThread], v0[kPerThread];
#pragma unroll
  for (int j = 0; j < kPerThread; ++j) {
    const int64_t i = min(i0 + j, x.n - 1);
    w0[j] = x.w[i];
    g0[j] = x.g[i];
    m0[j] = x.m[i];
    v0[j] = x.v[i];
  }
#pragma unroll
  for (int j = 0; j < kPerThread; ++j) {
    const int64_t i = i0 + j;
    if (i >= x.n) break;
    float p = w0[j];
    if (!skip) {
      float g = a.grad_scale ? g0[j] * inv_scale : g0[j];
      if (a.grad_mul) g = mul_f32(mul_f32(g, gm0), gm1);
      p -= a.lr * a.weight_decay * p;
      const float m = a.beta1 * m0[j] + (1.f - a.beta1) * g;
      const float v = a.beta2 * v0[j] + (1.f - a.beta2) * g * g;
      p -= step_size * m / (sqrtf(v) / bc2_sqrt + a.eps);
      x.m[i] = m;
      x.v[i] = v;
      x.w[i] = p;
    }
    write_copies(x, i, p, out);
  }
}

// The global 2-norm of the unscaled gradients, as GradScaler.unscale_ and clip_grad_norm_
// compute it: u = fl32(g * inv_scale) with inv_scale = fl32(1 / (double) scale) (unscale_'s
// reciprocal), then sqrt(sum of u^2). Pass 1: each workgroup's sum over its kPerThread x kThreads
// elements of one tensor and a flag for a non-finite u; pass 2 (one workgroup): the sums in
// workgroup order, the norm, the clipping coefficient min(max_norm / (norm + 1e-6), 1) (NaN
// kept, as clamp keeps it) and the inf flag.
__device__ __forceinline__ float unscale_factor(const float* scale) {
  return static_cast<float>(1.0 / static_cast<double>(*scale));
}

__global__ __launch_bounds__(kThreads) void grad_sq_kernel(const int64_t* __restrict__ table,
                                                           const float* __restrict__ scale,
                                                           float* __restrict__ part_sum,
                                                           float* __restrict__ part_bad) {
  __shared__ float red[2][kThreads / kWave];
  const Entry x = entry(table, blockIdx.y);
  const float inv = unscale_factor(scale);
  const int64_t i0 = (static_cast<int64_t>(blockIdx.x) * kThreads + threadIdx.x) * kPerThread;
  float sq = 0.f, bad = 0.f;
#pragma unroll
  for (int j = 0; j < kPerThread; ++j) {
    const int64_t i = i0 + j;
    if (i < x.n) {
      const float u = mul_f32(x.g[i], inv);
      sq += u * u;
      bad += isfinite(u) ? 0.f : 1.f;
    }
  }
  sq = wave_sum(sq);
  bad = wave_sum(bad);
  const int w = threadIdx.x / kWave;
  if (threadIdx.x % kWave == 0) {
    red[0][w] = sq;
    red[1][w] = bad;
  }
  __syncthreads();
  if (threadIdx.x == 0) {
    float s = 0.f, b = 0.f;
    for (int k = 0; k < kThreads / kWave; ++k) {
      s += red[0][k];
      b += red[1][k];
    }
    const int64_t at = static_cast<int64_t>(blockIdx.y) * gridDim.x + blockIdx.x;
    part_sum[at] = s;
    part_bad[at] = b;
  }
}

__global__ __launch_bounds__(kThreads) void grad_norm_kernel(const float* __restrict__ part_sum,
                                                             const float* __restrict__ part_bad,
                                                             int64_t n_parts,
                                                             const float* __restrict__ scale,
                                                             float max_norm,
                                                             float* __restrict__ stats) {
  __shared__ float red[2][kThreads / kWave];
  float s = 0.f, b = 0.f;
  for (int64_t k = threadIdx.x; k < n_parts; k += kThreads) {
    s += part_sum[k];
    b += part_bad[k];
  }
  s = wave_sum(s);
  b = wave_sum(b);
  if (threadIdx.x % kWave == 0) {
    red[0][threadIdx.x / kWave] = s;
    red[1][threadIdx.x / kWave] = b;
  }
  __syncthreads();
  if (threadIdx.x == 0) {
    float total = 0.f, flags = 0.f;
    for (int k = 0; k < kThreads / kWave; ++k) {
      total += red[0][k];
      flags += red[1][k];
    }
    const float norm = sqrtf(total);
    const float coef = max_norm / (norm + 1e-6f);
    stats[0] = flags != 0.f || !isfinite(norm) ? 1.f : 0.f;
    stats[1] = unscale_factor(scale);
    stats[2] = coef > 1.f ? 1.f : coef;
    stats[3] = norm;
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
  AdamArgs a{lr, beta1, beta2, eps, weight_decay, step_in, step_out, grad_scale, found_inf,
             nullptr};
  hipLaunchKernelGGL(lora_adamw_kernel, grid_for(n_tensors, max_numel), dim3(kThreads), 0,
                     as_stream(stream), table, a, out);
  return check_launch("lora_adamw");
}

TALM_API int64_t talm_lora_grad_norm_workspace(int32_t n_tensors, int64_t max_numel) {
  if (n_tensors < 0 || n_tensors > 65535 || max_numel < 0) return -1;
  const dim3 g = grid_for(n_tensors, max_numel);
  return static_cast<int64_t>(g.x) * g.y * 2 * 4;
}

TALM_API int talm_lora_grad_norm(const int64_t* table, int32_t n_tensors, int64_t max_numel,
                                 const float* scale, float max_norm, void* workspace,
                                 int64_t workspace_bytes, float* stats, void* stream) {
  if (n_tensors < 0 || n_tensors > 65535 || max_numel < 0)
    return fail(TALM_EINVAL, "lora_grad_norm: %d tensors, max_numel %lld", n_tensors,
                (long long)max_numel);
  if (!scale || !stats || (n_tensors > 0 && max_numel > 0 && (!table || !workspace)))
    return fail(TALM_EINVAL, "lora_grad_norm: null pointer");
  if (!aligned(table, 8) || !aligned(workspace, 4))
    return fail(TALM_EINVAL, "lora_grad_norm: table 8-byte, workspace 4-byte aligned");
  const int64_t need = talm_lora_grad_norm_workspace(n_tensors, max_numel);
  if (workspace_bytes < need)
    return fail(TALM_EINVAL, "lora_grad_norm: workspace of %lld bytes, %lld needed",
                (long long)workspace_bytes, (long long)need);
  const hipStream_t s = as_stream(stream);
  const dim3 g = grid_for(n_tensors, max_numel);
  const int64_t n_parts = static_cast<int64_t>(g.x) * g.y;
  float* part_sum = static_cast<float*>(workspace);
  float* part_bad = part_sum + n_parts;
  if (n_parts > 0)
    hipLaunchKernelGGL(grad_sq_kernel, g, dim3(kThreads), 0, s, table, scale, part_sum, part_bad);
  hipLaunchKernelGGL(grad_norm_kernel, dim3(1), dim3(kThreads), 0, s, part_sum, part_bad, n_parts,
                     scale, max_norm, stats);
  return check_launch("lora_grad_norm");
}

TALM_API int talm_lora_adamw_clipped(const int64_t* table, int32_t n_tensors, int64_t max_numel,
                                     float lr, float beta1, float beta2, float eps,
                                     float weight_decay, const float* step_in, float* step_out,
                                     const float* found_inf, const float* grad_mul,
                                     uint16_t* out, void* stream) {
  if (check_table("lora_adamw_clipped", table, n_tensors, max_numel, out)) return TALM_EINVAL;
  if (!step_in || !step_out || !found_inf || !grad_mul)
    return fail(TALM_EINVAL, "lora_adamw_clipped: null step counter, inf flag or multiplier");
  if (!(beta1 >= 0.f && beta1 < 1.f && beta2 >= 0.f && beta2 < 1.f && eps > 0.f && lr >= 0.f))
    return fail(TALM_EINVAL, "lora_adamw_clipped: betas in [0, 1), eps > 0 and lr >= 0");
  if (n_tensors == 0 || max_numel == 0) return ok();
  AdamArgs a{lr, beta1, beta2, eps, weight_decay, step_in, step_out, nullptr, found_inf, grad_mul};
  hipLaunchKernelGGL(lora_adamw_kernel, grid_for(n_tensors, max_numel), dim3(kThreads), 0,
                     as_stream(stream), table, a, out);
  return check_launch("lora_adamw_clipped");
}
