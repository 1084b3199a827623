// SwiGLU for gfx950: forward silu(gate) * up and its backward, fp16 storage with fp32 math.
// Flat, contiguous operands (or [rows, cols] views with row strides, the *_rows entry points);
// each thread moves 8 elements per 16-byte access. Aliasing the outputs onto the inputs is
// allowed (the in-place backward and the save-up forward): a thread loads its operands before
// storing at the same offsets.
#include "common.h"

#include <initializer_list>

namespace talm {
namespace {

constexpr int kThreads = 256;
constexpr int kVecPerThread = 2;  // 16 elements per thread per grid step

// sigmoid(x) = 1 / (1 + 2^(-x log2 e)) with v_exp_f32 and v_rcp_f32 (1 ulp each; an IEEE fp32
// division is a ~10-instruction sequence). At 8 elements per 16-byte access the kernels are
// close to VALU-bound on gfx950 (no packed fp32 math here), so the reciprocal matters: the
// results are fp16, far coarser than these roundings.
__device__ __forceinline__ float sigmoid(float x) {
  return __builtin_amdgcn_rcpf(1.0f + __builtin_amdgcn_exp2f(x * -1.44269504088896341f));
}

__device__ __forceinline__ void unpack8(const uint4& a, float* v) {
  v[0] = lo_f(a.x); v[1] = hi_f(a.x); v[2] = lo_f(a.y); v[3] = hi_f(a.y);
  v[4] = lo_f(a.z); v[5] = hi_f(a.z); v[6] = lo_f(a.w); v[7] = hi_f(a.w);
}

__device__ __forceinline__ uint4 pack8(const float* v) {
  return make_uint4(pack2(v[0], v[1]), pack2(v[2], v[3]), pack2(v[4], v[5]), pack2(v[6], v[7]));
}

typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

// Loads carry the non-temporal hint: the operands are read once, and on gfx950 the hinted loads
// stream from HBM markedly faster (config 3, same grid: the forward 0.64 -> 0.72 and the backward
// 0.64 -> 0.72 of 8 TB/s, against 0.73 for this build's own non-temporal 2-read / 1-write and
// 3-read / 2-write probes). The stores stay ordinary: the outputs are the next GEMM's operands
// and are best left in the last-level cache.
__device__ __forceinline__ uint4 load_nt(const uint4* p) {
  const u32x4 v = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(p));
  return make_uint4(v.x, v.y, v.z, v.w);
}

// Grid-stride over 16-byte vectors, kVecPerThread per thread and iteration (256 apart), with the
// next iteration's loads issued before this one's arithmetic and stores: two iterations' loads
// in flight. Indices past the end are clamped to the last vector (their stores are skipped), so
// the loads need no branch. Aliasing outputs onto inputs stays allowed: a thread loads an element
// before it stores at that offset, and the element loaded ahead is never one stored before it.
__global__ __launch_bounds__(kThreads) void swiglu_fwd_vec(const uint4* gate, const uint4* up,
                                                           uint4* out, int64_t n_vec) {
  const int64_t stride = static_cast<int64_t>(gridDim.x) * kThreads * kVecPerThread;
  int64_t base = static_cast<int64_t>(blockIdx.x) * kThreads * kVecPerThread + threadIdx.x;
  if (base >= n_vec) return;
  uint4 gv[kVecPerThread], uv[kVecPerThread];
  auto load = [&](int64_t b, uint4 (&g)[kVecPerThread], uint4 (&u)[kVecPerThread]) {
#pragma unroll
    for (int j = 0; j < kVecPerThread; ++j) {
      const int64_t i = min(b + j * kThreads, n_vec - 1);
      g[j] = load_nt(gate + i);
      u[j] = load_nt(up + i);
    }
  };
  load(base, gv, uv);
  for (;;) {
    const int64_t next = base + stride;
    const bool more = next < n_vec;
    uint4 ng[kVecPerThread], nu[kVecPerThread];
    if (more) load(next, ng, nu);
#pragma unroll
    for (int j = 0; j < kVecPerThread; ++j) {
      const int64_t i = base + j * kThreads;
      float g[8], u[8], o[8];
      unpack8(gv[j], g);
      unpack8(uv[j], u);
#pragma unroll
      for (int e = 0; e < 8; ++e) o[e] = g[e] * sigmoid(g[e]) * u[e];
      if (i < n_vec) out[i] = pack8(o);
    }
    if (!more) break;
    base = next;
#pragma unroll
    for (int j = 0; j < kVecPerThread; ++j) {
      gv[j] = ng[j];
      uv[j] = nu[j];
    }
  }
}

__global__ __launch_bounds__(kThreads) void swiglu_bwd_vec(const uint4* grad, const uint4* gate,
                                                           const uint4* up, uint4* dgate,
                                                           uint4* dup, int64_t n_vec) {
  const int64_t stride = static_cast<int64_t>(gridDim.x) * kThreads * kVecPerThread;
  int64_t base = static_cast<int64_t>(blockIdx.x) * kThreads * kVecPerThread + threadIdx.x;
  if (base >= n_vec) return;
  uint4 dv[kVecPerThread], gv[kVecPerThread], uv[kVecPerThread];
  auto load = [&](int64_t b, uint4 (&d)[kVecPerThread], uint4 (&g)[kVecPerThread],
                  uint4 (&u)[kVecPerThread]) {
#pragma unroll
    for (int j = 0; j < kVecPerThread; ++j) {
      const int64_t i = min(b + j * kThreads, n_vec - 1);
      d[j] = load_nt(grad + i);
      g[j] = load_nt(gate + i);
      u[j] = load_nt(up + i);
    }
  };
  load(base, dv, gv, uv);
  for (;;) {
    const int64_t next = base + stride;
    const bool more = next < n_vec;
    uint4 nd[kVecPerThread], ng[kVecPerThread], nu[kVecPerThread];
    if (more) load(next, nd, ng, nu);
#pragma unroll
    for (int j = 0; j < kVecPerThread; ++j) {
      const int64_t i = base + j * kThreads;
      float d[8], g[8], u[8], dg[8], du[8];
      unpack8(dv[j], d);
      unpack8(gv[j], g);
      unpack8(uv[j], u);
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        const float sig = sigmoid(g[e]);
        du[e] = d[e] * g[e] * sig;
        dg[e] = d[e] * u[e] * sig * (1.0f + g[e] * (1.0f - sig));
      }
      if (i < n_vec) {
        dgate[i] = pack8(dg);
        dup[i] = pack8(du);
      }
    }
    if (!more) break;
    base = next;
#pragma unroll
    for (int j = 0; j < kVecPerThread; ++j) {
      dv[j] = nd[j];
      gv[j] = ng[j];
      uv[j] = nu[j];
    }
  }
}

// Scalar tail / unaligned path.
__global__ __launch_bounds__(kThreads) void swiglu_fwd_any(const uint16_t* gate, const uint16_t* up,
                                                           uint16_t* out, int64_t n) {
  const int64_t i = static_cast<int64_t>(blockIdx.x) * kThreads + threadIdx.x;
  if (i >= n) return;
  const float g = h2f(gate[i]);
  out[i] = f2h(g * sigmoid(g) * h2f(up[i]));
}

__global__ __launch_bounds__(kThreads) void swiglu_bwd_any(const uint16_t* grad, const uint16_t* gate,
                                                           const uint16_t* up, uint16_t* dgate,
                                                           uint16_t* dup, int64_t n) {
  const int64_t i = static_cast<int64_t>(blockIdx.x) * kThreads + threadIdx.x;
  if (i >= n) return;
  const float d = h2f(grad[i]), g = h2f(gate[i]), u = h2f(up[i]);
  const float sig = sigmoid(g);
  dgate[i] = f2h(d * u * sig * (1.0f + g * (1.0f - sig)));
  dup[i] = f2h(d * g * sig);
}

// Row-strided operands ([rows, cols] views, row strides in 16-byte vectors): one vector per
// thread, row = blockIdx.y. Used where gate and up are the two halves of one [rows, 2 cols]
// buffer (the fused MLP's gate|up GEMM output).
struct RowArgs {
  int64_t cols_vec, ld0, ld1, ld2, ld3, ld4;  // row strides of the operands in vectors
};

__global__ __launch_bounds__(kThreads) void swiglu_fwd_rows(const uint4* gate, const uint4* up,
                                                            uint4* out, RowArgs r) {
  const int64_t c = static_cast<int64_t>(blockIdx.x) * kThreads + threadIdx.x;
  if (c >= r.cols_vec) return;
  const int64_t row = blockIdx.y;
  const uint4 gv = load_nt(gate + row * r.ld0 + c), uv = load_nt(up + row * r.ld1 + c);
  float g[8], u[8], o[8];
  unpack8(gv, g);
  unpack8(uv, u);
#pragma unroll
  for (int e = 0; e < 8; ++e) o[e] = g[e] * sigmoid(g[e]) * u[e];
  out[row * r.ld2 + c] = pack8(o);
}

__global__ __launch_bounds__(kThreads) void swiglu_bwd_rows(const uint4* grad, const uint4* gate,
                                                            const uint4* up, uint4* dgate,
                                                            uint4* dup, RowArgs r) {
  const int64_t c = static_cast<int64_t>(blockIdx.x) * kThreads + threadIdx.x;
  if (c >= r.cols_vec) return;
  const int64_t row = blockIdx.y;
  const uint4 dv = load_nt(grad + row * r.ld0 + c), gv = load_nt(gate + row * r.ld1 + c),
              uv = load_nt(up + row * r.ld2 + c);
  float d[8], g[8], u[8], dg[8], du[8];
  unpack8(dv, d);
  unpack8(gv, g);
  unpack8(uv, u);
#pragma unroll
  for (int e = 0; e < 8; ++e) {
    const float sig = sigmoid(g[e]);
    du[e] = d[e] * g[e] * sig;
    dg[e] = d[e] * u[e] * sig * (1.0f + g[e] * (1.0f - sig));
  }
  dgate[row * r.ld3 + c] = pack8(dg);
  dup[row * r.ld4 + c] = pack8(du);
}

// Workgroups of a grid-stride launch: `per_cu` per CU (measured on config 3 at 4, 8 and 16: the
// forward runs best at 16, the backward at 4), fewer when the vectors run out first.
unsigned vec_blocks(int64_t n_vec, int per_cu) {
  const int64_t per_block = static_cast<int64_t>(kThreads) * kVecPerThread;
  const int64_t need = (n_vec + per_block - 1) / per_block;
  const int64_t cap = static_cast<int64_t>(per_cu) * device_cus();
  return static_cast<unsigned>(need < cap ? need : cap);
}

}  // namespace
}  // namespace talm

using namespace talm;

TALM_API int talm_swiglu_fwd(const uint16_t* gate, const uint16_t* up, uint16_t* out, int64_t n,
                             void* stream) {
  if (n < 0) return fail(TALM_EINVAL, "swiglu_fwd: n %lld < 0", (long long)n);
  if (n == 0) return ok();
  if (!gate || !up || !out) return fail(TALM_EINVAL, "swiglu_fwd: null pointer");
  const hipStream_t s = as_stream(stream);
  int64_t head = 0;
  if (aligned(gate, 16) && aligned(up, 16) && aligned(out, 16)) {
    const int64_t n_vec = n / 8;
    head = n_vec * 8;
    if (n_vec)
      hipLaunchKernelGGL(swiglu_fwd_vec, dim3(vec_blocks(n_vec, 16)), dim3(kThreads), 0, s,
                         reinterpret_cast<const uint4*>(gate), reinterpret_cast<const uint4*>(up),
                         reinterpret_cast<uint4*>(out), n_vec);
  }
  const int64_t tail = n - head;
  if (tail)
    hipLaunchKernelGGL(swiglu_fwd_any, dim3(static_cast<unsigned>((tail + kThreads - 1) / kThreads)),
                       dim3(kThreads), 0, s, gate + head, up + head, out + head, tail);
  return check_launch("swiglu_fwd");
}

TALM_API int talm_swiglu_bwd(const uint16_t* grad, const uint16_t* gate, const uint16_t* up,
                             uint16_t* dgate, uint16_t* dup, int64_t n, void* stream) {
  if (n < 0) return fail(TALM_EINVAL, "swiglu_bwd: n %lld < 0", (long long)n);
  if (n == 0) return ok();
  if (!grad || !gate || !up || !dgate || !dup) return fail(TALM_EINVAL, "swiglu_bwd: null pointer");
  const hipStream_t s = as_stream(stream);
  int64_t head = 0;
  if (aligned(grad, 16) && aligned(gate, 16) && aligned(up, 16) && aligned(dgate, 16) &&
      aligned(dup, 16)) {
    const int64_t n_vec = n / 8;
    head = n_vec * 8;
    if (n_vec)
      hipLaunchKernelGGL(swiglu_bwd_vec, dim3(vec_blocks(n_vec, 4)), dim3(kThreads), 0, s,
                         reinterpret_cast<const uint4*>(grad), reinterpret_cast<const uint4*>(gate),
                         reinterpret_cast<const uint4*>(up), reinterpret_cast<uint4*>(dgate),
                         reinterpret_cast<uint4*>(dup), n_vec);
  }
  const int64_t tail = n - head;
  if (tail)
    hipLaunchKernelGGL(swiglu_bwd_any, dim3(static_cast<unsigned>((tail + kThreads - 1) / kThreads)),
                       dim3(kThreads), 0, s, grad + head, gate + head, up + head, dgate + head,
                       dup + head, tail);
  return check_launch("swiglu_bwd");
}

namespace {
int rows_check(const char* what, int64_t rows, int64_t cols, std::initializer_list<int64_t> lds,
               std::initializer_list<const void*> ptrs) {
  if (rows < 0 || cols < 0 || cols % 8 || rows > 65535)
    return fail(TALM_EINVAL, "%s: rows %lld (<= 65535), cols %lld (a multiple of 8)", what,
                (long long)rows, (long long)cols);
  for (int64_t ld : lds)
    if (ld < cols || ld % 8)
      return fail(TALM_EINVAL, "%s: row strides at least cols and multiples of 8", what);
  for (const void* p : ptrs) {
    if (!p) return fail(TALM_EINVAL, "%s: null pointer", what);
    if (!aligned(p, 16)) return fail(TALM_EINVAL, "%s: operands 16-byte aligned", what);
  }
  return TALM_OK;
}
}  // namespace

TALM_API int talm_swiglu_fwd_rows(const uint16_t* gate, int64_t ld_gate, const uint16_t* up,
                                  int64_t ld_up, uint16_t* out, int64_t ld_out, int64_t rows,
                                  int64_t cols, void* stream) {
  if (rows == 0 || cols == 0) return ok();
  if (int st = rows_check("swiglu_fwd_rows", rows, cols, {ld_gate, ld_up, ld_out},
                          {gate, up, out}))
    return st;
  RowArgs r{cols / 8, ld_gate / 8, ld_up / 8, ld_out / 8, 0, 0};
  hipLaunchKernelGGL(swiglu_fwd_rows,
                     dim3(static_cast<unsigned>((r.cols_vec + kThreads - 1) / kThreads),
                          static_cast<unsigned>(rows)),
                     dim3(kThreads), 0, as_stream(stream), reinterpret_cast<const uint4*>(gate),
                     reinterpret_cast<const uint4*>(up), reinterpret_cast<uint4*>(out), r);
  return check_launch("swiglu_fwd_rows");
}

TALM_API int talm_swiglu_bwd_rows(const uint16_t* grad, int64_t ld_grad, const uint16_t* gate,
                                  int64_t ld_gate, const uint16_t* up, int64_t ld_up,
                                  uint16_t* dgate, int64_t ld_dgate, uint16_t* dup,
                                  int64_t ld_dup, int64_t rows, int64_t cols, void* stream) {
  if (rows == 0 || cols == 0) return ok();
  if (int st = rows_check("swiglu_bwd_rows", rows, cols,
                          {ld_grad, ld_gate, ld_up, ld_dgate, ld_dup},
                          {grad, gate, up, dgate, dup}))
    return st;
  RowArgs r{cols / 8, ld_grad / 8, ld_gate / 8, ld_up / 8, ld_dgate / 8, ld_dup / 8};
  hipLaunchKernelGGL(swiglu_bwd_rows,
                     dim3(static_cast<unsigned>((r.cols_vec + kThreads - 1) / kThreads),
                          static_cast<unsigned>(rows)),
                     dim3(kThreads), 0, as_stream(stream), reinterpret_cast<const uint4*>(grad),
                     reinterpret_cast<const uint4*>(gate), reinterpret_cast<const uint4*>(up),
                     reinterpret_cast<uint4*>(dgate), reinterpret_cast<uint4*>(dup), r);
  return check_launch("swiglu_bwd_rows");
}
