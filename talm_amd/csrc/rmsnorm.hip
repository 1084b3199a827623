// Fused (residual-add +) RMSNorm for gfx950, forward and backward.
//
// One wavefront owns one row: lane l holds the 8-column chunks l, l + 64, ... of the row in
// registers (16-byte loads of fp16, 32-byte of fp32), so every operand is read once and written
// once, and the two row reductions (sum of squares forward, sum of g * xhat backward) are wave64
// butterfly sums with no LDS and no barrier. Rows whose width is not a multiple of 8 or wider
// than kMaxChunks * 8 * 64 columns take a generic path that reads the row twice.
#include "common.h"

namespace talm {
namespace {

constexpr int kThreads = 256;            // four rows per workgroup
constexpr int kRowsPerBlock = kThreads / kWave;
constexpr int kMaxChunks = 8;            // vector path: rows up to 8 * 8 * 64 = 4096 columns

// Row operands are read with the non-temporal hint (each is read once; on gfx950 hinted loads
// stream from HBM faster, as measured on the SwiGLU kernels' mixes); the weight, which every row
// reads, and all stores stay ordinary.
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef float f32x4 __attribute__((ext_vector_type(4)));

template <typename T>
struct IO;

template <>
struct IO<float> {
  static __device__ __forceinline__ void load8(const float* p, float* v) {
    const float4 a = reinterpret_cast<const float4*>(p)[0];
    const float4 b = reinterpret_cast<const float4*>(p)[1];
    v[0] = a.x; v[1] = a.y; v[2] = a.z; v[3] = a.w;
    v[4] = b.x; v[5] = b.y; v[6] = b.z; v[7] = b.w;
  }
  static __device__ __forceinline__ void load8_nt(const float* p, float* v) {
    const f32x4 a = __builtin_nontemporal_load(reinterpret_cast<const f32x4*>(p));
    const f32x4 b = __builtin_nontemporal_load(reinterpret_cast<const f32x4*>(p) + 1);
    v[0] = a.x; v[1] = a.y; v[2] = a.z; v[3] = a.w;
    v[4] = b.x; v[5] = b.y; v[6] = b.z; v[7] = b.w;
  }
  static __device__ __forceinline__ void store8(float* p, const float* v) {
    reinterpret_cast<float4*>(p)[0] = make_float4(v[0], v[1], v[2], v[3]);
    reinterpret_cast<float4*>(p)[1] = make_float4(v[4], v[5], v[6], v[7]);
  }
  static __device__ __forceinline__ float load1(const float* p) { return *p; }
  static __device__ __forceinline__ void store1(float* p, float v) { *p = v; }
};

template <>
struct IO<uint16_t> {
  static __device__ __forceinline__ void load8(const uint16_t* p, float* v) {
    const uint4 a = *reinterpret_cast<const uint4*>(p);
    v[0] = lo_f(a.x); v[1] = hi_f(a.x); v[2] = lo_f(a.y); v[3] = hi_f(a.y);
    v[4] = lo_f(a.z); v[5] = hi_f(a.z); v[6] = lo_f(a.w); v[7] = hi_f(a.w);
  }
  static __device__ __forceinline__ void load8_nt(const uint16_t* p, float* v) {
    const u32x4 a = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(p));
    v[0] = lo_f(a.x); v[1] = hi_f(a.x); v[2] = lo_f(a.y); v[3] = hi_f(a.y);
    v[4] = lo_f(a.z); v[5] = hi_f(a.z); v[6] = lo_f(a.w); v[7] = hi_f(a.w);
  }
  static __device__ __forceinline__ void store8(uint16_t* p, const float* v) {
    *reinterpret_cast<uint4*>(p) =
        make_uint4(pack2(v[0], v[1]), pack2(v[2], v[3]), pack2(v[4], v[5]), pack2(v[6], v[7]));
  }
  static __device__ __forceinline__ float load1(const uint16_t* p) { return h2f(*p); }
  static __device__ __forceinline__ void store1(uint16_t* p, float v) { *p = f2h(v); }
};

// Forward, vector path, NC 8-column chunks per lane (NC = ceil(chunks / 64)). x = a (+ p);
// q = x; h = w * xhat; xhat = x * rstd. Every load of the row is issued before any is used:
// chunk indices past the row are clamped to its last chunk (their values are masked out and
// their stores skipped), so no load waits behind a branch.
template <typename XT, typename OT, typename WT, bool ADD, int NC>
__global__ __launch_bounds__(kThreads) void rms_fwd_vec(const XT* __restrict__ a,
                                                        const OT* __restrict__ p, XT* __restrict__ q,
                                                        OT* __restrict__ h, OT* __restrict__ xhat,
                                                        const WT* __restrict__ w,
                                                        float* __restrict__ rstd, int64_t n_rows,
                                                        int n_cols, float eps) {
  const int lane = threadIdx.x % kWave;
  const int64_t row = static_cast<int64_t>(blockIdx.x) * kRowsPerBlock + threadIdx.x / kWave;
  if (row >= n_rows) return;
  const int n_chunks = n_cols / 8;
  const int64_t at = row * n_cols;
  float x[NC][8], wv[NC][8];
#pragma unroll
  for (int i = 0; i < NC; ++i) {
    const int c = min(lane + kWave * i, n_chunks - 1);
    IO<XT>::load8_nt(a + at + 8 * c, x[i]);
    IO<WT>::load8(w + 8 * c, wv[i]);
    if constexpr (ADD) {
      float pv[8];
      IO<OT>::load8_nt(p + at + 8 * c, pv);
#pragma unroll
      for (int e = 0; e < 8; ++e) x[i][e] += pv[e];
    }
  }
  float ss = 0.f;
#pragma unroll
  for (int i = 0; i < NC; ++i) {
    const int c = lane + kWave * i;
    if (c < n_chunks) {
      if constexpr (ADD) IO<XT>::store8(q + at + 8 * c, x[i]);
#pragma unroll
      for (int e = 0; e < 8; ++e) ss += x[i][e] * x[i][e];
    }
  }
  ss = wave_sum(ss);
  const float r = rsqrtf(ss / static_cast<float>(n_cols) + eps);
  if (lane == 0) rstd[row] = r;
#pragma unroll
  for (int i = 0; i < NC; ++i) {
    const int c = lane + kWave * i;
    if (c < n_chunks) {
      float xh[8], y[8];
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        xh[e] = x[i][e] * r;
        y[e] = wv[i][e] * xh[e];
      }
      IO<OT>::store8(h + at + 8 * c, y);
      IO<OT>::store8(xhat + at + 8 * c, xh);
    }
  }
}

// Backward, vector path. g = dy * w; dx = rstd * (g - xhat * mean(g * xhat)) (+ ds -> p; no q:
// ds = 0).
// Loads first, as in the forward.
template <typename XT, typename OT, typename WT, bool ADD, int NC>
__global__ __launch_bounds__(kThreads) void rms_bwd_vec(XT* __restrict__ a, OT* __restrict__ p,
                                                        const XT* __restrict__ q,
                                                        const OT* __restrict__ h,
                                                        const OT* __restrict__ xhat,
                                                        const WT* __restrict__ w,
                                                        const float* __restrict__ rstd,
                                                        int64_t n_rows, int n_cols) {
  const int lane = threadIdx.x % kWave;
  const int64_t row = static_cast<int64_t>(blockIdx.x) * kRowsPerBlock + threadIdx.x / kWave;
  if (row >= n_rows) return;
  const int n_chunks = n_cols / 8;
  const int64_t at = row * n_cols;
  float g[NC][8], xh[NC][8], ds[NC][8];
#pragma unroll
  for (int i = 0; i < NC; ++i) {
    const int c = min(lane + kWave * i, n_chunks - 1);
    float wv[8];
    IO<OT>::load8_nt(h + at + 8 * c, g[i]);
    IO<OT>::load8_nt(xhat + at + 8 * c, xh[i]);
    IO<WT>::load8(w + 8 * c, wv);
    if constexpr (ADD) {
      if (q) {
        IO<XT>::load8_nt(q + at + 8 * c, ds[i]);
      } else {
#pragma unroll
        for (int e = 0; e < 8; ++e) ds[i][e] = 0.f;  // no sum gradient: ds = 0
      }
    }
#pragma unroll
    for (int e = 0; e < 8; ++e) g[i][e] *= wv[e];
  }
  const float r = rstd[row];
  float dot = 0.f;
#pragma unroll
  for (int i = 0; i < NC; ++i)
    if (lane + kWave * i < n_chunks)
#pragma unroll
      for (int e = 0; e < 8; ++e) dot += g[i][e] * xh[i][e];
  const float cmean = wave_sum(dot) / static_cast<float>(n_cols);
#pragma unroll
  for (int i = 0; i < NC; ++i) {
    const int c = lane + kWave * i;
    if (c < n_chunks) {
      float dx[8];
#pragma unroll
      for (int e = 0; e < 8; ++e) dx[e] = r * (g[i][e] - xh[i][e] * cmean);
      if constexpr (ADD) {
#pragma unroll
        for (int e = 0; e < 8; ++e) dx[e] += ds[i][e];
        IO<OT>::store8(p + at + 8 * c, dx);
      }
      IO<XT>::store8(a + at + 8 * c, dx);
    }
  }
}

// Generic path (any width): the row is read twice, one element per lane per step.
template <typename XT, typename OT, typename WT, bool ADD>
__global__ __launch_bounds__(kThreads) void rms_fwd_any(const XT* __restrict__ a,
                                                        const OT* __restrict__ p, XT* __restrict__ q,
                                                        OT* __restrict__ h, OT* __restrict__ xhat,
                                                        const WT* __restrict__ w,
                                                        float* __restrict__ rstd, int64_t n_rows,
                                                        int n_cols, float eps) {
  const int lane = threadIdx.x % kWave;
  const int64_t row = static_cast<int64_t>(blockIdx.x) * kRowsPerBlock + threadIdx.x / kWave;
  if (row >= n_rows) return;
  const int64_t at = row * n_cols;
  float ss = 0.f;
  for (int j = lane; j < n_cols; j += kWave) {
    float x = IO<XT>::load1(a + at + j);
    if constexpr (ADD) {
      x += IO<OT>::load1(p + at + j);
      IO<XT>::store1(q + at + j, x);
    }
    ss += x * x;
  }
  ss = wave_sum(ss);
  const float r = rsqrtf(ss / static_cast<float>(n_cols) + eps);
  if (lane == 0) rstd[row] = r;
  for (int j = lane; j < n_cols; j += kWave) {
    float x = IO<XT>::load1(a + at + j);
    if constexpr (ADD) x += IO<OT>::load1(p + at + j);
    const float xh = x * r;
    IO<OT>::store1(h + at + j, IO<WT>::load1(w + j) * xh);
    IO<OT>::store1(xhat + at + j, xh);
  }
}

template <typename XT, typename OT, typename WT, bool ADD>
__global__ __launch_bounds__(kThreads) void rms_bwd_any(XT* __restrict__ a, OT* __restrict__ p,
                                                        const XT* __restrict__ q,
                                                        const OT* __restrict__ h,
                                                        const OT* __restrict__ xhat,
                                                        const WT* __restrict__ w,
                                                        const float* __restrict__ rstd,
                                                        int64_t n_rows, int n_cols) {
  const int lane = threadIdx.x % kWave;
  const int64_t row = static_cast<int64_t>(blockIdx.x) * kRowsPerBlock + threadIdx.x / kWave;
  if (row >= n_rows) return;
  const int64_t at = row * n_cols;
  float dot = 0.f;
  for (int j = lane; j < n_cols; j += kWave)
    dot += IO<OT>::load1(h + at + j) * IO<WT>::load1(w + j) * IO<OT>::load1(xhat + at + j);
  const float cmean = wave_sum(dot) / static_cast<float>(n_cols);
  const float r = rstd[row];
  for (int j = lane; j < n_cols; j += kWave) {
    const float g = IO<OT>::load1(h + at + j) * IO<WT>::load1(w + j);
    float dx = r * (g - IO<OT>::load1(xhat + at + j) * cmean);
    if constexpr (ADD) {
      if (q) dx += IO<XT>::load1(q + at + j);
      IO<OT>::store1(p + at + j, dx);
    }
    IO<XT>::store1(a + at + j, dx);
  }
}

template <typename XT, typename OT, typename WT, bool ADD>
void launch(void* a, void* q, void* h, void* xhat, void* p, const void* weight, float* rstd,
            int64_t n_rows, int n_cols, float eps, bool backward, bool vec, hipStream_t s) {
  const dim3 grid(static_cast<unsigned>((n_rows + kRowsPerBlock - 1) / kRowsPerBlock));
  const dim3 block(kThreads);
  XT* ax = static_cast<XT*>(a);
  XT* qx = static_cast<XT*>(q);
  OT* ho = static_cast<OT*>(h);
  OT* xo = static_cast<OT*>(xhat);
  OT* po = static_cast<OT*>(p);
  const WT* wv = static_cast<const WT*>(weight);
  const int nc = (n_cols / 8 + kWave - 1) / kWave;  // chunks per lane on the vector path
  if (!backward) {
    if (vec) {
      switch (nc) {
#define TALM_RMS_FWD(NC)                                                                          \
  case NC:                                                                                        \
    hipLaunchKernelGGL((rms_fwd_vec<XT, OT, WT, ADD, NC>), grid, block, 0, s, ax, po, qx, ho, xo, \
                       wv, rstd, n_rows, n_cols, eps);                                            \
    break;
        TALM_RMS_FWD(1) TALM_RMS_FWD(2) TALM_RMS_FWD(3) TALM_RMS_FWD(4)
        TALM_RMS_FWD(5) TALM_RMS_FWD(6) TALM_RMS_FWD(7) TALM_RMS_FWD(8)
#undef TALM_RMS_FWD
      }
    } else
      hipLaunchKernelGGL((rms_fwd_any<XT, OT, WT, ADD>), grid, block, 0, s, ax, po, qx, ho, xo, wv,
                         rstd, n_rows, n_cols, eps);
  } else {
    if (vec) {
      switch (nc) {
#define TALM_RMS_BWD(NC)                                                                          \
  case NC:                                                                                        \
    hipLaunchKernelGGL((rms_bwd_vec<XT, OT, WT, ADD, NC>), grid, block, 0, s, ax, po, qx, ho, xo, \
                       wv, rstd, n_rows, n_cols);                                                 \
    break;
        TALM_RMS_BWD(1) TALM_RMS_BWD(2) TALM_RMS_BWD(3) TALM_RMS_BWD(4)
        TALM_RMS_BWD(5) TALM_RMS_BWD(6) TALM_RMS_BWD(7) TALM_RMS_BWD(8)
#undef TALM_RMS_BWD
      }
    } else
      hipLaunchKernelGGL((rms_bwd_any<XT, OT, WT, ADD>), grid, block, 0, s, ax, po, qx, ho, xo, wv,
                         rstd, n_rows, n_cols);
  }
}

template <typename XT, typename OT, typename WT>
void dispatch_add(bool add, void* a, void* q, void* h, void* xhat, void* p, const void* weight,
                  float* rstd, int64_t n_rows, int n_cols, float eps, bool backward, bool vec,
                  hipStream_t s) {
  if (add)
    launch<XT, OT, WT, true>(a, q, h, xhat, p, weight, rstd, n_rows, n_cols, eps, backward, vec, s);
  else
    launch<XT, OT, WT, false>(a, q, h, xhat, p, weight, rstd, n_rows, n_cols, eps, backward, vec, s);
}

template <typename XT, typename OT>
void dispatch_w(int w_dtype, bool add, void* a, void* q, void* h, void* xhat, void* p,
                const void* weight, float* rstd, int64_t n_rows, int n_cols, float eps,
                bool backward, bool vec, hipStream_t s) {
  if (w_dtype == TALM_F32)
    dispatch_add<XT, OT, float>(add, a, q, h, xhat, p, weight, rstd, n_rows, n_cols, eps, backward, vec, s);
  else
    dispatch_add<XT, OT, uint16_t>(add, a, q, h, xhat, p, weight, rstd, n_rows, n_cols, eps, backward, vec, s);
}

}  // namespace
}  // namespace talm

using namespace talm;

TALM_API int talm_rmsnorm(void* a, void* q, void* h, void* xhat, void* p, const void* weight,
                          float* rstd, int64_t n_rows, int64_t n_cols, int32_t x_dtype,
                          int32_t out_dtype, int32_t w_dtype, float eps, int32_t backward,
                          int32_t add, void* stream) {
  for (int32_t dt : {x_dtype, out_dtype, w_dtype})
    if (dt != TALM_F32 && dt != TALM_F16) return fail(TALM_EINVAL, "rmsnorm: unsupported dtype code %d", dt);
  if (n_rows < 0 || n_cols < 1 || n_cols > (1 << 24))
    return fail(TALM_EINVAL, "rmsnorm: bad shape [%lld, %lld]", (long long)n_rows, (long long)n_cols);
  if (n_rows == 0) return ok();
  if (!a || !h || !xhat || !weight || !rstd || (add && (!p || (!q && !backward))))
    return fail(TALM_EINVAL, "rmsnorm: null pointer");
  const bool vec = n_cols % 8 == 0 && n_cols <= kMaxChunks * 8 * kWave && aligned(a, 16) &&
                   aligned(h, 16) && aligned(xhat, 16) && aligned(weight, 16) &&
                   (!add || (aligned(p, 16) && aligned(q, 16)));
  const hipStream_t s = as_stream(stream);
  const int cols = static_cast<int>(n_cols);
  const bool bwd = backward != 0, ad = add != 0;
  if (x_dtype == TALM_F32 && out_dtype == TALM_F16)
    dispatch_w<float, uint16_t>(w_dtype, ad, a, q, h, xhat, p, weight, rstd, n_rows, cols, eps, bwd, vec, s);
  else if (x_dtype == TALM_F32 && out_dtype == TALM_F32)
    dispatch_w<float, float>(w_dtype, ad, a, q, h, xhat, p, weight, rstd, n_rows, cols, eps, bwd, vec, s);
  else if (x_dtype == TALM_F16 && out_dtype == TALM_F16)
    dispatch_w<uint16_t, uint16_t>(w_dtype, ad, a, q, h, xhat, p, weight, rstd, n_rows, cols, eps, bwd, vec, s);
  else
    dispatch_w<uint16_t, float>(w_dtype, ad, a, q, h, xhat, p, weight, rstd, n_rows, cols, eps, bwd, vec, s);
  return check_launch("rmsnorm");
}

namespace talm {
namespace {

// The split-K forms: the branch (forward) or dy (backward) of a row given as a split-K GEMM's
// fp32 K-part partials [parts][n_rows][n_cols], summed in part order from +0 and rounded to
// fp16 (the values splitk_reduce_kernel would write for the vector kernels to read back), for
// XT fp32 (the residual stream) and OT fp16 (autocast). One workgroup per row and one 8-column
// chunk per thread (chunk 64 w + l in lane l of wavefront w), so there are as many threads in
// flight as in the plain reduction. The row's reduction is folded in the vector kernels' order
// (lane l accumulates chunks l, l + 64, ... in turn: wavefront w continues the fold of w - 1,
// handed over through LDS), then the same butterfly: the results are those of the reduction
// followed by the vector kernel, bit for bit.
template <int NW>
__device__ __forceinline__ float fold_row(float f, const float (&x)[8], const float (&y)[8],
                                          bool live, float* handoff) {
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
#pragma unroll
  for (int w = 0; w < NW; ++w) {
    if (wave == w) {
      if (w > 0) f = handoff[lane];
      if (live)
#pragma unroll
        for (int e = 0; e < 8; ++e) f += x[e] * y[e];
      if (w < NW - 1) handoff[lane] = f;
    }
    if (w < NW - 1) __syncthreads();
  }
  return f;  // the lane's whole fold in the last wavefront
}

__device__ __forceinline__ void part_sum8(const float* __restrict__ part, int parts, int64_t mn,
                                          int64_t at, float (&v)[8]) {
  float s[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
  for (int k0 = 0; k0 < parts; k0 += 8) {
    float t[8][8];
#pragma unroll
    for (int kk = 0; kk < 8; ++kk)
      IO<float>::load8_nt(part + static_cast<int64_t>(min(k0 + kk, parts - 1)) * mn + at, t[kk]);
#pragma unroll
    for (int kk = 0; kk < 8; ++kk) {
      const bool live = k0 + kk < parts;  // a part past the last adds +0
#pragma unroll
      for (int e = 0; e < 8; ++e) s[e] += live ? t[kk][e] : 0.f;
    }
  }
#pragma unroll
  for (int e = 0; e < 8; ++e) v[e] = h2f(f2h(s[e]));
}

template <typename WT, int NW>
__global__ __launch_bounds__(64 * NW) void rms_fwd_parts(
    const float* __restrict__ part, int parts, const float* __restrict__ a,
    const WT* __restrict__ w, float* __restrict__ q, uint16_t* __restrict__ h,
    uint16_t* __restrict__ xhat, float* __restrict__ rstd, int64_t n_rows, int n_cols,
    float eps) {
  __shared__ float handoff[kWave];
  __shared__ float r_shared;
  const int64_t row = blockIdx.x;
  const int n_chunks = n_cols / 8;
  const int c = static_cast<int>(threadIdx.x), cc = min(c, n_chunks - 1);
  const bool live = c < n_chunks;
  const int64_t at = row * n_cols + 8 * cc;
  float x[8], wv[8], pv[8];
  IO<float>::load8_nt(a + at, x);
  IO<WT>::load8(w + 8 * cc, wv);
  part_sum8(part, parts, n_rows * n_cols, at, pv);
#pragma unroll
  for (int e = 0; e < 8; ++e) x[e] += pv[e];
  if (live) IO<float>::store8(q + at, x);
  float ss = fold_row<NW>(0.f, x, x, live, handoff);
  if ((threadIdx.x >> 6) == NW - 1) {
    ss = wave_sum(ss);
    if ((threadIdx.x & 63) == 0) {
      const float r = rsqrtf(ss / static_cast<float>(n_cols) + eps);
      rstd[row] = r;
      r_shared = r;
    }
  }
  __syncthreads();
  const float r = r_shared;
  if (live) {
    float xh[8], y[8];
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      xh[e] = x[e] * r;
      y[e] = wv[e] * xh[e];
    }
    IO<uint16_t>::store8(h + at, y);
    IO<uint16_t>::store8(xhat + at, xh);
  }
}

template <typename WT, int NW>
__global__ __launch_bounds__(64 * NW) void rms_bwd_parts(
    const float* __restrict__ part, int parts, const uint16_t* __restrict__ xhat,
    const WT* __restrict__ w, const float* __restrict__ rstd, const float* __restrict__ ds,
    float* __restrict__ dx, uint16_t* __restrict__ dbranch, int64_t n_rows, int n_cols) {
  __shared__ float handoff[kWave];
  __shared__ float m_shared;
  const int64_t row = blockIdx.x;
  const int n_chunks = n_cols / 8;
  const int c = static_cast<int>(threadIdx.x), cc = min(c, n_chunks - 1);
  const bool live = c < n_chunks;
  const int64_t at = row * n_cols + 8 * cc;
  float xh[8], wv[8], dsv[8], g[8];
  IO<uint16_t>::load8_nt(xhat + at, xh);
  IO<WT>::load8(w + 8 * cc, wv);
  if (ds) {
    IO<float>::load8_nt(ds + at, dsv);
  } else {
#pragma unroll
    for (int e = 0; e < 8; ++e) dsv[e] = 0.f;  // no sum gradient: ds = 0
  }
  part_sum8(part, parts, n_rows * n_cols, at, g);
#pragma unroll
  for (int e = 0; e < 8; ++e) g[e] *= wv[e];
  float dot = fold_row<NW>(0.f, g, xh, live, handoff);
  if ((threadIdx.x >> 6) == NW - 1) {
    dot = wave_sum(dot);
    if ((threadIdx.x & 63) == 0) m_shared = dot / static_cast<float>(n_cols);
  }
  __syncthreads();
  const float cmean = m_shared, r = rstd[row];
  if (live) {
    float d[8];
#pragma unroll
    for (int e = 0; e < 8; ++e) d[e] = r * (g[e] - xh[e] * cmean);
#pragma unroll
    for (int e = 0; e < 8; ++e) d[e] += dsv[e];
    IO<uint16_t>::store8(dbranch + at, d);
    IO<float>::store8(dx + at, d);
  }
}

template <typename WT, bool BWD>
void launch_parts(const float* part, int parts, const float* resid, const float* ds,
                  const uint16_t* xhat_in, const void* weight, int64_t n_rows, int n_cols,
                  float eps, float* x_out, uint16_t* h, uint16_t* xhat, float* rstd,
                  hipStream_t s) {
  const dim3 grid(static_cast<unsigned>(n_rows));
  const WT* w = static_cast<const WT*>(weight);
  const int nw = (n_cols / 8 + kWave - 1) / kWave;
  switch (nw) {
#define TALM_RMS_PARTS(NW)                                                                  \
  case NW:                                                                                  \
    if constexpr (BWD)                                                                      \
      hipLaunchKernelGGL((rms_bwd_parts<WT, NW>), grid, dim3(64 * NW), 0, s, part, parts,   \
                         xhat_in, w, rstd, ds, x_out, h, n_rows, n_cols);                   \
    else                                                                                    \
      hipLaunchKernelGGL((rms_fwd_parts<WT, NW>), grid, dim3(64 * NW), 0, s, part, parts,   \
                         resid, w, x_out, h, xhat, rstd, n_rows, n_cols, eps);              \
    break;
    TALM_RMS_PARTS(1) TALM_RMS_PARTS(2) TALM_RMS_PARTS(3) TALM_RMS_PARTS(4)
#undef TALM_RMS_PARTS
  }
}

int check_parts(const char* what, const float* part, int32_t parts, int64_t n_rows,
                int64_t n_cols, int32_t w_dtype, const void* weight) {
  if (w_dtype != TALM_F32 && w_dtype != TALM_F16)
    return fail(TALM_EINVAL, "%s: unsupported weight dtype code %d", what, w_dtype);
  if (parts < 1 || parts > 4096 || n_rows < 0 || n_cols < 8 || n_cols % 8 || n_cols > 2048 ||
      n_rows * n_cols > (int64_t{1} << 40))
    return fail(TALM_EINVAL,
                "%s: bad shape (parts %d, rows %lld, columns %lld): columns a multiple of 8, at "
                "most 2048",
                what, parts, (long long)n_rows, (long long)n_cols);
  if (n_rows > 0 && (!part || !weight)) return fail(TALM_EINVAL, "%s: null pointer", what);
  if (!aligned(part, 16) || !aligned(weight, 16))
    return fail(TALM_EINVAL, "%s: partials and weight must be 16-byte aligned", what);
  return TALM_OK;
}

}  // namespace
}  // namespace talm

TALM_API int talm_splitk_add_rmsnorm(const float* partials, int32_t parts, const float* resid,
                                     const void* weight, int32_t w_dtype, float eps,
                                     int64_t n_rows, int64_t n_cols, float* sum_out,
                                     uint16_t* h, uint16_t* xhat, float* rstd, void* stream) {
  if (check_parts("splitk_add_rmsnorm", partials, parts, n_rows, n_cols, w_dtype, weight))
    return TALM_EINVAL;
  if (n_rows == 0) return ok();
  if (!resid || !sum_out || !h || !xhat || !rstd)
    return fail(TALM_EINVAL, "splitk_add_rmsnorm: null pointer");
  if (!aligned(resid, 16) || !aligned(sum_out, 16) || !aligned(h, 16) || !aligned(xhat, 16))
    return fail(TALM_EINVAL, "splitk_add_rmsnorm: row operands must be 16-byte aligned");
  const hipStream_t s = as_stream(stream);
  if (w_dtype == TALM_F32)
    launch_parts<float, false>(partials, parts, resid, nullptr, nullptr, weight, n_rows,
                               static_cast<int>(n_cols), eps, sum_out, h, xhat, rstd, s);
  else
    launch_parts<uint16_t, false>(partials, parts, resid, nullptr, nullptr, weight, n_rows,
                                  static_cast<int>(n_cols), eps, sum_out, h, xhat, rstd, s);
  return check_launch("splitk_add_rmsnorm");
}

TALM_API int talm_splitk_rmsnorm_bwd(const float* partials, int32_t parts, const uint16_t* xhat,
                                     const float* rstd, const void* weight, int32_t w_dtype,
                                     const float* ds, int64_t n_rows, int64_t n_cols, float* dx,
                                     uint16_t* dbranch, void* stream) {
  if (check_parts("splitk_rmsnorm_bwd", partials, parts, n_rows, n_cols, w_dtype, weight))
    return TALM_EINVAL;
  if (n_rows == 0) return ok();
  if (!xhat || !rstd || !dx || !dbranch)
    return fail(TALM_EINVAL, "splitk_rmsnorm_bwd: null pointer");
  if (!aligned(xhat, 16) || !aligned(dx, 16) || !aligned(dbranch, 16) || !aligned(ds, 16))
    return fail(TALM_EINVAL, "splitk_rmsnorm_bwd: row operands must be 16-byte aligned");
  const hipStream_t s = as_stream(stream);
  if (w_dtype == TALM_F32)
    launch_parts<float, true>(partials, parts, nullptr, ds, xhat, weight, n_rows,
                              static_cast<int>(n_cols), 0.f, dx, dbranch, nullptr,
                              const_cast<float*>(rstd), s);
  else
    launch_parts<uint16_t, true>(partials, parts, nullptr, ds, xhat, weight, n_rows,
                                 static_cast<int>(n_cols), 0.f, dx, dbranch, nullptr,
                                 const_cast<float*>(rstd), s);
  return check_launch("splitk_rmsnorm_bwd");
}
