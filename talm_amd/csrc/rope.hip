// Rotary position embedding of q and k for gfx950, forward and backward, in place or out of
// place. One thread owns 8 rotation pairs (columns d and d + D/2 of one head of one token): it
// loads both 16-byte halves and the matching 32-byte cos/sin pieces, rotates in fp32 and writes
// both halves back, so an in-place launch never reads what another thread wrote. The 14 heads of
// a token are consecutive threads: their q/k rows are contiguous in the projection output and
// the token's cos/sin rows are fetched from HBM once and then served from L2 / L1.
#include "common.h"

namespace talm {
namespace {

constexpr int kThreads = 256;

struct Geometry {
  int64_t n_tokens;
  int n_q_heads, n_heads, half, chunks;  // chunks: 8-pair groups per head (vector) or pairs
  int64_t qs_t, qs_h, ks_t, ks_h, oqs_t, oqs_h, oks_t, oks_h, cs_t;
};

__device__ __forceinline__ void rotate(float x1, float x2, float c1, float c2, float s1, float s2,
                                       bool backward, float& y1, float& y2) {
  if (!backward) {
    y1 = x1 * c1 - x2 * s1;
    y2 = x2 * c2 + x1 * s2;
  } else {
    y1 = x1 * c1 + x2 * s2;
    y2 = x2 * c2 - x1 * s1;
  }
}

__device__ __forceinline__ void load8f(const float* p, float* v) {
  const float4 a = reinterpret_cast<const float4*>(p)[0];
  const float4 b = reinterpret_cast<const float4*>(p)[1];
  v[0] = a.x; v[1] = a.y; v[2] = a.z; v[3] = a.w;
  v[4] = b.x; v[5] = b.y; v[6] = b.z; v[7] = b.w;
}

template <bool VEC>
__global__ __launch_bounds__(kThreads) void rope_kernel(const uint16_t* q, const uint16_t* k,
                                                        const float* __restrict__ cos,
                                                        const float* __restrict__ sin,
                                                        uint16_t* out_q, uint16_t* out_k,
                                                        Geometry g, int backward) {
  const int64_t idx = static_cast<int64_t>(blockIdx.x) * kThreads + threadIdx.x;
  const int64_t per_token = static_cast<int64_t>(g.n_heads) * g.chunks;
  if (idx >= g.n_tokens * per_token) return;
  const int64_t t = idx / per_token;
  const int rem = static_cast<int>(idx - t * per_token);
  const int head = rem / g.chunks;
  const int c = rem - head * g.chunks;
  const uint16_t* src;
  uint16_t* dst;
  if (head < g.n_q_heads) {
    src = q + t * g.qs_t + head * g.qs_h;
    dst = out_q + t * g.oqs_t + head * g.oqs_h;
  } else {
    const int kh = head - g.n_q_heads;
    src = k + t * g.ks_t + kh * g.ks_h;
    dst = out_k + t * g.oks_t + kh * g.oks_h;
  }
  const float* cs = cos + t * g.cs_t;
  const float* sn = sin + t * g.cs_t;
  const bool bwd = backward != 0;
  if constexpr (VEC) {
    const int d = 8 * c;
    // q / k with the non-temporal hint (read once, then written in place); cos / sin, which the
    // token's 14 heads share, ordinary
    typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
    const u32x4 av = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(src + d));
    const u32x4 bv = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(src + g.half + d));
    const uint4 a = make_uint4(av.x, av.y, av.z, av.w);
    const uint4 b = make_uint4(bv.x, bv.y, bv.z, bv.w);
    float c1[8], c2[8], s1[8], s2[8];
    load8f(cs + d, c1);
    load8f(cs + g.half + d, c2);
    load8f(sn + d, s1);
    load8f(sn + g.half + d, s2);
    const uint32_t aw[4] = {a.x, a.y, a.z, a.w};
    const uint32_t bw[4] = {b.x, b.y, b.z, b.w};
    uint32_t ow1[4], ow2[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      float y1a, y2a, y1b, y2b;
      rotate(lo_f(aw[i]), lo_f(bw[i]), c1[2 * i], c2[2 * i], s1[2 * i], s2[2 * i], bwd, y1a, y2a);
      rotate(hi_f(aw[i]), hi_f(bw[i]), c1[2 * i + 1], c2[2 * i + 1], s1[2 * i + 1], s2[2 * i + 1],
             bwd, y1b, y2b);
      ow1[i] = pack2(y1a, y1b);
      ow2[i] = pack2(y2a, y2b);
    }
    *reinterpret_cast<uint4*>(dst + d) = make_uint4(ow1[0], ow1[1], ow1[2], ow1[3]);
    *reinterpret_cast<uint4*>(dst + g.half + d) = make_uint4(ow2[0], ow2[1], ow2[2], ow2[3]);
  } else {
    const int d = c;
    const float x1 = h2f(src[d]), x2 = h2f(src[g.half + d]);
    float y1, y2;
    rotate(x1, x2, cs[d], cs[g.half + d], sn[d], sn[g.half + d], bwd, y1, y2);
    dst[d] = f2h(y1);
    dst[g.half + d] = f2h(y2);
  }
}

// The rotary tables themselves, as transformers' rotary embedding computes them for the default
// (and statically scaled) types: angle = inv_freq[j] * float(position) in fp32 (its K = 1
// product), cos / sin of it (the same libm calls) times the attention scaling, written to
// columns j and j + half of the token's row. One thread per (token, j).
__global__ __launch_bounds__(kThreads) void rope_table_kernel(
    const int64_t* __restrict__ pos, int64_t n, const float* __restrict__ inv_freq, int half,
    float scaling, float* __restrict__ cos_out, float* __restrict__ sin_out) {
  const int64_t i = static_cast<int64_t>(blockIdx.x) * kThreads + threadIdx.x;
  if (i >= n * half) return;
  const int64_t t = i / half;
  const int j = static_cast<int>(i - t * half);
  const float angle = mul_f32(inv_freq[j], static_cast<float>(pos[t]));
  const float c = mul_f32(cosf(angle), scaling), sn = mul_f32(sinf(angle), scaling);
  float* crow = cos_out + t * 2 * half;
  float* srow = sin_out + t * 2 * half;
  crow[j] = c;
  crow[j + half] = c;
  srow[j] = sn;
  srow[j + half] = sn;
}

}  // namespace
}  // namespace talm

using namespace talm;

TALM_API int talm_rope_table(const int64_t* positions, int64_t n_tokens, const float* inv_freq,
                             int32_t half, float scaling, float* cos, float* sin, void* stream) {
  if (n_tokens < 0 || half < 1 || half > 4096 || n_tokens * half >= (int64_t{1} << 40))
    return fail(TALM_EINVAL, "rope_table: bad shape tokens=%lld half=%d", (long long)n_tokens,
                half);
  if (n_tokens == 0) return ok();
  if (!positions || !inv_freq || !cos || !sin) return fail(TALM_EINVAL, "rope_table: null pointer");
  const int64_t blocks = (n_tokens * half + kThreads - 1) / kThreads;
  if (blocks > 0x7fffffff) return fail(TALM_EINVAL, "rope_table: too many tokens");
  hipLaunchKernelGGL(rope_table_kernel, dim3(static_cast<unsigned>(blocks)), dim3(kThreads), 0,
                     as_stream(stream), positions, n_tokens, inv_freq, half, scaling, cos, sin);
  return check_launch("rope_table");
}

TALM_API int talm_rope(const uint16_t* q, const uint16_t* k, const float* cos, const float* sin,
                       uint16_t* out_q, uint16_t* out_k, int64_t n_tokens, int32_t n_q_heads,
                       int32_t n_k_heads, int32_t head_dim, int64_t q_stride_tok,
                       int64_t q_stride_head, int64_t k_stride_tok, int64_t k_stride_head,
                       int64_t out_q_stride_tok, int64_t out_q_stride_head,
                       int64_t out_k_stride_tok, int64_t out_k_stride_head,
                       int64_t cs_stride_tok, int32_t backward, void* stream) {
  if (n_tokens < 0 || n_q_heads < 0 || n_k_heads < 0 || head_dim < 2 || head_dim % 2 ||
      head_dim > 512)
    return fail(TALM_EINVAL, "rope: bad shape tokens=%lld heads=%d+%d head_dim=%d",
                (long long)n_tokens, n_q_heads, n_k_heads, head_dim);
  if (n_tokens == 0 || n_q_heads + n_k_heads == 0) return ok();
  if (!cos || !sin || (n_q_heads && (!q || !out_q)) || (n_k_heads && (!k || !out_k)))
    return fail(TALM_EINVAL, "rope: null pointer");
  Geometry g{n_tokens, n_q_heads, n_q_heads + n_k_heads, head_dim / 2, 0,
             q_stride_tok, q_stride_head, k_stride_tok, k_stride_head,
             out_q_stride_tok, out_q_stride_head, out_k_stride_tok, out_k_stride_head,
             cs_stride_tok};
  bool vec = g.half % 8 == 0 && cs_stride_tok % 4 == 0 && aligned(cos, 16) && aligned(sin, 16);
  const int64_t hstrides[] = {q_stride_tok, q_stride_head, k_stride_tok, k_stride_head,
                              out_q_stride_tok, out_q_stride_head, out_k_stride_tok,
                              out_k_stride_head};
  for (int64_t st : hstrides) vec = vec && st % 8 == 0;
  if (n_q_heads) vec = vec && aligned(q, 16) && aligned(out_q, 16);
  if (n_k_heads) vec = vec && aligned(k, 16) && aligned(out_k, 16);
  g.chunks = vec ? g.half / 8 : g.half;
  const int64_t total = n_tokens * g.n_heads * g.chunks;
  const int64_t blocks = (total + kThreads - 1) / kThreads;
  if (blocks > 0x7fffffff) return fail(TALM_EINVAL, "rope: too many tokens");
  const hipStream_t s = as_stream(stream);
  if (vec)
    hipLaunchKernelGGL(rope_kernel<true>, dim3(static_cast<unsigned>(blocks)), dim3(kThreads), 0, s,
                       q, k, cos, sin, out_q, out_k, g, backward);
  else
    hipLaunchKernelGGL(rope_kernel<false>, dim3(static_cast<unsigned>(blocks)), dim3(kThreads), 0, s,
                       q, k, cos, sin, out_q, out_k, g, backward);
  return check_launch("rope");
}
