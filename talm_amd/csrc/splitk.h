// The K-split bookkeeping shared by the fp16 split-K GEMM (gemm.hip) and the NF4 dequant-GEMM
// (w4gemm.hip): how many K parts a product gets, and the ordered sum of the parts' fp32 partials.
#pragma once

#include "common.h"

#include <algorithm>

namespace talm {
namespace {

constexpr int kReduceThreads = 256;

// out[r][c .. c + 7] = fp16(sum over parts p = 0, 1, ... of part[p][r][c .. c + 7]).
__global__ __launch_bounds__(kReduceThreads) void splitk_reduce_kernel(
    const float* __restrict__ part, int parts, int64_t mn, int N, uint16_t* __restrict__ out,
    int64_t ldo) {
  const int64_t e0 = (static_cast<int64_t>(blockIdx.x) * kReduceThreads + threadIdx.x) * 8;
  if (e0 >= mn) return;
  float s[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
  for (int p = 0; p < parts; ++p) {
    const float4 x = *reinterpret_cast<const float4*>(part + p * mn + e0);
    const float4 y = *reinterpret_cast<const float4*>(part + p * mn + e0 + 4);
    s[0] += x.x; s[1] += x.y; s[2] += x.z; s[3] += x.w;
    s[4] += y.x; s[5] += y.y; s[6] += y.z; s[7] += y.w;
  }
  const int64_t r = e0 / N, c = e0 % N;
  *reinterpret_cast<uint4*>(out + r * ldo + c) =
      make_uint4(pack2(s[0], s[1]), pack2(s[2], s[3]), pack2(s[4], s[5]), pack2(s[6], s[7]));
}

// Sums `parts` partials of an [m, n] product (n a multiple of 8) into out on `s`.
inline void launch_splitk_reduce(const float* part, int parts, int64_t m, int64_t n, uint16_t* out,
                                 int64_t ldo, hipStream_t s) {
  const int64_t mn = m * n;
  hipLaunchKernelGGL(splitk_reduce_kernel,
                     dim3(static_cast<unsigned>((mn / 8 + kReduceThreads - 1) / kReduceThreads)),
                     dim3(kReduceThreads), 0, s, part, parts, mn, static_cast<int>(n), out, ldo);
}

struct SplitPlan {
  int parts, steps_per_part, n_mtiles, n_ntiles;
};

// Tiles of bm x bn over [m, n] and K cut into as many parts as fill the chip's CUs in one round
// with the output tiles, each of at least `min_steps` bk-deep steps; no empty part.
inline SplitPlan plan_split(int64_t m, int64_t n, int64_t k, int bm, int bn, int bk,
                            int min_steps = 16) {
  SplitPlan p{};
  p.n_mtiles = static_cast<int>((m + bm - 1) / bm);
  p.n_ntiles = static_cast<int>((n + bn - 1) / bn);
  const int64_t steps = (k + bk - 1) / bk;
  const int64_t tiles = static_cast<int64_t>(p.n_mtiles) * p.n_ntiles;
  const int64_t parts = std::max<int64_t>(
      1, std::min<int64_t>(device_cus() / std::max<int64_t>(tiles, 1), steps / min_steps));
  p.steps_per_part = static_cast<int>((steps + parts - 1) / parts);
  p.parts = static_cast<int>((steps + p.steps_per_part - 1) / p.steps_per_part);
  return p;
}

}  // namespace
}  // namespace talm
