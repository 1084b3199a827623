// The NF4 format's arithmetic on gfx950, shared by the dequant kernels (nf4.hip) and the fused
// dequant-GEMM (w4gemm.hip): the 16 levels, the double-quantized block scale and the level times
// scale product, each rounded exactly as the reference does (solution/qgroup.py:60-91).
//
// hipcc contracts a * b + c into v_fma_f32 by default (also through HIP's rounding-mode helpers,
// whose header definitions carry the contraction flag): contraction is switched off for every
// file that includes this header, and the products and sums below are plain operators, each
// rounded on its own.
#pragma once

#include "common.h"

#pragma clang fp contract(off)

namespace talm {
namespace {

// The 16 NormalFloat levels (QLoRA, Dettmers et al. 2023), as in solution/qgroup.py:60-63.
__constant__ float kNF4Levels[16] = {
    -1.0f, -0.6961928009986877f, -0.5250730514526367f, -0.39491748809814453f,
    -0.28444138169288635f, -0.18477343022823334f, -0.09105003625154495f, 0.0f,
    0.07958029955625534f, 0.16093020141124725f, 0.24611230194568634f, 0.33791524171829224f,
    0.44070982933044434f, 0.5626170039176941f, 0.7229568362236023f, 1.0f};

// The fp32 product, materialized: the empty asm keeps the backend from folding "multiply, then
// convert to fp16" into one v_fma_mix (a single rounding of the exact product).
__device__ __forceinline__ float mul_f32(float a, float b) {
  float p = a * b;
  asm("" : "+v"(p));
  return p;
}

// Eight weights of one packed word (4 bytes, high nibble first) scaled and packed to 4 x 2 fp16.
__device__ __forceinline__ uint4 dequant_word(uint32_t word, float scale, const float* levels) {
  uint32_t out[4];
#pragma unroll
  for (int b = 0; b < 4; ++b) {
    const uint32_t byte = (word >> (8 * b)) & 0xffu;
    const float first = mul_f32(levels[byte >> 4], scale);
    const float second = mul_f32(levels[byte & 15u], scale);
    out[b] = pack2(first, second);
  }
  return make_uint4(out[0], out[1], out[2], out[3]);
}

// The scale of one 64-weight block: the second-level code of its absmax byte times its group's
// fp32 scale, plus the offset, rounded after each step.
__device__ __forceinline__ float block_scale(float code, float absmax2, float offset2) {
  return mul_f32(code, absmax2) + offset2;
}

}  // namespace
}  // namespace talm
