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

// The 16 values fp16(fl32(level_j x scale)) of one block, held in registers as byte planes: lo[k]
// holds the low bytes of values 4k .. 4k + 3, hi[k] their high bytes. Each value is rounded as
// dequant_word rounds it (one fp32 product, one round-to-nearest-even conversion).
struct Nf4Table {
  uint32_t lo[4], hi[4];
};

typedef _Float16 nf4_half2_t __attribute__((ext_vector_type(2)));
typedef float nf4_float2_t __attribute__((ext_vector_type(2)));

__device__ __forceinline__ Nf4Table nf4_table(float scale) {
  uint32_t p[8];  // p[q] = value 2q | value 2q + 1 << 16
#pragma unroll
  for (int q = 0; q < 8; ++q)
    p[q] = __builtin_bit_cast(uint32_t, __builtin_convertvector(
                                            (nf4_float2_t){mul_f32(kNF4Levels[2 * q], scale),
                                                           mul_f32(kNF4Levels[2 * q + 1], scale)},
                                            nf4_half2_t));
  Nf4Table t;
  // v_perm_b32 (S0, S1, sel): selector byte 0..3 picks byte of S1, 4..7 byte of S0
#pragma unroll
  for (int k = 0; k < 4; ++k) {
    t.lo[k] = __builtin_amdgcn_perm(p[2 * k + 1], p[2 * k], 0x06040200u);
    t.hi[k] = __builtin_amdgcn_perm(p[2 * k + 1], p[2 * k], 0x07050301u);
  }
  return t;
}

// One byte plane's entries for four nibbles (one per byte): n7 holds each nibble's low three bits,
// m is 0xff in the bytes whose nibble is 8 or more.
__device__ __forceinline__ uint32_t nf4_pick(uint32_t n7, uint32_t m, const uint32_t (&plane)[4]) {
  const uint32_t a = __builtin_amdgcn_perm(plane[1], plane[0], n7);  // entries 0..7
  const uint32_t b = __builtin_amdgcn_perm(plane[3], plane[2], n7);  // entries 8..15
  return (a & ~m) | (b & m);
}

// dequant_word from a block's table: the eight weights of a packed word (high nibble first) as
// 4 x 2 fp16, bit-identical to dequant_word with the same scale, in VALU byte permutes only.
__device__ __forceinline__ uint4 nf4_lookup_word(uint32_t w, const Nf4Table& t) {
  // nibbles of the even elements (each byte's high nibble) and of the odd ones, one per byte;
  // selector bytes 0x0c / 0x0d make v_perm_b32 write 0x00 / 0xff
  const uint32_t nh = (w >> 4) & 0x07070707u, nl = w & 0x07070707u;
  const uint32_t mh = __builtin_amdgcn_perm(0u, 0u, ((w >> 7) & 0x01010101u) | 0x0c0c0c0cu);
  const uint32_t ml = __builtin_amdgcn_perm(0u, 0u, ((w >> 3) & 0x01010101u) | 0x0c0c0c0cu);
  const uint32_t lh = nf4_pick(nh, mh, t.lo), hh = nf4_pick(nh, mh, t.hi);
  const uint32_t ll = nf4_pick(nl, ml, t.lo), hl = nf4_pick(nl, ml, t.hi);
  const uint32_t e02 = __builtin_amdgcn_perm(hh, lh, 0x05010400u);  // element 0 | element 2 << 16
  const uint32_t e46 = __builtin_amdgcn_perm(hh, lh, 0x07030602u);
  const uint32_t e13 = __builtin_amdgcn_perm(hl, ll, 0x05010400u);
  const uint32_t e57 = __builtin_amdgcn_perm(hl, ll, 0x07030602u);
  return make_uint4(__builtin_amdgcn_perm(e13, e02, 0x05040100u),
                    __builtin_amdgcn_perm(e13, e02, 0x07060302u),
                    __builtin_amdgcn_perm(e57, e46, 0x05040100u),
                    __builtin_amdgcn_perm(e57, e46, 0x07060302u));
}

// The scale of one 64-weight block: the second-level code of its absmax byte times its group's
// fp32 scale, plus the offset, rounded after each step.
__device__ __forceinline__ float block_scale(float code, float absmax2, float offset2) {
  return mul_f32(code, absmax2) + offset2;
}

}  // namespace
}  // namespace talm
