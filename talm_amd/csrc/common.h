// Shared helpers of the gfx950 kernels: status reporting for the C-ABI, fp16 packing, wave64
// reductions. Device code is written for CDNA4 (64-lane wavefronts) only.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "../../include/talm.h"

#define TALM_API extern "C" __attribute__((visibility("default")))

namespace talm {

// Records the message of a failed call for talm_last_error() on this thread; returns `status`.
int fail(int status, const char* fmt, ...) __attribute__((format(printf, 2, 3)));
// TALM_OK after clearing the thread's message.
int ok();
// TALM_OK, or TALM_EHIP with the launch error of the last kernel enqueued on this thread.
int check_launch(const char* what);
// Compute units of the current device (queried once per device).
int device_cus();

constexpr int kWave = 64;

__device__ __forceinline__ float h2f(uint16_t bits) {
  return static_cast<float>(__builtin_bit_cast(_Float16, bits));
}

// IEEE round-to-nearest-even conversion (v_cvt_f16_f32 under the default rounding mode; fp16
// denormals are kept: hipcc does not flush them unless asked to).
__device__ __forceinline__ uint16_t f2h(float x) {
  return __builtin_bit_cast(uint16_t, static_cast<_Float16>(x));
}

// The fp32 product, materialized: the empty asm keeps the backend from folding "multiply, then
// convert to fp16" into one v_fma_mix (a single rounding of the exact product, and -0 turned
// into +0 by its zero addend), where the result must be rounded to fp32 first.
__device__ __forceinline__ float mul_f32(float a, float b) {
  float p = a * b;
  asm("" : "+v"(p));
  return p;
}

__device__ __forceinline__ uint32_t pack2(float lo, float hi) {
  return static_cast<uint32_t>(f2h(lo)) | (static_cast<uint32_t>(f2h(hi)) << 16);
}

__device__ __forceinline__ float lo_f(uint32_t w) { return h2f(static_cast<uint16_t>(w & 0xffffu)); }
__device__ __forceinline__ float hi_f(uint32_t w) { return h2f(static_cast<uint16_t>(w >> 16)); }

// Sum over the 64 lanes of a wavefront; every lane receives the total.
__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) v += __shfl_xor(v, off, kWave);
  return v;
}

__device__ __forceinline__ float wave_max(float v) {
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) v = fmaxf(v, __shfl_xor(v, off, kWave));
  return v;
}

inline bool aligned(const void* p, uintptr_t bytes) {
  return (reinterpret_cast<uintptr_t>(p) & (bytes - 1)) == 0;
}

inline hipStream_t as_stream(void* s) { return reinterpret_cast<hipStream_t>(s); }

}  // namespace talm
