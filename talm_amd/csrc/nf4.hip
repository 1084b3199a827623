// NF4 -> fp16 dequantization for gfx950: the grouped seven-projection launch of a decoder layer
// (double-quantized absmax rebuilt in the kernel) and the per-projection launch with an fp32
// absmax. HBM-bound, and write-heavy (0.5 B read, 2 B written per weight).
//
// Grouped kernel (blocks of >= 32 weights): a wavefront takes 2048 weights. Each lane reads one
// 16-byte chunk of codes (32 weights, half a 64-weight block) with one 128-bit load and forms
// its block's scale once; the chunks and scales go through LDS so that each of the four stores
// writes 1 KiB contiguous per wavefront (lane l stores word 64 k + l). Reading the codes per
// 8-weight word (one 32-bit load and three scale loads per word) was 15% slower, and storing
// each lane's own 64 bytes (16-byte stores 64 bytes apart) 35% slower than these coalesced
// stores; the kernel reaches ~97% of a copy kernel with the same traffic and no arithmetic.
//
// Both NF4 tables live in LDS: the 16 levels occupy 16 distinct banks, so the per-nibble gather
// is conflict-free (lanes reading the same level broadcast). The 256-entry second-level code
// table is gathered once per 64 weights (one absmax block).
//
// Arithmetic is the reference's bit for bit: the scale is rounded after the product and after
// the offset (no fused multiply-add anywhere in this file), the level times the scale is one
// fp32 product and one round-to-nearest-even to fp16.
#include "nf4_code.h"

namespace talm {
namespace {

constexpr int kThreads = 256;
constexpr int kWordsPerThread = 4;  // 32 weights per thread, four independent 128-bit stores

typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

// Grouped kernel, chunk path (qblock >= 32): a 16-byte chunk of codes (32 weights) lies in one
// absmax block; wavefront tile t covers chunks [64 t, 64 t + 64).
// kPow2: qblock2 is a power of two (its log2 in qblock2_shift), else qblock2 divides.
template <bool kPow2>
__global__ __launch_bounds__(kThreads) void nf4_group_chunks_kernel(
    const u32x4* __restrict__ packed, const uint8_t* __restrict__ absmax8,
    const float* __restrict__ code, const float* __restrict__ absmax2,
    const float* __restrict__ offset2, uint4* __restrict__ out, int64_t n_chunks,
    int chunk_shift, uint32_t qblock2, int qblock2_shift) {
  __shared__ float s_code[256];
  __shared__ float s_levels[16];
  __shared__ u32x4 s_chunks[kThreads / kWave][kWave];
  __shared__ float s_scale[kThreads / kWave][kWave];
  s_code[threadIdx.x] = code[threadIdx.x];
  if (threadIdx.x < 16) s_levels[threadIdx.x] = kNF4Levels[threadIdx.x];
  __syncthreads();
  const int lane = threadIdx.x & (kWave - 1), wave = threadIdx.x / kWave;
  const int64_t c0 = (static_cast<int64_t>(blockIdx.x) * (kThreads / kWave) + wave) * kWave;
  if (c0 >= n_chunks) return;  // no block barrier follows
  const int64_t c = min(c0 + lane, n_chunks - 1);
  const u32x4 codes = __builtin_nontemporal_load(packed + c);
  const int64_t row = c >> chunk_shift;
  const int64_t blk2 = kPow2 ? (row >> qblock2_shift)
                             : static_cast<int64_t>(static_cast<uint32_t>(row) / qblock2);
  const uint32_t a8 = absmax8[row];
  const float a2 = absmax2[blk2], o2 = offset2[blk2];
  s_chunks[wave][lane] = codes;
  s_scale[wave][lane] = block_scale(s_code[a8], a2, o2);
  __builtin_amdgcn_wave_barrier();
  const uint32_t* words = reinterpret_cast<const uint32_t*>(&s_chunks[wave][0]);
#pragma unroll
  for (int k = 0; k < 4; ++k) {
    const int src = 16 * k + lane / 4;  // the chunk holding word 64 k + lane
    if (c0 + src < n_chunks)
      out[c0 * 4 + 64 * k + lane] = dequant_word(words[64 * k + lane], s_scale[wave][src], s_levels);
  }
}

// Grouped kernel, word path (blocks of 8 or 16 weights, or codes not 16-byte aligned): word w
// covers weights [8w, 8w + 8) of absmax block w >> word_shift.
__global__ __launch_bounds__(kThreads) void nf4_group_kernel(
    const uint32_t* __restrict__ packed, const uint8_t* __restrict__ absmax8,
    const float* __restrict__ code, const float* __restrict__ absmax2,
    const float* __restrict__ offset2, uint4* __restrict__ out, int64_t n_words, int word_shift,
    uint32_t qblock2, int qblock2_shift) {
  __shared__ float s_code[256];
  __shared__ float s_levels[16];
  s_code[threadIdx.x] = code[threadIdx.x];
  if (threadIdx.x < 16) s_levels[threadIdx.x] = kNF4Levels[threadIdx.x];
  __syncthreads();

  const int64_t base = static_cast<int64_t>(blockIdx.x) * (kThreads * kWordsPerThread) + threadIdx.x;
  // Every load of every word is issued before any is used: indices past the end are clamped to
  // the last word (its store is skipped), so no load sits behind a branch and one wait covers
  // the thread's whole batch.
  uint32_t words[kWordsPerThread], codes[kWordsPerThread];
  float a2[kWordsPerThread], o2[kWordsPerThread];
#pragma unroll
  for (int j = 0; j < kWordsPerThread; ++j) {
    const int64_t w = min(base + j * kThreads, n_words - 1);
    words[j] = __builtin_nontemporal_load(packed + w);
    const int64_t row = w >> word_shift;
    const int64_t blk2 = qblock2_shift >= 0 ? (row >> qblock2_shift)
                                            : static_cast<int64_t>(static_cast<uint32_t>(row) / qblock2);
    codes[j] = absmax8[row];
    a2[j] = absmax2[blk2];
    o2[j] = offset2[blk2];
  }
  float scales[kWordsPerThread];
#pragma unroll
  for (int j = 0; j < kWordsPerThread; ++j) scales[j] = block_scale(s_code[codes[j]], a2[j], o2[j]);
#pragma unroll
  for (int j = 0; j < kWordsPerThread; ++j) {
    const int64_t w = base + j * kThreads;
    if (w < n_words) out[w] = dequant_word(words[j], scales[j], s_levels);
  }
}

// Per-projection kernel, word path: blocksize a multiple of 8.
__global__ __launch_bounds__(kThreads) void nf4_words_kernel(const uint32_t* __restrict__ packed,
                                                             const float* __restrict__ absmax,
                                                             uint4* __restrict__ out,
                                                             int64_t n_words, uint32_t words_per_block) {
  __shared__ float s_levels[16];
  if (threadIdx.x < 16) s_levels[threadIdx.x] = kNF4Levels[threadIdx.x];
  __syncthreads();
  const int64_t base = static_cast<int64_t>(blockIdx.x) * (kThreads * kWordsPerThread) + threadIdx.x;
  uint32_t words[kWordsPerThread];
  float scales[kWordsPerThread];
#pragma unroll
  for (int j = 0; j < kWordsPerThread; ++j) {  // all loads first (clamped indices, no branch)
    const int64_t w = min(base + j * kThreads, n_words - 1);
    words[j] = __builtin_nontemporal_load(packed + w);
    scales[j] = absmax[static_cast<uint32_t>(w) / words_per_block];
  }
#pragma unroll
  for (int j = 0; j < kWordsPerThread; ++j) {
    const int64_t w = base + j * kThreads;
    if (w < n_words) out[w] = dequant_word(words[j], scales[j], s_levels);
  }
}

// Per-projection kernel, byte path: any even blocksize / element count (one byte -> 2 fp16).
__global__ __launch_bounds__(kThreads) void nf4_bytes_kernel(const uint8_t* __restrict__ packed,
                                                             const float* __restrict__ absmax,
                                                             uint32_t* __restrict__ out,
                                                             int64_t n_bytes, uint32_t blocksize) {
  const int64_t i = static_cast<int64_t>(blockIdx.x) * kThreads + threadIdx.x;
  if (i >= n_bytes) return;
  const uint32_t byte = packed[i];
  const float scale = absmax[static_cast<uint32_t>(2 * i) / blocksize];
  out[i] = pack2(mul_f32(kNF4Levels[byte >> 4], scale), mul_f32(kNF4Levels[byte & 15u], scale));
}

int log2_exact(int64_t v) {
  if (v <= 0 || (v & (v - 1))) return -1;
  int s = 0;
  while ((int64_t{1} << s) < v) ++s;
  return s;
}

}  // namespace
}  // namespace talm

using namespace talm;

TALM_API int talm_nf4_group_dequant(const uint8_t* packed, const uint8_t* absmax8,
                                    const float* code, const float* absmax2,
                                    const float* offset2, uint16_t* out, int64_t n_rows,
                                    int32_t qblock, int32_t qblock2, void* stream) {
  const int qshift = log2_exact(qblock);
  if (n_rows < 0) return fail(TALM_EINVAL, "nf4_group_dequant: n_rows %lld < 0", (long long)n_rows);
  if (qshift < 3) return fail(TALM_EINVAL, "nf4_group_dequant: qblock %d is not a power of two >= 8", qblock);
  if (qblock2 < 1) return fail(TALM_EINVAL, "nf4_group_dequant: qblock2 %d < 1", qblock2);
  if (!aligned(packed, 4) || !aligned(out, 16))
    return fail(TALM_EINVAL, "nf4_group_dequant: packed must be 4-byte and out 16-byte aligned");
  if (n_rows == 0) return ok();
  if (!packed || !absmax8 || !code || !absmax2 || !offset2 || !out)
    return fail(TALM_EINVAL, "nf4_group_dequant: null pointer");
  const int64_t n_words = n_rows * (qblock / 8);
  if (n_rows > 0xffffffffLL) return fail(TALM_EINVAL, "nf4_group_dequant: too many weights");
  if (qshift >= 5 && aligned(packed, 16)) {
    const int64_t n_chunks = n_words / 4;
    const int64_t blocks = (n_chunks + kThreads - 1) / kThreads;
    if (blocks > 0x7fffffff) return fail(TALM_EINVAL, "nf4_group_dequant: too many weights");
    const int q2shift = log2_exact(qblock2);
    auto kernel = q2shift >= 0 ? nf4_group_chunks_kernel<true> : nf4_group_chunks_kernel<false>;
    hipLaunchKernelGGL(kernel, dim3(static_cast<unsigned>(blocks)), dim3(kThreads), 0,
                       as_stream(stream), reinterpret_cast<const u32x4*>(packed), absmax8, code,
                       absmax2, offset2, reinterpret_cast<uint4*>(out), n_chunks, qshift - 5,
                       static_cast<uint32_t>(qblock2), q2shift);
    return check_launch("nf4_group_dequant");
  }
  const int64_t per_block = kThreads * kWordsPerThread;
  const int64_t blocks = (n_words + per_block - 1) / per_block;
  if (blocks > 0x7fffffff) return fail(TALM_EINVAL, "nf4_group_dequant: too many weights");
  hipLaunchKernelGGL(nf4_group_kernel, dim3(static_cast<unsigned>(blocks)), dim3(kThreads), 0,
                     as_stream(stream), reinterpret_cast<const uint32_t*>(packed), absmax8, code,
                     absmax2, offset2, reinterpret_cast<uint4*>(out), n_words, qshift - 3,
                     static_cast<uint32_t>(qblock2), log2_exact(qblock2));
  return check_launch("nf4_group_dequant");
}

TALM_API int talm_nf4_dequant(const uint8_t* packed, const float* absmax, uint16_t* out, int64_t n,
                              int32_t blocksize, void* stream) {
  if (n < 0 || (n & 1)) return fail(TALM_EINVAL, "nf4_dequant: element count %lld is not even", (long long)n);
  if (blocksize < 2 || (blocksize & 1)) return fail(TALM_EINVAL, "nf4_dequant: blocksize %d is not even", blocksize);
  if (n == 0) return ok();
  if (!packed || !absmax || !out) return fail(TALM_EINVAL, "nf4_dequant: null pointer");
  if (!aligned(out, 4)) return fail(TALM_EINVAL, "nf4_dequant: out must be 4-byte aligned");
  if (n > 0xffffffffLL) return fail(TALM_EINVAL, "nf4_dequant: more than 2^32 weights");
  const hipStream_t s = as_stream(stream);
  if (blocksize % 8 == 0 && n % 8 == 0 && aligned(packed, 4) && aligned(out, 16)) {
    const int64_t n_words = n / 8;
    const int64_t per_block = kThreads * kWordsPerThread;
    hipLaunchKernelGGL(nf4_words_kernel, dim3(static_cast<unsigned>((n_words + per_block - 1) / per_block)),
                       dim3(kThreads), 0, s, reinterpret_cast<const uint32_t*>(packed), absmax,
                       reinterpret_cast<uint4*>(out), n_words, static_cast<uint32_t>(blocksize / 8));
  } else {
    const int64_t n_bytes = n / 2;
    hipLaunchKernelGGL(nf4_bytes_kernel, dim3(static_cast<unsigned>((n_bytes + kThreads - 1) / kThreads)),
                       dim3(kThreads), 0, s, packed, absmax, reinterpret_cast<uint32_t*>(out), n_bytes,
                       static_cast<uint32_t>(blocksize));
  }
  return check_launch("nf4_dequant");
}
