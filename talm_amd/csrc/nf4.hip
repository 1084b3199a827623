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

#include <algorithm>

namespace talm {
namespace {

constexpr int kThreads = 256;
constexpr int kWordsPerThread = 4;  // 32 weights per thread, four independent 128-bit stores

typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

// Grouped kernel, chunk path (qblock >= 32): a 16-byte chunk of codes (32 weights) lies in one
// absmax block; wavefront tile t covers chunks [64 t, 64 t + 64). The grid is persistent: each
// wavefront walks tiles t, t + stride, ... and issues the next tile's loads before it dequantizes
// and stores the current one (two tiles of loads in flight), and all four words of a lane are
// dequantized before its four stores go out back to back (6% faster than one-shot wavefronts
// storing each word as it is formed). kPow2: qblock2 is a power of two (its log2 in
// qblock2_shift), else qblock2 divides. kNt: non-temporal stores (the streaming entry point: the
// output is not read again soon, so it need not displace the last-level cache's contents).
template <bool kNt>
__device__ __forceinline__ void store16(uint4* p, uint4 v) {
  if constexpr (kNt)
    __builtin_nontemporal_store(u32x4{v.x, v.y, v.z, v.w}, reinterpret_cast<u32x4*>(p));
  else
    *p = v;
}

template <bool kPow2, bool kNt>
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
  const int64_t n_tiles = (n_chunks + kWave - 1) / kWave;
  const int64_t stride = static_cast<int64_t>(gridDim.x) * (kThreads / kWave);
  int64_t t = static_cast<int64_t>(blockIdx.x) * (kThreads / kWave) + wave;
  if (t >= n_tiles) return;  // no block barrier follows
  // a lane's chunk of tile t (the last chunk stands in past the end: its stores are skipped)
  auto load = [&](int64_t tile, u32x4& codes, uint32_t& a8, float& a2, float& o2) {
    const int64_t c = min(tile * kWave + lane, n_chunks - 1);
    codes = __builtin_nontemporal_load(packed + c);
    const int64_t row = c >> chunk_shift;
    const int64_t blk2 = kPow2 ? (row >> qblock2_shift)
                               : static_cast<int64_t>(static_cast<uint32_t>(row) / qblock2);
    a8 = absmax8[row];
    a2 = absmax2[blk2];
    o2 = offset2[blk2];
  };
  u32x4 codes;
  uint32_t a8;
  float a2, o2;
  load(t, codes, a8, a2, o2);
  for (;;) {
    const int64_t next = t + stride;
    const bool more = next < n_tiles;
    u32x4 n_codes = codes;
    uint32_t n_a8 = 0;
    float n_a2 = 0.f, n_o2 = 0.f;
    if (more) load(next, n_codes, n_a8, n_a2, n_o2);
    s_chunks[wave][lane] = codes;
    s_scale[wave][lane] = block_scale(s_code[a8], a2, o2);
    __builtin_amdgcn_wave_barrier();
    const uint32_t* words = reinterpret_cast<const uint32_t*>(&s_chunks[wave][0]);
    uint4 v[4];
#pragma unroll
    for (int k = 0; k < 4; ++k)  // word 64 k + lane lies in chunk 16 k + lane / 4
      v[k] = dequant_word(words[64 * k + lane], s_scale[wave][16 * k + lane / 4], s_levels);
    __builtin_amdgcn_wave_barrier();  // every lane has read the tile before the next is staged
    const int64_t c0 = t * kWave;
#pragma unroll
    for (int k = 0; k < 4; ++k)
      if (c0 + 16 * k + lane / 4 < n_chunks) store16<kNt>(out + c0 * 4 + 64 * k + lane, v[k]);
    if (!more) break;
    t = next;
    codes = n_codes;
    a8 = n_a8;
    a2 = n_a2;
    o2 = n_o2;
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

// Transposed grouped kernel: W^T of each projection of a packed layer, for the backward's
// input-gradient GEMMs (dX = dY W reads W^T as the k-contiguous operand). A tile is 64 weight
// rows x 256 columns of one projection (64-weight absmax blocks lie inside one row). Thread
// (p, ci) reads the 32 columns 32 ci .. of rows 2 p and 2 p + 1 with one 16-byte load each (eight
// lanes read a row's 128 bytes) and packs the two rows' values of each column into one 32-bit
// LDS word: the tile is stored transposed, [column][row pair], with the pair index XOR-ed by
// 4 ci so that the eight lanes writing one pair position hit different banks, and so that four
// consecutive pairs stay adjacent. Then each W^T row of the tile (64 values, 128 bytes) is
// written by eight lanes with 16-byte stores. Values are the grouped kernel's bit for bit.
constexpr int kTRows = 64, kTCols = 256;
constexpr int kTStride = kTRows / 2 + 4;  // words per LDS column: 16-byte aligned rows
constexpr int kMaxTSeg = 8;
static_assert(kTRows / 2 * (kTCols / 32) == kThreads, "one row pair and 32 columns per thread");

struct TSegs {
  int64_t start[kMaxTSeg];  // first weight element of the projection in the packed buffers
  int64_t dst[kMaxTSeg];    // element offset of its W^T (row 0, column 0) in the output
  int32_t rows[kMaxTSeg], cols[kMaxTSeg], ld[kMaxTSeg];  // W [rows, cols]; W^T row stride
  int32_t col_tiles[kMaxTSeg];
  int32_t tile0[kMaxTSeg + 1];  // first tile of each projection in the grid
  int n_seg;
};

// Persistent: workgroup b (on XCD b % 8) walks tiles first, first + stride, ... of its XCD's
// contiguous range, and the next tile's codes and scale inputs are loaded while the current one
// is dequantized, transposed through LDS and stored.
struct TTile {
  int g, r0, c0;  // projection, first weight row, first column
};

__device__ __forceinline__ TTile t_tile(const TSegs& s, int tile) {
  TTile t;
  t.g = 0;
  while (t.g + 1 < s.n_seg && tile >= s.tile0[t.g + 1]) ++t.g;
  const int local = tile - s.tile0[t.g];
  t.r0 = local / s.col_tiles[t.g] * kTRows;
  t.c0 = local % s.col_tiles[t.g] * kTCols;
  return t;
}

template <bool kPow2>
__global__ __launch_bounds__(kThreads) void nf4_group_t_kernel(
    const uint8_t* __restrict__ packed, const uint8_t* __restrict__ absmax8,
    const float* __restrict__ code, const float* __restrict__ absmax2,
    const float* __restrict__ offset2, uint16_t* __restrict__ out, TSegs s, int qblock_shift,
    uint32_t qblock2, int qblock2_shift) {
  __shared__ float s_code[256];
  __shared__ float s_levels[16];
  __shared__ __attribute__((aligned(16))) uint32_t s_t[kTCols * kTStride];
  s_code[threadIdx.x] = code[threadIdx.x];
  if (threadIdx.x < 16) s_levels[threadIdx.x] = kNF4Levels[threadIdx.x];
  // each XCD one contiguous range of tiles, so the neighbouring tiles of a row band, which read
  // the same cache lines of codes, share an L2
  const uint32_t n_tiles = static_cast<uint32_t>(s.tile0[s.n_seg]);
  uint32_t first = blockIdx.x, stride = gridDim.x, end = n_tiles;
  if (gridDim.x % 8 == 0) {
    const uint32_t x = blockIdx.x % 8, q = n_tiles / 8, r = n_tiles % 8;
    const uint32_t start = x * q + min(x, r);
    first = start + blockIdx.x / 8;
    stride = gridDim.x / 8;
    end = start + q + (x < r ? 1u : 0u);
  }
  __syncthreads();  // the tables in LDS
  if (first >= end) return;  // the whole workgroup; no barrier follows
  const int p = threadIdx.x >> 3, ci = threadIdx.x & 7;
  u32x4 w[2];
  uint32_t a8[2];
  float a2[2], o2[2];
  // thread (p, ci)'s codes of tile `tt`: columns 32 ci .. of rows 2 p and 2 p + 1 (rows past the
  // end clamped, a column chunk past the end reads the tile's first)
  auto load = [&](const TTile& tt, u32x4 (&lw)[2], uint32_t (&la8)[2], float (&la2)[2],
                  float (&lo2)[2]) {
    const int rows = s.rows[tt.g], cols = s.cols[tt.g];
    const int cc = tt.c0 + 32 * ci < cols ? tt.c0 + 32 * ci : tt.c0;
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      const int r = min(tt.r0 + 2 * p + h, rows - 1);
      const int64_t e = s.start[tt.g] + static_cast<int64_t>(r) * cols + cc;
      lw[h] = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(packed + e / 2));
      const int64_t blk = e >> qblock_shift;
      const int64_t blk2 = kPow2 ? (blk >> qblock2_shift)
                                 : static_cast<int64_t>(static_cast<uint32_t>(blk) / qblock2);
      la8[h] = absmax8[blk];
      la2[h] = absmax2[blk2];
      lo2[h] = offset2[blk2];
    }
  };
  TTile cur = t_tile(s, static_cast<int>(first));
  load(cur, w, a8, a2, o2);
  for (uint32_t tile = first;;) {
    const uint32_t next = tile + stride;
    const bool more = next < end;
    TTile nxt = cur;
    u32x4 nw[2] = {w[0], w[1]};
    uint32_t na8[2] = {0u, 0u};
    float na2[2] = {0.f, 0.f}, no2[2] = {0.f, 0.f};
    if (more) {
      nxt = t_tile(s, static_cast<int>(next));
      load(nxt, nw, na8, na2, no2);
    }
    float scale[2];
#pragma unroll
    for (int h = 0; h < 2; ++h) scale[h] = block_scale(s_code[a8[h]], a2[h], o2[h]);
    uint32_t* col = s_t + (32 * ci) * kTStride + (p ^ (4 * ci));
#pragma unroll
    for (int j = 0; j < 32; ++j) {  // word j / 8, byte (j % 8) / 2, high nibble first
      uint32_t pair = 0;
#pragma unroll
      for (int h = 0; h < 2; ++h) {
        const uint32_t word = w[h][j >> 3];
        const uint32_t byte = (word >> (8 * ((j & 7) >> 1))) & 0xffu;
        const uint32_t nib = (j & 1) ? (byte & 15u) : (byte >> 4);
        pair |= static_cast<uint32_t>(f2h(mul_f32(s_levels[nib], scale[h]))) << (16 * h);
      }
      col[j * kTStride] = pair;
    }
    __syncthreads();
    const int rows = s.rows[cur.g], cols = s.cols[cur.g];
    uint16_t* dst = out + s.dst[cur.g];
#pragma unroll
    for (int k = 0; k < kTCols * (kTRows / 8) / kThreads; ++k) {
      const int id = k * kThreads + threadIdx.x;
      const int c = id >> 3, oc = id & 7;  // W^T row c0 + c: rows r0 + 8 oc .. + 7 of W
      if (cur.c0 + c < cols && cur.r0 + 8 * oc < rows)
        *reinterpret_cast<uint4*>(dst + static_cast<int64_t>(cur.c0 + c) * s.ld[cur.g] + cur.r0 + 8 * oc) =
            *reinterpret_cast<const uint4*>(s_t + c * kTStride + ((4 * oc) ^ (4 * (c >> 5))));
    }
    if (!more) break;
    __syncthreads();  // every thread has read the tile before the next one is staged
    tile = next;
    cur = nxt;
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      w[h] = nw[h];
      a8[h] = na8[h];
      a2[h] = na2[h];
      o2[h] = no2[h];
    }
  }
}

int log2_exact(int64_t v) {
  if (v <= 0 || (v & (v - 1))) return -1;
  int s = 0;
  while ((int64_t{1} << s) < v) ++s;
  return s;
}

// scale[b] = block_scale(code[absmax8[b]], absmax2[b / qblock2], offset2[b / qblock2]): the
// double-quantized absmax of every block decoded once (the values dequant_word multiplies by).
// Grid (blocks of one second-level block / 256 threads, second-level blocks): no division.
__global__ __launch_bounds__(kThreads) void nf4_block_scales_kernel(
    const uint8_t* __restrict__ absmax8, const float* __restrict__ code,
    const float* __restrict__ absmax2, const float* __restrict__ offset2, int64_t n_blocks,
    uint32_t qblock2, float* __restrict__ out) {
  const uint32_t i = blockIdx.x * kThreads + threadIdx.x;
  const int64_t b2 = blockIdx.y, b = b2 * qblock2 + i;
  if (i >= qblock2 || b >= n_blocks) return;
  out[b] = block_scale(code[absmax8[b]], absmax2[b2], offset2[b2]);
}

}  // namespace
}  // namespace talm

using namespace talm;

namespace talm {
namespace {

int group_dequant(const uint8_t* packed, const uint8_t* absmax8, const float* code,
                  const float* absmax2, const float* offset2, uint16_t* out, int64_t n_rows,
                  int32_t qblock, int32_t qblock2, bool streaming, void* stream) {
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
    const int64_t tiles = (n_chunks + kWave - 1) / kWave;
    // persistent: up to 12 workgroups of four wavefronts per CU (measured best of 4 to 24 on
    // the config-1 layer, both store kinds), each wavefront walking its tiles
    const int64_t blocks = std::min<int64_t>((tiles + 3) / 4, 12 * static_cast<int64_t>(device_cus()));
    const int q2shift = log2_exact(qblock2);
    auto kernel = q2shift >= 0 ? (streaming ? nf4_group_chunks_kernel<true, true>
                                            : nf4_group_chunks_kernel<true, false>)
                               : (streaming ? nf4_group_chunks_kernel<false, true>
                                            : nf4_group_chunks_kernel<false, false>);
    hipLaunchKernelGGL(kernel, dim3(static_cast<unsigned>(blocks)), dim3(kThreads), 0,
                       as_stream(stream), reinterpret_cast<const u32x4*>(packed), absmax8, code,
                       absmax2, offset2, reinterpret_cast<uint4*>(out), n_chunks, qshift - 5,
                       static_cast<uint32_t>(qblock2), q2shift);
    return check_launch("nf4_group_dequant");
  }
  // blocks of 8 or 16 weights, or codes not 16-byte aligned: ordinary stores either way
  const int64_t per_block = kThreads * kWordsPerThread;
  const int64_t blocks = (n_words + per_block - 1) / per_block;
  if (blocks > 0x7fffffff) return fail(TALM_EINVAL, "nf4_group_dequant: too many weights");
  hipLaunchKernelGGL(nf4_group_kernel, dim3(static_cast<unsigned>(blocks)), dim3(kThreads), 0,
                     as_stream(stream), reinterpret_cast<const uint32_t*>(packed), absmax8, code,
                     absmax2, offset2, reinterpret_cast<uint4*>(out), n_words, qshift - 3,
                     static_cast<uint32_t>(qblock2), log2_exact(qblock2));
  return check_launch("nf4_group_dequant");
}

}  // namespace
}  // namespace talm

TALM_API int talm_nf4_group_dequant(const uint8_t* packed, const uint8_t* absmax8,
                                    const float* code, const float* absmax2,
                                    const float* offset2, uint16_t* out, int64_t n_rows,
                                    int32_t qblock, int32_t qblock2, void* stream) {
  return group_dequant(packed, absmax8, code, absmax2, offset2, out, n_rows, qblock, qblock2,
                       false, stream);
}

TALM_API int talm_nf4_group_dequant_streaming(const uint8_t* packed, const uint8_t* absmax8,
                                              const float* code, const float* absmax2,
                                              const float* offset2, uint16_t* out,
                                              int64_t n_rows, int32_t qblock, int32_t qblock2,
                                              void* stream) {
  return group_dequant(packed, absmax8, code, absmax2, offset2, out, n_rows, qblock, qblock2,
                       true, stream);
}

TALM_API int talm_nf4_block_scales(const uint8_t* absmax8, const float* code,
                                   const float* absmax2, const float* offset2, int64_t n_blocks,
                                   int32_t qblock2, float* out, void* stream) {
  if (n_blocks < 0 || qblock2 < 1)
    return fail(TALM_EINVAL, "nf4_block_scales: n_blocks %lld, qblock2 %d", (long long)n_blocks,
                qblock2);
  if (n_blocks == 0) return ok();
  if (!absmax8 || !code || !absmax2 || !offset2 || !out)
    return fail(TALM_EINVAL, "nf4_block_scales: null pointer");
  const int64_t groups = (n_blocks + qblock2 - 1) / qblock2;
  if (groups > 65535) return fail(TALM_EINVAL, "nf4_block_scales: too many second-level blocks");
  hipLaunchKernelGGL(nf4_block_scales_kernel,
                     dim3(static_cast<unsigned>((qblock2 + kThreads - 1) / kThreads),
                          static_cast<unsigned>(groups)),
                     dim3(kThreads), 0, as_stream(stream), absmax8, code, absmax2, offset2,
                     n_blocks, static_cast<uint32_t>(qblock2), out);
  return check_launch("nf4_block_scales");
}

TALM_API int talm_nf4_group_dequant_t(const uint8_t* packed, const uint8_t* absmax8,
                                      const float* code, const float* absmax2,
                                      const float* offset2, const int64_t* segs, int32_t n_seg,
                                      int32_t qblock, int32_t qblock2, uint16_t* out,
                                      int64_t out_numel, void* stream) {
  const int qshift = log2_exact(qblock);
  if (qshift < 6)
    return fail(TALM_EINVAL, "nf4_group_dequant_t: qblock %d is not a power of two >= 64", qblock);
  if (qblock2 < 1) return fail(TALM_EINVAL, "nf4_group_dequant_t: qblock2 %d < 1", qblock2);
  if (n_seg < 0 || n_seg > kMaxTSeg)
    return fail(TALM_EINVAL, "nf4_group_dequant_t: %d projections (at most %d)", n_seg, kMaxTSeg);
  if (n_seg == 0) return ok();
  if (!packed || !absmax8 || !code || !absmax2 || !offset2 || !out || !segs)
    return fail(TALM_EINVAL, "nf4_group_dequant_t: null pointer");
  if (!aligned(packed, 16) || !aligned(out, 16))
    return fail(TALM_EINVAL, "nf4_group_dequant_t: packed and out must be 16-byte aligned");
  TSegs t{};
  t.n_seg = n_seg;
  int64_t tiles = 0;
  for (int g = 0; g < n_seg; ++g) {
    const int64_t start = segs[5 * g], rows = segs[5 * g + 1], cols = segs[5 * g + 2];
    const int64_t dst = segs[5 * g + 3], ld = segs[5 * g + 4];
    if (start < 0 || start % qblock || rows < 8 || rows % 8 || cols < 64 || cols % 64 ||
        rows > (1 << 24) || cols > (1 << 24) || ld < rows || ld % 8 || ld > (1 << 30) ||
        dst < 0 || dst % 8 || dst + (cols - 1) * ld + rows > out_numel)
      return fail(TALM_EINVAL,
                  "nf4_group_dequant_t: projection %d (start %lld, [%lld, %lld], W^T at %lld "
                  "stride %lld): start a multiple of qblock, rows a multiple of 8, columns of "
                  "64, stride >= rows and a multiple of 8, inside the %lld-element output",
                  g, (long long)start, (long long)rows, (long long)cols, (long long)dst,
                  (long long)ld, (long long)out_numel);
    t.start[g] = start;
    t.dst[g] = dst;
    t.rows[g] = static_cast<int32_t>(rows);
    t.cols[g] = static_cast<int32_t>(cols);
    t.ld[g] = static_cast<int32_t>(ld);
    t.col_tiles[g] = static_cast<int32_t>((cols + kTCols - 1) / kTCols);
    t.tile0[g] = static_cast<int32_t>(tiles);
    tiles += (rows + kTRows - 1) / kTRows * t.col_tiles[g];
    if (tiles > 0x7fffffff) return fail(TALM_EINVAL, "nf4_group_dequant_t: too many weights");
  }
  t.tile0[n_seg] = static_cast<int32_t>(tiles);
  const int q2shift = log2_exact(qblock2);
  auto kernel = q2shift >= 0 ? nf4_group_t_kernel<true> : nf4_group_t_kernel<false>;
  // persistent workgroups, four per CU (a multiple of 8 in all), or one per tile; measured on the
  // step's transposed layer (q|k|v, o, down): 14.5 us with one workgroup per tile, 20.2 / 15.1 /
  // 13.4 / 12.5 / 14.3 / 14.3 us with 1 / 2 / 3 / 4 / 6 / 8 per CU
  int64_t wgs = std::min<int64_t>(tiles, 4 * static_cast<int64_t>(device_cus()));
  if (wgs >= 8) wgs -= wgs % 8;
  hipLaunchKernelGGL(kernel, dim3(static_cast<unsigned>(wgs)), dim3(kThreads), 0,
                     as_stream(stream), packed, absmax8, code, absmax2, offset2, out, t, qshift,
                     static_cast<uint32_t>(qblock2), q2shift);
  return check_launch("nf4_group_dequant_t");
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
