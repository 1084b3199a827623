// y = x W^T with W in the layer group's NF4 form (double-quantized absmax, 64-weight blocks),
// fp16 MFMA on gfx950: the weight is dequantized into LDS inside the GEMM, never written to HBM
// (SURVEY's W4A16 row; replaces the dequantization of the layer's buffer + hipBLASLt's fp16
// GEMM for the projections it serves, solution/qgroup.py:72-99 and :346-355).
//
// Tiles of 128 tokens x 256 weight rows, 8 wavefronts of 64 x 64 (v_mfma_f32_32x32x16_f16),
// 64-deep k steps (one NF4 block per weight row and step). Both operands go through registers
// into 2-slot LDS buffers in the swizzled layout the MFMA fragment reads expect (mfma_tile.h):
//   A (x): two 16-byte chunks per thread and step;
//   B: each thread loads 16 bytes (32 weights of one row) and the row's block-scale inputs, then
//      dequantizes them exactly as nf4_group_kernel does (fp32 level x scale, one rounding to
//      fp16) into four 16-byte chunks.
// Step kt: barrier; MFMAs on slot kt % 2; the registers of step kt + 1 (loaded kDepth steps
// earlier, into register set (kt + 1) % kDepth) into slot (kt + 1) % 2; loads of step
// kt + 1 + kDepth into that register set. kDepth steps of MFMAs and dequantization cover each
// load's latency (one step, ~0.5 µs, does not). Loads past the last step are clamped, so no load
// sits behind a branch (the compiler would wait for it at the join). (Operand DMA straight into LDS, as in the other GEMMs, would make
// the compiler wait for it before every LDS access of the dequantization.)
// The fp16 weights are bit-identical to the dequantized buffer's; the products are the fp16
// GEMM's with fp32 accumulation (only the summation order differs from hipBLASLt's).
#include "mfma_tile.h"
#include "nf4_code.h"

namespace talm {
namespace {

typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

using W4Shape = TileShape<128, 256, 64, 2, 2, 4>;
constexpr int kW4AStage = W4Shape::kAChunks * 16;          // 16 KiB of x per step
constexpr int kW4BStage = W4Shape::kBN * W4Shape::kBK * 2;  // 32 KiB of fp16 weights per step
constexpr int kW4Lds = 2 * kW4AStage + 2 * kW4BStage;
constexpr int kW4APer = W4Shape::kAChunks / W4Shape::kThreads;  // A chunks per thread and step
static_assert(kW4APer * W4Shape::kThreads == W4Shape::kAChunks, "whole A chunks per thread");
constexpr int kDepth = 2;  // register sets of loaded steps in flight (even: LDS slots stay static)
static_assert(kDepth % 2 == 0, "an even depth keeps the two LDS slots' indices constant");
constexpr int kW4ZS = W4Shape::kBN + 8;  // staged output tile row stride (halfs)
static_assert(W4Shape::kBM * kW4ZS * 2 <= kW4Lds, "the staged tile reuses the operand buffers");
static_assert(W4Shape::kThreads == 2 * W4Shape::kBN, "two threads per weight row and step");

struct W4Args {
  const uint16_t* x;       // [n_tokens][ldx]
  int64_t ldx;
  int n_tokens, k;         // k: multiple of 64
  const uint8_t* packed;   // [n_out][k / 2], two weights per byte, high nibble first
  const uint8_t* absmax8;  // [n_out * k / 64]: second-level code index of each block
  const float* code;       // [256]
  const float* absmax2;    // [(n_out * k) / 16384]
  const float* offset2;    // [(n_out * k) / 16384]
  int n_out;
  uint16_t* out;           // [n_tokens][ldo]
  int64_t ldo;
  int n_mtiles, n_ntiles;
};

__global__ __launch_bounds__(W4Shape::kThreads, 1) void w4_gemm_kernel(W4Args a) {
  using S = W4Shape;
  __shared__ __attribute__((aligned(1024))) unsigned char smem[kW4Lds];
  __shared__ float s_code[256];
  __shared__ float s_levels[16];
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int wm = wave / S::kWavesN, wn = wave % S::kWavesN;
  if (tid < 256) s_code[tid] = a.code[tid];
  if (tid < 16) s_levels[tid] = kNF4Levels[tid];

  // consecutive tiles walk the token tiles of one weight panel (the panel stays in L2)
  const uint32_t tile = xcd_tile(blockIdx.x, static_cast<uint32_t>(a.n_mtiles * a.n_ntiles));
  const int ntile = static_cast<int>(tile / a.n_mtiles), mtile = static_cast<int>(tile % a.n_mtiles);
  const int m0 = mtile * S::kBM, n0 = ntile * S::kBN;
  const int nk = a.k / S::kBK;

  uint4* const a_slot[2] = {reinterpret_cast<uint4*>(smem),
                            reinterpret_cast<uint4*>(smem + kW4AStage)};
  uint4* const b_slot[2] = {reinterpret_cast<uint4*>(smem + 2 * kW4AStage),
                            reinterpret_cast<uint4*>(smem + 2 * kW4AStage + kW4BStage)};

  // A: chunk c = tid + j * threads of the stage is row c / 8, k chunk c % 8; rows past the
  // batch read its last row (their outputs are not stored)
  const uint16_t* a_src[kW4APer];
  int a_dst[kW4APer];
#pragma unroll
  for (int j = 0; j < kW4APer; ++j) {
    const int c = tid + j * S::kThreads, row = c / S::kCpr, kc = c % S::kCpr;
    a_src[j] = a.x + static_cast<int64_t>(min(m0 + row, a.n_tokens - 1)) * a.ldx + 8 * kc;
    a_dst[j] = swz<S::kCpr>(row, kc);
  }
  u32x4 ar[kDepth][kW4APer];
  auto a_load = [&](int r, int kt) {
    kt = min(kt, nk - 1);
#pragma unroll
    for (int j = 0; j < kW4APer; ++j)
      ar[r][j] = *reinterpret_cast<const u32x4*>(a_src[j] + S::kBK * kt);
  };
  auto a_store = [&](int r, uint4* slot) {
#pragma unroll
    for (int j = 0; j < kW4APer; ++j)
      slot[a_dst[j]] = make_uint4(ar[r][j][0], ar[r][j][1], ar[r][j][2], ar[r][j][3]);
  };

  // B: this thread's weight row (clamped past n_out: its columns are not stored) and 16-byte half
  const int br = tid >> 1, bh = tid & 1;
  const int64_t brow = min(n0 + br, a.n_out - 1);
  const uint8_t* const bp = a.packed + brow * (a.k / 2) + 16 * bh;
  const uint8_t* const b8 = a.absmax8 + brow * (a.k / 64);
  const int64_t belem = brow * a.k;
  u32x4 bw[kDepth];
  uint32_t bcode[kDepth];
  float ba2[kDepth], bo2[kDepth];
  auto b_load = [&](int r, int kt) {
    kt = min(kt, nk - 1);
    bw[r] = *reinterpret_cast<const u32x4*>(bp + 32 * kt);
    bcode[r] = b8[kt];
    const int64_t blk = (belem + 64 * static_cast<int64_t>(kt)) >> 14;
    ba2[r] = a.absmax2[blk];
    bo2[r] = a.offset2[blk];
  };
  auto b_store = [&](int r, uint4* slot) {
    const float scale = block_scale(s_code[bcode[r]], ba2[r], bo2[r]);
#pragma unroll
    for (int j = 0; j < 4; ++j)
      slot[swz<S::kCpr>(br, 4 * bh + j)] = dequant_word(bw[r][j], scale, s_levels);
  };

  Acc<S> acc;
#pragma unroll
  for (int i = 0; i < S::kFragM; ++i)
#pragma unroll
    for (int j = 0; j < S::kFragN; ++j)
#pragma unroll
      for (int v = 0; v < 16; ++v) acc[i][j][v] = 0.f;

#pragma unroll
  for (int r = 0; r < kDepth; ++r) {
    a_load(r, r);
    b_load(r, r);
  }
  __syncthreads();  // the code / level tables
  a_store(0, a_slot[0]);
  b_store(0, b_slot[0]);
  a_load(0, kDepth);
  b_load(0, kDepth);
  // step kt + h: slot h % 2 holds it; the register set of step kt + h + 1 goes into the other
  // slot and is reloaded with step kt + h + 1 + kDepth (kt a multiple of kDepth: the indices are
  // constants once h is)
  auto step = [&](int kt, int h) {
    __syncthreads();  // the stores of the step before are visible; the slot it read is free
    mma_step<S>(a_slot[h & 1], b_slot[h & 1], acc, lane, wm, wn);
    const int r = (h + 1) % kDepth;
    a_store(r, a_slot[(h + 1) & 1]);
    b_store(r, b_slot[(h + 1) & 1]);
    a_load(r, kt + h + 1 + kDepth);
    b_load(r, kt + h + 1 + kDepth);
  };
  int kt = 0;
  for (; kt + kDepth <= nk; kt += kDepth) {
#pragma unroll
    for (int h = 0; h < kDepth; ++h) step(kt, h);
  }
  // the last nk % kDepth steps (outside the loop: its back edge then only sees whole trips, and
  // the compiler's waits there stay kDepth steps deep)
#pragma unroll
  for (int h = 0; h < kDepth - 1; ++h)
    if (kt + h < nk) step(kt, h);
  __syncthreads();  // every wavefront is done with the operand buffers

  // epilogue: fp16 tile staged in LDS, then 16-byte row stores
  uint16_t* zs = reinterpret_cast<uint16_t*>(smem);
#pragma unroll
  for (int i = 0; i < S::kFragM; ++i)
#pragma unroll
    for (int j = 0; j < S::kFragN; ++j) {
      const int col = acc_col<S>(wn, j, lane);
#pragma unroll
      for (int v = 0; v < 16; ++v) zs[acc_row<S>(wm, i, v, lane) * kW4ZS + col] = f2h(acc[i][j][v]);
    }
  __syncthreads();
  constexpr int kChunksPerRow = S::kBN / 8;
#pragma unroll
  for (int it = 0; it < (S::kBM * kChunksPerRow) / S::kThreads; ++it) {
    const int c = it * S::kThreads + tid, row = c / kChunksPerRow, kc = c % kChunksPerRow;
    const int gr = m0 + row, gc = n0 + kc * 8;
    if (gr < a.n_tokens && gc < a.n_out)
      *reinterpret_cast<uint4*>(a.out + static_cast<int64_t>(gr) * a.ldo + gc) =
          *reinterpret_cast<const uint4*>(zs + row * kW4ZS + kc * 8);
  }
}

}  // namespace
}  // namespace talm

using namespace talm;

TALM_API int talm_nf4_gemm(const uint16_t* x, int64_t ldx, int64_t n_tokens, int64_t k,
                           const uint8_t* packed, const uint8_t* absmax8, const float* code,
                           const float* absmax2, const float* offset2, int64_t n_out,
                           int32_t blocksize, int32_t blocksize2, uint16_t* out, int64_t ldo,
                           void* stream) {
  using S = W4Shape;
  if (blocksize != 64 || blocksize2 != 256)
    return fail(TALM_EINVAL, "nf4_gemm: blocksizes %d / %d (64 / 256 supported)", blocksize,
                blocksize2);
  if (n_tokens < 0 || k < 64 || k % 64 || n_out < 1 || ldx < k || ldx % 8 || ldo < n_out ||
      ldo % 8 || n_out % 8 || n_tokens > (1 << 30) || n_out > (1 << 30) || k > (1 << 20) ||
      (n_out * k) % 16384 || !(S::kBM * ldx * 2 < (int64_t{1} << 31)))
    return fail(TALM_EINVAL,
                "nf4_gemm: bad shape (tokens %lld, k %lld, n_out %lld, ldx %lld, ldo %lld): k a "
                "multiple of 64, n_out a multiple of 8, n_out * k whole 16384-weight groups",
                (long long)n_tokens, (long long)k, (long long)n_out, (long long)ldx,
                (long long)ldo);
  if (n_tokens == 0) return ok();
  if (!x || !packed || !absmax8 || !code || !absmax2 || !offset2 || !out)
    return fail(TALM_EINVAL, "nf4_gemm: null pointer");
  if (!aligned(x, 16) || !aligned(packed, 16) || !aligned(out, 16))
    return fail(TALM_EINVAL, "nf4_gemm: x, packed and out must be 16-byte aligned");
  W4Args a{};
  a.x = x; a.ldx = ldx; a.n_tokens = static_cast<int>(n_tokens); a.k = static_cast<int>(k);
  a.packed = packed; a.absmax8 = absmax8; a.code = code; a.absmax2 = absmax2; a.offset2 = offset2;
  a.n_out = static_cast<int>(n_out); a.out = out; a.ldo = ldo;
  a.n_mtiles = static_cast<int>((n_tokens + S::kBM - 1) / S::kBM);
  a.n_ntiles = static_cast<int>((n_out + S::kBN - 1) / S::kBN);
  hipLaunchKernelGGL(w4_gemm_kernel, dim3(static_cast<unsigned>(a.n_mtiles * a.n_ntiles)),
                     dim3(S::kThreads), 0, as_stream(stream), a);
  return check_launch("nf4_gemm");
}
