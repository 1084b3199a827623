// The decoder's products on a weight W [rows, cols] held in the layer group's NF4 form
// (double-quantized absmax, 64-weight blocks along a row), fp16 MFMA on gfx950, with the weight
// dequantized into LDS inside the GEMM and never written to HBM (SURVEY's W4A16 row; it replaces
// the dequantization of the layer's buffer + the fp16 GEMM on it for the projections it serves,
// solution/qgroup.py:72-99 and :346-355):
//   forward     out [M, rows] = x [M, cols] W^T        ("nt": the reduction runs along W's rows)
//   input grad  out [M, cols] = dy [M, rows] W         ("nn": the reduction runs across W's rows)
//
// Why it pays on this chip: the fp16 GEMMs of the step are bound by the operand stream from L2
// into the CUs (about 16 bytes per clock per CU for direct-to-LDS loads), not by the MFMA pipe.
// A 256 x 256 tile of fp16 operands moves 64 KiB per 64-deep step; with the weight read as NF4
// codes it moves 32 KiB of activations plus 8 KiB of codes, and the dequantization (VALU and LDS
// writes) runs beside the MFMAs of the other wavefronts.
//
// Tiles of 256 tokens x 256 output columns, 8 wavefronts of 128 x 64 (v_mfma_f32_32x32x16_f16),
// 64-deep steps through a two-slot LDS ring:
//   A (activations) streams from global memory straight into LDS (buffer_load ... lds, the
//     swizzled layout of mfma_tile.h);
//   B (weights): each thread loads 16 bytes of codes (32 weights of one row and one block) and
//     the block's scale inputs two steps ahead into registers, and dequantizes them exactly as
//     the group dequant kernel does (fp32 level x scale, one rounding to fp16) into the other
//     slot while the MFMAs read this one. "nt" stores them as [256 out rows][64 k] (the MFMA
//     fragment layout); "nn" stores W's rows as they are, [64 k rows][256 out columns], and
//     reads its fragments with the transposing ds_read_b64_tr_b16.
// K is cut into parts when the output has too few tiles to fill the chip (fp32 partials summed
// in part order by splitk_reduce_kernel, deterministic). The fp16 weights are bit-identical to
// talm_nf4_group_dequant's; the products are fp16 GEMMs with fp32 accumulation.
#include "mfma_tile.h"
#include "nf4_code.h"
#include "splitk.h"

namespace talm {
namespace {

typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

using W4Shape = TileShape<256, 256, 64, 2, 2, 4>;
constexpr int kW4ASlots = 3, kW4BSlots = 2;         // A two steps ahead, B one
constexpr int kW4ABytes = W4Shape::kAChunks * 16;  // 32 KiB of activations per step
constexpr int kW4BBytes = W4Shape::kBChunks * 16;  // 32 KiB of fp16 weights per step
constexpr int kW4Ring = kW4ASlots * kW4ABytes + kW4BSlots * kW4BBytes;
constexpr int kW4ZS = W4Shape::kBN + 8;  // staged fp16 output row stride (halfs)
constexpr int kW4Lds = kW4Ring > W4Shape::kBM * kW4ZS * 2 ? kW4Ring : W4Shape::kBM * kW4ZS * 2;
static_assert(kW4Lds <= 160 * 1024, "LDS per CU");
static_assert(W4Shape::kThreads == 512, "the B mapping assumes 512 threads");

struct W4Args {
  const uint16_t* a;       // [M][lda]: x ("nt") or dy ("nn")
  int64_t lda;
  int M, N, K;             // out [M, N], reduction K
  int w_cols;              // W's row length (the NF4 blocks run along it)
  const uint8_t* packed;   // W [rows][w_cols], two weights per byte, high nibble first
  const float* scale;      // [rows * w_cols / 64]: each 64-weight block's decoded absmax
  uint16_t* out;           // [M][ldo] when parts == 1
  int64_t ldo;
  float* part;             // [parts][M][N] when parts > 1 or partial_out
  int steps_per_part, n_mtiles, n_ntiles, n_tiles, parts;
  int partial_out;         // fp32 partials even for one part (the caller sums them)
};

// One step of the wavefront's 128 x 64 block: per 16-deep slice ks its fragments, its MFMAs, then
// extra(ks) (the dequantization of the next stage, interleaved so that its VALU work issues
// while the slice's MFMAs run).
template <bool kNN, class Extra>
__device__ __forceinline__ void w4_mma(const uint4* __restrict__ As, const unsigned char* __restrict__ Bs,
                                       Acc<W4Shape>& acc, int lane, int wm, int wn, Extra&& extra) {
  using S = W4Shape;
  constexpr int kSteps = S::kBK / 16;
#pragma unroll
  for (int ks = 0; ks < kSteps; ++ks) {
    half8_t a[S::kFragM], b[S::kFragN];
    const int kc = ks * 2 + (lane >> 5);
#pragma unroll
    for (int i = 0; i < S::kFragM; ++i)
      a[i] = __builtin_bit_cast(half8_t, As[swz<S::kCpr>(wm * S::kWaveM + i * 32 + (lane & 31), kc)]);
#pragma unroll
    for (int j = 0; j < S::kFragN; ++j) {
      if constexpr (!kNN) {
        b[j] = __builtin_bit_cast(
            half8_t, reinterpret_cast<const uint4*>(Bs)[swz<S::kCpr>(wn * S::kWaveN + j * 32 + (lane & 31), kc)]);
      } else {
        b[j] = nn_b_fragment(Bs, ks, wn * S::kWaveN + j * 32, lane);
      }
    }
#pragma unroll
    for (int i = 0; i < S::kFragM; ++i)
#pragma unroll
      for (int j = 0; j < S::kFragN; ++j)
        acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_f16(a[i], b[j], acc[i][j], 0, 0, 0);
    extra(ks);
  }
}

// Word j (8 weights) of the 16 bytes of codes a thread loaded for a step, looked up in its
// block's table of scaled levels, into its 16-byte chunk of the B stage. The pointers are restrict-qualified, so
// these LDS accesses carry alias scopes of their own.
template <bool kNN>
__device__ __forceinline__ void w4_dequant_word(uint32_t word, const Nf4Table& table,
                                                uint4* __restrict__ bs, int tid, int j) {
  const uint4 v = nf4_lookup_word(word, table);
  if constexpr (!kNN)
    bs[swz<W4Shape::kCpr>(tid >> 1, 4 * (tid & 1) + j)] = v;
  else
    bs[nn_pos(tid >> 3, 4 * (tid & 7) + j)] = v;
}

template <bool kNN>
__global__ __launch_bounds__(W4Shape::kThreads, 1) void w4_gemm_kernel(W4Args a) {
  using S = W4Shape;
  // one LDS object (A ring, B ring; the output staging afterwards): with several, the compiler
  // tags their accesses with alias scopes and then waits for the ring's direct-to-LDS loads
  // before every LDS access of the same object
  __shared__ __attribute__((aligned(1024))) unsigned char smem[kW4Lds];
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int wm = wave / S::kWavesN, wn = wave % S::kWavesN;

  // row tiles vary fastest, then column tiles, then K parts: tiles in flight on one XCD share
  // the codes of their column tile and K part in its L2
  const uint32_t tile = xcd_tile(blockIdx.x, static_cast<uint32_t>(a.n_tiles));
  const int mt = static_cast<int>(tile % a.n_mtiles);
  const int rest = static_cast<int>(tile / a.n_mtiles);
  const int nt = rest % a.n_ntiles, kp = rest / a.n_ntiles;
  const int m0 = mt * S::kBM, n0 = nt * S::kBN;
  const int k0 = kp * a.steps_per_part * S::kBK;
  const int nk = min(a.steps_per_part, a.K / S::kBK - kp * a.steps_per_part);  // >= 1

  Loader<S, S::kBM> la;
  la.init(a.a + static_cast<int64_t>(m0) * a.lda + k0, a.lda, a.M - m0, nk * S::kBK, wave, lane);

  // B: this thread's 16 bytes of codes per step. "nt": weight row n0 + tid / 2 (clamped: the
  // columns of rows past N are not stored), k half tid % 2 (a row's 32 bytes of codes in two
  // adjacent lanes: storing 16 rows' halves per phase is a 2-way LDS bank conflict, and one
  // row per lane with the halves 256 threads apart measured slower). "nn": weight row k0 + 64 kt + tid / 8
  // (below K: K is a multiple of 64), 32 columns n0 + 32 (tid % 8) (clamped to the last 32 of the
  // row: columns past N are not stored). e0 is the first weight's element index at step 0, e_step
  // the advance per step (rows * cols < 2^31).
  uint32_t e0, e_step;
  if constexpr (!kNN) {
    e0 = static_cast<uint32_t>(min(n0 + (tid >> 1), a.N - 1)) * a.w_cols + k0 + 32 * (tid & 1);
    e_step = S::kBK;
  } else {
    e0 = static_cast<uint32_t>(k0 + (tid >> 3)) * a.w_cols + min(n0 + 32 * (tid & 7), a.w_cols - 32);
    e_step = static_cast<uint32_t>(S::kBK) * a.w_cols;
  }
  u32x4 bw[2];
  float bscale[2];
  auto b_load = [&](int r, int kt) {  // two loads: the codes and their block's scale
    const uint32_t e = e0 + e_step * static_cast<uint32_t>(min(kt, nk - 1));
    bw[r] = *reinterpret_cast<const u32x4*>(a.packed + (e >> 1));
    bscale[r] = a.scale[e >> 6];
  };

  Acc<S> acc;
#pragma unroll
  for (int i = 0; i < S::kFragM; ++i)
#pragma unroll
    for (int j = 0; j < S::kFragN; ++j)
#pragma unroll
      for (int v = 0; v < 16; ++v) acc[i][j][v] = 0.f;

  unsigned char* const b_ring = smem + kW4ASlots * kW4ABytes;
  // Step kt computes A slot kt % 3 and B slot kt % 2 while A(kt + 2) and the codes of step
  // kt + 2 load and the codes of step kt + 1 (register set (kt + 1) % 2, loaded in the step
  // before) are dequantized into B slot (kt + 1) % 2. Vector-memory issue order: A(0), codes(0),
  // A(1), codes(1), then per step A(kt + 2), codes(kt + 2); at step kt's top A(kt) is complete once
  // at most A(kt + 1) and codes(kt + 1) (6 loads) remain in flight (the codes of step kt were
  // waited for by the step before, which dequantized them). A is issued past the last step too
  // (its k window reads zeros into a retired slot), so the count holds to the end.
  la.issue(smem, 0, wave);
  b_load(0, 0);
  la.issue(smem + kW4ABytes, S::kBK, wave);
  b_load(1, 1);
  {
    const Nf4Table table = nf4_table(bscale[0]);
#pragma unroll
    for (int j = 0; j < 4; ++j)
      w4_dequant_word<kNN>(bw[0][j], table, reinterpret_cast<uint4*>(b_ring), tid, j);
  }
  auto step = [&](int kt, int h) {  // h = kt % 6: slots and register sets are constants
    wait_vmcnt<6>();
    lds_barrier();  // A(kt) landed, B(kt) stored; every wavefront is done with step kt - 1
    la.issue(smem + ((h + 2) % kW4ASlots) * kW4ABytes, (kt + 2) * S::kBK, wave);
    b_load(h & 1, kt + 2);  // set h % 2 held the codes of step kt, dequantized in the step before
    // the loads stay here, a step ahead of their use (the scheduler would sink them to their
    // first use to shorten the registers' lives)
    __builtin_amdgcn_sched_barrier(0);
    const Nf4Table table = nf4_table(bscale[(h + 1) & 1]);
    uint4* const b_next = reinterpret_cast<uint4*>(b_ring + ((h + 1) & 1) * kW4BBytes);
    w4_mma<kNN>(reinterpret_cast<const uint4*>(smem + (h % kW4ASlots) * kW4ABytes),
                b_ring + (h & 1) * kW4BBytes, acc, lane, wm, wn,
                [&](int ks) { w4_dequant_word<kNN>(bw[(h + 1) & 1][ks], table, b_next, tid, ks); });
  };
  for (int kb = 0; kb < nk; kb += 6) {
#pragma unroll
    for (int h = 0; h < 6; ++h) {
      if (kb + h >= nk) break;
      step(kb + h, h);
    }
  }
  __syncthreads();  // every wavefront is done with the ring (and every load has landed)

  if (a.parts > 1 || a.partial_out) {
    float* P = a.part + static_cast<int64_t>(kp) * a.M * a.N;
#pragma unroll
    for (int i = 0; i < S::kFragM; ++i)
#pragma unroll
      for (int j = 0; j < S::kFragN; ++j) {
        const int gc = n0 + acc_col<S>(wn, j, lane);
#pragma unroll
        for (int v = 0; v < 16; ++v) {
          const int gr = m0 + acc_row<S>(wm, i, v, lane);
          if (gr < a.M && gc < a.N) P[static_cast<int64_t>(gr) * a.N + gc] = acc[i][j][v];
        }
      }
    return;
  }
  // fp16 tile staged in LDS, then 16-byte row stores
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
#pragma unroll 4
  for (int it = 0; it < (S::kBM * kChunksPerRow) / S::kThreads; ++it) {
    const int c = it * S::kThreads + tid, row = c / kChunksPerRow, kc = c % kChunksPerRow;
    const int gr = m0 + row, gc = n0 + kc * 8;
    if (gr < a.M && gc < a.N)
      *reinterpret_cast<uint4*>(a.out + static_cast<int64_t>(gr) * a.ldo + gc) =
          *reinterpret_cast<const uint4*>(zs + row * kW4ZS + kc * 8);
  }
}

SplitPlan w4_plan(int64_t m, int64_t n, int64_t k) {
  return plan_split(m, n, k, W4Shape::kBM, W4Shape::kBN, W4Shape::kBK);
}

// rows x cols of W, the product's (M, N, K) and whether W's layout supports it
bool w4_shape_ok(bool nn, int64_t m, int64_t rows, int64_t cols) {
  if (m < 0 || m > (1 << 24) || rows < 64 || cols < 64 || rows > (1 << 20) || cols > (1 << 20) ||
      rows * cols >= (int64_t{1} << 31))
    return false;
  if (cols % 64 || (rows * cols) % 16384) return false;
  return nn ? rows % 64 == 0 : rows % 8 == 0;
}

}  // namespace
}  // namespace talm

using namespace talm;

TALM_API int64_t talm_nf4_gemm_workspace(int64_t n_tokens, int64_t rows, int64_t cols,
                                         int32_t transpose) {
  const bool nn = transpose != 0;
  if (!w4_shape_ok(nn, n_tokens, rows, cols)) return -1;
  const int64_t n = nn ? cols : rows, k = nn ? rows : cols;
  const SplitPlan p = w4_plan(n_tokens, n, k);
  return p.parts > 1 ? static_cast<int64_t>(p.parts) * n_tokens * n * 4 : 0;
}

namespace talm {
namespace {

// out == nullptr: fp32 partials [parts][n_tokens][n] in the workspace (also for one part), left
// for the caller's next launch to sum.
int nf4_gemm_impl(const char* what, const uint16_t* x, int64_t ldx, int64_t n_tokens,
                  const uint8_t* packed, const float* scale, int64_t rows, int64_t cols,
                  int32_t transpose, int32_t blocksize, uint16_t* out, int64_t ldo,
                  void* workspace, int64_t workspace_bytes, hipStream_t s) {
  using S = W4Shape;
  const bool nn = transpose != 0;
  if (blocksize != 64)
    return fail(TALM_EINVAL, "%s: blocksize %d (64 supported)", what, blocksize);
  const int64_t n = nn ? cols : rows, k = nn ? rows : cols;
  if (!w4_shape_ok(nn, n_tokens, rows, cols) || ldx < k || ldx % 8 ||
      (out && (ldo < n || ldo % 8)) || !(S::kBM * ldx * 2 < (int64_t{1} << 31)))
    return fail(TALM_EINVAL,
                "%s: bad shape (tokens %lld, W [%lld, %lld], %s, ldx %lld, ldo %lld): W's "
                "row length a multiple of 64, its rows a multiple of %d, whole 16384-weight "
                "groups, strides multiples of 8 covering the rows",
                what, (long long)n_tokens, (long long)rows, (long long)cols,
                nn ? "dy W" : "x W^T", (long long)ldx, (long long)ldo, nn ? 64 : 8);
  if (n_tokens == 0) return ok();
  if (!x || !packed || !scale) return fail(TALM_EINVAL, "%s: null pointer", what);
  if (!aligned(x, 16) || !aligned(packed, 16) || !aligned(out, 16) || !aligned(scale, 4))
    return fail(TALM_EINVAL, "%s: x, packed and out must be 16-byte aligned, scale 4-byte", what);
  const SplitPlan p = w4_plan(n_tokens, n, k);
  if (p.parts > 1 || !out) {
    const int64_t need = static_cast<int64_t>(p.parts) * n_tokens * n * 4;
    if (!workspace || workspace_bytes < need || !aligned(workspace, 16))
      return fail(TALM_EINVAL, "%s: workspace of %lld bytes, %lld needed (16-byte aligned)",
                  what, (long long)workspace_bytes, (long long)need);
  }
  W4Args a{};
  a.a = x; a.lda = ldx;
  a.M = static_cast<int>(n_tokens); a.N = static_cast<int>(n); a.K = static_cast<int>(k);
  a.w_cols = static_cast<int>(cols);
  a.packed = packed; a.scale = scale;
  a.out = out; a.ldo = ldo;
  a.part = static_cast<float*>(workspace);
  a.steps_per_part = p.steps_per_part;
  a.n_mtiles = p.n_mtiles; a.n_ntiles = p.n_ntiles; a.parts = p.parts;
  a.n_tiles = p.n_mtiles * p.n_ntiles * p.parts;
  a.partial_out = out ? 0 : 1;
  if (nn)
    hipLaunchKernelGGL(w4_gemm_kernel<true>, dim3(static_cast<unsigned>(a.n_tiles)),
                       dim3(S::kThreads), 0, s, a);
  else
    hipLaunchKernelGGL(w4_gemm_kernel<false>, dim3(static_cast<unsigned>(a.n_tiles)),
                       dim3(S::kThreads), 0, s, a);
  if (out && p.parts > 1)
    launch_splitk_reduce(static_cast<const float*>(workspace), p.parts, n_tokens, n, out, ldo, s);
  return check_launch(what);
}

}  // namespace
}  // namespace talm

TALM_API int talm_nf4_gemm(const uint16_t* x, int64_t ldx, int64_t n_tokens, const uint8_t* packed,
                           const float* scale, int64_t rows, int64_t cols, int32_t transpose,
                           int32_t blocksize, uint16_t* out, int64_t ldo, void* workspace,
                           int64_t workspace_bytes, void* stream) {
  if (!out && n_tokens > 0) return fail(TALM_EINVAL, "nf4_gemm: null pointer");
  return nf4_gemm_impl("nf4_gemm", x, ldx, n_tokens, packed, scale, rows, cols, transpose,
                       blocksize, out, ldo, workspace, workspace_bytes, as_stream(stream));
}

TALM_API int64_t talm_nf4_gemm_parts(int64_t n_tokens, int64_t rows, int64_t cols,
                                     int32_t transpose) {
  const bool nn = transpose != 0;
  if (!w4_shape_ok(nn, n_tokens, rows, cols)) return -1;
  return w4_plan(n_tokens, nn ? cols : rows, nn ? rows : cols).parts;
}

TALM_API int talm_nf4_gemm_partials(const uint16_t* x, int64_t ldx, int64_t n_tokens,
                                    const uint8_t* packed, const float* scale, int64_t rows,
                                    int64_t cols, int32_t transpose, int32_t blocksize,
                                    float* partials, int64_t partials_bytes, void* stream) {
  return nf4_gemm_impl("nf4_gemm_partials", x, ldx, n_tokens, packed, scale, rows, cols,
                       transpose, blocksize, nullptr, 0, partials, partials_bytes,
                       as_stream(stream));
}
