// Vocabulary-chunked fused LM head + cross-entropy for gfx950 (fp16 MFMA, fp32 statistics).
//
// The reference (solution/fused_head.py:315-393 with fused_head_vocab_kernel, :88-182) walks the
// vocabulary in slices of `vchunk` columns: per slice, fp16 logits z = fp16(H W_c^T), the online
// per-row statistics (max m, s = sum e^{z-m}, t = sum e^{z-m} z, first argmax, z at the target),
// and for labelled rows the gradient accumulator: acc = e^{m_old - m} acc + fp16(e^{z-m}) W_c,
// with m the running maximum after slice c; at the end dH = acc / s - W[target].
//
// The same recurrence here, shaped for MI355X. Slices are processed `group` at a time:
//   head_logits   Z = H W^T over the group's columns; the epilogue rounds to fp16, stages the
//                 tile in LDS and emits, per (row, 128-column tile), the tile's max m_t, first
//                 argmax, sum e^{z-m_t} and sum e^{z-m_t} z; for labelled rows it also writes
//                 P_t = fp16(e^{z - m_t}) to the group's buffer (the only copy of the logits
//                 that reaches global memory).
//   head_merge    one wavefront per row folds the tiles of each slice, in column order, into the
//                 running statistics exactly as the reference's per-slice update, recording the
//                 slice's running max m_c and rescale e^{m_old - m_c}, and for labelled rows the
//                 per-tile factors fp16(e^{m_t - m_c}); after the last slice it writes token
//                 loss, entropy, argmax and correctness.
//   head_grad     Y_c = P_c W_c for every slice of the group side by side, against the
//                 transposed weight W^T [hidden, vocab] so that both operands are k-contiguous;
//                 P_c = fp16(P_t e^{m_t - m_c}), the reference's fp16(e^{z - m_c}) up to one
//                 more fp16 rounding, is formed on the A fragments between LDS and the MFMAs.
//   head_combine  acc = e^{m_old - m_c} acc + Y_c in slice order (the reference's rescale then
//                 add), and after the last slice dH = acc / s - W16[target] in fp16.
// The full [N, V] logits never exist: one group of slices (group * vchunk columns) at a time.
//
// Both GEMMs run the tile core of mfma_tile.h (v_mfma_f32_32x32x16_f16, operands streamed by
// buffer_load_dwordx4 ... lds straight into an LDS ring, 16-byte chunks XOR-swizzled so that
// fragment reads are free of bank conflicts, tiles mapped to XCDs so the tiles that share an
// operand panel share an L2) in one of two shapes picked per launch: Narrow, 256 x 128 tiles
// with a three-stage ring of 32-deep steps and two workgroups per CU, or Wide, 256 x 256 tiles
// with a two-stage ring of 64-deep steps and one workgroup of eight wavefronts per CU.
#include "mfma_tile.h"

#include <algorithm>

namespace talm {
namespace {

constexpr int kThreads = 256;        // block size of the merge, combine and transpose kernels
constexpr int kTile = 128;           // statistics granule (columns)

// GEMM tile shapes of the head: 256 x BN, every wavefront 128 x 64, two wavefronts per SIMD.
// Narrow runs two 256-thread workgroups per CU; Wide one 512-thread workgroup that moves a third
// fewer bytes per FLOP. The logits epilogue stages the fp16 tile in LDS ([256][BN + 8] halfs).
template <int BN, int BK, int STAGES>
struct HeadShape : TileShape<256, BN, BK, STAGES, 2, BN / 64> {
  static constexpr int kZS = BN + 8;
  static constexpr int kRingBytes = TileShape<256, BN, BK, STAGES, 2, BN / 64>::kRing;
  static constexpr int kLds = kRingBytes > 256 * kZS * 2 ? kRingBytes : 256 * kZS * 2;
  static_assert(kLds <= 160 * 1024, "LDS per CU");
};
using Narrow = HeadShape<128, 32, 3>;  // 72 KiB ring
using Wide = HeadShape<256, 64, 2>;    // 128 KiB ring, 135 KiB with the staged logits tile
// head_grad runs the same tiles with wavefronts of 64 x 128: half as many A fragments per
// wavefront, each of which it scales between LDS and the MFMAs.
using GradNarrow = TileShape<256, 128, 32, 3, 4, 1>;
using GradWide = TileShape<256, 256, 64, 2, 4, 2>;
static_assert(GradNarrow::kThreads == Narrow::kThreads && GradWide::kThreads == Wide::kThreads &&
              GradNarrow::kPerCu == Narrow::kPerCu && GradWide::kPerCu == Wide::kPerCu,
              "head_grad shapes launch like the logits shapes");
constexpr int kBM = 256;

struct Stat {
  float m, s, t;
  int idx;
};

// Merge two partial statistics; ties of the maximum keep the smaller column (first argmax).
__device__ __forceinline__ Stat merge(Stat a, Stat b) {
  Stat r;
  r.m = fmaxf(a.m, b.m);
  if (r.m == -INFINITY) {
    r.s = 0.f;
    r.t = 0.f;
  } else {
    const float ea = a.m == -INFINITY ? 0.f : __expf(a.m - r.m);
    const float eb = b.m == -INFINITY ? 0.f : __expf(b.m - r.m);
    r.s = a.s * ea + b.s * eb;
    r.t = a.t * ea + b.t * eb;
  }
  if (a.m > b.m) r.idx = a.idx;
  else if (b.m > a.m) r.idx = b.idx;
  else r.idx = min(a.idx, b.idx);
  return r;
}

__device__ __forceinline__ Stat shfl_stat(Stat v, int off) {
  Stat r;
  r.m = __shfl_xor(v.m, off, kWave);
  r.s = __shfl_xor(v.s, off, kWave);
  r.t = __shfl_xor(v.t, off, kWave);
  r.idx = __shfl_xor(v.idx, off, kWave);
  return r;
}

// ------------------------------------------------------------------------------------------
// GEMM1: z[r][j] = fp16(sum_k H[r][k] W[j][k]) for the group's columns j < group_cols (W starts
// at the group's first vocabulary row) and the per-(row, 128-column tile) partial statistics;
// rows r < n_p (the labelled rows when the gradient is wanted) store P[r][j] = fp16(e^{z - m_t})
// with m_t the max of the row's 128-column tile, 0 past group_cols.
// ------------------------------------------------------------------------------------------
template <class S>
__global__ __launch_bounds__(S::kThreads, S::kPerCu) void head_logits_kernel(
    const uint16_t* __restrict__ H, int64_t ldh, const uint16_t* __restrict__ W, int64_t ldw,
    int n_rows, int K, int group_cols, int first_col, uint16_t* __restrict__ Z, int64_t ldz,
    float4* __restrict__ part, int parts_per_row, int n_mtiles, int n_ntiles,
    const int64_t* __restrict__ targets, float* __restrict__ ztarget, int n_p) {
  constexpr int kBN = S::kBN, kZS = S::kZS;
  __shared__ __attribute__((aligned(1024))) unsigned char smem[S::kLds];

  // row tiles vary fastest inside an XCD's range: the tiles in flight on one XCD share weight rows
  const uint32_t tile = xcd_tile(blockIdx.x, static_cast<uint32_t>(n_mtiles * n_ntiles));
  const int ntile = static_cast<int>(tile / n_mtiles);
  const int mtile = static_cast<int>(tile % n_mtiles);
  const int m0 = mtile * kBM, n0 = ntile * kBN;
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int wm = wave / S::kWavesN, wn = wave % S::kWavesN;

  Loader<S, kBM> la;
  Loader<S, kBN> lb;
  la.init(H + static_cast<int64_t>(m0) * ldh, ldh, n_rows - m0, K, wave, lane);
  lb.init(W + static_cast<int64_t>(n0) * ldw, ldw, group_cols - n0, K, wave, lane);
  Acc<S> acc;
  ring_gemm<S>(
      smem, (K + S::kBK - 1) / S::kBK,
      [&](unsigned char* slot, int kt) {
        la.issue(slot, kt * S::kBK, wave);
        lb.issue(slot + S::kAChunks * 16, kt * S::kBK, wave);
      },
      acc, lane, wave);

  // Epilogue 1: fp16 logits tile into LDS ([kBM][kZS] halfs).
  uint16_t* Zs = reinterpret_cast<uint16_t*>(smem);
#pragma unroll
  for (int i = 0; i < S::kFragM; ++i)
#pragma unroll
    for (int j = 0; j < S::kFragN; ++j)
#pragma unroll
      for (int v = 0; v < 16; ++v) {
        const int row = wm * 128 + i * 32 + 8 * (v >> 2) + 4 * (lane >> 5) + (v & 3);
        const int col = wn * 64 + j * 32 + (lane & 31);
        Zs[row * kZS + col] = f2h(acc[i][j][v]);
      }
  __syncthreads();

  // Epilogue 2: partial statistics of one (row, 128-column statistics tile) per thread, which
  // then replaces its z with P in LDS (stored for rows < n_p).
  {
    const int row = tid % kBM, st = tid / kBM, gr = m0 + row;
    const int c0 = n0 + st * kTile;  // the statistics tile's first column in the group
    const int valid = min(kTile, group_cols - c0);
    if (gr < n_rows && valid > 0) {
      uint16_t* zr = Zs + row * kZS + st * kTile;
      uint4 zv[kTile / 8];
#pragma unroll
      for (int c = 0; c < kTile / 8; ++c) zv[c] = *reinterpret_cast<const uint4*>(zr + 8 * c);
      float m = -INFINITY;
      int idx = 0;
#pragma unroll
      for (int c = 0; c < kTile / 8; ++c) {
        const uint32_t w4[4] = {zv[c].x, zv[c].y, zv[c].z, zv[c].w};
#pragma unroll
        for (int e = 0; e < 8; ++e) {
          const int col = 8 * c + e;
          const float z = (e & 1) ? hi_f(w4[e >> 1]) : lo_f(w4[e >> 1]);
          if (col < valid && z > m) {
            m = z;
            idx = col;
          }
        }
      }
      // the logit at the target, when the target column is in this tile (one tile per row)
      const int64_t rel = targets[gr] - (first_col + c0);
      if (rel >= 0 && rel < valid) ztarget[gr] = h2f(zr[static_cast<int>(rel)]);
      float sum = 0.f, t = 0.f;
#pragma unroll
      for (int c = 0; c < kTile / 8; ++c) {
        const uint32_t w4[4] = {zv[c].x, zv[c].y, zv[c].z, zv[c].w};
        float ez[8];
#pragma unroll
        for (int e = 0; e < 8; ++e) {
          const int col = 8 * c + e;
          const float z = (e & 1) ? hi_f(w4[e >> 1]) : lo_f(w4[e >> 1]);
          // columns past the group are z = 0 (zero weight rows) and get e^{-inf} = 0: no branch
          ez[e] = __expf(col < valid ? z - m : -INFINITY);
          sum += ez[e];
          t += ez[e] * z;
        }
        *reinterpret_cast<uint4*>(zr + 8 * c) = make_uint4(
              pack2(ez[0], ez[1]), pack2(ez[2], ez[3]), pack2(ez[4], ez[5]), pack2(ez[6], ez[7]));
      }
      part[static_cast<int64_t>(gr) * parts_per_row + c0 / kTile] =
          make_float4(m, sum, t, __int_as_float(first_col + c0 + idx));
    }
  }
  if (n_p <= m0) return;
  __syncthreads();

  // Epilogue 3: the P rows of the tile to global memory in 16-byte chunks (kBN / 8 per row); the
  // chunk that holds the group's last column carries the zeros past it (head_grad reads chunks).
#pragma unroll
  for (int it = 0; it < (kBM * kBN / 8) / S::kThreads; ++it) {
    const int c = it * S::kThreads + tid, row = c / (kBN / 8), kc = c % (kBN / 8);
    const int gr = m0 + row, gc = n0 + kc * 8;
    if (gr < n_p && gc < group_cols)
      *reinterpret_cast<uint4*>(Z + static_cast<int64_t>(gr) * ldz + gc) =
          *reinterpret_cast<const uint4*>(Zs + row * kZS + kc * 8);
  }
}

// ------------------------------------------------------------------------------------------
// Running statistics, one wavefront per row, over the slices of one group.
// ------------------------------------------------------------------------------------------
// Factor of labelled row r and the group's 128-column tile t, e^{m_t - m_c} in fp16, where it
// sits for head_grad: 128-row blocks b = r / 128 of [tile][block][128] halfs, and inside a block
// the four rows r % 32 + 32 i (i < 4) next to each other, so that one 8-byte load gives a lane of
// a 128-row wavefront the factors of its four A-fragment rows.
__device__ __forceinline__ int64_t scale_index(int row, int tile, int n_blocks) {
  return (static_cast<int64_t>(tile) * n_blocks + (row >> 7)) * 128 + (row & 31) * 4 + ((row >> 5) & 3);
}

struct MergeArgs {
  const float4* part;
  int parts_per_row;
  uint16_t* scale;         // per-(labelled row, tile) factors, see scale_index
  int scale_blocks;        // 128-row blocks per tile in `scale`
  const int64_t* targets;
  const float* ztarget;    // [n_rows] the logit at the target (written by head_logits)
  int n_rows;
  int n_grad;
  int n_slices;            // slices in this group
  int slice_cols[8];       // columns of each slice (the last may be narrower)
  int slice_col0[8];       // first vocabulary column of each slice
  int vchunk;              // columns per full slice (a multiple of kTile)
  int first_slice;         // this group holds the first slice of the vocabulary
  int last_slice;          // this group holds the last slice
  float* run;              // [6][n_rows]: m, s, t, best, zt, best_idx (as int bits)
  float* alpha;            // [n_slices][n_rows]: e^{m_old - m} of each slice (0 for the first)
  float* token_loss;
  float* entropy;
  int32_t* best_idx;
  int32_t* correct;
};

__global__ __launch_bounds__(kThreads) void head_merge_kernel(MergeArgs a) {
  const int lane = threadIdx.x & 63;
  const int row = blockIdx.x * (kThreads / kWave) + (threadIdx.x >> 6);
  if (row >= a.n_rows) return;
  const int64_t target = a.targets[row];
  const bool labelled = target >= 0;
  float* run = a.run;
  const int n = a.n_rows;
  float m, s, t, best, zt;
  int bidx;
  if (a.first_slice) {
    m = -INFINITY; s = 0.f; t = 0.f; best = -INFINITY; zt = 0.f; bidx = 0;
  } else {
    m = run[row]; s = run[n + row]; t = run[2 * n + row]; best = run[3 * n + row];
    zt = run[4 * n + row]; bidx = __float_as_int(run[5 * n + row]);
  }
  for (int c = 0; c < a.n_slices; ++c) {
    const int tiles = (a.slice_cols[c] + kTile - 1) / kTile;
    const int tile0 = c * (a.vchunk / kTile);
    Stat acc{-INFINITY, 0.f, 0.f, 0x7fffffff};
    for (int tt = lane; tt < tiles; tt += kWave) {
      const float4 p = a.part[static_cast<int64_t>(row) * a.parts_per_row + tile0 + tt];
      acc = merge(acc, Stat{p.x, p.y, p.z, __float_as_int(p.w)});
    }
#pragma unroll
    for (int off = 32; off >= 1; off >>= 1) acc = merge(acc, shfl_stat(acc, off));
    // the slice into the running statistics (solution/fused_head.py:136-153)
    const float m_old = m;
    const float m_new = fmaxf(m, acc.m);
    const float e_old = m == -INFINITY ? 0.f : __expf(m - m_new);
    const float e_new = acc.m == -INFINITY ? 0.f : __expf(acc.m - m_new);
    s = s * e_old + acc.s * e_new;
    t = t * e_old + acc.t * e_new;
    m = m_new;
    if (acc.m > best) {
      best = acc.m;
      bidx = acc.idx;
    }
    const int64_t rel = target - a.slice_col0[c];
    if (labelled && rel >= 0 && rel < a.slice_cols[c]) zt = a.ztarget[row];
    if (row < a.n_grad) {
      // P_t = fp16(e^{z - m_t}) of each tile becomes the reference's fp16(e^{z - m_c})
      // (solution/fused_head.py:178-182) through e^{m_t - m_c}, applied by head_grad
      for (int tt = lane; tt < tiles; tt += kWave) {
        const float mt = a.part[static_cast<int64_t>(row) * a.parts_per_row + tile0 + tt].x;
        const float f = mt == -INFINITY ? 0.f : __expf(mt - m);
        a.scale[scale_index(row, tile0 + tt, a.scale_blocks)] = f2h(f);
      }
    }
    if (lane == 0) {
      a.alpha[static_cast<int64_t>(c) * n + row] =
          (a.first_slice && c == 0) || m_old == -INFINITY ? 0.f : __expf(m_old - m);
    }
  }
  if (lane != 0) return;
  run[row] = m; run[n + row] = s; run[2 * n + row] = t; run[3 * n + row] = best;
  run[4 * n + row] = zt; run[5 * n + row] = __int_as_float(bidx);
  if (a.last_slice) {  // solution/fused_head.py:160-169
    const float ls = __logf(s);
    const float lse = m + ls;
    a.entropy[row] = lse - t / s;
    a.token_loss[row] = labelled ? ls + (m - zt) : 0.f;
    a.best_idx[row] = bidx;
    a.correct[row] = (labelled && static_cast<int64_t>(bidx) == target) ? 1 : 0;
  }
}

// ------------------------------------------------------------------------------------------
// GEMM2: Y_c[r][h] = sum_j P_c[r][zc + j] W^T[h][col0 + zc + j] over slice c's columns (zc = c *
// vchunk inside the group), for the first n_grad rows (the labelled rows, put first by the
// caller); P_c = fp16(P_t e^{m_t - m_c}) from head_logits' P_t and head_merge's factors.
// ------------------------------------------------------------------------------------------

// The A-fragment hook of head_grad: ring step kt covers columns [zc + kt BK, + BK) of one 128-column
// tile (BK divides 128, zc is a multiple of BK); lane l of the wavefront owning rows
// [r0, r0 + 32 FRAGS) multiplies fragment i (row r0 + 32 i + l % 32) by the row's factor of that
// tile. r0 is a multiple of 32 FRAGS, so the lane's FRAGS factors are adjacent: one load per step,
// into the register set of the step's ring slot.
template <int BK, int FRAGS, int SLOTS>
struct TileScale {
  static_assert(FRAGS == 2 || FRAGS == 4, "two or four 32-row A fragments per wavefront");
  using Word = typename std::conditional<FRAGS == 4, uint2, uint32_t>::type;
  const uint16_t* base;  // &scale[scale_index(r0 + lane % 32, 0, blocks)]
  int64_t tile_stride;   // blocks * 128
  int zc;
  Word f[SLOTS];
  __device__ __forceinline__ void prefetch(int kt, int slot) {
    f[slot] = *reinterpret_cast<const Word*>(base + ((zc + kt * BK) >> 7) * tile_stride);
  }
  __device__ __forceinline__ half8_t apply(half8_t a, int i, int slot) const {
    uint32_t w;
    if constexpr (FRAGS == 4) w = i < 2 ? f[slot].x : f[slot].y;
    else w = f[slot];
    const uint16_t h = static_cast<uint16_t>((i & 1) ? w >> 16 : w & 0xffffu);
    return a * __builtin_bit_cast(_Float16, h);
  }
};
struct GradArgs {
  const uint16_t* Z;
  int64_t ldz;
  const uint16_t* WT;     // transposed weight [hidden][ldwt], columns past the vocabulary zero
  int64_t ldwt;
  int col0;               // the group's first vocabulary column
  int n_grad;
  int hidden;
  int vchunk;
  int slice_cols[8];
  int ksplit;             // parts of each slice's columns, each with its own partial
  const uint16_t* scale;  // per-(row, tile) factors of head_merge, see scale_index
  int scale_blocks;
  float* Y;               // [n_slices * ksplit][n_grad][hidden] fp32
  int n_mtiles, n_ntiles, n_tiles;
};

template <class S>
__global__ __launch_bounds__(S::kThreads, S::kPerCu) void head_grad_kernel(GradArgs a) {
  constexpr int kBN = S::kBN;
  __shared__ __attribute__((aligned(1024))) unsigned char smem[S::kRing];

  // hidden tiles vary fastest inside an XCD's range: the tiles in flight on one XCD share P rows
  const uint32_t tile = xcd_tile(blockIdx.x, static_cast<uint32_t>(a.n_tiles));
  const int ntile = static_cast<int>(tile % a.n_ntiles);
  const int rest = static_cast<int>(tile / a.n_ntiles);
  const int mtile = rest % a.n_mtiles, piece = rest / a.n_mtiles;
  const int slice = piece / a.ksplit, kpart = piece % a.ksplit;
  const int m0 = mtile * kBM, n0 = ntile * kBN;
  const int cols = a.slice_cols[slice];
  // this part's columns of the slice, in whole steps
  const int span = (cols + a.ksplit - 1) / a.ksplit;
  const int per = (span + S::kBK - 1) / S::kBK * S::kBK;
  const int k0 = min(kpart * per, cols), kn = min(cols - k0, per);
  const int zc = slice * a.vchunk + k0;
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int wm = wave / S::kWavesN, wn = wave % S::kWavesN;

  Loader<S, kBM> la;
  Loader<S, kBN> lb;
  la.init(a.Z + static_cast<int64_t>(m0) * a.ldz + zc, a.ldz, a.n_grad - m0, kn, wave, lane);
  lb.init(a.WT + static_cast<int64_t>(n0) * a.ldwt + a.col0 + zc, a.ldwt, a.hidden - n0, kn,
          wave, lane);
  TileScale<S::kBK, S::kFragM, S::kStages> sc;
  sc.base = a.scale + scale_index(m0 + wm * S::kWaveM + (lane & 31), 0, a.scale_blocks);
  sc.tile_stride = static_cast<int64_t>(a.scale_blocks) * 128;
  sc.zc = kn > 0 ? zc : 0;  // an empty part (zc may be the group's end) still loads in range
  Acc<S> acc;
  ring_gemm<S>(
      smem, (kn + S::kBK - 1) / S::kBK,
      [&](unsigned char* slot, int kt) {
        la.issue(slot, kt * S::kBK, wave);
        lb.issue(slot + S::kAChunks * 16, kt * S::kBK, wave);
      },
      acc, lane, wave, sc);

  float* Y = a.Y + static_cast<int64_t>(piece) * a.n_grad * a.hidden;
#pragma unroll
  for (int i = 0; i < S::kFragM; ++i)
#pragma unroll
    for (int j = 0; j < S::kFragN; ++j)
#pragma unroll
      for (int v = 0; v < 16; ++v) {
        const int gr = m0 + acc_row<S>(wm, i, v, lane);
        const int gc = n0 + acc_col<S>(wn, j, lane);
        if (gr < a.n_grad && gc < a.hidden) Y[static_cast<int64_t>(gr) * a.hidden + gc] = acc[i][j][v];
      }
}

// ------------------------------------------------------------------------------------------
// acc = e^{m_old - m_c} acc + Y_c in slice order; after the last slice dH = acc / s - W[target].
// One thread per 4 hidden columns of one row.
// ------------------------------------------------------------------------------------------
struct CombineArgs {
  float* acc;              // [n_grad][hidden]
  const float* Y;          // [n_slices * ksplit][n_grad][hidden]: ksplit partials per slice
  const float* alpha;      // [n_slices][n_rows]
  const float* run;        // running statistics (s at [n_rows + row])
  const int64_t* targets;
  const uint16_t* W;       // full weight (row = vocabulary column)
  int64_t ldw;
  int64_t vocab;
  uint16_t* grad;          // [n_rows][hidden] fp16 (written after the last slice)
  int n_rows, n_grad, hidden, n_slices, ksplit, first_slice, last_slice;
};

__global__ __launch_bounds__(kThreads) void head_combine_kernel(CombineArgs a) {
  const int q = a.hidden / 4;
  const int64_t idx = static_cast<int64_t>(blockIdx.x) * kThreads + threadIdx.x;
  const int64_t rows = a.last_slice ? a.n_rows : a.n_grad;
  if (idx >= rows * q) return;
  const int row = static_cast<int>(idx / q), col = static_cast<int>(idx % q) * 4;
  if (row >= a.n_grad) {  // unlabelled rows: zero gradient
    *reinterpret_cast<uint2*>(a.grad + static_cast<int64_t>(row) * a.hidden + col) = make_uint2(0u, 0u);
    return;
  }
  const int64_t at = static_cast<int64_t>(row) * a.hidden + col;
  float4 v = a.first_slice ? make_float4(0.f, 0.f, 0.f, 0.f) : *reinterpret_cast<const float4*>(a.acc + at);
  for (int c = 0; c < a.n_slices; ++c) {
    const float al = a.alpha[static_cast<int64_t>(c) * a.n_rows + row];
    float4 y = make_float4(0.f, 0.f, 0.f, 0.f);
    for (int p = 0; p < a.ksplit; ++p) {
      const float4 yp = *reinterpret_cast<const float4*>(
          a.Y + static_cast<int64_t>(c * a.ksplit + p) * a.n_grad * a.hidden + at);
      y.x += yp.x; y.y += yp.y; y.z += yp.z; y.w += yp.w;
    }
    if (a.first_slice && c == 0) {
      v = y;
    } else {
      v.x = v.x * al + y.x; v.y = v.y * al + y.y; v.z = v.z * al + y.z; v.w = v.w * al + y.w;
    }
  }
  if (!a.last_slice) {
    *reinterpret_cast<float4*>(a.acc + at) = v;
    return;
  }
  const float s = a.run[a.n_rows + row];
  const int64_t tgt = a.targets[row];
  if (tgt < 0) {  // an ignored row among the gradient rows: zero gradient, as for the others
    *reinterpret_cast<uint2*>(a.grad + at) = make_uint2(0u, 0u);
    return;
  }
  // a target at or past the vocabulary (a broken contract) must not make the kernel read
  // outside the weight: its W[target] term is left out
  uint2 wv = make_uint2(0u, 0u);
  if (tgt >= 0 && tgt < a.vocab) wv = *reinterpret_cast<const uint2*>(a.W + tgt * a.ldw + col);
  const float g0 = v.x / s - lo_f(wv.x), g1 = v.y / s - hi_f(wv.x);
  const float g2 = v.z / s - lo_f(wv.y), g3 = v.w / s - hi_f(wv.y);
  *reinterpret_cast<uint2*>(a.grad + at) = make_uint2(pack2(g0, g1), pack2(g2, g3));
}

// ------------------------------------------------------------------------------------------
// WT[h][v] = W[v][h] for v < vocab, 0 for vocab <= v < ldwt: the k-contiguous B operand of
// head_grad. 64 x 64 blocks through LDS, 16-byte loads and stores.
// ------------------------------------------------------------------------------------------
__global__ __launch_bounds__(kThreads) void weight_t_kernel(const uint16_t* __restrict__ W,
                                                            int64_t ldw, int vocab, int hidden,
                                                            uint16_t* __restrict__ WT,
                                                            int64_t ldwt) {
  __shared__ uint16_t tile[64][64 + 2];
  const int v0 = blockIdx.x * 64, h0 = blockIdx.y * 64;
  const int tid = threadIdx.x;
#pragma unroll
  for (int it = 0; it < 2; ++it) {  // 64 vocabulary rows x 8 chunks of 8 hidden columns
    const int c = it * kThreads + tid, r = c >> 3, hc = (c & 7) * 8;
    const int v = v0 + r, h = h0 + hc;
    uint4 x = make_uint4(0, 0, 0, 0);
    if (v < vocab && h < hidden) x = *reinterpret_cast<const uint4*>(W + static_cast<int64_t>(v) * ldw + h);
    const uint32_t w4[4] = {x.x, x.y, x.z, x.w};
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      tile[hc + 2 * e][r] = static_cast<uint16_t>(w4[e] & 0xffffu);
      tile[hc + 2 * e + 1][r] = static_cast<uint16_t>(w4[e] >> 16);
    }
  }
  __syncthreads();
#pragma unroll
  for (int it = 0; it < 2; ++it) {  // 64 hidden rows x 8 chunks of 8 vocabulary columns
    const int c = it * kThreads + tid, r = c >> 3, vc = (c & 7) * 8;
    const int h = h0 + r, v = v0 + vc;
    if (h >= hidden || v >= ldwt) continue;
    uint32_t w4[4];
#pragma unroll
    for (int e = 0; e < 4; ++e)
      w4[e] = static_cast<uint32_t>(tile[r][vc + 2 * e]) | (static_cast<uint32_t>(tile[r][vc + 2 * e + 1]) << 16);
    *reinterpret_cast<uint4*>(WT + static_cast<int64_t>(h) * ldwt + v) = make_uint4(w4[0], w4[1], w4[2], w4[3]);
  }
}

size_t align_up(size_t v, size_t a) { return (v + a - 1) / a * a; }

constexpr int kCus = 256;  // MI355X compute units

// Fraction of the launch's workgroup slots that hold work, over the rounds it takes.
double fill(int64_t blocks, int per_cu) {
  const int64_t slots = static_cast<int64_t>(kCus) * per_cu;
  const int64_t rounds = (blocks + slots - 1) / slots;
  return rounds ? static_cast<double>(blocks) / static_cast<double>(rounds * slots) : 0.0;
}

// The Wide shape moves a third fewer bytes per FLOP (~20% faster per tile); pick it unless the
// launch fills the chip clearly worse with it.
constexpr double kWideGain = 1.2;

bool logits_wide(int64_t n_rows, int64_t gcols) {
  const int64_t mt = (n_rows + kBM - 1) / kBM;
  return kWideGain * fill(mt * ((gcols + Wide::kBN - 1) / Wide::kBN), Wide::kPerCu) >=
         fill(mt * ((gcols + Narrow::kBN - 1) / Narrow::kBN), Narrow::kPerCu);
}

// The gradient GEMM's output [n_grad, hidden] per slice is small: besides the shape, each slice's
// columns may be split into `ksplit` parts (each its own fp32 partial, summed by head_combine) so
// the launch fills the chip. Each extra part costs a little partial traffic.
struct GradPlan {
  bool wide;
  int ksplit;
};

GradPlan plan_grad(int64_t n_grad, int64_t hidden, int ns) {
  const int64_t mt = (n_grad + kBM - 1) / kBM;
  GradPlan best{true, 1};
  double best_score = -1.0;
  for (int wide = 1; wide >= 0; --wide) {
    const int bn = wide ? Wide::kBN : Narrow::kBN;
    for (int ks = 1; ks <= 4; ++ks) {
      const int64_t blocks = mt * ((hidden + bn - 1) / bn) * ns * ks;
      const double score = (wide ? kWideGain : 1.0) * (1.0 - 0.03 * (ks - 1)) *
                           fill(blocks, wide ? Wide::kPerCu : Narrow::kPerCu);
      if (score > best_score + 1e-9) {
        best_score = score;
        best = GradPlan{wide != 0, ks};
      }
    }
  }
  return best;
}

struct Layout {
  size_t z, part, scale, run, ztarget, alpha, y, acc, total;
  int64_t ldz;
  int parts_per_row;
  int scale_blocks;  // 128-row blocks of the factor table: whole 256-row tiles of head_grad
};

Layout layout(int64_t n_rows, int64_t hidden, int64_t vocab, int64_t vchunk, int64_t n_grad,
              int group) {
  Layout l{};
  l.ldz = align_up(static_cast<size_t>(group * vchunk), 8);
  l.parts_per_row = static_cast<int>(group * vchunk / kTile);
  // fp32 partials for the largest group: a full one, or the last (narrower) one
  const int64_t slices = (vocab + vchunk - 1) / vchunk;
  const int last = static_cast<int>(slices - (slices - 1) / group * group);
  const int64_t pieces = n_grad > 0 ? std::max<int64_t>(group * plan_grad(n_grad, hidden, group).ksplit,
                                                        last * plan_grad(n_grad, hidden, last).ksplit)
                                    : 0;
  l.scale_blocks = static_cast<int>((n_grad + kBM - 1) / kBM * 2);
  size_t off = 0;
  l.z = off;      off = align_up(off + static_cast<size_t>(n_grad) * l.ldz * 2, 256);
  l.part = off;   off = align_up(off + static_cast<size_t>(n_rows) * l.parts_per_row * 16, 256);
  l.scale = off;  off = align_up(off + static_cast<size_t>(l.parts_per_row) * l.scale_blocks * 128 * 2, 256);
  l.run = off;    off = align_up(off + static_cast<size_t>(n_rows) * 6 * 4, 256);
  l.ztarget = off; off = align_up(off + static_cast<size_t>(n_rows) * 4, 256);
  l.alpha = off;  off = align_up(off + static_cast<size_t>(group) * n_rows * 4, 256);
  l.y = off;      off = align_up(off + static_cast<size_t>(pieces) * n_grad * hidden * 4, 256);
  l.acc = off;    off = align_up(off + static_cast<size_t>(n_grad) * hidden * 4, 256);
  l.total = off;
  return l;
}

}  // namespace
}  // namespace talm

using namespace talm;

TALM_API int64_t talm_head_ce_workspace(int64_t n_rows, int64_t hidden, int64_t vocab,
                                        int64_t vchunk, int64_t n_grad, int32_t group) {
  if (n_rows < 0 || hidden < 1 || vocab < 1 || vchunk < kTile || vchunk % kTile || n_grad < 0 ||
      n_grad > n_rows || group < 1 || group > 8)
    return -1;
  const int64_t slices = (vocab + vchunk - 1) / vchunk;
  const int g = static_cast<int>(slices < group ? slices : group);
  return static_cast<int64_t>(layout(n_rows, hidden, vocab, vchunk, n_grad, g).total);
}

TALM_API int talm_head_weight_t(const uint16_t* weight, int64_t ldw, int64_t vocab,
                                int64_t hidden, uint16_t* weight_t, int64_t ldwt, void* stream) {
  if (vocab < 1 || hidden < 8 || hidden % 8 || ldw < hidden || ldw % 8 || ldwt < vocab ||
      ldwt % 8 || vocab > (1 << 30) || hidden > (1 << 20))
    return fail(TALM_EINVAL,
                "head_weight_t: bad shape (vocab %lld, hidden %lld, ldw %lld, ldwt %lld): hidden "
                "and both strides multiples of 8, ldw >= hidden, ldwt >= vocab",
                (long long)vocab, (long long)hidden, (long long)ldw, (long long)ldwt);
  if (!weight || !weight_t) return fail(TALM_EINVAL, "head_weight_t: null pointer");
  if (!aligned(weight, 16) || !aligned(weight_t, 16))
    return fail(TALM_EINVAL, "head_weight_t: weight and weight_t must be 16-byte aligned");
  const dim3 grid(static_cast<unsigned>((ldwt + 63) / 64), static_cast<unsigned>((hidden + 63) / 64));
  hipLaunchKernelGGL(weight_t_kernel, grid, dim3(kThreads), 0, as_stream(stream), weight, ldw,
                     static_cast<int>(vocab), static_cast<int>(hidden), weight_t, ldwt);
  return check_launch("head_weight_t");
}

TALM_API int talm_head_ce(const uint16_t* hidden_states, int64_t ldh, const uint16_t* weight,
                          int64_t ldw, const uint16_t* weight_t, int64_t ldwt,
                          const int64_t* targets, int64_t n_rows, int64_t hidden,
                          int64_t vocab, int64_t vchunk, int64_t n_grad, int32_t group,
                          float* token_loss, float* entropy, int32_t* best_idx, int32_t* correct,
                          uint16_t* grad_hidden, void* workspace, int64_t workspace_bytes,
                          void* stream) {
  if (n_rows < 0 || hidden < 8 || hidden % 8 || vocab < 1 || vchunk < kTile || vchunk % kTile ||
      n_grad < 0 || n_grad > n_rows || group < 1 || group > 8 || ldh < hidden || ldh % 8 ||
      ldw < hidden || ldw % 8)
    return fail(TALM_EINVAL,
                "head_ce: bad shape (rows %lld, hidden %lld, vocab %lld, vchunk %lld, n_grad "
                "%lld, group %d, ldh %lld, ldw %lld): hidden and strides multiples of 8, vchunk "
                "a multiple of %d, 1 <= group <= 8",
                (long long)n_rows, (long long)hidden, (long long)vocab, (long long)vchunk,
                (long long)n_grad, group, (long long)ldh, (long long)ldw, kTile);
  if (n_rows > (1 << 30) || vocab > (1 << 30) || hidden > (1 << 20) || ldh >= (1 << 22) ||
      ldw >= (1 << 22))
    return fail(TALM_EINVAL, "head_ce: sizes beyond 32-bit indexing (row strides below 2^22)");
  const bool with_grad = n_grad > 0 && grad_hidden;
  if (with_grad && (ldwt < vocab || ldwt % 8 || ldwt >= (1 << 22)))
    return fail(TALM_EINVAL, "head_ce: weight_t row stride %lld: at least vocab (%lld), a "
                             "multiple of 8", (long long)ldwt, (long long)vocab);
  if (n_rows == 0) return ok();
  if (!hidden_states || !weight || !targets || !token_loss || !entropy || !best_idx || !correct ||
      !workspace || (n_grad > 0 && !grad_hidden) || (with_grad && !weight_t))
    return fail(TALM_EINVAL, "head_ce: null pointer");
  if (!aligned(hidden_states, 16) || !aligned(weight, 16) || !aligned(workspace, 256) ||
      (grad_hidden && !aligned(grad_hidden, 16)) || (with_grad && !aligned(weight_t, 16)))
    return fail(TALM_EINVAL, "head_ce: hidden states, weight, weight_t and dH must be 16-byte "
                             "aligned, the workspace 256-byte aligned");
  const int64_t slices = (vocab + vchunk - 1) / vchunk;
  const int g = static_cast<int>(slices < group ? slices : group);
  const Layout l = layout(n_rows, hidden, vocab, vchunk, n_grad, g);
  if (l.ldz >= (1 << 22))
    return fail(TALM_EINVAL, "head_ce: group * vchunk = %lld columns per step, below 2^22 needed",
                (long long)l.ldz);
  if (workspace_bytes < static_cast<int64_t>(l.total))
    return fail(TALM_EINVAL, "head_ce: workspace of %lld bytes, %zu needed",
                (long long)workspace_bytes, l.total);
  unsigned char* ws = static_cast<unsigned char*>(workspace);
  uint16_t* Z = reinterpret_cast<uint16_t*>(ws + l.z);
  float4* part = reinterpret_cast<float4*>(ws + l.part);
  uint16_t* scale = reinterpret_cast<uint16_t*>(ws + l.scale);
  float* run = reinterpret_cast<float*>(ws + l.run);
  float* ztarget = reinterpret_cast<float*>(ws + l.ztarget);
  float* alpha = reinterpret_cast<float*>(ws + l.alpha);
  float* Y = reinterpret_cast<float*>(ws + l.y);
  float* accbuf = reinterpret_cast<float*>(ws + l.acc);
  const hipStream_t s = as_stream(stream);
  const int rows = static_cast<int>(n_rows);
  const int mt = (rows + kBM - 1) / kBM;
  const int n_p = grad_hidden ? static_cast<int>(n_grad) : 0;  // rows whose P is stored

  for (int64_t s0 = 0; s0 < slices; s0 += g) {
    const int ns = static_cast<int>(slices - s0 < g ? slices - s0 : g);
    const int64_t col0 = s0 * vchunk;
    const int64_t gcols = (s0 + ns == slices) ? vocab - col0 : ns * vchunk;
    if (logits_wide(rows, gcols)) {
      const int nt = static_cast<int>((gcols + Wide::kBN - 1) / Wide::kBN);
      hipLaunchKernelGGL((head_logits_kernel<Wide>), dim3(static_cast<unsigned>(mt * nt)),
                         dim3(Wide::kThreads), 0, s, hidden_states, ldh, weight + col0 * ldw, ldw,
                         rows, static_cast<int>(hidden), static_cast<int>(gcols),
                         static_cast<int>(col0), Z, l.ldz, part, l.parts_per_row, mt, nt, targets,
                         ztarget, n_p);
    } else {
      const int nt = static_cast<int>((gcols + Narrow::kBN - 1) / Narrow::kBN);
      hipLaunchKernelGGL((head_logits_kernel<Narrow>), dim3(static_cast<unsigned>(mt * nt)),
                         dim3(Narrow::kThreads), 0, s, hidden_states, ldh, weight + col0 * ldw,
                         ldw, rows, static_cast<int>(hidden), static_cast<int>(gcols),
                         static_cast<int>(col0), Z, l.ldz, part, l.parts_per_row, mt, nt, targets,
                         ztarget, n_p);
    }
    MergeArgs ma{};
    ma.part = part; ma.parts_per_row = l.parts_per_row;
    ma.scale = scale; ma.scale_blocks = l.scale_blocks;
    ma.targets = targets; ma.ztarget = ztarget; ma.n_rows = rows;
    ma.n_grad = n_p;
    ma.n_slices = ns; ma.vchunk = static_cast<int>(vchunk);
    for (int c = 0; c < ns; ++c) {
      const int64_t c0 = col0 + c * vchunk;
      ma.slice_col0[c] = static_cast<int>(c0);
      ma.slice_cols[c] = static_cast<int>(vocab - c0 < vchunk ? vocab - c0 : vchunk);
    }
    ma.first_slice = s0 == 0;
    ma.last_slice = s0 + ns == slices;
    ma.run = run; ma.alpha = alpha;
    ma.token_loss = token_loss; ma.entropy = entropy; ma.best_idx = best_idx; ma.correct = correct;
    hipLaunchKernelGGL(head_merge_kernel, dim3(static_cast<unsigned>((rows + 3) / 4)), dim3(kThreads),
                       0, s, ma);
    if (n_grad > 0 && grad_hidden) {
      GradArgs ga{};
      ga.Z = Z; ga.ldz = l.ldz; ga.WT = weight_t; ga.ldwt = ldwt; ga.col0 = static_cast<int>(col0);
      ga.n_grad = static_cast<int>(n_grad); ga.hidden = static_cast<int>(hidden);
      ga.vchunk = static_cast<int>(vchunk);
      for (int c = 0; c < ns; ++c) ga.slice_cols[c] = ma.slice_cols[c];
      ga.scale = scale; ga.scale_blocks = l.scale_blocks;
      ga.Y = Y;
      const GradPlan gp = plan_grad(n_grad, hidden, ns);
      const int bn = gp.wide ? Wide::kBN : Narrow::kBN;
      ga.ksplit = gp.ksplit;
      ga.n_mtiles = static_cast<int>((n_grad + kBM - 1) / kBM);
      ga.n_ntiles = static_cast<int>((hidden + bn - 1) / bn);
      ga.n_tiles = ga.n_mtiles * ga.n_ntiles * ns * gp.ksplit;
      if (gp.wide)
        hipLaunchKernelGGL((head_grad_kernel<GradWide>), dim3(static_cast<unsigned>(ga.n_tiles)),
                           dim3(GradWide::kThreads), 0, s, ga);
      else
        hipLaunchKernelGGL((head_grad_kernel<GradNarrow>), dim3(static_cast<unsigned>(ga.n_tiles)),
                           dim3(GradNarrow::kThreads), 0, s, ga);
      CombineArgs ca{};
      ca.acc = accbuf; ca.Y = Y; ca.alpha = alpha; ca.run = run; ca.targets = targets;
      ca.W = weight; ca.ldw = ldw; ca.vocab = vocab; ca.grad = grad_hidden; ca.n_rows = rows;
      ca.n_grad = static_cast<int>(n_grad); ca.hidden = static_cast<int>(hidden);
      ca.n_slices = ns; ca.ksplit = gp.ksplit;
      ca.first_slice = ma.first_slice; ca.last_slice = ma.last_slice;
      const int64_t work = (ca.last_slice ? n_rows : n_grad) * (hidden / 4);
      hipLaunchKernelGGL(head_combine_kernel, dim3(static_cast<unsigned>((work + kThreads - 1) / kThreads)),
                         dim3(kThreads), 0, s, ca);
    } else if (grad_hidden && s0 + ns == slices) {
      // no labelled row: the gradient is zero everywhere
      CombineArgs ca{};
      ca.grad = grad_hidden; ca.n_rows = rows; ca.n_grad = 0; ca.hidden = static_cast<int>(hidden);
      ca.last_slice = 1;
      const int64_t work = n_rows * (hidden / 4);
      hipLaunchKernelGGL(head_combine_kernel, dim3(static_cast<unsigned>((work + kThreads - 1) / kThreads)),
                         dim3(kThreads), 0, s, ca);
    }
  }
  return check_launch("head_ce");
}
