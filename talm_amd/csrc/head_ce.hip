// Vocabulary-chunked fused LM head + cross-entropy for gfx950 (fp16 MFMA, fp32 statistics).
//
// The reference (solution/fused_head.py:315-393 with fused_head_vocab_kernel, :88-182) walks the
// vocabulary in slices of `vchunk` columns: per slice, fp16 logits z = fp16(H W_c^T), the online
// per-row statistics (max m, s = sum e^{z-m}, t = sum e^{z-m} z, first argmax, z at the target),
// and for labelled rows the gradient accumulator: acc = e^{m_old - m} acc + fp16(e^{z-m}) W_c,
// with m the running maximum after slice c; at the end dH = acc / s - W[target].
//
// The same recurrence here, shaped for MI355X. Slices are processed `group` at a time:
//   head_logits   Z = H W^T over the group's columns (v_mfma_f32_32x32x16_f16, 256x128 tiles,
//                 LDS double buffer, XOR-swizzled 16-byte chunks); the epilogue rounds to fp16,
//                 stages the tile in LDS, writes it to the group's logits buffer and emits, per
//                 (row, 128-column tile), the tile's max, first argmax, sum e^{z-max} and
//                 sum e^{z-max} z.
//   head_merge    one wavefront per row folds the tiles of each slice, in column order, into the
//                 running statistics exactly as the reference's per-slice update, recording the
//                 slice's running max m_c and rescale e^{m_old - m_c}; after the last slice it
//                 writes token loss, entropy, argmax and correctness.
//   head_grad     Y_c = P_c W_c with P_c = fp16(e^{z - m_c}) formed while the logits tile is
//                 staged into LDS (never stored); one workgroup per (slice, 256-row, 128-col)
//                 tile, so the small [n_lab, H] output of each slice still fills the chip.
//   head_combine  acc = e^{m_old - m_c} acc + Y_c in slice order (the reference's rescale then
//                 add), and after the last slice dH = acc / s - W16[target] in fp16.
// The full [N, V] logits never exist: one group of slices (group * vchunk columns) at a time.
#include "common.h"

namespace talm {
namespace {

typedef _Float16 half8_t __attribute__((ext_vector_type(8)));
typedef float f32x16 __attribute__((ext_vector_type(16)));

constexpr int kThreads = 256;        // 4 wavefronts, 2 x 2 over the tile
constexpr int kBM = 256;             // tile rows (hidden-state rows)
constexpr int kBN = 128;             // tile columns
constexpr int kBK = 32;              // reduction step: two 32x32x16 MFMAs deep
constexpr int kWM = 4, kWN = 2;      // 32x32 MFMA blocks per wavefront (128 x 64)
constexpr int kTile = 128;           // statistics granule (columns) == kBN
constexpr int kZS = kBN + 8;         // LDS row stride (halfs) of the staged logits tile
constexpr int kXcds = 8;

// Row-major [rows][kBK] fp16 tile as 16-byte chunks (4 per row), XOR-swizzled so that the 8
// lanes of a ds_read_b128 phase (8 consecutive rows, one chunk column) hit 8 distinct bank groups.
__device__ __forceinline__ int swz(int row, int kc) { return row * 4 + (kc ^ ((row >> 1) & 3)); }

__device__ __forceinline__ uint32_t xcd_tile(uint32_t bid, uint32_t n_tiles) {
  // Workgroups are dispatched round-robin over the 8 XCDs; give each XCD a contiguous range of
  // tiles (tiles that share weight columns share that XCD's L2).
  if (n_tiles % kXcds) return bid;
  return (bid % kXcds) * (n_tiles / kXcds) + bid / kXcds;
}

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
// GEMM1: Z[r][j] = fp16(sum_k H[r][k] W[col0 + j][k]) for the group's columns j < group_cols,
// plus the per-(row, 128-column tile) partial statistics.
// ------------------------------------------------------------------------------------------
__global__ __launch_bounds__(kThreads, 2) void head_logits_kernel(
    const uint16_t* __restrict__ H, int64_t ldh, const uint16_t* __restrict__ W, int64_t ldw,
    int n_rows, int K, int group_cols, int first_col, uint16_t* __restrict__ Z, int64_t ldz,
    float4* __restrict__ part, int parts_per_row, int n_mtiles, int n_ntiles,
    const int64_t* __restrict__ targets, float* __restrict__ ztarget) {
  constexpr int kLdsMain = 2 * (kBM + kBN) * kBK * 2;   // double-buffered A and B tiles
  constexpr int kLdsEpi = kBM * kZS * 2;                 // staged logits tile
  constexpr int kLds = kLdsMain > kLdsEpi ? kLdsMain : kLdsEpi;
  __shared__ __attribute__((aligned(16))) unsigned char smem[kLds];
  uint4* As = reinterpret_cast<uint4*>(smem);            // [2][kBM * 4] chunks
  uint4* Bs = As + 2 * kBM * 4;                          // [2][kBN * 4] chunks

  const uint32_t tile = xcd_tile(blockIdx.x, static_cast<uint32_t>(n_mtiles * n_ntiles));
  const int ntile = static_cast<int>(tile / n_mtiles);
  const int mtile = static_cast<int>(tile % n_mtiles);
  const int m0 = mtile * kBM, n0 = ntile * kBN;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int wm = wave >> 1, wn = wave & 1;

  // Global -> register staging: A 256 rows x 4 chunks (4 per thread), B 128 x 4 (2 per thread).
  uint4 ra[4], rb[2];
  auto load = [&](int k0) {
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const int c = tid + kThreads * r, row = c >> 2, kc = c & 3;
      const int gr = m0 + row, gk = k0 + kc * 8;
      ra[r] = (gr < n_rows && gk < K)
                  ? *reinterpret_cast<const uint4*>(H + static_cast<int64_t>(gr) * ldh + gk)
                  : make_uint4(0, 0, 0, 0);
    }
#pragma unroll
    for (int r = 0; r < 2; ++r) {
      const int c = tid + kThreads * r, row = c >> 2, kc = c & 3;
      const int gc = n0 + row, gk = k0 + kc * 8;
      rb[r] = (gc < group_cols && gk < K)
                  ? *reinterpret_cast<const uint4*>(W + static_cast<int64_t>(gc) * ldw + gk)
                  : make_uint4(0, 0, 0, 0);
    }
  };
  auto store = [&](int buf) {
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const int c = tid + kThreads * r;
      As[buf * kBM * 4 + swz(c >> 2, c & 3)] = ra[r];
    }
#pragma unroll
    for (int r = 0; r < 2; ++r) {
      const int c = tid + kThreads * r;
      Bs[buf * kBN * 4 + swz(c >> 2, c & 3)] = rb[r];
    }
  };

  f32x16 acc[kWM][kWN];
#pragma unroll
  for (int i = 0; i < kWM; ++i)
#pragma unroll
    for (int j = 0; j < kWN; ++j)
#pragma unroll
      for (int v = 0; v < 16; ++v) acc[i][j][v] = 0.f;

  const int nk = (K + kBK - 1) / kBK;
  load(0);
  store(0);
  __syncthreads();
  for (int kt = 0; kt < nk; ++kt) {
    const int buf = kt & 1;
    if (kt + 1 < nk) load((kt + 1) * kBK);
#pragma unroll
    for (int ks = 0; ks < 2; ++ks) {
      const int kc = ks * 2 + (lane >> 5);
      half8_t a[kWM], b[kWN];
#pragma unroll
      for (int i = 0; i < kWM; ++i) {
        const uint4 v = As[buf * kBM * 4 + swz(wm * 128 + i * 32 + (lane & 31), kc)];
        a[i] = __builtin_bit_cast(half8_t, v);
      }
#pragma unroll
      for (int j = 0; j < kWN; ++j) {
        const uint4 v = Bs[buf * kBN * 4 + swz(wn * 64 + j * 32 + (lane & 31), kc)];
        b[j] = __builtin_bit_cast(half8_t, v);
      }
#pragma unroll
      for (int i = 0; i < kWM; ++i)
#pragma unroll
        for (int j = 0; j < kWN; ++j)
          acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_f16(a[i], b[j], acc[i][j], 0, 0, 0);
    }
    if (kt + 1 < nk) store(buf ^ 1);
    __syncthreads();
  }

  // Epilogue 1: fp16 logits tile into LDS ([kBM][kZS] halfs).
  uint16_t* Zs = reinterpret_cast<uint16_t*>(smem);
#pragma unroll
  for (int i = 0; i < kWM; ++i)
#pragma unroll
    for (int j = 0; j < kWN; ++j)
#pragma unroll
      for (int v = 0; v < 16; ++v) {
        const int row = wm * 128 + i * 32 + 8 * (v >> 2) + 4 * (lane >> 5) + (v & 3);
        const int col = wn * 64 + j * 32 + (lane & 31);
        Zs[row * kZS + col] = f2h(acc[i][j][v]);
      }
  __syncthreads();

  // Epilogue 2: partial statistics of row `tid` over this tile's valid columns.
  {
    const int row = tid, gr = m0 + row;
    const int valid = min(kBN, group_cols - n0);
    if (gr < n_rows) {
      uint4 zv[kBN / 8];
#pragma unroll
      for (int c = 0; c < kBN / 8; ++c) zv[c] = *reinterpret_cast<const uint4*>(Zs + row * kZS + 8 * c);
      float m = -INFINITY;
      int idx = 0;
#pragma unroll
      for (int c = 0; c < kBN / 8; ++c) {
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
      float s = 0.f, t = 0.f;
#pragma unroll
      for (int c = 0; c < kBN / 8; ++c) {
        const uint32_t w4[4] = {zv[c].x, zv[c].y, zv[c].z, zv[c].w};
#pragma unroll
        for (int e = 0; e < 8; ++e) {
          const int col = 8 * c + e;
          const float z = (e & 1) ? hi_f(w4[e >> 1]) : lo_f(w4[e >> 1]);
          if (col < valid) {
            const float ez = __expf(z - m);
            s += ez;
            t += ez * z;
          }
        }
      }
      part[static_cast<int64_t>(gr) * parts_per_row + ntile] =
          make_float4(m, s, t, __int_as_float(first_col + n0 + idx));
      // the logit at the target, when the target column is in this tile (one tile per row)
      const int64_t rel = targets[gr] - (first_col + n0);
      if (rel >= 0 && rel < valid) ztarget[gr] = h2f(Zs[row * kZS + static_cast<int>(rel)]);
    }
  }

  // Epilogue 3: the logits tile to global memory in 16-byte chunks (16 per row).
#pragma unroll
  for (int it = 0; it < (kBM * kBN / 8) / kThreads; ++it) {
    const int c = it * kThreads + tid, row = c >> 4, kc = c & 15;
    const int gr = m0 + row, gc = n0 + kc * 8;
    if (gr < n_rows && gc < group_cols)
      *reinterpret_cast<uint4*>(Z + static_cast<int64_t>(gr) * ldz + gc) =
          *reinterpret_cast<const uint4*>(Zs + row * kZS + kc * 8);
  }
}

// ------------------------------------------------------------------------------------------
// Running statistics, one wavefront per row, over the slices of one group.
// ------------------------------------------------------------------------------------------
struct MergeArgs {
  const float4* part;
  int parts_per_row;
  uint16_t* Z;             // the group's logits; rows < n_grad become P = fp16(e^{z - m_c})
  int64_t ldz;
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
      // the slice's logits of a labelled row become fp16(e^{z - m_c}) in place
      // (solution/fused_head.py:178-182), the A operand of head_grad
      uint16_t* zrow = a.Z + static_cast<int64_t>(row) * a.ldz + (a.slice_col0[c] - a.slice_col0[0]);
      for (int e0 = lane * 8; e0 < a.slice_cols[c]; e0 += kWave * 8) {
        uint4 v = *reinterpret_cast<const uint4*>(zrow + e0);
        uint32_t w[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
        for (int q = 0; q < 4; ++q) w[q] = pack2(__expf(lo_f(w[q]) - m), __expf(hi_f(w[q]) - m));
        *reinterpret_cast<uint4*>(zrow + e0) = make_uint4(w[0], w[1], w[2], w[3]);
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
// GEMM2: Y_c[r][h] = sum_j fp16(e^{Z[r][j] - m_c[r]}) W[col0_c + j][h] over slice c's columns,
// for the first n_grad rows (the labelled rows, put first by the caller).
// ------------------------------------------------------------------------------------------
struct GradArgs {
  const uint16_t* Z;
  int64_t ldz;
  const uint16_t* W;      // weight row of the group's first vocabulary column
  int64_t ldw;
  int n_rows;
  int n_grad;
  int hidden;
  int vchunk;
  int slice_cols[8];
  float* Y;               // [n_slices][n_grad][hidden] fp32
  int n_mtiles, n_ntiles;
};

__global__ __launch_bounds__(kThreads, 2) void head_grad_kernel(GradArgs a) {
  constexpr int kLdsA = 2 * kBM * kBK * 2;   // P tiles, swizzled chunks
  constexpr int kLdsB = 2 * kBN * kBK * 2;   // weight tiles transposed to [n][k], swizzled chunks
  __shared__ __attribute__((aligned(16))) unsigned char smem[kLdsA + kLdsB];
  uint4* As = reinterpret_cast<uint4*>(smem);
  uint4* Bs = reinterpret_cast<uint4*>(smem + kLdsA);

  const uint32_t per_slice = static_cast<uint32_t>(a.n_mtiles * a.n_ntiles);
  const int slice = static_cast<int>(blockIdx.x / per_slice);
  const uint32_t tile = xcd_tile(blockIdx.x % per_slice, per_slice);
  const int ntile = static_cast<int>(tile / a.n_mtiles);
  const int mtile = static_cast<int>(tile % a.n_mtiles);
  const int m0 = mtile * kBM, n0 = ntile * kBN;
  const int cols = a.slice_cols[slice];
  const int zcol0 = slice * a.vchunk;  // slice's first column inside the group's logits
  const uint16_t* Wc = a.W + static_cast<int64_t>(zcol0) * a.ldw;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int wm = wave >> 1, wn = wave & 1;
  // B staging: thread = (k pair kp, 8-column group ng): rows k, k+1 of 8 weight columns
  const int kp = tid & 15, ng = tid >> 4;

  uint4 ra[4], rb[2];
  auto load = [&](int k0) {
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const int c = tid + kThreads * r, row = c >> 2, kc = c & 3;
      const int gr = m0 + row, gk = k0 + kc * 8;
      uint4 v = make_uint4(0, 0, 0, 0);
      if (gr < a.n_grad && gk < cols) {
        v = *reinterpret_cast<const uint4*>(a.Z + static_cast<int64_t>(gr) * a.ldz + zcol0 + gk);
        if (gk + 8 > cols) {  // the last slice's tail: columns past `cols` hold no P
          uint32_t w[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
          for (int e = 0; e < 4; ++e) {
            if (gk + 2 * e >= cols) w[e] = 0u;
            else if (gk + 2 * e + 1 >= cols) w[e] &= 0xffffu;
          }
          v = make_uint4(w[0], w[1], w[2], w[3]);
        }
      }
      ra[r] = v;
    }
#pragma unroll
    for (int r = 0; r < 2; ++r) {
      const int gk = k0 + 2 * kp + r, gn = n0 + 8 * ng;
      rb[r] = (gk < cols && gn < a.hidden)
                  ? *reinterpret_cast<const uint4*>(Wc + static_cast<int64_t>(gk) * a.ldw + gn)
                  : make_uint4(0, 0, 0, 0);
    }
  };
  auto store = [&](int buf) {
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const int c = tid + kThreads * r;
      As[buf * kBM * 4 + swz(c >> 2, c & 3)] = ra[r];
    }
    // transpose 2 (k) x 8 (n) into 8 rows of [n][k]: one 32-bit (k, k+1) pair per row
    uint32_t* Bw = reinterpret_cast<uint32_t*>(Bs + buf * kBN * 4);
    const uint32_t lo[4] = {rb[0].x, rb[0].y, rb[0].z, rb[0].w};
    const uint32_t hi[4] = {rb[1].x, rb[1].y, rb[1].z, rb[1].w};
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      const uint32_t even = (lo[q] & 0xffffu) | (hi[q] << 16);
      const uint32_t odd = (lo[q] >> 16) | (hi[q] & 0xffff0000u);
      Bw[swz(8 * ng + 2 * q, kp >> 2) * 4 + (kp & 3)] = even;
      Bw[swz(8 * ng + 2 * q + 1, kp >> 2) * 4 + (kp & 3)] = odd;
    }
  };

  f32x16 acc[kWM][kWN];
#pragma unroll
  for (int i = 0; i < kWM; ++i)
#pragma unroll
    for (int j = 0; j < kWN; ++j)
#pragma unroll
      for (int v = 0; v < 16; ++v) acc[i][j][v] = 0.f;

  const int nk = (cols + kBK - 1) / kBK;
  load(0);
  store(0);
  __syncthreads();
  for (int kt = 0; kt < nk; ++kt) {
    const int buf = kt & 1;
    if (kt + 1 < nk) load((kt + 1) * kBK);
#pragma unroll
    for (int ks = 0; ks < 2; ++ks) {
      const int kc = ks * 2 + (lane >> 5);
      half8_t av[kWM], bv[kWN];
#pragma unroll
      for (int i = 0; i < kWM; ++i) {
        const uint4 v = As[buf * kBM * 4 + swz(wm * 128 + i * 32 + (lane & 31), kc)];
        av[i] = __builtin_bit_cast(half8_t, v);
      }
#pragma unroll
      for (int j = 0; j < kWN; ++j) {
        const uint4 v = Bs[buf * kBN * 4 + swz(wn * 64 + j * 32 + (lane & 31), kc)];
        bv[j] = __builtin_bit_cast(half8_t, v);
      }
#pragma unroll
      for (int i = 0; i < kWM; ++i)
#pragma unroll
        for (int j = 0; j < kWN; ++j)
          acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_f16(av[i], bv[j], acc[i][j], 0, 0, 0);
    }
    if (kt + 1 < nk) store(buf ^ 1);
    __syncthreads();
  }

  float* Y = a.Y + static_cast<int64_t>(slice) * a.n_grad * a.hidden;
#pragma unroll
  for (int i = 0; i < kWM; ++i)
#pragma unroll
    for (int j = 0; j < kWN; ++j)
#pragma unroll
      for (int v = 0; v < 16; ++v) {
        const int gr = m0 + wm * 128 + i * 32 + 8 * (v >> 2) + 4 * (lane >> 5) + (v & 3);
        const int gc = n0 + wn * 64 + j * 32 + (lane & 31);
        if (gr < a.n_grad && gc < a.hidden) Y[static_cast<int64_t>(gr) * a.hidden + gc] = acc[i][j][v];
      }
}

// ------------------------------------------------------------------------------------------
// acc = e^{m_old - m_c} acc + Y_c in slice order; after the last slice dH = acc / s - W[target].
// One thread per 4 hidden columns of one row.
// ------------------------------------------------------------------------------------------
struct CombineArgs {
  float* acc;              // [n_grad][hidden]
  const float* Y;          // [n_slices][n_grad][hidden]
  const float* alpha;      // [n_slices][n_rows]
  const float* run;        // running statistics (s at [n_rows + row])
  const int64_t* targets;
  const uint16_t* W;       // full weight (row = vocabulary column)
  int64_t ldw;
  int64_t vocab;
  uint16_t* grad;          // [n_rows][hidden] fp16 (written after the last slice)
  int n_rows, n_grad, hidden, n_slices, first_slice, last_slice;
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
    const float4 y = *reinterpret_cast<const float4*>(a.Y + static_cast<int64_t>(c) * a.n_grad * a.hidden + at);
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
  // rows [0, n_grad) are labelled by contract; a target outside [0, vocab) (a broken contract)
  // must not make the kernel read outside the weight: its W[target] term is left out
  uint2 wv = make_uint2(0u, 0u);
  if (tgt >= 0 && tgt < a.vocab) wv = *reinterpret_cast<const uint2*>(a.W + tgt * a.ldw + col);
  const float g0 = v.x / s - lo_f(wv.x), g1 = v.y / s - hi_f(wv.x);
  const float g2 = v.z / s - lo_f(wv.y), g3 = v.w / s - hi_f(wv.y);
  *reinterpret_cast<uint2*>(a.grad + at) = make_uint2(pack2(g0, g1), pack2(g2, g3));
}

size_t align_up(size_t v, size_t a) { return (v + a - 1) / a * a; }

struct Layout {
  size_t z, part, run, ztarget, alpha, y, acc, total;
  int64_t ldz;
  int parts_per_row;
};

Layout layout(int64_t n_rows, int64_t hidden, int64_t vchunk, int64_t n_grad, int group) {
  Layout l{};
  l.ldz = align_up(static_cast<size_t>(group * vchunk), 8);
  l.parts_per_row = static_cast<int>(group * vchunk / kTile);
  size_t off = 0;
  l.z = off;      off = align_up(off + static_cast<size_t>(n_rows) * l.ldz * 2, 256);
  l.part = off;   off = align_up(off + static_cast<size_t>(n_rows) * l.parts_per_row * 16, 256);
  l.run = off;    off = align_up(off + static_cast<size_t>(n_rows) * 6 * 4, 256);
  l.ztarget = off; off = align_up(off + static_cast<size_t>(n_rows) * 4, 256);
  l.alpha = off;  off = align_up(off + static_cast<size_t>(group) * n_rows * 4, 256);
  l.y = off;      off = align_up(off + static_cast<size_t>(group) * n_grad * hidden * 4, 256);
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
  return static_cast<int64_t>(layout(n_rows, hidden, vchunk, n_grad, g).total);
}

TALM_API int talm_head_ce(const uint16_t* hidden_states, int64_t ldh, const uint16_t* weight,
                          int64_t ldw, const int64_t* targets, int64_t n_rows, int64_t hidden,
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
  if (n_rows > (1 << 30) || vocab > (1 << 30) || hidden > (1 << 20))
    return fail(TALM_EINVAL, "head_ce: sizes beyond 32-bit indexing");
  if (n_rows == 0) return ok();
  if (!hidden_states || !weight || !targets || !token_loss || !entropy || !best_idx || !correct ||
      !workspace || (n_grad > 0 && !grad_hidden))
    return fail(TALM_EINVAL, "head_ce: null pointer");
  if (!aligned(hidden_states, 16) || !aligned(weight, 16) || !aligned(workspace, 256) ||
      (grad_hidden && !aligned(grad_hidden, 16)))
    return fail(TALM_EINVAL, "head_ce: hidden states, weight and dH must be 16-byte aligned, the "
                             "workspace 256-byte aligned");
  const int64_t slices = (vocab + vchunk - 1) / vchunk;
  const int g = static_cast<int>(slices < group ? slices : group);
  const Layout l = layout(n_rows, hidden, vchunk, n_grad, g);
  if (workspace_bytes < static_cast<int64_t>(l.total))
    return fail(TALM_EINVAL, "head_ce: workspace of %lld bytes, %zu needed",
                (long long)workspace_bytes, l.total);
  unsigned char* ws = static_cast<unsigned char*>(workspace);
  uint16_t* Z = reinterpret_cast<uint16_t*>(ws + l.z);
  float4* part = reinterpret_cast<float4*>(ws + l.part);
  float* run = reinterpret_cast<float*>(ws + l.run);
  float* ztarget = reinterpret_cast<float*>(ws + l.ztarget);
  float* alpha = reinterpret_cast<float*>(ws + l.alpha);
  float* Y = reinterpret_cast<float*>(ws + l.y);
  float* accbuf = reinterpret_cast<float*>(ws + l.acc);
  const hipStream_t s = as_stream(stream);
  const int rows = static_cast<int>(n_rows);
  const int mt = (rows + kBM - 1) / kBM;

  for (int64_t s0 = 0; s0 < slices; s0 += g) {
    const int ns = static_cast<int>(slices - s0 < g ? slices - s0 : g);
    const int64_t col0 = s0 * vchunk;
    const int64_t gcols = (s0 + ns == slices) ? vocab - col0 : ns * vchunk;
    const int nt = static_cast<int>((gcols + kBN - 1) / kBN);
    hipLaunchKernelGGL(head_logits_kernel, dim3(static_cast<unsigned>(mt * nt)), dim3(kThreads), 0, s,
                       hidden_states, ldh, weight + col0 * ldw, ldw, rows, static_cast<int>(hidden),
                       static_cast<int>(gcols), static_cast<int>(col0), Z, l.ldz, part,
                       l.parts_per_row, mt, nt, targets, ztarget);
    MergeArgs ma{};
    ma.part = part; ma.parts_per_row = l.parts_per_row; ma.Z = Z; ma.ldz = l.ldz;
    ma.targets = targets; ma.ztarget = ztarget; ma.n_rows = rows;
    ma.n_grad = grad_hidden ? static_cast<int>(n_grad) : 0;
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
      ga.Z = Z; ga.ldz = l.ldz; ga.W = weight + col0 * ldw; ga.ldw = ldw;
      ga.n_rows = rows; ga.n_grad = static_cast<int>(n_grad); ga.hidden = static_cast<int>(hidden);
      ga.vchunk = static_cast<int>(vchunk);
      for (int c = 0; c < ns; ++c) ga.slice_cols[c] = ma.slice_cols[c];
      ga.Y = Y;
      ga.n_mtiles = static_cast<int>((n_grad + kBM - 1) / kBM);
      ga.n_ntiles = static_cast<int>((hidden + kBN - 1) / kBN);
      hipLaunchKernelGGL(head_grad_kernel, dim3(static_cast<unsigned>(ga.n_mtiles * ga.n_ntiles * ns)),
                         dim3(kThreads), 0, s, ga);
      CombineArgs ca{};
      ca.acc = accbuf; ca.Y = Y; ca.alpha = alpha; ca.run = run; ca.targets = targets;
      ca.W = weight; ca.ldw = ldw; ca.vocab = vocab; ca.grad = grad_hidden; ca.n_rows = rows;
      ca.n_grad = static_cast<int>(n_grad); ca.hidden = static_cast<int>(hidden);
      ca.n_slices = ns; ca.first_slice = ma.first_slice; ca.last_slice = ma.last_slice;
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
