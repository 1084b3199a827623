// The fp16 MFMA tile core shared by the head (head_ce.hip) and the q|k|v projection (qkv.hip):
// C[BM x BN] = A B^T with both operands k-contiguous, on gfx950.
//
// Operands stream from global memory straight into an LDS ring with buffer_load_dwordx4 ... lds
// (no register staging: lane l of a 1 KiB wavefront block fills the block's l-th 16-byte chunk).
// Chunks are XOR-swizzled so that the ds_read_b128 fragment reads of v_mfma_f32_32x32x16_f16 are
// free of bank conflicts. Out-of-range rows / k-chunks get a buffer offset past the descriptor's
// range and read as zeros, so tails need no branches. One barrier per step; the ring keeps
// STAGES - 1 steps in flight. Every wavefront owns (BM / WM) x (BN / WN) of the tile.
#pragma once

#include "common.h"

#include <type_traits>

namespace talm {
namespace {

typedef _Float16 half8_t __attribute__((ext_vector_type(8)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef __attribute__((address_space(3))) void* lds_ptr_t;
typedef short s16x4 __attribute__((ext_vector_type(4)));
typedef __attribute__((address_space(3))) s16x4* lds_s16x4_ptr;

constexpr int kXcds = 8;
constexpr uint32_t kOob = 0x80000000u;  // buffer offset past every range: the load returns 0

// A BM x BN output tile in BK-deep steps through a STAGES-slot LDS ring, WM x WN wavefronts.
// `kPerCu` workgroups share a CU so that two wavefronts run per SIMD.
template <int BM, int BN, int BK, int STAGES, int WM, int WN>
struct TileShape {
  static constexpr int kBM = BM, kBN = BN, kBK = BK, kStages = STAGES;
  static constexpr int kWaves = WM * WN, kWavesN = WN;
  static constexpr int kThreads = 64 * kWaves;
  static constexpr int kWaveM = BM / WM, kWaveN = BN / WN;  // the wavefront's share of the tile
  static constexpr int kFragM = kWaveM / 32, kFragN = kWaveN / 32;  // 32x32 MFMA blocks
  static constexpr int kCpr = BK / 8;                         // 16-byte chunks per row of a stage
  static constexpr int kAChunks = BM * kCpr, kBChunks = BN * kCpr;
  static constexpr int kStageBytes = (kAChunks + kBChunks) * 16;
  static constexpr int kRing = STAGES * kStageBytes;
  static constexpr int kPerCu = 512 / kThreads;
  static_assert(STAGES >= 2 && STAGES <= 4, "ring depth");
  static_assert(kWaveM % 32 == 0 && kWaveN % 32 == 0, "32x32 MFMA blocks");
  static_assert(BK == 32 || BK == 64, "swizzle keys exist for 4 and 8 chunks per row");
  static_assert(kRing <= 160 * 1024, "LDS per CU");
};

// [rows][BK] fp16 stage as 16-byte chunks, CPR per row. The chunk column is XOR-ed with a key of
// the row so that the rows read by one ds_read_b128 phase (8 consecutive rows on 32 banks, 16 on
// 64 banks, one chunk column) land on distinct banks: ((row >> 1) ^ (row >> 2)) & 3 for 64-byte
// rows, (row ^ (row >> 3)) & 7 for 128-byte rows.
template <int CPR>
__device__ __forceinline__ int swz_key(int row) {
  if constexpr (CPR == 4) return ((row >> 1) ^ (row >> 2)) & 3;
  else return (row ^ (row >> 3)) & 7;
}
template <int CPR>
__device__ __forceinline__ int swz(int row, int kc) { return row * CPR + (kc ^ swz_key<CPR>(row)); }

// Wait until at most N vector-memory operations of this wavefront are outstanding (vmcnt only).
template <int N>
__device__ __forceinline__ void wait_vmcnt() {
  static_assert(N >= 0 && N < 64, "vmcnt range");
  __builtin_amdgcn_s_waitcnt((N & 15) | (7 << 4) | (15 << 8) | ((N >> 4) << 14));
}

// Workgroup barrier that orders LDS accesses only: the LDS reads issued before it have returned
// (lgkmcnt 0), and the compiler moves no memory access across it. Unlike __syncthreads() it does
// not drain the wavefront's outstanding buffer ... lds transfers, which the ring keeps in flight
// and waits for with wait_vmcnt.
__device__ __forceinline__ void lds_barrier() {
  asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
}

// Workgroups are dispatched round-robin over the 8 XCDs (workgroup b runs on XCD b % 8). Give
// each XCD one contiguous range of tile indices (a bijection for any tile count), so tiles that
// are neighbours in the caller's order share that XCD's L2.
__device__ __forceinline__ uint32_t xcd_tile(uint32_t bid, uint32_t n_tiles) {
  const uint32_t x = bid % kXcds, i = bid / kXcds;
  const uint32_t q = n_tiles / kXcds, r = n_tiles % kXcds;
  return x * q + min(x, r) + i;
}

__device__ __forceinline__ __amdgpu_buffer_rsrc_t buffer_rsrc(const uint16_t* base) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<uint16_t*>(base), 0, 0x7fffffff, 0x00020000);
}

__device__ __forceinline__ void dma16(__amdgpu_buffer_rsrc_t rsrc, unsigned char* dst, uint32_t off) {
  __builtin_amdgcn_raw_ptr_buffer_load_lds(rsrc, (lds_ptr_t)dst, 16, off, 0, 0, 0);
}

// One operand of the tile: kRows rows of fp16 with k contiguous, from `base` (the tile's first
// row, k = 0) with row stride `ld` halfs (row * ld * 2 below 2^31). Each step every wavefront
// moves its 1 KiB blocks of the stage: lane l loads the global chunk that the swizzle puts at
// the block's l-th chunk. Chunks of rows past `rows_valid`, or starting outside
// [k_lo, k_valid), get an out-of-range offset and read as zeros (only in-window chunks are read,
// so `base` may point before the operand when k_lo > 0).
template <class S, int kRows>
struct Loader {
  static constexpr int kPer = kRows * S::kCpr / S::kThreads;  // DMA instructions per step
  static constexpr int kRowsPerBlock = 64 / S::kCpr;
  static_assert(kPer * S::kThreads == kRows * S::kCpr, "whole 1 KiB blocks per wavefront");
  __amdgpu_buffer_rsrc_t rsrc;
  uint32_t off[kPer];
  int kc8[kPer];
  int k_lo, k_valid;

  __device__ __forceinline__ void init(const uint16_t* base, int64_t ld, int rows_valid,
                                       int k_valid_, int wave, int lane, int k_lo_ = 0) {
    rsrc = buffer_rsrc(base);
    k_lo = k_lo_;
    k_valid = k_valid_;
#pragma unroll
    for (int p = 0; p < kPer; ++p) {
      const int row = kRowsPerBlock * (p * S::kWaves + wave) + lane / S::kCpr;
      const int kc = (lane % S::kCpr) ^ swz_key<S::kCpr>(row);
      kc8[p] = kc * 8;
      off[p] = row < rows_valid ? static_cast<uint32_t>((row * ld + kc * 8) * 2) : kOob;
    }
  }
  // The same operand with rows past `rows_valid` cut off by the descriptor's range instead of by
  // per-lane offsets: `lanes` sets the offsets, which depend on the lane only (all rows read), once;
  // `rows` points the descriptor at a tile (scalar registers only), so a kernel that walks tiles
  // keeps one set of offsets. rows_valid * ld * 2 must stay below 2^32.
  __device__ __forceinline__ void lanes(int64_t ld, int k_valid_, int wave, int lane) {
    k_lo = 0;
    k_valid = k_valid_;
#pragma unroll
    for (int p = 0; p < kPer; ++p) {
      const int row = kRowsPerBlock * (p * S::kWaves + wave) + lane / S::kCpr;
      const int kc = (lane % S::kCpr) ^ swz_key<S::kCpr>(row);
      kc8[p] = kc * 8;
      off[p] = static_cast<uint32_t>((row * ld + kc * 8) * 2);
    }
  }
  __device__ __forceinline__ void rows(const uint16_t* base, int64_t ld, int rows_valid) {
    rsrc = __builtin_amdgcn_make_buffer_rsrc(const_cast<uint16_t*>(base), 0,
                                             static_cast<int>(rows_valid * ld * 2), 0x00020000);
  }
  // operands of step k0 into the stage block at `dst`
  __device__ __forceinline__ void issue(unsigned char* dst, int k0, int wave) {
#pragma unroll
    for (int p = 0; p < kPer; ++p) {
      const int k = k0 + kc8[p];
      const uint32_t v = k >= k_lo && k < k_valid ? off[p] + static_cast<uint32_t>(k0 * 2) : kOob;
      dma16(rsrc, dst + (p * S::kWaves + wave) * 1024, v);
    }
  }
};

// An "nn" B stage: [BK k rows][256 n columns] fp16 (the operand's rows as they lie in memory, n
// contiguous), 32 chunks of 16 bytes per row, chunk c of row r at position
// c ^ (4 (r & 3) + (c / 16 + 2 (r & 1)) % 4) (an XOR of the low four bits, so a bijection on each
// row that keeps bit 4). gfx950's LDS serves 16 lanes of a 16-byte access, or 32 of an 8-byte
// one, per phase over 64 four-byte banks: 16 chunk positions mod 16. 16-byte stores of two rows
// (chunks 4 cc + j of cc = 0..7 per phase) and the transposing 8-byte fragment reads (4
// consecutive rows x 4 adjacent chunks per phase) both meet 16 distinct positions mod 16.
__device__ __forceinline__ int nn_key(int row, int chunk) {
  return (((chunk >> 4) + 2 * (row & 1)) & 3) | ((row & 3) << 2);
}
__device__ __forceinline__ int nn_pos(int row, int chunk) { return row * 32 + (chunk ^ nn_key(row, chunk)); }

// The B operand of v_mfma_f32_32x32x16_f16 for the 32 columns [col0, col0 + 32) and k-slice ks of
// an nn stage, read with the transposing ds_read_b64_tr_b16: lane (g = lane / 16, i = lane % 16)
// points at row 16 ks + 8 (g / 2) + i / 4 (and 4 rows on), columns col .. col + 3 with col =
// col0 + 16 (g % 2) + 4 (i % 4), and receives k-slots 8 (g / 2) + 0..3 (+ 4..7) of column
// col0 + lane % 32.
__device__ __forceinline__ half8_t nn_b_fragment(const unsigned char* Bs, int ks, int col0, int lane) {
  const int g = lane >> 4, i = lane & 15;
  const int row = ks * 16 + 8 * (g >> 1) + (i >> 2);
  const int col = col0 + 16 * (g & 1) + 4 * (i & 3);
  const unsigned char* p0 = Bs + nn_pos(row, col >> 3) * 16 + (col & 7) * 2;
  const unsigned char* p1 = Bs + nn_pos(row + 4, col >> 3) * 16 + (col & 7) * 2;
  const s16x4 lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s16x4_ptr)(p0));
  const s16x4 hi = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s16x4_ptr)(p1));
  return __builtin_bit_cast(half8_t, __builtin_shufflevector(lo, hi, 0, 1, 2, 3, 4, 5, 6, 7));
}

// An nn operand streamed into nn stages: rows [kt BK, kt BK + BK) of the matrix at `base` (row
// stride `ld` halfs, n contiguous), its 256 columns from `base` on. A wavefront's 1 KiB DMA block
// b covers stage positions [64 b, 64 b + 64), i.e. rows 2 b and 2 b + 1, so lane l loads the
// global chunk that the swizzle puts at position l % 32 of row 2 b + l / 32. Rows at or past
// `rows_valid` and chunks at or past `cols_valid` columns read as zeros (out-of-range offsets),
// so the operand may end inside a step. rows_valid * ld * 2 stays below 2^31.
template <class S>
struct LoaderNN {
  static_assert(S::kBN == 256, "32 chunks per stage row");
  static constexpr int kPer = S::kBK * 32 / S::kThreads;  // DMA instructions per step
  static_assert(kPer * S::kThreads == S::kBK * 32, "whole 1 KiB blocks per wavefront");
  __amdgpu_buffer_rsrc_t rsrc;
  uint32_t off[kPer];
  int row[kPer];
  int rows_valid;
  uint32_t step_bytes;
  __device__ __forceinline__ void init(const uint16_t* base, int64_t ld, int rows_valid_,
                                       int cols_valid, int wave, int lane) {
    rsrc = buffer_rsrc(base);
    rows_valid = rows_valid_;
    step_bytes = static_cast<uint32_t>(S::kBK * ld * 2);
#pragma unroll
    for (int p = 0; p < kPer; ++p) {
      const int r = 2 * (p * S::kWaves + wave) + lane / 32, pos = lane % 32;
      const int c = pos ^ nn_key(r, pos);
      row[p] = r;
      off[p] = c * 8 < cols_valid ? static_cast<uint32_t>((r * ld + c * 8) * 2) : kOob;
    }
  }
  __device__ __forceinline__ void issue(unsigned char* dst, int kt, int wave) {
#pragma unroll
    for (int p = 0; p < kPer; ++p) {
      const uint32_t v = kt * S::kBK + row[p] < rows_valid && off[p] != kOob
                             ? off[p] + static_cast<uint32_t>(kt) * step_bytes : kOob;
      dma16(rsrc, dst + (p * S::kWaves + wave) * 1024, v);
    }
  }
};

template <class S>
using Acc = f32x16[S::kFragM][S::kFragN];

// DMA instructions per thread and step of the B operand, k-contiguous or nn stages.
template <class S, bool kBnn>
constexpr int b_dma_per_step() {
  if constexpr (kBnn) return LoaderNN<S>::kPer;
  else return Loader<S, S::kBN>::kPer;
}

// A per-step hook of the ring. The default does nothing; a hook loads step kt's own operands
// (kLoads vector-memory operations per thread) into its register set `slot` (the step's ring
// slot) in prefetch(kt, slot), issued right before step kt's DMA group so that the wait for that
// group covers them too. apply(a, i, slot) may scale fragment i of the wavefront's A fragments
// between their LDS read and the MFMAs; after(stage, slot, kt) runs once the step's MFMAs are
// issued, with the step's stage still in LDS (more MFMAs on the same A block). The ring is
// unrolled by its depth, so `slot` is a compile-time index and no register is copied (a copy of a
// loaded register would wait for its load).
struct NoScale {
  static constexpr int kLoads = 0;
  __device__ __forceinline__ void prefetch(int, int) {}
  __device__ __forceinline__ half8_t apply(half8_t a, int, int) const { return a; }
  __device__ __forceinline__ void after(const unsigned char*, int, int) {}
};

// One step of the wavefront's block: BK / 16 x (kFragM A + kFragN B fragments, their MFMAs).
template <class S, class Scale = NoScale, bool kBnn = false>
__device__ __forceinline__ void mma_step(const uint4* __restrict__ As, const uint4* __restrict__ Bs,
                                         Acc<S>& acc, int lane, int wm, int wn,
                                         const Scale& scale = Scale(), int slot = 0) {
  constexpr int kSteps = S::kBK / 16;
  half8_t a[kSteps][S::kFragM], b[kSteps][S::kFragN];
#pragma unroll
  for (int ks = 0; ks < kSteps; ++ks) {
    const int kc = ks * 2 + (lane >> 5);
#pragma unroll
    for (int i = 0; i < S::kFragM; ++i)
      a[ks][i] = scale.apply(__builtin_bit_cast(
          half8_t, As[swz<S::kCpr>(wm * S::kWaveM + i * 32 + (lane & 31), kc)]), i, slot);
#pragma unroll
    for (int j = 0; j < S::kFragN; ++j) {
      if constexpr (kBnn)
        b[ks][j] = nn_b_fragment(reinterpret_cast<const unsigned char*>(Bs), ks, wn * S::kWaveN + j * 32, lane);
      else
        b[ks][j] = __builtin_bit_cast(
            half8_t, Bs[swz<S::kCpr>(wn * S::kWaveN + j * 32 + (lane & 31), kc)]);
    }
  }
#pragma unroll
  for (int ks = 0; ks < kSteps; ++ks)
#pragma unroll
    for (int i = 0; i < S::kFragM; ++i)
#pragma unroll
      for (int j = 0; j < S::kFragN; ++j)
        acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_f16(a[ks][i], b[ks][j], acc[i][j], 0, 0, 0);
}

// Wait until at most `later` whole groups of N operations are in flight (later <= 2).
template <int N>
__device__ __forceinline__ void wait_groups(int later) {
  if (later >= 2) wait_vmcnt<2 * N>();
  else if (later == 1) wait_vmcnt<N>();
  else wait_vmcnt<0>();
}

// acc = sum over nk steps. issue(slot, kt) enqueues step kt's A block at `slot` and its B block
// at slot + A bytes, exactly Loader<S, BM>::kPer + Loader<S, BN>::kPer DMA instructions per
// thread. Step kt lives in ring slot kt % STAGES, and STAGES - 1 steps are in flight ahead of the
// one being computed: step kt waits for its own group only (the groups of steps kt + 1 ..
// kt + STAGES - 2 stay in flight), one barrier makes every wavefront's data visible and retires
// the slot read in step kt - 1, which then receives step kt + STAGES - 1. With a scaling hook,
// step kt's factors are loaded right before its group and every step issues a full group (past
// nk the loaders read zeros into a retired slot) and the hook's loads (clamped to the last step,
// step 0 when nk is 0), so every wait counts whole groups. The step loop is unrolled by STAGES: slot indices and LDS
// offsets are compile-time constants.
template <class S, bool kBnn = false, class Issue, class Scale = NoScale>
__device__ __forceinline__ void ring_gemm(unsigned char* smem, int nk, Issue&& issue, Acc<S>& acc,
                                          int lane, int wave, Scale&& scale = Scale()) {
  constexpr int kHookLoads = std::decay_t<Scale>::kLoads;
  constexpr bool kScaled = kHookLoads > 0;
  constexpr int kBPer = b_dma_per_step<S, kBnn>();
  constexpr int kGroup = Loader<S, S::kBM>::kPer + kBPer + kHookLoads;
  constexpr int kSt = S::kStages;
  const int wm = wave / S::kWavesN, wn = wave % S::kWavesN;
#pragma unroll
  for (int i = 0; i < S::kFragM; ++i)
#pragma unroll
    for (int j = 0; j < S::kFragN; ++j)
#pragma unroll
      for (int v = 0; v < 16; ++v) acc[i][j][v] = 0.f;
  auto issue_step = [&](int slot, int kt) {
    if (kScaled) {
      asm volatile("" ::: "memory");  // the factor load stays right before its group
      scale.prefetch(kt < nk ? kt : (nk > 0 ? nk - 1 : 0), slot);  // in range when nk is 0
      asm volatile("" ::: "memory");
    }
    issue(smem + slot * S::kStageBytes, kt);
  };
#pragma unroll
  for (int st = 0; st < kSt - 1; ++st)
    if (kScaled || st < nk) issue_step(st, st);
  for (int kb = 0; kb < nk; kb += kSt) {
#pragma unroll
    for (int i = 0; i < kSt; ++i) {  // step kt = kb + i in slot i
      const int kt = kb + i;
      if (kt >= nk) break;
      wait_groups<kGroup>(kScaled ? kSt - 2 : min(kSt - 2, nk - 1 - kt));
      lds_barrier();
      if (kScaled || kt + kSt - 1 < nk) issue_step((i + kSt - 1) % kSt, kt + kSt - 1);
      const unsigned char* st = smem + i * S::kStageBytes;
      mma_step<S, std::decay_t<Scale>, kBnn>(reinterpret_cast<const uint4*>(st),
                  reinterpret_cast<const uint4*>(st + S::kAChunks * 16), acc, lane, wm, wn, scale,
                  i);
      scale.after(st, i, kt);
    }
  }
  __syncthreads();  // every wavefront is done with the ring before the caller reuses the LDS
}

// Row and column, inside the tile, of accumulator element v of 32x32 block (i, j) on `lane`.
template <class S>
__device__ __forceinline__ int acc_row(int wm, int i, int v, int lane) {
  return wm * S::kWaveM + i * 32 + 8 * (v >> 2) + 4 * (lane >> 5) + (v & 3);
}
template <class S>
__device__ __forceinline__ int acc_col(int wn, int j, int lane) {
  return wn * S::kWaveN + j * 32 + (lane & 31);
}

}  // namespace
}  // namespace talm
