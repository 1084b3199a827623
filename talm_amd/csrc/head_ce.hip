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
//                 running statistics exactly as the reference's per-slice update; for labelled
//                 rows it writes the per-tile factors fp16(e^{m_t - m_G}) against the running max
//                 m_G after the group and the accumulator's rescale e^{m_prev - m_G}; after the
//                 last slice it writes token loss, entropy, argmax and correctness.
//   head_grad     Y = P W over the group's columns, cut into K parts that fill the chip, against
//                 the transposed weight W^T [hidden, vocab] so that both operands are
//                 k-contiguous; P = fp16(P_t e^{m_t - m_G}) is formed on the A fragments between
//                 LDS and the MFMAs. The reference's per-slice rescales e^{m_old - m_c} of its
//                 accumulator telescope over a group into e^{m_c - m_G}, so this is its
//                 accumulator update up to one more fp16 rounding of P.
//   head_combine  acc = e^{m_prev - m_G} acc + the parts' sum, and after the last group
//                 dH = acc / s - W16[target] in fp16.
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

// head_logits: 256 vocabulary rows (A = W) x 256 token rows (B = H) per tile, 64-deep steps
// through a two-slot ring, eight wavefronts of 128 vocabulary rows x 64 tokens. In the
// accumulator layout of v_mfma_f32_32x32x16_f16 a lane holds one column (a token) and 16 rows
// (vocabulary entries) of each 32 x 32 block, so a wavefront's 128 rows, one statistics tile,
// are 64 values in lane l and 64 in lane l ^ 32 for each of its tokens: the per-token statistics
// need no LDS staging and one cross-lane exchange.
using LogitsShape = TileShape<256, 256, 64, 2, 2, 4>;
static_assert(LogitsShape::kWaveM == 128 && LogitsShape::kFragM == 4,
              "one statistics tile of 4 x 32 rows per wavefront");
// head_grad: 256 (labelled rows) x 256 (hidden) tiles, 64-deep steps through a two-slot ring,
// eight wavefronts of 64 x 128 (two A fragments, each scaled between LDS and the MFMAs). The B
// operand is the weight's rows as they lie ([64 vocabulary entries][256 hidden columns] per
// stage), transposed by the fragment reads: no transposed copy of the weight.
using GradShape = TileShape<256, 256, 64, 2, 4, 2>;
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

// The value of lane l ^ 32. v_permlane32_swap exchanges the upper 32 lanes of its first operand
// with the lower 32 lanes of its second: with a register as both, lanes >= 32 find their
// partner's value in the first result, lanes < 32 in the second.
__device__ __forceinline__ uint32_t other_half(uint32_t v) {
  const auto r = __builtin_amdgcn_permlane32_swap(v, v, false, false);
  return (threadIdx.x & 32) ? r[0] : r[1];
}
__device__ __forceinline__ float other_half(float v) {
  return __builtin_bit_cast(float, other_half(__builtin_bit_cast(uint32_t, v)));
}
__device__ __forceinline__ int other_half(int v) {
  return static_cast<int>(other_half(static_cast<uint32_t>(v)));
}

// ------------------------------------------------------------------------------------------
// GEMM1: z[r][j] = fp16(sum_k H[r][k] W[j][k]) for the group's columns j < group_cols (W starts
// at the group's first vocabulary row) and the per-(row, 128-column tile) partial statistics
// (max m_t, first argmax, sum e^{z - m_t}, sum e^{z - m_t} z, and the logit at the target when
// the tile holds it); rows r < n_p (the labelled rows when the gradient is wanted) store
// P[r][j] = fp16(e^{z - m_t}), 0 past group_cols.
//
// Persistent: one workgroup per CU walks its tiles (each XCD one contiguous range, token tiles
// fastest, so the tiles in flight on an XCD share weight rows in its L2). When a tile's last ring
// step is read, the next tile's first step is issued into the ring and lands while the epilogue
// of the finished tile runs from registers.
// ------------------------------------------------------------------------------------------
struct LogitsArgs {
  const uint16_t* H;
  int64_t ldh;
  const uint16_t* W;  // the group's first vocabulary row
  int64_t ldw;
  int n_rows, K, group_cols, first_col;
  uint16_t* Z;
  int64_t ldz;
  float4* part;
  int parts_per_row;
  const int64_t* targets;
  float* ztarget;
  int n_p;
  int n_ttiles, n_tiles;
};

constexpr float kLog2e = 1.4426950408889634f;

// Row of the statistics tile held in z[k] of a lane in half h (lane >> 5): i * 32 + 8 q + 4 h + w
// for k = i * 16 + 4 q + w (the accumulator layout of block i).
__device__ __forceinline__ int stat_row(int k, int h) {
  return (k >> 4) * 32 + 8 * ((k >> 2) & 3) + 4 * h + (k & 3);
}

__device__ __forceinline__ void put_part(const LogitsArgs& a, int tok, int c0, float m, float s,
                                         float t, int idx) {
  a.part[static_cast<int64_t>(tok) * a.parts_per_row + (c0 >> 7)] =
      make_float4(m, s, t, __int_as_float(a.first_col + c0 + idx));
}

// Whether this lane holds the target's row of the statistics tile (rarely: one tile per row), and
// the target's index k in z; `valid` counts the group's columns from the tile's first on.
__device__ __forceinline__ bool target_here(int64_t target, int valid, int tok, int c0, int h,
                                            const LogitsArgs& a, int& k) {
  const int64_t rel = target - (a.first_col + c0);
  const int r = static_cast<int>(rel & 127);
  k = ((r >> 5) << 4) | (((r >> 3) & 3) << 2) | (r & 3);
  return tok < a.n_rows && rel >= 0 && rel < min(valid, 128) && ((rel >> 2) & 1) == h;
}

typedef _Float16 half2_t __attribute__((ext_vector_type(2)));
typedef float float2_t __attribute__((ext_vector_type(2)));

// Statistics and P of one (token, statistics tile) from this lane's 64 rounded logits, packed in
// pairs: zp[k / 2] holds rows stat_row(k, h) and stat_row(k + 1, h) (k even), and the 64 of lane
// l ^ 32. When a lane of the wavefront holds its token's target row, the pairs also go to the
// lanes' 128-byte LDS rows `zs`, from which that lane reads the target's logit. Rows at or past
// `valid` (the tile holding the group's end) are not vocabulary: their logits are -65504 (see
// the kernel), which gives e = 0 and P = 0 and takes no part in the maximum or the argmax.
__device__ __forceinline__ uint32_t pack_h2(float lo, float hi) {  // v_cvt_pk_f16_f32
  return __builtin_bit_cast(uint32_t, __builtin_convertvector((float2_t){lo, hi}, half2_t));
}

// The epilogue's LDS row accesses (the rare target-logit path) as assembly. A plain LDS access
// here makes the compiler wait for every direct-to-LDS load in flight first (it cannot tell
// that the next tile's first ring step lands in the other slot, where the rows are not), which
// would drain the prefetch the persistent loop keeps in flight under this epilogue.
// lds_store16: 16 bytes into the row. lds_u16_now: one fp16 read back and waited for in the same
// block; both blocks are ordered ("memory" clobbers), and a wavefront's LDS operations complete
// in order, so the read sees the stores.
__device__ __forceinline__ void lds_store16(uint16_t* p, uint4 v) {
  const uint32_t addr = static_cast<uint32_t>(reinterpret_cast<uintptr_t>(
      (__attribute__((address_space(3))) uint16_t*)(p)));
  typedef uint32_t u32x4_t __attribute__((ext_vector_type(4)));
  const u32x4_t d = {v.x, v.y, v.z, v.w};
  asm volatile("ds_write_b128 %0, %1" : : "v"(addr), "v"(d) : "memory");
}

__device__ __forceinline__ uint16_t lds_u16_now(const uint16_t* p) {
  const uint32_t addr = static_cast<uint32_t>(reinterpret_cast<uintptr_t>(
      (__attribute__((address_space(3))) const uint16_t*)(p)));
  uint32_t r;
  asm volatile("ds_read_u16 %0, %1\n\ts_waitcnt lgkmcnt(0)" : "=v"(r) : "v"(addr) : "memory");
  return static_cast<uint16_t>(r);
}

__device__ __forceinline__ void tile_stats(const uint32_t (&zp)[32], float mx, uint16_t* zs,
                                           int lane, int tok, int64_t target, int c0, int valid,
                                           const LogitsArgs& a) {
  const int h = lane >> 5;
  int kt;
  const bool hit = target_here(target, valid, tok, c0, h, a, kt);
  if (__builtin_amdgcn_ballot_w64(hit)) {
#pragma unroll
    for (int k = 0; k < 32; k += 4)
      lds_store16(zs + 2 * k, make_uint4(zp[k], zp[k + 1], zp[k + 2], zp[k + 3]));
  }
  auto zh = [&](int k) {  // row stat_row(k, h) as fp16
    return __builtin_bit_cast(half2_t, zp[k >> 1])[k & 1];
  };
  // maximum of the rounded logits (`mx`: of this lane's)
  const float m = fmaxf(mx, other_half(mx));
  const _Float16 m16 = static_cast<_Float16>(m);  // exact
  // first argmax: the smallest row whose logit equals the maximum (-0 and +0 compare equal)
  int idx = 1 << 30;
#pragma unroll
  for (int k = 63; k >= 0; --k) {
    // the row (without 4 h, added once below) through a scalar register set right here: as
    // plain constants, the 64 rows would be hoisted into vector registers across the tile loop
    int row;
    asm volatile("s_mov_b32 %0, %1" : "=s"(row) : "i"(stat_row(k, 0)));
    if (zh(k) >= m16) idx = row;
  }
  idx += 4 * h;
  idx = min(idx, other_half(idx));
  // e = e^{z - m} = 2^u with u = z log2(e) - m log2(e), the sums s = sum e and
  // t = sum e z = m s + (sum e u) / log2(e), and P, block by block: after exchanging half of the
  // fp16 pairs with lane l ^ 32, a lane holds the 8 consecutive rows i * 32 + 8 (q + h) for
  // q = 0, 2, one 16-byte store each
  const float nm = -m * kLog2e;
  float s = 0.f, tu = 0.f;
  const bool store_p = tok < a.n_p;
  uint16_t* zrow = a.Z + static_cast<int64_t>(tok) * a.ldz + c0;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    uint32_t pk[8];
#pragma unroll
    for (int v = 0; v < 16; v += 2) {
      float e2[2];
#pragma unroll
      for (int u = 0; u < 2; ++u) {
        const float arg = fmaf(static_cast<float>(zh(i * 16 + v + u)), kLog2e, nm);
        const float e = __builtin_amdgcn_exp2f(arg);
        s += e;
        tu = fmaf(e, arg, tu);
        e2[u] = e;
      }
      pk[v >> 1] = pack_h2(e2[0], e2[1]);
    }
#pragma unroll
    for (int q = 0; q < 4; q += 2) {
      uint32_t x[2] = {pk[2 * q], pk[2 * q + 1]};
      uint32_t y[2] = {pk[2 * q + 2], pk[2 * q + 3]};
#pragma unroll
      for (int u = 0; u < 2; ++u) {
        // lanes < 32 receive the other half's x in y, lanes >= 32 the other half's y in x
        const auto r = __builtin_amdgcn_permlane32_swap(x[u], y[u], false, false);
        x[u] = r[0];
        y[u] = r[1];
      }
      if (store_p)
        *reinterpret_cast<uint4*>(zrow + i * 32 + 8 * (q + h)) = make_uint4(x[0], x[1], y[0], y[1]);
    }
  }
  s += other_half(s);
  tu += other_half(tu);
  const float t = fmaf(tu, 1.f / kLog2e, m * s);
  if (tok < a.n_rows && h == 0) put_part(a, tok, c0, m, s, t, idx);
  if (hit) a.ztarget[tok] = h2f(lds_u16_now(zs + kt));
}

// One ring step of the logits kernel: for each 16-deep slice ks, the wavefront's 4 A and 2 B
// fragments and their 8 MFMAs. With 128-byte rows (8 chunks), the swizzled chunk of slice ks is
// the slice-0 chunk with bits 1-2 XOR-ed by ks, so every fragment's address is its slice-0 byte
// offset `fo` XOR 32 ks. The XOR goes through an opaque scalar: otherwise the compiler keeps all
// 24 addresses of the step (and those of the other slot) in registers across the tile loop.
template <class S>
__device__ __forceinline__ void logits_step(const unsigned char* st, const uint32_t (&fo)[6],
                                            Acc<S>& acc) {
  static_assert(S::kCpr == 8 && S::kFragM == 4 && S::kFragN == 2, "the logits tile shape");
#pragma unroll
  for (int ks = 0; ks < S::kBK / 16; ++ks) {
    uint32_t x;
    asm volatile("s_mov_b32 %0, %1" : "=s"(x) : "i"(32 * ks));
    half8_t f[6];
#pragma unroll
    for (int q = 0; q < 6; ++q) f[q] = *reinterpret_cast<const half8_t*>(st + (fo[q] ^ x));
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
      for (int j = 0; j < 2; ++j)
        acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_f16(f[i], f[4 + j], acc[i][j], 0, 0, 0);
  }
}

template <class S>
__global__ __launch_bounds__(S::kThreads, 1) void head_logits_kernel(LogitsArgs a) {
  __shared__ __attribute__((aligned(1024))) unsigned char smem[S::kRing];
  constexpr int kSt = S::kStages;
  static_assert(kSt == 2, "the first step of each tile waits for every outstanding operation");
  static_assert(S::kStageBytes >= S::kThreads * 128, "a 128-byte LDS row per lane in slot 1");
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int wm = wave / S::kWavesN, wn = wave % S::kWavesN;

  // this workgroup's tiles: first, first + stride, ... below end
  const uint32_t nwg = gridDim.x, n_tiles = static_cast<uint32_t>(a.n_tiles);
  uint32_t first = blockIdx.x, stride = nwg, end = n_tiles;
  if (nwg % kXcds == 0) {  // workgroup b runs on XCD b % 8: give each XCD a contiguous range
    const uint32_t x = blockIdx.x % kXcds, q = n_tiles / kXcds, r = n_tiles % kXcds;
    const uint32_t start = x * q + min(x, r);
    first = start + blockIdx.x / kXcds;
    stride = nwg / kXcds;
    end = start + q + (x < r ? 1u : 0u);
  }
  const int nk = (a.K + S::kBK - 1) / S::kBK;

  // slice-0 byte offsets of the wavefront's fragments in a stage: A (weight rows) then B (tokens)
  uint32_t fo[6];
#pragma unroll
  for (int i = 0; i < 4; ++i)
    fo[i] = 16u * swz<S::kCpr>(wm * S::kWaveM + i * 32 + (lane & 31), lane >> 5);
#pragma unroll
  for (int j = 0; j < 2; ++j)
    fo[4 + j] = S::kAChunks * 16u + 16u * swz<S::kCpr>(wn * S::kWaveN + j * 32 + (lane & 31), lane >> 5);

  Loader<S, S::kBM> la;
  Loader<S, S::kBN> lb;
  la.lanes(a.ldw, a.K, wave, lane);
  lb.lanes(a.ldh, a.K, wave, lane);
  auto start_tile = [&](uint32_t tile) {
    const int tt = static_cast<int>(tile % a.n_ttiles), vt = static_cast<int>(tile / a.n_ttiles);
    la.rows(a.W + static_cast<int64_t>(vt) * S::kBM * a.ldw, a.ldw, min(a.group_cols - vt * S::kBM, S::kBM));
    lb.rows(a.H + static_cast<int64_t>(tt) * S::kBN * a.ldh, a.ldh, min(a.n_rows - tt * S::kBN, S::kBN));
    if (nk > 0) {
      // step 0 through an opaque zero: the addresses are tile-invariant, and hoisting them out of
      // the tile loop would hold eight more registers across it
      int k0;
      asm volatile("s_mov_b32 %0, 0" : "=s"(k0));
      la.issue(smem, k0, wave);
      lb.issue(smem + S::kAChunks * 16, k0, wave);
    }
  };
  if (first >= end) return;
  start_tile(first);
  for (uint32_t tile = first;;) {
    const int tt = static_cast<int>(tile % a.n_ttiles), vt = static_cast<int>(tile / a.n_ttiles);
    const int c0 = vt * S::kBM + wm * S::kWaveM;  // the wavefront's first column in the group
    const int valid = a.group_cols - c0;         // of its rows, those that are vocabulary
    // the targets of the lane's two tokens, loaded before the K loop (whose first wait covers
    // them): loaded in the epilogue, after the next tile's first ring step was issued, their
    // wait would also wait for that step's loads (vector-memory loads complete in order), and
    // the epilogue would not overlap the prefetch. Held as int32 (-1: none; a label past 2^31
    // is past any vocabulary and can hit no column either).
    int tgt[S::kFragN];
#pragma unroll
    for (int j = 0; j < S::kFragN; ++j) {
      const int tok = tt * S::kBN + wn * S::kWaveN + j * 32 + (lane & 31);
      const int64_t t = tok < a.n_rows ? a.targets[tok] : -1;
      tgt[j] = t < 0 || t > 0x7fffffff ? -1 : static_cast<int>(t);
    }
    // Accumulators start at 0, or at -65504 (fp16's lowest finite value) for rows past the group's
    // end: their weight rows read as zeros, so their logits stay -65504 exactly, and e^{z - m}
    // is 0 for them whenever a vocabulary logit of the tile exceeds -65400 (a tile whose logits
    // all round to -65504 or below has overflowed fp16 anyway). Row i * 32 + 8 q + 4 h + w is past
    // the end when (valid - 1 - 4 h) - (i * 32 + 8 q + w) < 0: its sign bit selects the value
    // without a mask register per row.
    Acc<S> acc;
#pragma unroll
    for (int i = 0; i < S::kFragM; ++i)
#pragma unroll
      for (int j = 0; j < S::kFragN; ++j)
#pragma unroll
        for (int v = 0; v < 16; ++v) acc[i][j][v] = 0.f;
    if (valid < S::kWaveM) {  // uniform, rare
      asm volatile("");  // keeps the branch (no selects on every tile)
      const int lim = valid - 1 - 4 * (lane >> 5);
      constexpr int kLowest = static_cast<int>(0xc77fe000u);  // -65504.f
#pragma unroll
      for (int i = 0; i < S::kFragM; ++i)
#pragma unroll
        for (int j = 0; j < S::kFragN; ++j)
#pragma unroll
          for (int v = 0; v < 16; ++v)
            acc[i][j][v] =
                __int_as_float(((lim - (i * 32 + 8 * (v >> 2) + (v & 3))) >> 31) & kLowest);
    }
    for (int kb = 0; kb < nk; kb += kSt) {
#pragma unroll
      for (int i = 0; i < kSt; ++i) {  // step kt = kb + i in slot i
        const int kt = kb + i;
        if (kt >= nk) break;
        wait_vmcnt<0>();  // this step's group (and, at step 0, the previous epilogue's stores)
        lds_barrier();
        if (kt + 1 < nk) {
          unsigned char* slot = smem + ((i + 1) % kSt) * S::kStageBytes;
          la.issue(slot, (kt + 1) * S::kBK, wave);
          lb.issue(slot + S::kAChunks * 16, (kt + 1) * S::kBK, wave);
        }
        logits_step<S>(smem + i * S::kStageBytes, fo, acc);
      }
    }
    // the targets count as written here, where nothing else is in flight: their wait (if the
    // loop's own did not cover them) is placed here and not after the next step's loads below
    asm volatile("" : "+v"(tgt[0]), "+v"(tgt[1]));
    static_assert(S::kFragN == 2, "two token columns per wavefront");
    // every wavefront has read the last step: slot 0 takes the next tile's first step, slot 1
    // serves the epilogue's rare paths (a 128-byte row per lane)
    lds_barrier();
    const uint32_t next = tile + stride;
    if (next < end) start_tile(next);

    // epilogue from registers: the wavefront's statistics tile and two 32-token columns, rounded
    // to fp16 first (the logits the reference sees; half the registers of the sums)
    uint32_t zp[S::kFragN][32];
    float mx[S::kFragN];
#pragma unroll
    for (int j = 0; j < S::kFragN; ++j) {
      half2_t m2;
#pragma unroll
      for (int i = 0; i < S::kFragM; ++i)
#pragma unroll
        for (int v = 0; v < 16; v += 2) {
          const half2_t z2 = __builtin_convertvector((float2_t){acc[i][j][v], acc[i][j][v + 1]}, half2_t);
          m2 = i == 0 && v == 0 ? z2 : __builtin_elementwise_max(m2, z2);
          zp[j][i * 8 + v / 2] = __builtin_bit_cast(uint32_t, z2);
        }
      mx[j] = fmaxf(static_cast<float>(m2[0]), static_cast<float>(m2[1]));
    }
    uint16_t* zs = reinterpret_cast<uint16_t*>(smem + S::kStageBytes) + tid * 64;
    if (valid > 0) {
#pragma unroll
      for (int j = 0; j < S::kFragN; ++j) {
        const int tok = tt * S::kBN + wn * S::kWaveN + j * 32 + (lane & 31);
        tile_stats(zp[j], mx[j], zs, lane, tok, tgt[j], c0, valid, a);
      }
    }
    if (next >= end) break;
    tile = next;
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
  float* alpha;            // [n_rows]: e^{m_prev - m_G}, the accumulator's rescale for this group
  float* token_loss;
  float* entropy;
  int32_t* best_idx;
  int32_t* correct;
};

// One wavefront per row. With slices of at most 64 tiles (vchunk <= 8192) a lane holds one tile of
// each slice, and every load the row needs (the group's tiles, the running statistics, the
// target's logit) is issued before the first reduction: one memory round trip per row instead
// of two per slice. Wider slices take the tiles in lane-strided loops. Same merges in the same
// order either way.
template <bool kOne>
__device__ __forceinline__ void merge_row(const MergeArgs& a, int row, int lane) {
  constexpr int kMaxSlices = 8;
  const int n = a.n_rows;
  const float4* prow = a.part + static_cast<int64_t>(row) * a.parts_per_row;
  const int tiles_per_slice = a.vchunk / kTile;
  float4 p[kMaxSlices];
  if constexpr (kOne) {
#pragma unroll
    for (int c = 0; c < kMaxSlices; ++c) {
      const int tiles = c < a.n_slices ? (a.slice_cols[c] + kTile - 1) / kTile : 0;
      p[c] = lane < tiles ? prow[c * tiles_per_slice + lane] : make_float4(-INFINITY, 0.f, 0.f, 0.f);
    }
  }
  const int64_t target = a.targets[row];
  const bool labelled = target >= 0;
  const float zt_new = a.ztarget[row];  // meaningful only when the target is in this group
  float* run = a.run;
  float m, s, t, best, zt;
  int bidx;
  if (a.first_slice) {
    m = -INFINITY; s = 0.f; t = 0.f; best = -INFINITY; zt = 0.f; bidx = 0;
  } else {
    m = run[row]; s = run[n + row]; t = run[2 * n + row]; best = run[3 * n + row];
    zt = run[4 * n + row]; bidx = __float_as_int(run[5 * n + row]);
  }
  auto slice = [&](int c) {
    const int tiles = (a.slice_cols[c] + kTile - 1) / kTile;
    const int tile0 = c * tiles_per_slice;
    Stat acc{-INFINITY, 0.f, 0.f, 0x7fffffff};
    if constexpr (kOne) {
      if (lane < tiles) acc = merge(acc, Stat{p[c].x, p[c].y, p[c].z, __float_as_int(p[c].w)});
    } else {
      for (int tt = lane; tt < tiles; tt += kWave) {
        const float4 q = prow[tile0 + tt];
        acc = merge(acc, Stat{q.x, q.y, q.z, __float_as_int(q.w)});
      }
    }
#pragma unroll
    for (int off = 32; off >= 1; off >>= 1) acc = merge(acc, shfl_stat(acc, off));
    // the slice into the running statistics (solution/fused_head.py:136-153)
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
    if (labelled && rel >= 0 && rel < a.slice_cols[c]) zt = zt_new;
  };
  const float m_prev = m;  // the running maximum before this group
  if constexpr (kOne) {
#pragma unroll
    for (int c = 0; c < kMaxSlices; ++c)
      if (c < a.n_slices) slice(c);
  } else {
    for (int c = 0; c < a.n_slices; ++c) slice(c);
  }
  // The reference adds fp16(e^{z - m_c}) W_c into its fp32 accumulator after rescaling it by
  // e^{m_old - m_c} at every slice (solution/fused_head.py:170-182); the rescales of one group's
  // slices telescope, so the group's contribution is sum_c e^{m_c - m_G} fp16(e^{z - m_c}) W_c with
  // m_G the running maximum after the group. Here each tile's P_t = fp16(e^{z - m_t}) is scaled by
  // fp16(e^{m_t - m_G}) in head_grad (one more fp16 rounding than the reference's P, as before),
  // so the group's columns form one plain reduction that head_grad may cut anywhere, and
  // head_combine rescales the accumulator once per group by e^{m_prev - m_G}.
  auto factors = [&](int c) {
      const int tiles = (a.slice_cols[c] + kTile - 1) / kTile;
      const int tile0 = c * tiles_per_slice;
      if constexpr (kOne) {
        if (lane < tiles) {
          const float mt = p[c].x;
          a.scale[scale_index(row, tile0 + lane, a.scale_blocks)] = f2h(mt == -INFINITY ? 0.f : __expf(mt - m));
        }
      } else {
        for (int tt = lane; tt < tiles; tt += kWave) {
          const float mt = prow[tile0 + tt].x;
          a.scale[scale_index(row, tile0 + tt, a.scale_blocks)] = f2h(mt == -INFINITY ? 0.f : __expf(mt - m));
        }
      }
  };
  if (row < a.n_grad) {
    if constexpr (kOne) {
#pragma unroll
      for (int c = 0; c < kMaxSlices; ++c)
        if (c < a.n_slices) factors(c);
    } else {
      for (int c = 0; c < a.n_slices; ++c) factors(c);
    }
  }
  if (lane == 0)
    a.alpha[row] = a.first_slice || m_prev == -INFINITY ? 0.f : __expf(m_prev - m);
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

__global__ __launch_bounds__(kThreads) void head_merge_kernel(MergeArgs a) {
  const int lane = threadIdx.x & 63;
  const int row = blockIdx.x * (kThreads / kWave) + (threadIdx.x >> 6);
  if (row >= a.n_rows) return;
  if (a.vchunk <= kTile * kWave) merge_row<true>(a, row, lane);
  else merge_row<false>(a, row, lane);
}

// ------------------------------------------------------------------------------------------
// GEMM2: Y_p[r][h] = sum_j P[r][j] W^T[h][col0 + j] over part p of the group's columns (a range of
// whole 64-column steps; the group's slices lie side by side in P and in W^T), for the first
// n_grad rows (the labelled rows, put first by the caller); P = fp16(P_t e^{m_t - m_G}) from
// head_logits' P_t and head_merge's factors. The group's K steps are cut into `parts` equal
// ranges so that (row tiles x hidden tiles x parts) workgroups fill the chip whatever the
// number of labelled rows.
// ------------------------------------------------------------------------------------------

// The A-fragment hook of head_grad: ring step kt covers columns [zc + kt BK, + BK) of one 128-column
// tile (BK divides 128, zc is a multiple of BK); lane l of the wavefront owning rows
// [r0, r0 + 32 FRAGS) multiplies fragment i (row r0 + 32 i + l % 32) by the row's factor of that
// tile. r0 is a multiple of 32 FRAGS, so the lane's FRAGS factors are adjacent: one load per step,
// into the register set of the step's ring slot.
template <int BK, int FRAGS, int SLOTS>
struct TileScale {
  static_assert(FRAGS == 2 || FRAGS == 4, "two or four 32-row A fragments per wavefront");
  static constexpr int kLoads = 1;
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
  __device__ __forceinline__ void after(const unsigned char*, int, int) {}
};
struct GradArgs {
  const uint16_t* Z;
  int64_t ldz;
  const uint16_t* W;      // the weight [vocab][ldw]: the B operand's rows as they lie (nn stages)
  int64_t ldw;
  int vocab;
  int col0;               // the group's first vocabulary column
  int n_grad;
  int hidden;
  int group_cols;         // the group's columns
  int parts;              // K ranges of the group's columns, each with its own partial
  int steps_per_part;     // 64-column steps per part (the last part may have fewer or none)
  const uint16_t* scale;  // per-(row, tile) factors of head_merge, see scale_index
  int scale_blocks;
  float* Y;               // [parts][n_grad][hidden] fp32
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
  const int m0 = mtile * kBM, n0 = ntile * kBN;
  // this part's columns of the group, in whole steps (BK divides 128: a step lies in one tile)
  static_assert(kTile % S::kBK == 0, "a ring step inside one statistics tile");
  const int per = a.steps_per_part * S::kBK;
  const int zc = min(piece * per, a.group_cols), kn = min(a.group_cols - zc, per);
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int wm = wave / S::kWavesN, wn = wave % S::kWavesN;

  Loader<S, kBM> la;
  LoaderNN<S> lb;
  la.init(a.Z + static_cast<int64_t>(m0) * a.ldz + zc, a.ldz, a.n_grad - m0, kn, wave, lane);
  // W's rows col0 + zc .. (the part's vocabulary entries, none past the vocabulary), columns
  // n0 .. n0 + 255 of the hidden dimension, transposed by the fragment reads
  lb.init(a.W + static_cast<int64_t>(a.col0 + zc) * a.ldw + n0, a.ldw,
          min(kn, a.vocab - a.col0 - zc), a.hidden - n0, wave, lane);
  TileScale<S::kBK, S::kFragM, S::kStages> sc;
  sc.base = a.scale + scale_index(m0 + wm * S::kWaveM + (lane & 31), 0, a.scale_blocks);
  sc.tile_stride = static_cast<int64_t>(a.scale_blocks) * 128;
  sc.zc = kn > 0 ? zc : 0;  // an empty part (zc may be the group's end) still loads in range
  Acc<S> acc;
  ring_gemm<S, true>(
      smem, (kn + S::kBK - 1) / S::kBK,
      [&](unsigned char* slot, int kt) {
        la.issue(slot, kt * S::kBK, wave);
        lb.issue(slot + S::kAChunks * 16, kt, wave);
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
// acc = e^{m_prev - m_G} acc + sum_p Y_p (parts in order); after the last group dH = acc / s -
// W[target]. One thread per 4 hidden columns of one row.
// ------------------------------------------------------------------------------------------
struct CombineArgs {
  float* acc;              // [n_grad][hidden]
  const float* Y;          // [parts][n_grad][hidden]
  const float* alpha;      // [n_rows]: e^{m_prev - m_G}
  const float* run;        // running statistics (s at [n_rows + row])
  const int64_t* targets;
  const uint16_t* W;       // full weight (row = vocabulary column)
  int64_t ldw;
  int64_t vocab;
  uint16_t* grad;          // [n_rows][hidden] fp16 (written after the last slice)
  int n_rows, n_grad, hidden, parts, first_slice, last_slice;
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
  // the row's other inputs are loaded beside the parts (one memory round trip; the weight row
  // of the target follows)
  float al = 0.f, s = 1.f;
  float4 o = make_float4(0.f, 0.f, 0.f, 0.f);
  int64_t tgt = -1;
  if (!a.first_slice) {
    al = a.alpha[row];
    o = *reinterpret_cast<const float4*>(a.acc + at);
  }
  if (a.last_slice) {
    s = a.run[a.n_rows + row];
    tgt = a.targets[row];
  }
  // the parts in order, eight loads in flight before their adds (selects, not a branch, so that
  // no load is sunk to its add; parts past the last add +0)
  const int64_t part_stride = static_cast<int64_t>(a.n_grad) * a.hidden;
  float4 y = make_float4(0.f, 0.f, 0.f, 0.f);
  for (int p0 = 0; p0 < a.parts; p0 += 8) {
    float4 yp[8];
#pragma unroll
    for (int j = 0; j < 8; ++j)
      yp[j] = *reinterpret_cast<const float4*>(a.Y + min(p0 + j, a.parts - 1) * part_stride + at);
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      const bool in = p0 + j < a.parts;
      y.x += in ? yp[j].x : 0.f; y.y += in ? yp[j].y : 0.f;
      y.z += in ? yp[j].z : 0.f; y.w += in ? yp[j].w : 0.f;
    }
  }
  float4 v = y;
  if (!a.first_slice) {
    v.x = o.x * al + y.x; v.y = o.y * al + y.y; v.z = o.z * al + y.z; v.w = o.w * al + y.w;
  }
  if (!a.last_slice) {
    *reinterpret_cast<float4*>(a.acc + at) = v;
    return;
  }
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
// WT[h][v] = W[v][h] for v < vocab, 0 for vocab <= v < ldwt (talm_head_weight_t). 64 x 64 blocks
// through LDS, 16-byte loads and stores.
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

// The gradient GEMM's output [n_grad, hidden] is small against its reduction (a group's columns):
// the group's K steps are cut into `parts` ranges, each with its own fp32 partial (summed by
// head_combine), so that the launch fills the chip. The plan minimizes a time model: rounds of
// workgroups x steps per part x a 64-deep step's time with every CU busy (1.7 us, measured),
// plus each part's partial written and read back at 5 TB/s.
constexpr double kStepUs = 1.7, kPartialBytesPerUs = 5e6;
constexpr int kMaxParts = 16;

struct GradPlan {
  int parts;           // parts holding work
  int steps_per_part;  // 64-deep ring steps per part
};

GradPlan plan_grad(int64_t n_grad, int64_t hidden, int64_t group_cols) {
  using S = GradShape;
  const int64_t tiles = (n_grad + S::kBM - 1) / S::kBM * ((hidden + S::kBN - 1) / S::kBN);
  const int64_t total = std::max<int64_t>(1, (group_cols + S::kBK - 1) / S::kBK);
  GradPlan best{1, static_cast<int>(total)};
  double best_t = 1e300;
  for (int64_t p = 1; p <= std::min<int64_t>(kMaxParts, total); ++p) {
    const int64_t steps = (total + p - 1) / p;
    const int64_t parts = (total + steps - 1) / steps;
    const int64_t rounds = (tiles * parts + kCus - 1) / kCus;
    const double t = static_cast<double>(rounds * steps) * kStepUs +
                     static_cast<double>(parts * n_grad * hidden) * 8.0 / kPartialBytesPerUs;
    if (t < best_t - 1e-9) {
      best_t = t;
      best = GradPlan{static_cast<int>(parts), static_cast<int>(steps)};
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
  // fp32 partials for the group with the most parts: a full one, or the last (narrower) one
  const int64_t slices = (vocab + vchunk - 1) / vchunk;
  const int64_t last_cols = vocab - (slices - 1) / group * group * vchunk;
  const int64_t pieces = n_grad > 0 ? std::max<int64_t>(plan_grad(n_grad, hidden, group * vchunk).parts,
                                                        plan_grad(n_grad, hidden, last_cols).parts)
                                    : 0;
  l.scale_blocks = static_cast<int>((n_grad + kBM - 1) / kBM * 2);
  size_t off = 0;
  l.z = off;      off = align_up(off + static_cast<size_t>(n_grad) * l.ldz * 2, 256);
  l.part = off;   off = align_up(off + static_cast<size_t>(n_rows) * l.parts_per_row * 16, 256);
  l.scale = off;  off = align_up(off + static_cast<size_t>(l.parts_per_row) * l.scale_blocks * 128 * 2, 256);
  l.run = off;    off = align_up(off + static_cast<size_t>(n_rows) * 6 * 4, 256);
  l.ztarget = off; off = align_up(off + static_cast<size_t>(n_rows) * 4, 256);
  l.alpha = off;  off = align_up(off + static_cast<size_t>(n_rows) * 4, 256);
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
  if (n_rows > (1 << 30) || vocab > (1 << 30) || hidden > (1 << 20) || ldh >= (1 << 22) ||
      ldw >= (1 << 22))
    return fail(TALM_EINVAL, "head_ce: sizes beyond 32-bit indexing (row strides below 2^22)");
  const bool with_grad = n_grad > 0 && grad_hidden;
  if (n_rows == 0) return ok();
  if (!hidden_states || !weight || !targets || !token_loss || !entropy || !best_idx || !correct ||
      !workspace || (n_grad > 0 && !grad_hidden))
    return fail(TALM_EINVAL, "head_ce: null pointer");
  if (!aligned(hidden_states, 16) || !aligned(weight, 16) || !aligned(workspace, 256) ||
      (grad_hidden && !aligned(grad_hidden, 16)))
    return fail(TALM_EINVAL, "head_ce: hidden states, weight and dH must be 16-byte "
                             "aligned, the workspace 256-byte aligned");
  const int64_t slices = (vocab + vchunk - 1) / vchunk;
  const int g = static_cast<int>(slices < group ? slices : group);
  const Layout l = layout(n_rows, hidden, vocab, vchunk, n_grad, g);
  if (l.ldz >= (1 << 22))
    return fail(TALM_EINVAL, "head_ce: group * vchunk = %lld columns per step, below 2^22 needed",
                (long long)l.ldz);
  if (with_grad && static_cast<int64_t>(g) * vchunk * ldw * 2 >= (int64_t{1} << 31))
    return fail(TALM_EINVAL, "head_ce: a group's weight rows (%lld x %lld halfs) beyond 2^31 bytes",
                (long long)(g * vchunk), (long long)ldw);
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
  const int n_p = grad_hidden ? static_cast<int>(n_grad) : 0;  // rows whose P is stored

  for (int64_t s0 = 0; s0 < slices; s0 += g) {
    const int ns = static_cast<int>(slices - s0 < g ? slices - s0 : g);
    const int64_t col0 = s0 * vchunk;
    const int64_t gcols = (s0 + ns == slices) ? vocab - col0 : ns * vchunk;
    LogitsArgs la{};
    la.H = hidden_states; la.ldh = ldh; la.W = weight + col0 * ldw; la.ldw = ldw;
    la.n_rows = rows; la.K = static_cast<int>(hidden); la.group_cols = static_cast<int>(gcols);
    la.first_col = static_cast<int>(col0); la.Z = Z; la.ldz = l.ldz; la.part = part;
    la.parts_per_row = l.parts_per_row; la.targets = targets; la.ztarget = ztarget; la.n_p = n_p;
    la.n_ttiles = (rows + LogitsShape::kBN - 1) / LogitsShape::kBN;
    la.n_tiles = la.n_ttiles * static_cast<int>((gcols + LogitsShape::kBM - 1) / LogitsShape::kBM);
    // one workgroup per CU (a multiple of 8, one range per XCD) or one per tile, if fewer
    int wgs = std::min(la.n_tiles, device_cus());
    if (wgs >= kXcds) wgs -= wgs % kXcds;
    hipLaunchKernelGGL((head_logits_kernel<LogitsShape>), dim3(static_cast<unsigned>(wgs)),
                       dim3(LogitsShape::kThreads), 0, s, la);
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
      ga.Z = Z; ga.ldz = l.ldz; ga.W = weight; ga.ldw = ldw; ga.vocab = static_cast<int>(vocab);
      ga.col0 = static_cast<int>(col0);
      ga.n_grad = static_cast<int>(n_grad); ga.hidden = static_cast<int>(hidden);
      ga.group_cols = static_cast<int>(gcols);
      ga.scale = scale; ga.scale_blocks = l.scale_blocks;
      ga.Y = Y;
      const GradPlan gp = plan_grad(n_grad, hidden, gcols);
      constexpr int bn = GradShape::kBN;
      ga.parts = gp.parts;
      ga.steps_per_part = gp.steps_per_part;
      ga.n_mtiles = static_cast<int>((n_grad + kBM - 1) / kBM);
      ga.n_ntiles = static_cast<int>((hidden + bn - 1) / bn);
      ga.n_tiles = ga.n_mtiles * ga.n_ntiles * gp.parts;
      hipLaunchKernelGGL((head_grad_kernel<GradShape>), dim3(static_cast<unsigned>(ga.n_tiles)),
                         dim3(GradShape::kThreads), 0, s, ga);
      CombineArgs ca{};
      ca.acc = accbuf; ca.Y = Y; ca.alpha = alpha; ca.run = run; ca.targets = targets;
      ca.W = weight; ca.ldw = ldw; ca.vocab = vocab; ca.grad = grad_hidden; ca.n_rows = rows;
      ca.n_grad = static_cast<int>(n_grad); ca.hidden = static_cast<int>(hidden);
      ca.parts = gp.parts;
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
