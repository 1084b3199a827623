// The q|k|v projection of a decoder layer with its LoRA adapters, on gfx950 fp16 MFMA.
//
// The reference (solution/fused_proj.py:88-218 with PEFT's LoRA arithmetic, solution/lora.py:
// 151-231) computes [q|k|v] = x W^T + b as one GEMM, then per adapter t = x A^T,
// branch = t B^T and out[:, seg] += scaling * branch, and the rotary embedding on q and k.
// Here that is two launches:
//   lora_down   t = x A_g^T for every adapter g (rank 16 each) and ts = scaling_g * t: a
//               register-only v_mfma_f32_16x16x32_f16 kernel, the reduction split over the eight
//               wavefronts of a workgroup (t is what the backward keeps, as in the reference).
//   qkv_fwd     out = [x | ts] [W | B]^T + b with the rotary embedding applied in the epilogue:
//               the LoRA up-projection is one more 64-deep step of the tile GEMM (the adapter's
//               16 columns of ts against its 16 columns of B, zeros elsewhere), so the adapter
//               term is accumulated in fp32 with the base product and rounded once. Tiles of
//               128 columns are whole heads, so the epilogue rotates each (j, j + 64) pair of
//               the staged fp16 tile in LDS before the coalesced store.
#include <mutex>

#include "mfma_tile.h"

namespace talm {
namespace {

typedef float f32x4 __attribute__((ext_vector_type(4)));

constexpr int kRank = 16;         // LoRA rank of the MFMA path (one 16x16x32 column block)
constexpr int kMaxAdapters = 2;

// ------------------------------------------------------------------------------------------
// t[r][16 g + i] = fp16(sum_k x[r][k] A_g[i][k]); ts = fp16(scaling_g * the same fp32 sum).
// One workgroup per 16 tokens, wavefront w takes the 32-deep k-steps w, w + 8, ... of the
// workgroup's chunk list, issuing the loads of up to kDownBatch steps before their MFMAs.
// ------------------------------------------------------------------------------------------
// Adapter g reduces over x's columns [xcol_g, xcol_g + k_g) against A_g [16][k_g] (the forward:
// both over all of x; the backward: u = dy_seg B_g over each adapter's own output columns).
// With `a_kmajor` the A_g are given as [k_g][16] (the backward passes B_g as it is stored):
// each lane then gathers its 8 k-consecutive values with 2-byte loads.
constexpr int kDownWaves = 8;
constexpr int kDownBatch = 8;

// How a workgroup walks its reduction: the 32-deep k-steps of adapter 0 ([0, n0)) then those of
// adapter 1 ([n0, n0 + n1)) form ONE list of chunks, dealt to the wavefronts round-robin, so the
// loads of both adapters are in flight together (one memory round trip, not one per adapter).
// kDownShared (the forward: both adapters over the same x columns and depth): a chunk is one x
// load for both adapters' MFMAs. kDownKmajor (the backward's B_g given as [k][16]): each lane
// gathers its 8 k-consecutive A values with 2-byte loads.
enum DownMode { kDownSplit = 0, kDownKmajor = 1, kDownShared = 2 };

template <int kMode>
__global__ __launch_bounds__(64 * kDownWaves) void lora_down_kernel(
    const uint16_t* __restrict__ x, int64_t ldx, int n_tokens, int k0len, int k1len, int xcol0,
    int xcol1, const uint16_t* __restrict__ a0, const uint16_t* __restrict__ a1, int n_adapters,
    float s0, float s1, uint16_t* __restrict__ t, uint16_t* __restrict__ ts, int64_t ldt) {
  constexpr bool kKmajor = kMode == kDownKmajor, kShared = kMode == kDownShared;
  __shared__ float red[kDownWaves][kMaxAdapters][16][16 + 1];
  const int m0 = blockIdx.x * 16;
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int row = lane & 15, kq = 8 * (lane >> 4);
  const uint16_t* xr = x + static_cast<int64_t>(m0) * ldx;
  const __amdgpu_buffer_rsrc_t rx0 = buffer_rsrc(xr + xcol0);
  const __amdgpu_buffer_rsrc_t rx1 = buffer_rsrc(xr + xcol1);
  const __amdgpu_buffer_rsrc_t ra0 = buffer_rsrc(a0);
  const __amdgpu_buffer_rsrc_t ra1 = buffer_rsrc(a1);
  const uint32_t xoff = m0 + row < n_tokens ? static_cast<uint32_t>((row * ldx + kq) * 2) : kOob;
  const uint32_t aoff0 = static_cast<uint32_t>((row * k0len + kq) * 2);
  const uint32_t aoff1 = static_cast<uint32_t>((row * k1len + kq) * 2);
  const int n0 = k0len >> 5, n1 = n_adapters > 1 ? k1len >> 5 : 0;
  const int chunks = kShared ? n0 : n0 + n1;
  f32x4 acc0 = {0.f, 0.f, 0.f, 0.f}, acc1 = acc0;
  for (int base = wave; base < chunks; base += kDownWaves * kDownBatch) {
    // slot j of the pass is chunk base + 8 j; a slot past the list loads through an offset
    // beyond every buffer (the load returns 0 and fetches nothing) and its MFMA adds zeros.
    // Every load is unconditional: branches between them would make the compiler wait on
    // earlier loads inside the chain.
    half8_t xa[kDownBatch], wa[kDownBatch], wb[kShared ? kDownBatch : 1];
    uint16_t g[kKmajor ? kDownBatch : 1][8];
#pragma unroll
    for (int j = 0; j < kDownBatch; ++j) {
      const int c = base + kDownWaves * j;
      const bool live = c < chunks, second = !kShared && c >= n0;
      const uint32_t kbytes = static_cast<uint32_t>((second ? c - n0 : c) * 64);
      xa[j] = __builtin_bit_cast(half8_t, __builtin_amdgcn_raw_buffer_load_b128(
                                              second ? rx1 : rx0, live ? xoff + kbytes : kOob, 0, 0));
      if constexpr (kKmajor) {
        // A_g [k][16]: element (k, i) at byte 32 k + 2 i; this lane's k = kbytes / 2 + kq + e
        const uint32_t at = kbytes * 16 + static_cast<uint32_t>((kq * 16 + row) * 2);
#pragma unroll
        for (int e = 0; e < 8; ++e)
          g[j][e] = __builtin_amdgcn_raw_buffer_load_b16(second ? ra1 : ra0,
                                                         live ? at + 32 * e : kOob, 0, 0);
      } else {
        wa[j] = __builtin_bit_cast(half8_t, __builtin_amdgcn_raw_buffer_load_b128(
                                                second ? ra1 : ra0,
                                                live ? (second ? aoff1 : aoff0) + kbytes : kOob, 0, 0));
      }
      if constexpr (kShared)
        wb[j] = __builtin_bit_cast(half8_t, __builtin_amdgcn_raw_buffer_load_b128(
                                                ra1, live ? aoff1 + kbytes : kOob, 0, 0));
    }
    // the empty statements take the loaded registers, so the compiler waits for the whole pass
    // here and not load by load
#pragma unroll
    for (int j = 0; j < kDownBatch; ++j) {
      asm volatile("" : "+v"(xa[j]));
      if constexpr (kKmajor) {
#pragma unroll
        for (int e = 0; e < 8; ++e) asm volatile("" : "+v"(g[j][e]));
      } else {
        asm volatile("" : "+v"(wa[j]));
      }
      if constexpr (kShared) asm volatile("" : "+v"(wb[j]));
    }
#pragma unroll
    for (int j = 0; j < kDownBatch; ++j) {
      if constexpr (kKmajor) {
        uint4 w;
        w.x = g[j][0] | (uint32_t{g[j][1]} << 16); w.y = g[j][2] | (uint32_t{g[j][3]} << 16);
        w.z = g[j][4] | (uint32_t{g[j][5]} << 16); w.w = g[j][6] | (uint32_t{g[j][7]} << 16);
        wa[j] = __builtin_bit_cast(half8_t, w);
      }
      if constexpr (kShared) {
        acc0 = __builtin_amdgcn_mfma_f32_16x16x32_f16(xa[j], wa[j], acc0, 0, 0, 0);
        acc1 = __builtin_amdgcn_mfma_f32_16x16x32_f16(xa[j], wb[j], acc1, 0, 0, 0);
      } else if (base + kDownWaves * j >= n0) {
        acc1 = __builtin_amdgcn_mfma_f32_16x16x32_f16(xa[j], wa[j], acc1, 0, 0, 0);
      } else {
        acc0 = __builtin_amdgcn_mfma_f32_16x16x32_f16(xa[j], wa[j], acc0, 0, 0, 0);
      }
    }
  }
  // accumulator element v of lane l: token 4 * (l / 16) + v, rank l % 16
#pragma unroll
  for (int v = 0; v < 4; ++v) {
    red[wave][0][4 * (lane >> 4) + v][lane & 15] = acc0[v];
    red[wave][1][4 * (lane >> 4) + v][lane & 15] = acc1[v];
  }
  __syncthreads();
  const int tid = threadIdx.x;
  for (int e = tid; e < n_adapters * 256; e += 64 * kDownWaves) {
    const int g_ = e >> 8, r = (e >> 4) & 15, i = e & 15;
    if (m0 + r >= n_tokens) continue;
    float sum = 0.f;
#pragma unroll
    for (int w = 0; w < kDownWaves; ++w) sum += red[w][g_][r][i];
    const int64_t at = static_cast<int64_t>(m0 + r) * ldt + g_ * kRank + i;
    t[at] = f2h(sum);
    ts[at] = f2h((g_ == 0 ? s0 : s1) * sum);
  }
}

// ------------------------------------------------------------------------------------------
// out = [x | ts] [W | B]^T + bias, rotary embedding on the columns below rope_cols.
// ------------------------------------------------------------------------------------------
// 64 x 128 tiles of 4 wavefronts of 32 x 64, a 3-slot ring (72 KiB) and two workgroups per CU:
// the token count gives few row tiles, so the smaller tile doubles the workgroups in flight and
// each keeps its own L2 -> LDS stream busy.
using QkvShape = TileShape<64, 128, 64, 3, 2, 2>;
constexpr int kQZS = QkvShape::kBN + 8;             // staged tile row stride (halfs)
static_assert(QkvShape::kBM * kQZS * 2 <= QkvShape::kRing, "the staged tile reuses the ring");

// An operand whose k range has two parts: steps [0, nk1) read `base1` (k < k1), the steps after
// them read `base2` (k in [lo2, hi2), counted from 0 again). The per-lane row and chunk do not depend on the part; the
// part's base, stride and bounds are chosen by value each step (scalar selects), so nothing is
// indexed through a selected address and the loader stays in registers.
template <class S, int kRows>
struct TwoPartLoader {
  static constexpr int kPer = Loader<S, kRows>::kPer;
  static constexpr int kRowsPerBlock = Loader<S, kRows>::kRowsPerBlock;
  __amdgpu_buffer_rsrc_t r1, r2;
  int row[kPer], kc8[kPer];
  int ld1, ld2, rows1, rows2, k1, lo2, hi2, nk1;

  __device__ __forceinline__ void init(const uint16_t* base1, int64_t ld1_, int rows1_, int k1_,
                                       const uint16_t* base2, int64_t ld2_, int rows2_, int lo2_,
                                       int hi2_, int wave, int lane) {
    r1 = buffer_rsrc(base1);
    r2 = buffer_rsrc(base2);
    ld1 = static_cast<int>(ld1_);
    ld2 = static_cast<int>(ld2_);
    rows1 = rows1_;
    rows2 = rows2_;
    k1 = k1_;
    lo2 = lo2_;
    hi2 = hi2_;
    nk1 = (k1_ + S::kBK - 1) / S::kBK;
#pragma unroll
    for (int p = 0; p < kPer; ++p) {
      row[p] = kRowsPerBlock * (p * S::kWaves + wave) + lane / S::kCpr;
      kc8[p] = ((lane % S::kCpr) ^ swz_key<S::kCpr>(row[p])) * 8;
    }
  }
  __device__ __forceinline__ void issue(unsigned char* dst, int kt, int wave) {
    const bool second = kt >= nk1;
    const int k0 = (second ? kt - nk1 : kt) * S::kBK;
    const __amdgpu_buffer_rsrc_t r = second ? r2 : r1;
    const int ld = second ? ld2 : ld1, rows = second ? rows2 : rows1;
    const int lo = second ? lo2 : 0, hi = second ? hi2 : k1;
#pragma unroll
    for (int p = 0; p < kPer; ++p) {
      const int k = k0 + kc8[p];
      const uint32_t v = row[p] < rows && k >= lo && k < hi
                             ? static_cast<uint32_t>((row[p] * ld + k) * 2)
                             : kOob;
      dma16(r, dst + (p * S::kWaves + wave) * 1024, v);
    }
  }
};

struct QkvArgs {
  const uint16_t* x;
  int64_t ldx;
  int n_tokens, hidden;
  const uint16_t* w;      // [n_out][ldw]: B rows of the main product (k = hidden)
  int64_t ldw;
  int n_out;
  const uint16_t* bias;   // [n_out] or null
  const uint16_t* ts;     // [n_tokens][ldt]: A of the extra step (k in a segment's window)
  int64_t ldt;
  int n_segs;             // output-column segments that get the extra step (at most 2)
  const uint16_t* b[kMaxAdapters];  // B of the extra step for segment g, row = output column
  int64_t ldb[kMaxAdapters];
  int seg_begin[kMaxAdapters], seg_end[kMaxAdapters];
  int k_lo[kMaxAdapters], k_hi[kMaxAdapters];  // the segment's k window of the extra step
  const float* cos;       // [n_tokens][cs_stride] or null (no rotary embedding)
  const float* sin;
  int64_t cs_stride;
  int rope_cols;          // columns [0, rope_cols) are heads of 128 to rotate
  uint16_t* out;          // [n_tokens][ldo]
  int64_t ldo;
  int n_mtiles, n_ntiles;
  // proj_ext_kernel<true>: the adapters' down-projection inside the GEMM (ts unused): A_g
  // [16][lda] fp16, t = x A_g^T written to t_out [n_tokens][ldt_out] (adapter g's 16 columns from
  // 16 g) by the first column tile of the segment
  const uint16_t* adown[kMaxAdapters];
  int64_t lda;
  float scaling[kMaxAdapters];
  uint16_t* t_out;
  int64_t ldt_out;
};

// The forward's LoRA down-projection inside the q|k|v GEMM (proj_ext_kernel<true>): each ring
// step of the main product also accumulates t = x A_g^T over the tile's 64 rows, wavefront w
// taking rows 16 w .. 16 w + 15 with two v_mfma_f32_16x16x32_f16 per 64-deep step. Their A
// operand is the x block already in the step's stage; their B operand is the adapter's 16 x 64
// slice of A_g, which the workgroup streams into a three-slot ring of its own beside the tile
// ring (2 KiB per step: each wavefront one direct-to-LDS load of four rows, its lanes past 32
// masked off), issued and waited with the step's stage. Slice row r holds chunk c at position
// c ^ (r / 2): the 16 lanes of a read phase (rows 0 .. 15, one chunk) meet 16 bank groups.
constexpr int kDownSlice = kRank * 64 * 2;  // bytes of one step's A_g slice

template <class S>
struct DownHook {
  static constexpr int kLoads = 1;
  __amdgpu_buffer_rsrc_t ra;
  unsigned char* ring;  // kStages slices of kDownSlice bytes
  uint32_t off;         // this lane's global byte offset at step 0 (lanes below 32)
  int klim;             // k below which A_g is read: the hidden size, 0 outside the adapters
  int kc;               // this lane's k inside a step (lanes below 32)
  int dst;              // this wavefront's 512 bytes of a slice
  int row;              // the lane's x row in the stage: 16 wave + lane % 16
  int lane;
  bool live;            // the tile is in an adapter's columns
  f32x4 t;
  __device__ __forceinline__ void prefetch(int kt, int slot) {
    const int k = kt * S::kBK + kc;
    // one compare, no branch around the address: a select between two offsets
    const uint32_t o = k < klim ? off + static_cast<uint32_t>(kt * S::kBK * 2) : kOob;
    if (lane < 32) dma16(ra, ring + slot * kDownSlice + dst, o);
  }
  __device__ __forceinline__ half8_t apply(half8_t a, int, int) const { return a; }
  __device__ __forceinline__ void after(const unsigned char* st, int slot, int) {
    if (!live) return;  // uniform over the workgroup
    const uint4* As = reinterpret_cast<const uint4*>(st);
    const uint4* Bs = reinterpret_cast<const uint4*>(ring + slot * kDownSlice);
    const int r = lane & 15;
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      const int c = 4 * h + (lane >> 4);
      t = __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(half8_t, As[swz<S::kCpr>(row, c)]),
                                                  __builtin_bit_cast(half8_t, Bs[r * 8 + (c ^ (r >> 1))]),
                                                  t, 0, 0, 0);
    }
  }
};

// out = x w^T (+ the extra step on the tile's segment) (+ bias), optionally rotated: the forward
// (extra step = the adapter term) and the backward dX (extra step = u A over all columns).
// kDown: the forward with the adapters' t = x A_g^T computed by the tile itself during the main
// product (DownHook) and the adapter term added after it as ts B_g^T (ts = fp16(scaling t),
// two v_mfma_f32_32x32x16_f16 per wavefront, K = the rank 16), in place of the extra step.
constexpr int kTsOff = 32 * 1024;  // ts [64][kTsLd] in the ring after the main product
constexpr int kTsLd = 24;          // 48-byte rows: a 16-lane phase of 16-byte reads meets 16 bank groups
static_assert(kTsOff >= QkvShape::kBM * kQZS * 2 && kTsOff + QkvShape::kBM * kTsLd * 2 <= QkvShape::kRing,
              "ts beside the staged tile");

template <bool kDown>
__global__ __launch_bounds__(QkvShape::kThreads, QkvShape::kPerCu) void proj_ext_kernel(QkvArgs a) {
  using S = QkvShape;
  static_assert(S::kFragM == 1 && S::kWaveM == 32 && S::kWaves == 4 && S::kBM == 64 &&
                    S::kBK == 64 && S::kCpr == 8,
                "the down-projection hook assumes four wavefronts on 64 rows, 64-deep steps");
  // the tile ring, then (kDown) the adapter slices' ring
  __shared__ __attribute__((aligned(1024))) unsigned char smem[S::kRing + (kDown ? S::kStages * kDownSlice : 0)];
  const uint32_t tile = xcd_tile(blockIdx.x, static_cast<uint32_t>(a.n_mtiles * a.n_ntiles));
  const int ntile = static_cast<int>(tile / a.n_mtiles), mtile = static_cast<int>(tile % a.n_mtiles);
  const int m0 = mtile * S::kBM, n0 = ntile * S::kBN;
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int wm = wave / S::kWavesN, wn = wave % S::kWavesN;

  // the segment whose output columns hold this tile (segments are whole tiles); selected with
  // conditionals, not by indexing the argument arrays (which would copy them to scratch)
  const bool in0 = a.n_segs > 0 && n0 >= a.seg_begin[0] && n0 < a.seg_end[0];
  const bool in1 = a.n_segs > 1 && n0 >= a.seg_begin[1] && n0 < a.seg_end[1];
  const int g = in1 ? 1 : (in0 ? 0 : -1);
  const bool g1 = g > 0;
  const uint16_t* bg = g1 ? a.b[1] : a.b[0];
  const int64_t ldb = g1 ? a.ldb[1] : a.ldb[0];
  const int sb = g1 ? a.seg_begin[1] : a.seg_begin[0], se = g1 ? a.seg_end[1] : a.seg_end[0];
  const int lo = g1 ? a.k_lo[1] : a.k_lo[0], hi = g1 ? a.k_hi[1] : a.k_hi[0];
  // A: x, then ts's k window; B: w's rows, then the segment's B (indexed from k = lo)
  TwoPartLoader<S, S::kBM> la;
  TwoPartLoader<S, S::kBN> lb;
  la.init(a.x + static_cast<int64_t>(m0) * a.ldx, a.ldx, a.n_tokens - m0, a.hidden,
          a.ts + static_cast<int64_t>(m0) * a.ldt, a.ldt, a.n_tokens - m0, lo, hi, wave, lane);
  lb.init(a.w + static_cast<int64_t>(n0) * a.ldw, a.ldw, a.n_out - n0, a.hidden,
          bg + static_cast<int64_t>(n0 - sb) * ldb - lo, ldb, se - n0, lo, hi, wave, lane);
  const int nk1 = (a.hidden + S::kBK - 1) / S::kBK;
  Acc<S> acc;
  if constexpr (!kDown) {
    ring_gemm<S>(
        smem, nk1 + (g >= 0 ? (hi + S::kBK - 1) / S::kBK : 0),
        [&](unsigned char* slot, int kt) {
          la.issue(slot, kt, wave);
          lb.issue(slot + S::kAChunks * 16, kt, wave);
        },
        acc, lane, wave);
  } else {
    // the adapter's B rows for this wavefront's two 32-column blocks (B_g [segment][16]: lane
    // gets output column n0 + 64 wn + 32 j + lane % 32, k-slots 8 (lane / 32) .. + 7), loaded
    // now so that they have landed when the product ends
    half8_t bfr[S::kFragN];
    const __amdgpu_buffer_rsrc_t rb = buffer_rsrc(bg);
#pragma unroll
    for (int j = 0; j < S::kFragN; ++j) {
      const int col = n0 + wn * S::kWaveN + 32 * j + (lane & 31);
      bfr[j] = __builtin_bit_cast(
          half8_t, __builtin_amdgcn_raw_buffer_load_b128(
                       rb, g >= 0 && col < se ? static_cast<uint32_t>(((col - sb) * kRank + 8 * (lane >> 5)) * 2) : kOob,
                       0, 0));
    }
    DownHook<S> hook;
    hook.ra = buffer_rsrc(g1 ? a.adown[1] : a.adown[0]);
    {
      // lane l < 32 of wavefront w fills slice row 4 w + l / 8, position l % 8: the global chunk
      // the swizzle puts there
      const int r = 4 * wave + (lane >> 3) % 4, c = (lane & 7) ^ (r >> 1);
      hook.off = static_cast<uint32_t>((r * a.lda + 8 * c) * 2);
      hook.kc = 8 * c;
    }
    hook.ring = smem + S::kRing;
    hook.dst = wave * 512;
    hook.lane = lane;
    hook.klim = g >= 0 ? a.hidden : 0;
    hook.row = 16 * wave + (lane & 15);
    hook.live = g >= 0;
    hook.t = f32x4{0.f, 0.f, 0.f, 0.f};
    ring_gemm<S>(
        smem, nk1,
        [&](unsigned char* slot, int kt) {
          la.issue(slot, kt, wave);
          lb.issue(slot + S::kAChunks * 16, kt, wave);
        },
        acc, lane, wave, hook);
    // ts = fp16(scaling t) into LDS for the adapter term; t itself, which the backward keeps, to
    // t_out from the segment's first column tile (lane: rank lane % 16, rows 4 (lane / 16) + v)
    uint16_t* tsl = reinterpret_cast<uint16_t*>(smem + kTsOff);
    if (g >= 0) {
      const float sg = g1 ? a.scaling[1] : a.scaling[0];
#pragma unroll
      for (int v = 0; v < 4; ++v) {
        const int r = 16 * wave + 4 * (lane >> 4) + v;
        tsl[r * kTsLd + (lane & 15)] = f2h(sg * hook.t[v]);
        if (n0 == sb && m0 + r < a.n_tokens)
          a.t_out[static_cast<int64_t>(m0 + r) * a.ldt_out + kRank * g + (lane & 15)] = f2h(hook.t[v]);
      }
    }
    __syncthreads();  // every wavefront's ts rows are in LDS
    if (g >= 0) {
      const half8_t tsa = *reinterpret_cast<const half8_t*>(&tsl[(wm * S::kWaveM + (lane & 31)) * kTsLd + 8 * (lane >> 5)]);
#pragma unroll
      for (int j = 0; j < S::kFragN; ++j)
        acc[0][j] = __builtin_amdgcn_mfma_f32_32x32x16_f16(tsa, bfr[j], acc[0][j], 0, 0, 0);
    }
  }

  // Epilogue: + bias, fp16, staged in LDS ([kBM][kQZS] halfs)
  uint16_t* Zs = reinterpret_cast<uint16_t*>(smem);
#pragma unroll
  for (int i = 0; i < S::kFragM; ++i)
#pragma unroll
    for (int j = 0; j < S::kFragN; ++j) {
      const int col = acc_col<S>(wn, j, lane);
      const float bv = a.bias && n0 + col < a.n_out ? h2f(a.bias[n0 + col]) : 0.f;
#pragma unroll
      for (int v = 0; v < 16; ++v) Zs[acc_row<S>(wm, i, v, lane) * kQZS + col] = f2h(acc[i][j][v] + bv);
    }
  __syncthreads();
  if (a.cos && n0 < a.rope_cols) {
    // one head: y1 = x1 c1 - x2 s1, y2 = x2 c2 + x1 s2 on the pairs (j, j + 64)
    for (int e = tid; e < S::kBM * 64; e += S::kThreads) {
      const int row = e >> 6, j = e & 63, gr = m0 + row;
      if (gr >= a.n_tokens) continue;
      const float* cr = a.cos + static_cast<int64_t>(gr) * a.cs_stride;
      const float* sr = a.sin + static_cast<int64_t>(gr) * a.cs_stride;
      const float x1 = h2f(Zs[row * kQZS + j]), x2 = h2f(Zs[row * kQZS + j + 64]);
      Zs[row * kQZS + j] = f2h(x1 * cr[j] - x2 * sr[j]);
      Zs[row * kQZS + j + 64] = f2h(x2 * cr[j + 64] + x1 * sr[j + 64]);
    }
    __syncthreads();
  }
#pragma unroll
  for (int it = 0; it < (S::kBM * S::kBN / 8) / S::kThreads; ++it) {
    const int c = it * S::kThreads + tid, row = c >> 4, kc = c & 15;
    const int gr = m0 + row, gc = n0 + kc * 8;
    if (gr < a.n_tokens && gc < a.n_out)
      *reinterpret_cast<uint4*>(a.out + static_cast<int64_t>(gr) * a.ldo + gc) =
          *reinterpret_cast<const uint4*>(Zs + row * kQZS + kc * 8);
  }
}

// ------------------------------------------------------------------------------------------
// The backward's operand: dcat = [rope_back(dq) | rope_back(dk) | dv] ([N, q + k + v] fp16).
// dx1 = dy1 c1 + dy2 s2, dx2 = dy2 c2 - dy1 s1 on each (j, j + 64) pair of a 128-wide head
// (solution/rope.py:145-157). One workgroup per token row, one thread per 8 columns.
// ------------------------------------------------------------------------------------------
__global__ __launch_bounds__(256) void qkv_bwd_prep_kernel(
    const uint16_t* __restrict__ dq, int64_t ldq, const uint16_t* __restrict__ dk, int64_t ldk,
    const uint16_t* __restrict__ dv, int64_t ldv, int q_cols, int k_cols, int v_cols,
    const float* __restrict__ cos, const float* __restrict__ sin, int64_t cs_stride,
    uint16_t* __restrict__ dcat, int64_t ldc) {
  const int r = blockIdx.x;
  const int rope_cols = q_cols + k_cols, total = rope_cols + v_cols;
  for (int c = threadIdx.x * 8; c < total; c += 256 * 8) {
    auto chunk = [&](int col) {
      const uint16_t* p = col < q_cols ? dq + static_cast<int64_t>(r) * ldq + col
                          : col < rope_cols ? dk + static_cast<int64_t>(r) * ldk + (col - q_cols)
                                            : dv + static_cast<int64_t>(r) * ldv + (col - rope_cols);
      return *reinterpret_cast<const uint4*>(p);
    };
    uint4 v = chunk(c);
    if (c < rope_cols && cos) {
      const int j = c & 127, first = j < 64;
      const uint4 o = chunk(first ? c + 64 : c - 64);  // the partner half of the same head
      const float* cr = cos + static_cast<int64_t>(r) * cs_stride;
      const float* sr = sin + static_cast<int64_t>(r) * cs_stride;
      const uint32_t mine[4] = {v.x, v.y, v.z, v.w}, other[4] = {o.x, o.y, o.z, o.w};
      uint32_t res[4];
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        float y[2];
#pragma unroll
        for (int h = 0; h < 2; ++h) {
          const int jj = j + 2 * e + h, pj = first ? jj + 64 : jj - 64;
          const float me = h ? hi_f(mine[e]) : lo_f(mine[e]);
          const float ot = h ? hi_f(other[e]) : lo_f(other[e]);
          // first half: dy1 c1 + dy2 s2; second half: dy2 c2 - dy1 s1
          y[h] = first ? me * cr[jj] + ot * sr[pj] : me * cr[jj] - ot * sr[pj];
        }
        res[e] = pack2(y[0], y[1]);
      }
      v = make_uint4(res[0], res[1], res[2], res[3]);
    }
    *reinterpret_cast<uint4*>(dcat + static_cast<int64_t>(r) * ldc + c) = v;
  }
}

// ------------------------------------------------------------------------------------------
// The adapters' weight gradients (reductions over tokens), fp32, in two passes:
//   dA_g[i][h] = sum_r u[r][16 g + i] x[r][h]                 (i < 16, h < hidden)
//   dB_g[j][i] = scaling_g sum_r dy[r][lo_g + j] t[r][16 g + i]  (j < seg_g)
// (solution/fused_proj.py:211-215, solution/lora.py:229-230: dA = u^T xd, dB = g^T t with
// g = scaling dy). Pass 1: workgroup (column block, token chunk) accumulates one column per
// thread over its chunk's tokens, the chunk's u / t rows broadcast from LDS, and writes a
// partial; pass 2 sums the chunks in order (deterministic) into the fp32 gradients.
// ------------------------------------------------------------------------------------------
constexpr int kWgChunk = 64;  // tokens per partial

struct WgradArgs {
  const uint16_t* x;      // [N][ldx]
  int64_t ldx;
  const uint16_t* dy;     // [N][ldy]: the node's output gradient (after the RoPE backward)
  int64_t ldy;
  const uint16_t* u;      // [N][ldu]: 16 columns per adapter
  int64_t ldu;
  const uint16_t* t;      // [N][ldt]
  int64_t ldt;
  int n_tokens, hidden, n_adapters;
  int lo[kMaxAdapters], seg[kMaxAdapters];
  float scaling[kMaxAdapters];
  float* part;            // [chunks][cols][32] fp32, cols = hidden + seg_0 + seg_1
  float* da[kMaxAdapters];  // [16][hidden]
  float* db[kMaxAdapters];  // [seg_g][16]
  int cols, chunks;
};

__global__ __launch_bounds__(256) void lora_wgrad_partial_kernel(WgradArgs a) {
  // every lane reads the same row (a broadcast): rows of 32 floats, 16-byte aligned
  __shared__ __attribute__((aligned(16))) float su[kWgChunk][32];
  __shared__ __attribute__((aligned(16))) float st[kWgChunk][32];
  const int chunk = blockIdx.y, r0 = chunk * kWgChunk;
  const int rn = min(kWgChunk, a.n_tokens - r0);
  const int rank = 16 * a.n_adapters;
  for (int e = threadIdx.x; e < kWgChunk * 32; e += 256) {
    const int r = e >> 5, i = e & 31;
    const bool ok = r < rn && i < rank;
    su[r][i] = ok ? h2f(a.u[static_cast<int64_t>(r0 + r) * a.ldu + i]) : 0.f;
    st[r][i] = ok ? h2f(a.t[static_cast<int64_t>(r0 + r) * a.ldt + i]) : 0.f;
  }
  __syncthreads();
  const int c = blockIdx.x * 256 + threadIdx.x;
  if (c >= a.cols) return;
  float acc[32];
#pragma unroll
  for (int i = 0; i < 32; ++i) acc[i] = 0.f;
  float* out = a.part + (static_cast<int64_t>(chunk) * a.cols + c) * 32;
  // the chunk's column values are all loaded before use (rows past the batch are clamped to its
  // last row and zeroed); their u / t rows in LDS are zero too
  float v[kWgChunk];
  if (c < a.hidden) {  // dA column h: both adapters' u
    const uint16_t* xc = a.x + static_cast<int64_t>(r0) * a.ldx + c;
#pragma unroll
    for (int r = 0; r < kWgChunk; ++r) v[r] = h2f(xc[static_cast<int64_t>(min(r, rn - 1)) * a.ldx]);
#pragma unroll
    for (int r = 0; r < kWgChunk; ++r) {
      const float xv = r < rn ? v[r] : 0.f;
#pragma unroll
      for (int i = 0; i < 32; ++i) acc[i] += su[r][i] * xv;
    }
  } else {  // dB row j of adapter g: its t
    const int cb = c - a.hidden, g = cb >= a.seg[0] ? 1 : 0;
    const int j = g ? cb - a.seg[0] : cb, col = (g ? a.lo[1] : a.lo[0]) + j;
    const uint16_t* yc = a.dy + static_cast<int64_t>(r0) * a.ldy + col;
#pragma unroll
    for (int r = 0; r < kWgChunk; ++r) v[r] = h2f(yc[static_cast<int64_t>(min(r, rn - 1)) * a.ldy]);
#pragma unroll
    for (int r = 0; r < kWgChunk; ++r) {
      const float yv = r < rn ? v[r] : 0.f;
#pragma unroll
      for (int i = 0; i < 16; ++i) acc[i] += st[r][16 * g + i] * yv;
    }
  }
#pragma unroll
  for (int i = 0; i < 32; i += 4)
    *reinterpret_cast<float4*>(out + i) = make_float4(acc[i], acc[i + 1], acc[i + 2], acc[i + 3]);
}

__global__ __launch_bounds__(256) void lora_wgrad_reduce_kernel(WgradArgs a) {
  // one thread per (column, i): the dA columns carry 32 values, the dB rows 16
  const int64_t e = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x;
  if (e >= static_cast<int64_t>(a.cols) * 32) return;
  const int c = static_cast<int>(e >> 5), i = static_cast<int>(e & 31);
  // the chunks in order; eight loads in flight before their adds (one memory round trip per
  // eight chunks instead of one per chunk; selects, not a branch, so that no load is sunk to its
  // add; chunks past the last add +0)
  const float* pc = a.part + static_cast<int64_t>(c) * 32 + i;
  const int64_t chunk_stride = static_cast<int64_t>(a.cols) * 32;
  float sum = 0.f;
  for (int k0 = 0; k0 < a.chunks; k0 += 8) {
    float v[8];
#pragma unroll
    for (int j = 0; j < 8; ++j) v[j] = pc[min(k0 + j, a.chunks - 1) * chunk_stride];
#pragma unroll
    for (int j = 0; j < 8; ++j) sum += k0 + j < a.chunks ? v[j] : 0.f;
  }
  if (c < a.hidden) {
    const int g = i >> 4;
    if (g < a.n_adapters) (g ? a.da[1] : a.da[0])[static_cast<int64_t>(i & 15) * a.hidden + c] = sum;
  } else if (i < 16) {
    const int cb = c - a.hidden, g = cb >= a.seg[0] ? 1 : 0;
    const int j = g ? cb - a.seg[0] : cb;
    (g ? a.db[1] : a.db[0])[static_cast<int64_t>(j) * 16 + i] = (g ? a.scaling[1] : a.scaling[0]) * sum;
  }
}

// The same partials on MFMA (v_mfma_f32_32x32x16_f16), for 128-token chunks. Workgroup
// (128 columns, chunk) stages the chunk's column values transposed in LDS, [column][token], a
// token pair written as one dword, so that a fragment's 8 tokens are one 16-byte read; u^T and
// t^T ([i][token], 32 columns each) sit next to them. Each wavefront reduces its 32 columns
// against the 32 u columns (dA columns) or the 32 t columns (dB rows; the adapter's 16 are kept)
// over the chunk's tokens: C[column][i] = sum_token X^T[column][token] M^T[i][token]. Needs
// hidden % 32 == 0 and 8-aligned segments, offsets and row strides (16-byte loads); other shapes
// take the kernel above. Same partial layout, so the same ordered reduction follows.
constexpr int kWmTok = 128;         // tokens per chunk
constexpr int kWmCols = 128;        // columns per workgroup: 4 wavefronts x 32
constexpr int kWmLd = kWmTok + 8;   // LDS row stride in halves (272 bytes, 16-byte multiple)

__device__ __forceinline__ void put_pair_columns(uint16_t (*rows)[kWmLd], int col, int pair,
                                                 uint4 va, uint4 vb) {
  // va / vb: 8 consecutive columns of tokens 2 pair and 2 pair + 1
  const uint32_t wa[4] = {va.x, va.y, va.z, va.w}, wb[4] = {vb.x, vb.y, vb.z, vb.w};
#pragma unroll
  for (int e = 0; e < 4; ++e) {
    *reinterpret_cast<uint32_t*>(&rows[col + 2 * e][2 * pair]) = (wa[e] & 0xffffu) | (wb[e] << 16);
    *reinterpret_cast<uint32_t*>(&rows[col + 2 * e + 1][2 * pair]) =
        (wa[e] >> 16) | (wb[e] & 0xffff0000u);
  }
}

__global__ __launch_bounds__(256) void lora_wgrad_mfma_kernel(WgradArgs a) {
  __shared__ __attribute__((aligned(16))) uint16_t xs[kWmCols][kWmLd];
  __shared__ __attribute__((aligned(16))) uint16_t ms[2][32][kWmLd];  // u^T, t^T
  constexpr int kPairs = kWmTok / 2;
  const int chunk = blockIdx.y, r0 = chunk * kWmTok;
  const int rn = min(kWmTok, a.n_tokens - r0);
  const int c0 = blockIdx.x * kWmCols;
  const int tid = threadIdx.x;
  const uint4 zero = make_uint4(0u, 0u, 0u, 0u);
  // Every global load of the workgroup is issued before the first LDS store (one memory round
  // trip): the column values, item = (8-column group, token pair), then u^T and t^T, item =
  // (which, 8-column group of 32, token pair). Rows past the batch are clamped to its last row
  // for the load and zeroed; columns of a missing adapter are zero.
  constexpr int kXItems = (kWmCols / 8) * kPairs / 256;  // 4 per thread
  constexpr int kMItems = 2 * 4 * kPairs / 256;          // 2 per thread
  static_assert(kXItems * 256 == (kWmCols / 8) * kPairs && kMItems * 256 == 2 * 4 * kPairs,
                "whole items per thread");
  uint4 xa[kXItems], xb[kXItems], ma[kMItems], mb[kMItems];
#pragma unroll
  for (int q = 0; q < kXItems; ++q) {
    const int it = q * 256 + tid, p = it % kPairs, g = it / kPairs;
    const int c = c0 + 8 * g;
    xa[q] = xb[q] = zero;
    if (c < a.cols) {
      const uint16_t* src;
      int64_t ld;
      if (c < a.hidden) {
        src = a.x + c;
        ld = a.ldx;
      } else {
        const int cb = c - a.hidden;
        src = a.dy + (cb >= a.seg[0] ? a.lo[1] + cb - a.seg[0] : a.lo[0] + cb);
        ld = a.ldy;
      }
      const int ra = min(2 * p, rn - 1), rb = min(2 * p + 1, rn - 1);
      xa[q] = *reinterpret_cast<const uint4*>(src + static_cast<int64_t>(r0 + ra) * ld);
      xb[q] = *reinterpret_cast<const uint4*>(src + static_cast<int64_t>(r0 + rb) * ld);
    }
  }
  const bool need_u = c0 < a.hidden, need_t = c0 + kWmCols > a.hidden;
  const int rank = kRank * a.n_adapters;
#pragma unroll
  for (int q = 0; q < kMItems; ++q) {
    const int it = q * 256 + tid, p = it % kPairs, gq = (it / kPairs) % 4, which = it / (4 * kPairs);
    ma[q] = mb[q] = zero;
    if ((which ? need_t : need_u) && 8 * gq < rank) {
      const uint16_t* src = (which ? a.t : a.u) + 8 * gq;
      const int64_t ld = which ? a.ldt : a.ldu;
      const int ra = min(2 * p, rn - 1), rb = min(2 * p + 1, rn - 1);
      ma[q] = *reinterpret_cast<const uint4*>(src + static_cast<int64_t>(r0 + ra) * ld);
      mb[q] = *reinterpret_cast<const uint4*>(src + static_cast<int64_t>(r0 + rb) * ld);
    }
  }
#pragma unroll
  for (int q = 0; q < kXItems; ++q) {
    const int it = q * 256 + tid, p = it % kPairs, g = it / kPairs;
    put_pair_columns(xs, 8 * g, p, 2 * p < rn ? xa[q] : zero, 2 * p + 1 < rn ? xb[q] : zero);
  }
#pragma unroll
  for (int q = 0; q < kMItems; ++q) {
    const int it = q * 256 + tid, p = it % kPairs, gq = (it / kPairs) % 4, which = it / (4 * kPairs);
    if (which ? !need_t : !need_u) continue;
    put_pair_columns(ms[which], 8 * gq, p, 2 * p < rn ? ma[q] : zero, 2 * p + 1 < rn ? mb[q] : zero);
  }
  __syncthreads();
  const int wave = tid >> 6, lane = tid & 63;
  const int cw = c0 + 32 * wave;
  if (cw >= a.cols) return;  // no barrier follows
  const int which = cw < a.hidden ? 0 : 1;  // hidden % 32 == 0: one kind per wavefront
  f32x16 acc = {};
#pragma unroll
  for (int ks = 0; ks < kWmTok / 16; ++ks) {
    const int kc = ks * 2 + (lane >> 5);
    const half8_t av = *reinterpret_cast<const half8_t*>(&xs[32 * wave + (lane & 31)][8 * kc]);
    const half8_t bv = *reinterpret_cast<const half8_t*>(&ms[which][lane & 31][8 * kc]);
    acc = __builtin_amdgcn_mfma_f32_32x32x16_f16(av, bv, acc, 0, 0, 0);
  }
  const int n = lane & 31;
  float* out = a.part + static_cast<int64_t>(chunk) * a.cols * 32;
#pragma unroll
  for (int v = 0; v < 16; ++v) {
    const int c = cw + 8 * (v >> 2) + 4 * (lane >> 5) + (v & 3);
    if (c >= a.cols) continue;
    int i = n;
    if (which) {  // dB row of adapter g: its 16 t columns, stored at 0..15
      i = n - (c - a.hidden >= a.seg[0] ? kRank : 0);
      if (i < 0 || i >= kRank) continue;
    }
    out[static_cast<int64_t>(c) * 32 + i] = acc[v];
  }
}

bool fits32(int64_t rows, int64_t ld) { return rows * ld * 2 < (int64_t{1} << 31); }

}  // namespace
}  // namespace talm

using namespace talm;

TALM_API int talm_lora_down(const uint16_t* x, int64_t ldx, int64_t n_tokens, int64_t k0,
                            int64_t k1, int64_t xcol0, int64_t xcol1, const uint16_t* a0,
                            const uint16_t* a1, int32_t n_adapters, int32_t a_kmajor,
                            float scaling0, float scaling1, uint16_t* t, uint16_t* ts, int64_t ldt,
                            void* stream) {
  const bool two = n_adapters > 1;
  if (n_tokens < 0 || n_adapters < 1 || n_adapters > kMaxAdapters || k0 < 32 || k0 % 32 ||
      (two && (k1 < 32 || k1 % 32)) || xcol0 < 0 || xcol0 % 8 || xcol0 + k0 > ldx ||
      (two && (xcol1 < 0 || xcol1 % 8 || xcol1 + k1 > ldx)) || ldx % 8 ||
      ldt < kRank * n_adapters || !fits32(16, ldx) || !fits32(16, k0) || !fits32(16, k1) ||
      n_tokens > (1 << 30))
    return fail(TALM_EINVAL,
                "lora_down: bad shape (tokens %lld, k %lld/%lld at columns %lld/%lld, ldx %lld, "
                "adapters %d, ldt %lld): reductions of a multiple of 32 inside x's rows, 1-2 "
                "adapters of rank 16",
                (long long)n_tokens, (long long)k0, (long long)k1, (long long)xcol0,
                (long long)xcol1, (long long)ldx, n_adapters, (long long)ldt);
  if (n_tokens == 0) return ok();
  if (!x || !a0 || (two && !a1) || !t || !ts) return fail(TALM_EINVAL, "lora_down: null pointer");
  if (!aligned(x, 16) || !aligned(a0, 16) || (two && !aligned(a1, 16)))
    return fail(TALM_EINVAL, "lora_down: x and the A matrices must be 16-byte aligned");
  const int mode = a_kmajor ? kDownKmajor
                   : two && xcol0 == xcol1 && k0 == k1 ? kDownShared : kDownSplit;
  const dim3 grid(static_cast<unsigned>((n_tokens + 15) / 16)), block(64 * kDownWaves);
  const uint16_t* a1s = two ? a1 : a0;
  const int k1s = static_cast<int>(two ? k1 : k0), x1s = static_cast<int>(two ? xcol1 : xcol0);
#define TALM_LORA_DOWN(M)                                                                     \
  hipLaunchKernelGGL(lora_down_kernel<M>, grid, block, 0, as_stream(stream), x, ldx,          \
                     static_cast<int>(n_tokens), static_cast<int>(k0), k1s,                   \
                     static_cast<int>(xcol0), x1s, a0, a1s, n_adapters, scaling0, scaling1, t, \
                     ts, ldt)
  if (mode == kDownKmajor)
    TALM_LORA_DOWN(kDownKmajor);
  else if (mode == kDownShared)
    TALM_LORA_DOWN(kDownShared);
  else
    TALM_LORA_DOWN(kDownSplit);
#undef TALM_LORA_DOWN
  return check_launch("lora_down");
}

namespace talm {
namespace {

int check_proj(const char* what, int64_t ldx, int64_t n_tokens, int64_t hidden, int64_t ldw,
               int64_t n_out, int64_t ldo) {
  using S = QkvShape;
  if (n_tokens < 0 || hidden < 8 || hidden % 8 || ldx < hidden || ldx % 8 || n_out < 1 ||
      ldw < hidden || ldw % 8 || ldo < n_out || ldo % 8 || n_tokens > (1 << 30) ||
      n_out > (1 << 30) || !fits32(S::kBM, ldx) || !fits32(S::kBN, ldw))
    return fail(TALM_EINVAL,
                "%s: bad shape (tokens %lld, hidden %lld, n_out %lld, ldx %lld, ldw %lld, ldo "
                "%lld): sizes and strides multiples of 8",
                what, (long long)n_tokens, (long long)hidden, (long long)n_out, (long long)ldx,
                (long long)ldw, (long long)ldo);
  return TALM_OK;
}

void launch_proj(QkvArgs& a, hipStream_t stream) {
  using S = QkvShape;
  a.n_mtiles = (a.n_tokens + S::kBM - 1) / S::kBM;
  a.n_ntiles = (a.n_out + S::kBN - 1) / S::kBN;
  hipLaunchKernelGGL(proj_ext_kernel<false>, dim3(static_cast<unsigned>(a.n_mtiles * a.n_ntiles)),
                     dim3(S::kThreads), 0, stream, a);
}

void launch_proj_down(QkvArgs& a, hipStream_t stream) {
  using S = QkvShape;
  a.n_mtiles = (a.n_tokens + S::kBM - 1) / S::kBM;
  a.n_ntiles = (a.n_out + S::kBN - 1) / S::kBN;
  hipLaunchKernelGGL(proj_ext_kernel<true>, dim3(static_cast<unsigned>(a.n_mtiles * a.n_ntiles)),
                     dim3(S::kThreads), 0, stream, a);
}

}  // namespace
}  // namespace talm

TALM_API int talm_qkv_lora_fwd(const uint16_t* x, int64_t ldx, int64_t n_tokens, int64_t hidden,
                               const uint16_t* weight, int64_t ldw, int64_t n_out,
                               const uint16_t* bias, const uint16_t* ts, int64_t ldt,
                               int32_t n_adapters, const uint16_t* b0, int64_t seg0_begin,
                               int64_t seg0_end, const uint16_t* b1, int64_t seg1_begin,
                               int64_t seg1_end, const float* cos, const float* sin,
                               int64_t cs_stride, int64_t rope_cols, uint16_t* out, int64_t ldo,
                               void* stream) {
  using S = QkvShape;
  if (check_proj("qkv_lora_fwd", ldx, n_tokens, hidden, ldw, n_out, ldo)) return TALM_EINVAL;
  if (n_adapters < 0 || n_adapters > kMaxAdapters)
    return fail(TALM_EINVAL, "qkv_lora_fwd: %d adapters (0-2)", n_adapters);
  const int64_t begins[2] = {seg0_begin, seg1_begin}, ends[2] = {seg0_end, seg1_end};
  for (int g = 0; g < n_adapters; ++g)
    if (begins[g] < 0 || ends[g] <= begins[g] || ends[g] > n_out || begins[g] % S::kBN ||
        (ends[g] % S::kBN && ends[g] != n_out))
      return fail(TALM_EINVAL,
                  "qkv_lora_fwd: adapter %d columns [%lld, %lld) must be whole %d-column tiles "
                  "of [0, %lld)",
                  g, (long long)begins[g], (long long)ends[g], S::kBN, (long long)n_out);
  if (n_adapters > 0 && ldt < kRank * n_adapters)
    return fail(TALM_EINVAL, "qkv_lora_fwd: ldt %lld < %d", (long long)ldt, kRank * n_adapters);
  if (cos && (rope_cols < 0 || rope_cols % 128 || rope_cols > n_out || cs_stride < 128))
    return fail(TALM_EINVAL,
                "qkv_lora_fwd: rotary columns %lld must be whole 128-column heads of the output "
                "(cos/sin row stride %lld >= 128)",
                (long long)rope_cols, (long long)cs_stride);
  if (n_tokens == 0) return ok();
  if (!x || !weight || !out || (n_adapters > 0 && (!ts || !b0)) || (n_adapters > 1 && !b1) ||
      (cos && !sin))
    return fail(TALM_EINVAL, "qkv_lora_fwd: null pointer");
  if (!aligned(x, 16) || !aligned(weight, 16) || !aligned(out, 16) || (ts && !aligned(ts, 16)) ||
      (b0 && !aligned(b0, 16)) || (b1 && !aligned(b1, 16)))
    return fail(TALM_EINVAL, "qkv_lora_fwd: x, weight, out, ts and B must be 16-byte aligned");
  QkvArgs a{};
  a.x = x; a.ldx = ldx; a.n_tokens = static_cast<int>(n_tokens); a.hidden = static_cast<int>(hidden);
  a.w = weight; a.ldw = ldw; a.n_out = static_cast<int>(n_out); a.bias = bias;
  a.ts = ts; a.ldt = ldt; a.n_segs = n_adapters;
  a.b[0] = b0; a.b[1] = b1;
  for (int g = 0; g < 2; ++g) {
    a.ldb[g] = kRank;
    a.seg_begin[g] = static_cast<int>(begins[g]);
    a.seg_end[g] = static_cast<int>(ends[g]);
    a.k_lo[g] = kRank * g;        // adapter g's 16 columns of ts
    a.k_hi[g] = kRank * (g + 1);
  }
  a.cos = cos; a.sin = sin; a.cs_stride = cs_stride; a.rope_cols = static_cast<int>(rope_cols);
  a.out = out; a.ldo = ldo;
  launch_proj(a, as_stream(stream));
  return check_launch("qkv_lora_fwd");
}

TALM_API int talm_qkv_lora_fwd_down(const uint16_t* x, int64_t ldx, int64_t n_tokens,
                                    int64_t hidden, const uint16_t* weight, int64_t ldw,
                                    int64_t n_out, const uint16_t* bias, int32_t n_adapters,
                                    const uint16_t* a0, const uint16_t* a1, int64_t lda,
                                    float scaling0, float scaling1, const uint16_t* b0,
                                    int64_t seg0_begin, int64_t seg0_end, const uint16_t* b1,
                                    int64_t seg1_begin, int64_t seg1_end, const float* cos,
                                    const float* sin, int64_t cs_stride, int64_t rope_cols,
                                    uint16_t* t, int64_t ldt, uint16_t* out, int64_t ldo,
                                    void* stream) {
  using S = QkvShape;
  if (check_proj("qkv_lora_fwd_down", ldx, n_tokens, hidden, ldw, n_out, ldo)) return TALM_EINVAL;
  if (n_adapters < 0 || n_adapters > kMaxAdapters)
    return fail(TALM_EINVAL, "qkv_lora_fwd_down: %d adapters (0-2)", n_adapters);
  const int64_t begins[2] = {seg0_begin, seg1_begin}, ends[2] = {seg0_end, seg1_end};
  for (int g = 0; g < n_adapters; ++g)
    if (begins[g] < 0 || ends[g] <= begins[g] || ends[g] > n_out || begins[g] % S::kBN ||
        (ends[g] % S::kBN && ends[g] != n_out))
      return fail(TALM_EINVAL,
                  "qkv_lora_fwd_down: adapter %d columns [%lld, %lld) must be whole %d-column "
                  "tiles of [0, %lld)",
                  g, (long long)begins[g], (long long)ends[g], S::kBN, (long long)n_out);
  if (n_adapters > 1 && ends[0] > begins[1] && ends[1] > begins[0])
    return fail(TALM_EINVAL, "qkv_lora_fwd_down: the adapters' columns overlap");
  if (n_adapters > 0 && (ldt < kRank * n_adapters || lda < hidden || lda % 8 || !fits32(16, lda)))
    return fail(TALM_EINVAL, "qkv_lora_fwd_down: ldt %lld < %d or A row stride %lld",
                (long long)ldt, kRank * n_adapters, (long long)lda);
  if (cos && (rope_cols < 0 || rope_cols % 128 || rope_cols > n_out || cs_stride < 128))
    return fail(TALM_EINVAL,
                "qkv_lora_fwd_down: rotary columns %lld must be whole 128-column heads of the "
                "output (cos/sin row stride %lld >= 128)",
                (long long)rope_cols, (long long)cs_stride);
  if (n_tokens == 0) return ok();
  if (!x || !weight || !out || (n_adapters > 0 && (!a0 || !b0 || !t)) ||
      (n_adapters > 1 && (!a1 || !b1)) || (cos && !sin))
    return fail(TALM_EINVAL, "qkv_lora_fwd_down: null pointer");
  if (!aligned(x, 16) || !aligned(weight, 16) || !aligned(out, 16) || (a0 && !aligned(a0, 16)) ||
      (a1 && !aligned(a1, 16)) || (b0 && !aligned(b0, 16)) || (b1 && !aligned(b1, 16)))
    return fail(TALM_EINVAL, "qkv_lora_fwd_down: x, weight, out, A and B must be 16-byte aligned");
  QkvArgs a{};
  a.x = x; a.ldx = ldx; a.n_tokens = static_cast<int>(n_tokens); a.hidden = static_cast<int>(hidden);
  a.w = weight; a.ldw = ldw; a.n_out = static_cast<int>(n_out); a.bias = bias;
  a.n_segs = n_adapters;
  a.b[0] = b0; a.b[1] = b1;
  for (int g = 0; g < 2; ++g) {
    a.ldb[g] = kRank;
    a.seg_begin[g] = static_cast<int>(begins[g]);
    a.seg_end[g] = static_cast<int>(ends[g]);
  }
  a.adown[0] = a0; a.adown[1] = a1; a.lda = lda;
  a.scaling[0] = scaling0; a.scaling[1] = scaling1;
  a.t_out = t; a.ldt_out = ldt;
  a.cos = cos; a.sin = sin; a.cs_stride = cs_stride; a.rope_cols = static_cast<int>(rope_cols);
  a.out = out; a.ldo = ldo;
  launch_proj_down(a, as_stream(stream));
  return check_launch("qkv_lora_fwd_down");
}

TALM_API int talm_qkv_bwd_prep(const uint16_t* dq, int64_t ldq, const uint16_t* dk, int64_t ldk,
                               const uint16_t* dv, int64_t ldv, int64_t n_tokens, int64_t q_cols,
                               int64_t k_cols, int64_t v_cols, const float* cos, const float* sin,
                               int64_t cs_stride, uint16_t* dcat, int64_t ldc, void* stream) {
  const int64_t total = q_cols + k_cols + v_cols;
  if (n_tokens < 0 || q_cols < 0 || k_cols < 0 || v_cols < 0 || q_cols % 8 || k_cols % 8 ||
      v_cols % 8 || total < 8 || ldc < total || ldc % 8 || (q_cols && (ldq < q_cols || ldq % 8)) ||
      (k_cols && (ldk < k_cols || ldk % 8)) || (v_cols && (ldv < v_cols || ldv % 8)) ||
      n_tokens > (1 << 30) || total > (1 << 30))
    return fail(TALM_EINVAL,
                "qkv_bwd_prep: bad shape (tokens %lld, columns %lld/%lld/%lld, ldc %lld): column "
                "counts and row strides multiples of 8",
                (long long)n_tokens, (long long)q_cols, (long long)k_cols, (long long)v_cols,
                (long long)ldc);
  if (cos && (q_cols % 128 || k_cols % 128 || cs_stride < 128))
    return fail(TALM_EINVAL, "qkv_bwd_prep: the rotated q and k need whole 128-column heads");
  if (n_tokens == 0) return ok();
  if (!dcat || (q_cols && !dq) || (k_cols && !dk) || (v_cols && !dv) || (cos && !sin))
    return fail(TALM_EINVAL, "qkv_bwd_prep: null pointer");
  if (!aligned(dcat, 16) || (dq && !aligned(dq, 16)) || (dk && !aligned(dk, 16)) ||
      (dv && !aligned(dv, 16)))
    return fail(TALM_EINVAL, "qkv_bwd_prep: gradients must be 16-byte aligned");
  hipLaunchKernelGGL(qkv_bwd_prep_kernel, dim3(static_cast<unsigned>(n_tokens)), dim3(256), 0,
                     as_stream(stream), dq, ldq, dk, ldk, dv, ldv, static_cast<int>(q_cols),
                     static_cast<int>(k_cols), static_cast<int>(v_cols), cos, sin, cs_stride, dcat,
                     ldc);
  return check_launch("qkv_bwd_prep");
}

TALM_API int talm_qkv_lora_bwd_dx(const uint16_t* dcat, int64_t ldc, int64_t n_tokens,
                                  int64_t n_out, const uint16_t* weight_t, int64_t ldwt,
                                  int64_t hidden, const uint16_t* u, int64_t ldu, int64_t rank,
                                  const uint16_t* a_t, int64_t ldat, uint16_t* dx, int64_t lddx,
                                  void* stream) {
  // dx [N, hidden] = dcat [N, n_out] W [n_out, hidden] + u [N, rank] A [rank, hidden], as the
  // NT product [dcat | u] [W^T | A^T]^T: the kernel's "x" is dcat, its "w" is W^T
  if (check_proj("qkv_lora_bwd_dx", ldc, n_tokens, n_out, ldwt, hidden, lddx)) return TALM_EINVAL;
  if (rank < 0 || rank > 64 || rank % 8 || (rank && (ldu < rank || ldu % 8 || ldat < rank ||
                                                      ldat % 8)))
    return fail(TALM_EINVAL, "qkv_lora_bwd_dx: rank %lld (a multiple of 8, at most 64)",
                (long long)rank);
  if (n_tokens == 0) return ok();
  if (!dcat || !weight_t || !dx || (rank && (!u || !a_t)))
    return fail(TALM_EINVAL, "qkv_lora_bwd_dx: null pointer");
  if (!aligned(dcat, 16) || !aligned(weight_t, 16) || !aligned(dx, 16) ||
      (rank && (!aligned(u, 16) || !aligned(a_t, 16))))
    return fail(TALM_EINVAL, "qkv_lora_bwd_dx: operands must be 16-byte aligned");
  QkvArgs a{};
  a.x = dcat; a.ldx = ldc; a.n_tokens = static_cast<int>(n_tokens); a.hidden = static_cast<int>(n_out);
  a.w = weight_t; a.ldw = ldwt; a.n_out = static_cast<int>(hidden); a.bias = nullptr;
  a.ts = u; a.ldt = ldu; a.n_segs = rank ? 1 : 0;
  a.b[0] = a.b[1] = a_t; a.ldb[0] = a.ldb[1] = ldat;
  a.seg_begin[0] = 0; a.seg_end[0] = static_cast<int>(hidden);
  a.k_lo[0] = 0; a.k_hi[0] = static_cast<int>(rank);
  a.out = dx; a.ldo = lddx;
  launch_proj(a, as_stream(stream));
  return check_launch("qkv_lora_bwd_dx");
}

TALM_API int64_t talm_lora_wgrad_workspace(int64_t n_tokens, int64_t hidden, int64_t seg0,
                                          int64_t seg1) {
  if (n_tokens < 0 || hidden < 1 || seg0 < 0 || seg1 < 0) return -1;
  const int64_t chunks = (n_tokens + kWgChunk - 1) / kWgChunk;
  return chunks * (hidden + seg0 + seg1) * 32 * 4;
}

namespace {

// Validates the arguments of the two wgrad entry points (everything but the workspace) and fills
// `a` (partials not yet assigned); TALM_OK or TALM_EINVAL with the message set.
int wgrad_args(const uint16_t* x, int64_t ldx, const uint16_t* dy, int64_t ldy, const uint16_t* u,
               int64_t ldu, const uint16_t* t, int64_t ldt, int64_t n_tokens, int64_t hidden,
               int32_t n_adapters, int64_t lo0, int64_t seg0, float scaling0, float* da0,
               float* db0, int64_t lo1, int64_t seg1, float scaling1, float* da1, float* db1,
               WgradArgs& a) {
  const bool two = n_adapters > 1;
  if (n_tokens < 0 || hidden < 1 || n_adapters < 1 || n_adapters > kMaxAdapters || seg0 < 1 ||
      lo0 < 0 || (two && (seg1 < 1 || lo1 < 0)) || ldx < hidden || ldu < 16 * n_adapters ||
      ldt < 16 * n_adapters || ldy < lo0 + seg0 || (two && ldy < lo1 + seg1) ||
      n_tokens > (1 << 30) || hidden + seg0 + seg1 > (1 << 24))
    return fail(TALM_EINVAL,
                "lora_wgrad: bad shape (tokens %lld, hidden %lld, adapters %d, segments "
                "%lld+%lld / %lld+%lld)",
                (long long)n_tokens, (long long)hidden, n_adapters, (long long)lo0,
                (long long)seg0, (long long)lo1, (long long)seg1);
  if (n_tokens > 0 && (!x || !dy || !u || !t || !da0 || !db0 || (two && (!da1 || !db1))))
    return fail(TALM_EINVAL, "lora_wgrad: null pointer");
  a = WgradArgs{};
  a.x = x; a.ldx = ldx; a.dy = dy; a.ldy = ldy; a.u = u; a.ldu = ldu; a.t = t; a.ldt = ldt;
  a.n_tokens = static_cast<int>(n_tokens); a.hidden = static_cast<int>(hidden);
  a.n_adapters = n_adapters;
  a.lo[0] = static_cast<int>(lo0); a.seg[0] = static_cast<int>(seg0); a.scaling[0] = scaling0;
  a.da[0] = da0; a.db[0] = db0;
  a.lo[1] = two ? static_cast<int>(lo1) : 0; a.seg[1] = two ? static_cast<int>(seg1) : 0;
  a.scaling[1] = two ? scaling1 : 0.f; a.da[1] = two ? da1 : da0; a.db[1] = two ? db1 : db0;
  a.cols = static_cast<int>(hidden + seg0 + (two ? seg1 : 0));
  return TALM_OK;
}

// Enqueues the two passes of the weight gradients on `s` with the partials at `a.part` (every
// partial the reduction uses is written by the first pass: nothing needs clearing).
int wgrad_launch(WgradArgs& a, hipStream_t s) {
  const bool two = a.n_adapters > 1;
  const bool mfma = a.hidden % 32 == 0 && a.seg[0] % 8 == 0 && a.lo[0] % 8 == 0 &&
                    (!two || (a.seg[1] % 8 == 0 && a.lo[1] % 8 == 0)) && a.ldx % 8 == 0 &&
                    a.ldy % 8 == 0 && a.ldu % 8 == 0 && a.ldt % 8 == 0 && aligned(a.x, 16) &&
                    aligned(a.dy, 16) && aligned(a.u, 16) && aligned(a.t, 16);
  if (mfma) {
    a.chunks = (a.n_tokens + kWmTok - 1) / kWmTok;
    hipLaunchKernelGGL(lora_wgrad_mfma_kernel,
                       dim3(static_cast<unsigned>((a.cols + kWmCols - 1) / kWmCols),
                            static_cast<unsigned>(a.chunks)),
                       dim3(256), 0, s, a);
  } else {
    a.chunks = (a.n_tokens + kWgChunk - 1) / kWgChunk;
    hipLaunchKernelGGL(lora_wgrad_partial_kernel,
                       dim3(static_cast<unsigned>((a.cols + 255) / 256), static_cast<unsigned>(a.chunks)),
                       dim3(256), 0, s, a);
  }
  hipLaunchKernelGGL(lora_wgrad_reduce_kernel,
                     dim3(static_cast<unsigned>((static_cast<int64_t>(a.cols) * 32 + 255) / 256)),
                     dim3(256), 0, s, a);
  return check_launch("lora_wgrad");
}

// The partials of the allocation-free entry point: one array per GPU, in the code object's
// device memory (allocated when the module loads on that GPU, held until the process ends).
// Host code never passes `scratch` itself to a kernel (on the host it names a stand-in, not
// the device address): the address comes from hipGetSymbolAddress, once per device.
constexpr int64_t kWgradScratchBytes = TALM_LORA_WGRAD_SCRATCH_BYTES;
static __device__ __align__(256) float scratch[kWgradScratchBytes / sizeof(float)];

constexpr int kMaxDevices = 64;
std::mutex g_scratch_mutex;
float* g_scratch[kMaxDevices] = {};  // device address of `scratch` per device, set once

// The current device's address of `scratch` (looked up on the first call on that device).
int wgrad_scratch(float** out) {
  int device = 0;
  hipError_t err = hipGetDevice(&device);
  if (err != hipSuccess)
    return fail(TALM_EHIP, "lora_wgrad_noalloc: hipGetDevice: %s", hipGetErrorString(err));
  if (device < 0 || device >= kMaxDevices)
    return fail(TALM_EINVAL, "lora_wgrad_noalloc: device %d beyond %d", device, kMaxDevices);
  std::lock_guard<std::mutex> lock(g_scratch_mutex);
  if (!g_scratch[device]) {
    void* ptr = nullptr;
    err = hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch));
    if (err != hipSuccess || !ptr)
      return fail(TALM_EHIP, "lora_wgrad_noalloc: hipGetSymbolAddress: %s",
                  hipGetErrorString(err));
    g_scratch[device] = static_cast<float*>(ptr);
  }
  *out = g_scratch[device];
  return TALM_OK;
}

}  // namespace

TALM_API int talm_lora_wgrad(const uint16_t* x, int64_t ldx, const uint16_t* dy, int64_t ldy,
                             const uint16_t* u, int64_t ldu, const uint16_t* t, int64_t ldt,
                             int64_t n_tokens, int64_t hidden, int32_t n_adapters,
                             int64_t lo0, int64_t seg0, float scaling0, float* da0, float* db0,
                             int64_t lo1, int64_t seg1, float scaling1, float* da1, float* db1,
                             void* workspace, int64_t workspace_bytes, void* stream) {
  WgradArgs a;
  int status = wgrad_args(x, ldx, dy, ldy, u, ldu, t, ldt, n_tokens, hidden, n_adapters, lo0,
                          seg0, scaling0, da0, db0, lo1, seg1, scaling1, da1, db1, a);
  if (status != TALM_OK) return status;
  const int64_t need =
      talm_lora_wgrad_workspace(n_tokens, hidden, seg0, n_adapters > 1 ? seg1 : 0);
  if (workspace_bytes < need)
    return fail(TALM_EINVAL, "lora_wgrad: workspace of %lld bytes, %lld needed",
                (long long)workspace_bytes, (long long)need);
  if (n_tokens == 0) return ok();  // the caller zeroes the gradients of an empty batch
  if (!workspace) return fail(TALM_EINVAL, "lora_wgrad: null pointer");
  a.part = static_cast<float*>(workspace);
  return wgrad_launch(a, as_stream(stream));
}

TALM_API int talm_lora_wgrad_noalloc(const uint16_t* x, int64_t ldx, const uint16_t* dy,
                                     int64_t ldy, const uint16_t* u, int64_t ldu,
                                     const uint16_t* t, int64_t ldt, int64_t n_tokens,
                                     int64_t hidden, int32_t n_adapters, int64_t lo0,
                                     int64_t seg0, float scaling0, float* da0, float* db0,
                                     int64_t lo1, int64_t seg1, float scaling1, float* da1,
                                     float* db1, void* stream) {
  WgradArgs a;
  int status = wgrad_args(x, ldx, dy, ldy, u, ldu, t, ldt, n_tokens, hidden, n_adapters, lo0,
                          seg0, scaling0, da0, db0, lo1, seg1, scaling1, da1, db1, a);
  if (status != TALM_OK) return status;
  const int64_t need =
      talm_lora_wgrad_workspace(n_tokens, hidden, seg0, n_adapters > 1 ? seg1 : 0);
  if (need > kWgradScratchBytes)
    return fail(TALM_EINVAL,
                "lora_wgrad_noalloc: %lld tokens x %d columns need %lld bytes of partials, "
                "above the fixed scratch of %lld bytes (use talm_lora_wgrad with a workspace)",
                (long long)n_tokens, a.cols, (long long)need, (long long)kWgradScratchBytes);
  if (n_tokens == 0) return ok();
  status = wgrad_scratch(&a.part);
  if (status != TALM_OK) return status;
  return wgrad_launch(a, as_stream(stream));
}
