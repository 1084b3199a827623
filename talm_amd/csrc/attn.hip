// Variable-length causal attention with grouped KV heads (GQA), forward and backward, on gfx950
// fp16 MFMA with fp32 softmax statistics.
//
// Packed tokens: sequence s holds rows [cu[s], cu[s+1]); row i of a sequence attends to keys
// j <= i of the same sequence. q [N, Hq, D], k / v [N, Hkv, D] (any token / head strides, unit
// column stride), query head h reads KV head h / (Hq / Hkv); D = 128. This replaces the
// reference's per-KV-head memory-efficient attention launches (solution/unpad.py:199-294), whose
// semantics are per-row causal SDPA (solution/unpad.py:121-134).
//
// The forward is a flash-attention pass per (sequence, 32-row query tile, query heads of one KV
// head), its key tiles of 64 split between two groups of wavefronts and streamed with
// direct-to-LDS loads. Scores are computed transposed, S^T = K Q^T (v_mfma_f32_32x32x16_f16), so
// each lane owns one query row (its accumulator column): the online max / sum and the output
// rescale are per-lane scalars. The exponentiated scores are already in the B-operand layout of
// O^T = V^T P^T: the reduction over keys takes the accumulator's key order as its k-slot order,
// and V^T is read in that same order from the row-major V tile with transposing LDS reads. The
// row statistics are kept in base 2 (scores times scale * log2 e); lse is written in natural-log
// units, [Hq, N].
//
// The backward (FlashAttention-2's recurrences: P = exp(S - lse), dV = P^T dO, dP = dO V^T,
// dS = P (dP - rowsum(dO O)), dQ = scale dS K, dK = scale dS^T Q) runs as
//   attn_bwd_dot    Dd[h][t] = sum_d dO O (fp32);
//   attn_bwd_dq     per (sequence, query head, 128-row query tile): the forward's loop with
//                   dP^T = V dO^T next to S^T, and dQ^T += K^T dS^T with K^T read transposed
//                   from the K tile;
//   attn_bwd_dkdv   per (sequence, query head, 128-key tile): each lane owns a key (S and dP
//                   computed untransposed, so keys are accumulator columns), looping over
//                   64-row query tiles: dV^T += dO^T P and dK^T += Q^T dS with Q^T and dO^T read
//                   transposed from the row-major tiles; fp32 partials per query head;
//   attn_bwd_reduce the partials of a KV head's query heads summed in head order (deterministic)
//                   into dK, dV fp16.
// The dQ and dK / dV bodies run in one launch.
#include "mfma_tile.h"

namespace talm {
namespace {

typedef uint16_t half4_t __attribute__((ext_vector_type(4)));
// 16-byte register chunks as a native vector: HIP's uint4 struct is copied with memcpy, which
// keeps a register array of them on the stack when it is stored whole into LDS.
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

constexpr int kD = 128;         // head dim
constexpr int kKeys = 64;       // keys per tile
constexpr int kKS = kD + 8;     // row stride (halfs) of a [keys][D] tile in LDS
constexpr float kLn2 = 0.693147180559945309f;

__device__ __forceinline__ float exp2_(float x) { return __builtin_amdgcn_exp2f(x); }

struct FwdArgs {
  const uint16_t* q;
  int64_t q_tok, q_head;
  const uint16_t* k;
  int64_t k_tok, k_head;
  const uint16_t* v;
  int64_t v_tok, v_head;
  const int32_t* cu;
  int group;          // query heads per KV head
  int head_chunks;    // workgroups per KV head (group / heads per workgroup)
  int n_tiles;        // 32-row query tiles per sequence (of the longest)
  float scale_log2;   // softmax scale * log2(e)
  uint16_t* out;
  int64_t o_tok, o_head;
  float* lse;         // [Hq, n_tokens]
  int64_t n_tokens;
};

// K and V tiles of the forward in LDS: [64 keys][128 d] fp16 without padding, 16 chunks of 16
// bytes per row, chunk c of row r at position c ^ tile_swz(r). The direct-to-LDS loads write
// 1 KiB per wavefront instruction contiguously (4 rows). gfx950's LDS serves a 16-byte read in
// phases of 16 lanes over 64 four-byte banks (measured with the SQ_LDS_BANK_CONFLICT counter), so
// a 256-byte row spans every bank once and a chunk's banks depend on its position alone. The
// 4-bit key makes both reads conflict-free: the 16-byte row reads of the S = K Q^T operand
// (16 consecutive rows of one chunk per phase: the key takes 16 distinct values on them) and the
// transposing 8-byte reads (4 consecutive rows x 4 adjacent chunks per 32-lane phase: with
// r = 4a + t and c = 4b + u the position is 4 (b ^ t) + (u ^ a % 4), 16 distinct values).
constexpr int kTileBytes = kKeys * kD * 2;  // 16 KiB

__device__ __forceinline__ int tile_swz(int row) { return ((row & 3) << 2) | ((row >> 2) & 3); }
__device__ __forceinline__ int tile_chunk(int row, int chunk) { return row * 16 + (chunk ^ tile_swz(row)); }

// ds_read_b64_tr_b16 (gfx950): within each 16-lane group, lane i receives element e (0..3) from
// row 4 e + i / 4 of the 16 x 4 matrix formed by the four halves at each lane's address, column
// i % 4 (checked on the GPU with an in-bounds probe). With lane j pointing at row K0 + j / 4,
// columns D0 + 4 (j % 4) of a row-major [keys][d] tile, lane i gets keys K0 .. K0 + 3 of column
// D0 + i: the transpose of 4 x 16 elements.
// A 32 x 16 operand of v_mfma_f32_32x32x16_f16 read transposed from a swizzled [rows][128]
// tile: A[m][k] = tile[row0 + key(k)][col0 + m], lane l holding m = l % 32 and k-slots
// 8 (l / 32) .. + 7, whose rows follow the accumulator order of the 32-row blocks: slots
// 8 hh + e hold rows row0 + 4 hh + e (e < 4) and row0 + 8 + 4 hh + e - 4 (e >= 4).
// The same operand's two halves issued as inline assembly. The compiler does not track these
// reads: it adds no wait for the direct-to-LDS loads in flight before them (it cannot tell that
// those write the other ring slot, and would wait for all of them), and the caller waits for the
// results itself with lgkm_wait8 before using them.
__device__ __forceinline__ half4_t read_tr_untracked(const unsigned char* lds) {
  const uint32_t addr = static_cast<uint32_t>(reinterpret_cast<uintptr_t>(
      (__attribute__((address_space(3))) const unsigned char*)(lds)));
  half4_t r;
  asm volatile("ds_read_b64_tr_b16 %0, %1" : "=v"(r) : "v"(addr));
  return r;
}
__device__ __forceinline__ void read_tr_operand_untracked(const unsigned char* tile, int row0,
                                                          int col0, int lane, half4_t& lo,
                                                          half4_t& hi) {
  const int g = lane >> 4, i = lane & 15, hh = g >> 1;
  const int col = col0 + 16 * (g & 1) + 4 * (i & 3);
  const int row = row0 + 4 * hh + (i >> 2);
  lo = read_tr_untracked(tile + tile_chunk(row, col >> 3) * 16 + (col & 7) * 2);
  hi = read_tr_untracked(tile + tile_chunk(row + 8, col >> 3) * 16 + (col & 7) * 2);
}
typedef float f32x4_t __attribute__((ext_vector_type(4)));
__device__ __forceinline__ f32x4_t read_f4_untracked(const float* lds) {
  const uint32_t addr = static_cast<uint32_t>(reinterpret_cast<uintptr_t>(
      (__attribute__((address_space(3))) const float*)(lds)));
  f32x4_t r;
  asm volatile("ds_read_b128 %0, %1" : "=v"(r) : "v"(addr));
  return r;
}
__device__ __forceinline__ void lgkm_wait_f4(f32x4_t (&r)[4]) {
  asm volatile("s_waitcnt lgkmcnt(0)" : "+v"(r[0]), "+v"(r[1]), "+v"(r[2]), "+v"(r[3]));
}
// Wait until every LDS (and scalar-memory) operation of the wavefront has returned; the eight
// registers count as rewritten here, so no copy of them is made before the wait.
__device__ __forceinline__ void lgkm_wait8(half4_t (&r)[8]) {
  asm volatile("s_waitcnt lgkmcnt(0)"
               : "+v"(r[0]), "+v"(r[1]), "+v"(r[2]), "+v"(r[3]), "+v"(r[4]), "+v"(r[5]),
                 "+v"(r[6]), "+v"(r[7]));
}

// 16 bytes stored at byte offset `off` of the range that starts at `base`. A row past the
// sequence gets off = kOob, past the descriptor's range, and the hardware drops the store: the
// epilogues issue all their LDS reads and then all their stores, with no branch per row (a branch
// holding a read and its store made each read wait for the one before).
__device__ __forceinline__ __amdgpu_buffer_rsrc_t store_rsrc(void* base) {
  return __builtin_amdgcn_make_buffer_rsrc(base, 0, 0x7fffffff, 0x00020000);
}
__device__ __forceinline__ void store16(__amdgpu_buffer_rsrc_t r, uint32_t off, u32x4 v) {
  __builtin_amdgcn_raw_buffer_store_b128(v, r, off, 0, 0);
}

// One [64][128] tile from global rows base[r * ld + c] (r < rows_valid, else zeros) into `dst`
// with direct-to-LDS 16-byte loads: block b (rows 4 b .. 4 b + 3) by wavefront b % W.
template <int W>
__device__ __forceinline__ void dma_tile(const uint16_t* base, int64_t ld, int rows_valid,
                                         unsigned char* dst, int wave, int lane) {
  const __amdgpu_buffer_rsrc_t rsrc = buffer_rsrc(base);
  const int row_in = lane >> 4, pos = lane & 15;
#pragma unroll
  for (int it = 0; it < (kKeys / 4 + W - 1) / W; ++it) {
    const int b = wave + it * W;
    if (b >= kKeys / 4) break;
    const int row = 4 * b + row_in;
    const int chunk = pos ^ tile_swz(row);
    const uint32_t off = row < rows_valid ? static_cast<uint32_t>((row * ld + chunk * 8) * 2) : kOob;
    dma16(rsrc, dst + b * 1024, off);
  }
}

// Forward, one workgroup per (sequence, 32-row query tile, W query heads of one KV head), with
// S groups of W wavefronts: group g takes the key tiles g, g + S, g + 2 S, ..., one wavefront per
// head, so the serial key loop of a long query tile is S times shorter (its length, not the
// chip, bounds the kernel at these sequence lengths); the groups' partial results are merged
// through LDS at the end. The K / V tiles of the KV head are loaded once for the W heads.
// Scores are computed transposed, S^T = K Q^T, so each lane owns one query row: the online
// max / sum and the output rescale are per-lane scalars, and the exponentiated scores are
// already the B operand of O^T = V^T P^T, whose A operand is read transposed from the row-major
// V tile. Two LDS slots per group: the next tiles' loads fly during this step's math.
template <int W, int S>
__global__ __launch_bounds__(64 * W * S) void attn_fwd_kernel(FwdArgs a) {
  constexpr int kStepBytes = S * 2 * kTileBytes;        // the K and V tiles of one step
  constexpr int kRing = 2 * kStepBytes;
  constexpr int kMerge = (S - 1) * W * (64 * 64 * 4 + 64 * 8);  // partial O, m, l per wavefront
  constexpr int kStage = W * 32 * kKS * 2;              // fp16 output rows per head
  constexpr int kSmem = kRing > kMerge + kStage ? kRing : kMerge + kStage;
  __shared__ __attribute__((aligned(1024))) unsigned char smem[kSmem];

  const int seq = blockIdx.z;
  const int kvh = static_cast<int>(blockIdx.y) / a.head_chunks;
  const int hc = static_cast<int>(blockIdx.y) % a.head_chunks;
  const int tile = a.n_tiles - 1 - static_cast<int>(blockIdx.x);  // longest tiles first
  const int s0 = a.cu[seq], len = a.cu[seq + 1] - s0;
  const int q0 = tile * 32;
  if (q0 >= len) return;  // the whole workgroup, before any barrier
  const int tid = threadIdx.x, lane = tid & 63;
  // the wavefront index in a scalar register: everything the branches, loop bounds and the
  // direct-to-LDS addresses derive from it stays wavefront-uniform
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int hw = wave % W, grp = wave / W;  // head slot, key group
  const int hh = lane >> 5, l32 = lane & 31;
  const int head = kvh * a.group + hc * W + hw;

  // this lane's query row and its Q fragments (the B operand: k-slots d = 16 s + 8 hh .. + 8)
  const int qrow = q0 + l32;
  const int qr = min(qrow, len - 1);
  half8_t qf[kD / 16];
  {
    const uint16_t* qp = a.q + static_cast<int64_t>(s0 + qr) * a.q_tok + head * a.q_head + 8 * hh;
#pragma unroll
    for (int s = 0; s < kD / 16; ++s) qf[s] = *reinterpret_cast<const half8_t*>(qp + 16 * s);
  }

  const int kend = min(len, q0 + 32);  // keys any row of this tile can see
  const int n_kt = (kend + kKeys - 1) / kKeys;
  const int n_steps = (n_kt + S - 1) / S;
  const int key_lim = min(qrow, len - 1);  // the last key this lane's row may see
  const uint16_t* kbase = a.k + static_cast<int64_t>(s0) * a.k_tok + kvh * a.k_head;
  const uint16_t* vbase = a.v + static_cast<int64_t>(s0) * a.v_tok + kvh * a.v_head;
  // the group's W wavefronts load its tile: 16 blocks of 1 KiB per K or V tile, block b by
  // wavefront b % W of the group
  auto slot_of = [&](int step) { return smem + (step & 1) * kStepBytes + grp * 2 * kTileBytes; };
  auto issue = [&](int step) {  // the group's tile of `step`, if it exists
    const int kt = step * S + grp;
    if (kt >= n_kt) return;
    unsigned char* slot = slot_of(step);
    const int r0 = kt * kKeys;
    dma_tile<W>(kbase + static_cast<int64_t>(r0) * a.k_tok, a.k_tok, len - r0, slot, hw, lane);
    dma_tile<W>(vbase + static_cast<int64_t>(r0) * a.v_tok, a.v_tok, len - r0, slot + kTileBytes,
                hw, lane);
  };

  f32x16 o[kD / 32];
#pragma unroll
  for (int j = 0; j < kD / 32; ++j)
#pragma unroll
    for (int v = 0; v < 16; ++v) o[j][v] = 0.f;
  // m: the reference maximum of the row's scaled scores (log2 units), raised only when the
  // row's maximum exceeds it by more than kLazy (the exponentials stay <= 2^kLazy, far inside
  // fp16, and the final O / l uses the same reference: exact up to rounding)
  constexpr float kLazy = 8.f;
  float m = -INFINITY, lsum = 0.f;
  const float c = a.scale_log2;

  issue(0);
  for (int step = 0; step < n_steps; ++step) {
    const int kt = step * S + grp;
    // this group's tile of the step has landed (the next step's loads are not issued yet)
    wait_vmcnt<0>();
    lds_barrier();  // every group's tile has; everyone is done with step - 1 (its slots are free)
    issue(step + 1);
    if (kt >= n_kt) continue;  // this group has no tile left (barriers stay matched: no return)
    const unsigned char* ks = slot_of(step);
    const unsigned char* vs = ks + kTileBytes;
    const uint4* k16 = reinterpret_cast<const uint4*>(ks);
    const int k0 = kt * kKeys;
    // S^T for keys k0 + 32 b + (8 (v / 4) + 4 hh + v % 4), this lane's query column
    f32x16 st[2];
#pragma unroll
    for (int b = 0; b < 2; ++b) {
#pragma unroll
      for (int v = 0; v < 16; ++v) st[b][v] = 0.f;
      // the block's 8 operand reads issued before its MFMAs
      half8_t ka[kD / 16];
#pragma unroll
      for (int s = 0; s < kD / 16; ++s)
        ka[s] = __builtin_bit_cast(half8_t, k16[tile_chunk(32 * b + l32, 2 * s + hh)]);
      __builtin_amdgcn_sched_group_barrier(0x100, 8, 0);
      __builtin_amdgcn_sched_group_barrier(0x008, 8, 0);
#pragma unroll
      for (int s = 0; s < kD / 16; ++s)
        st[b] = __builtin_amdgcn_mfma_f32_32x32x16_f16(ka[s], qf[s], st[b], 0, 0, 0);
    }
    // causal / length mask only on a tile that reaches past the first query row of the
    // workgroup or past the sequence: a real (uniform) branch; the empty volatile asm keeps the
    // compiler from turning it into selects executed on every tile
    if (k0 + kKeys - 1 > q0 || k0 + kKeys > len) {
      asm volatile("");
#pragma unroll
      for (int b = 0; b < 2; ++b)
#pragma unroll
        for (int v = 0; v < 16; ++v) {
          const int key = k0 + 32 * b + 8 * (v >> 2) + 4 * hh + (v & 3);
          st[b][v] = key > key_lim ? -INFINITY : st[b][v];
        }
    }
    float mt = -INFINITY;
#pragma unroll
    for (int b = 0; b < 2; ++b)
#pragma unroll
      for (int v = 0; v < 16; ++v) mt = fmaxf(mt, st[b][v]);
    mt = c * fmaxf(mt, __shfl_xor(mt, 32, kWave));
    const bool grow = mt > m + kLazy;
    if (__ballot(grow)) {  // some row's maximum moved: rescale those rows
      asm volatile("");
      const float m_new = grow ? mt : m;
      const float alpha = exp2_(m - m_new);  // 0 on the first tile (m = -inf), 1 if unchanged
      m = m_new;
      lsum *= alpha;
#pragma unroll
      for (int j = 0; j < kD / 32; ++j)
#pragma unroll
        for (int v = 0; v < 16; ++v) o[j][v] *= alpha;
    }
    // V^T operands of the four 16-key groups (b, h), read untracked two groups at a time
    half4_t vt[2][8];
    auto read_v = [&](int grp16, int buf) {
#pragma unroll
      for (int j = 0; j < kD / 32; ++j)
        read_tr_operand_untracked(vs, 16 * grp16, 32 * j, lane, vt[buf][2 * j], vt[buf][2 * j + 1]);
    };
    read_v(0, 0);
    float ps = 0.f;
#pragma unroll
    for (int b = 0; b < 2; ++b)
#pragma unroll
      for (int v = 0; v < 16; ++v) {
        const float pv = exp2_(__builtin_fmaf(st[b][v], c, -m));
        st[b][v] = pv;
        ps += pv;
      }
    lsum += ps;
    // O^T[d][q] += V^T[d][key] P^T[key][q], 16 keys per step in the accumulator's key order
#pragma unroll
    for (int g16 = 0; g16 < 4; ++g16) {
      const int b = g16 >> 1, h = g16 & 1, buf = g16 & 1;
      lgkm_wait8(vt[buf]);  // group g16's reads have returned
      if (g16 < 3) read_v(g16 + 1, buf ^ 1);  // the next group's fly during these MFMAs
      half8_t pb;
#pragma unroll
      for (int e = 0; e < 8; ++e) pb[e] = static_cast<_Float16>(st[b][8 * h + e]);
#pragma unroll
      for (int j = 0; j < kD / 32; ++j)
        o[j] = __builtin_amdgcn_mfma_f32_32x32x16_f16(
            __builtin_bit_cast(half8_t, __builtin_shufflevector(vt[buf][2 * j], vt[buf][2 * j + 1],
                                                                0, 1, 2, 3, 4, 5, 6, 7)),
            pb, o[j], 0, 0, 0);
    }
  }
  lsum += __shfl_xor(lsum, 32, kWave);  // the row's sum over both halves of the lanes

  // merge the groups into group 0: each other group's wavefront leaves its (m, l, O) in LDS
  __syncthreads();  // every wavefront is done with the tiles
  float* part_o = reinterpret_cast<float*>(smem);                        // [group-1][W][64][64]
  float* part_ml = part_o + (S - 1) * W * 64 * 64;                       // [group-1][W][64][2]
  if (grp > 0) {
    float* po = part_o + ((grp - 1) * W + hw) * 64 * 64;
#pragma unroll
    for (int j = 0; j < kD / 32; ++j)
#pragma unroll
      for (int v = 0; v < 16; ++v) po[(16 * j + v) * 64 + lane] = o[j][v];
    float* pml = part_ml + ((grp - 1) * W + hw) * 64 * 2;
    pml[2 * lane] = m;
    pml[2 * lane + 1] = lsum;
  }
  __syncthreads();
  if (grp > 0) return;  // no barrier follows for the other groups
#pragma unroll
  for (int g = 1; g < S; ++g) {
    const float* po = part_o + ((g - 1) * W + hw) * 64 * 64;
    const float* pml = part_ml + ((g - 1) * W + hw) * 64 * 2;
    const float m2 = pml[2 * lane], l2 = pml[2 * lane + 1];
    const float m_new = fmaxf(m, m2);
    const float a1 = m == -INFINITY ? 0.f : exp2_(m - m_new);
    const float a2 = m2 == -INFINITY ? 0.f : exp2_(m2 - m_new);
    m = m_new;
    lsum = lsum * a1 + l2 * a2;
#pragma unroll
    for (int j = 0; j < kD / 32; ++j)
#pragma unroll
      for (int v = 0; v < 16; ++v) o[j][v] = o[j][v] * a1 + po[(16 * j + v) * 64 + lane] * a2;
  }

  // O = O^T / l through LDS: each head stages its 32 rows x D, then 16-byte row stores
  const float inv = 1.f / lsum;
  uint16_t* os = reinterpret_cast<uint16_t*>(smem + kMerge) + hw * 32 * kKS;
#pragma unroll
  for (int j = 0; j < kD / 32; ++j)
#pragma unroll
    for (int g = 0; g < 4; ++g) {
      const int d0 = 32 * j + 8 * g + 4 * hh;
      uint2 w;
      w.x = pack2(o[j][4 * g] * inv, o[j][4 * g + 1] * inv);
      w.y = pack2(o[j][4 * g + 2] * inv, o[j][4 * g + 3] * inv);
      *reinterpret_cast<uint2*>(&os[l32 * kKS + d0]) = w;
    }
  if (hh == 0 && qrow < len)
    a.lse[static_cast<int64_t>(head) * a.n_tokens + s0 + qrow] = (m + __log2f(lsum)) * kLn2;
  // the wavefront reads back its own staging rows (the other groups have exited: no workgroup
  // barrier): its LDS writes complete first, and the compiler keeps the order
  asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
  constexpr int kOut = (32 * kD / 8) / 64;  // 16-byte chunks per lane
  u32x4 ov[kOut];
#pragma unroll
  for (int it = 0; it < kOut; ++it) {
    const int cc16 = it * 64 + lane, r = cc16 / (kD / 8), cc = cc16 % (kD / 8);
    ov[it] = *reinterpret_cast<const u32x4*>(&os[r * kKS + 8 * cc]);
  }
  const __amdgpu_buffer_rsrc_t ors =
      store_rsrc(a.out + static_cast<int64_t>(s0 + q0) * a.o_tok + head * a.o_head);
#pragma unroll
  for (int it = 0; it < kOut; ++it) {
    const int cc16 = it * 64 + lane, r = cc16 / (kD / 8), cc = cc16 % (kD / 8);
    store16(ors, q0 + r < len ? static_cast<uint32_t>((r * a.o_tok + 8 * cc) * 2) : kOob, ov[it]);
  }
}

// ------------------------------------------------------------------------------------------
// Backward
// ------------------------------------------------------------------------------------------
struct BwdArgs {
  const uint16_t* q;
  int64_t q_tok, q_head;
  const uint16_t* k;
  int64_t k_tok, k_head;
  const uint16_t* v;
  int64_t v_tok, v_head;
  const uint16_t* o;
  int64_t o_tok, o_head;
  const uint16_t* dout;
  int64_t do_tok, do_head;
  const float* lse;    // [Hq, n_tokens], natural log
  const int32_t* cu;
  int group, n_q_heads, n_kv_heads;
  int n_tiles;         // tiles per sequence (of the longest)
  float scale, scale_log2;
  int64_t n_tokens;
  float* dd;           // [Hq, n_tokens]: rowsum(dO * O)
  float* lse2;         // [Hq, n_tokens]: lse in base-2 units (lse * log2 e)
  float* dk_part;      // [Hq, n_tokens, D] fp32
  float* dv_part;      // [Hq, n_tokens, D] fp32
  uint16_t* dq;
  int64_t dq_tok, dq_head;
  uint16_t* dk;
  int64_t dk_tok, dk_head;
  uint16_t* dv;
  int64_t dv_tok, dv_head;
  // the rotary embedding's backward folded into the outputs (null: none): cos / sin fp32
  // [n_tokens][cs_tok], and every 128-wide head of dq and dk is rotated back on its (d, d + 64)
  // pairs: dx1 = dy1 c1 + dy2 s2, dx2 = dy2 c2 - dy1 s1 (solution/rope.py:145-157)
  const float* cos;
  const float* sin;
  int64_t cs_tok;
};

// The rotary embedding's backward on one (d, d + 64) pair of four columns each: x = dy at
// columns d .. d + 3, y at d + 64 .. d + 67, of the token whose cos / sin rows are cr / sr.
__device__ __forceinline__ void rope_back4(float (&x)[4], float (&y)[4], const float* cr,
                                          const float* sr, int d) {
  const float4 c1 = *reinterpret_cast<const float4*>(cr + d);
  const float4 c2 = *reinterpret_cast<const float4*>(cr + d + kD / 2);
  const float4 s1 = *reinterpret_cast<const float4*>(sr + d);
  const float4 s2 = *reinterpret_cast<const float4*>(sr + d + kD / 2);
  const float cc1[4] = {c1.x, c1.y, c1.z, c1.w}, cc2[4] = {c2.x, c2.y, c2.z, c2.w};
  const float ss1[4] = {s1.x, s1.y, s1.z, s1.w}, ss2[4] = {s2.x, s2.y, s2.z, s2.w};
#pragma unroll
  for (int e = 0; e < 4; ++e) {
    const float a = x[e], b = y[e];
    x[e] = a * cc1[e] + b * ss2[e];
    y[e] = b * cc2[e] - a * ss1[e];
  }
}

// Dd[h][t] = sum_d dO[t][h][d] * O[t][h][d] and lse2[h][t] = lse[h][t] log2 e (the exponent offset
// both backward bodies subtract): 16 lanes per (token, head), 8 columns each.
__global__ __launch_bounds__(256) void attn_bwd_dot_kernel(BwdArgs a) {
  const int64_t row = (static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x) >> 4;  // t * Hq + h
  const int sub = threadIdx.x & 15;
  const int64_t rows = a.n_tokens * a.n_q_heads;
  const int64_t r = row < rows ? row : rows - 1;
  const int64_t t = r / a.n_q_heads;
  const int h = static_cast<int>(r % a.n_q_heads);
  const u32x4 x = *reinterpret_cast<const u32x4*>(a.o + t * a.o_tok + h * a.o_head + 8 * sub);
  const u32x4 y = *reinterpret_cast<const u32x4*>(a.dout + t * a.do_tok + h * a.do_head + 8 * sub);
  float acc = lo_f(x.x) * lo_f(y.x) + hi_f(x.x) * hi_f(y.x) + lo_f(x.y) * lo_f(y.y) +
              hi_f(x.y) * hi_f(y.y) + lo_f(x.z) * lo_f(y.z) + hi_f(x.z) * hi_f(y.z) +
              lo_f(x.w) * lo_f(y.w) + hi_f(x.w) * hi_f(y.w);
#pragma unroll
  for (int off = 8; off >= 1; off >>= 1) acc += __shfl_xor(acc, off, 16);
  if (sub == 0 && row < rows) {
    const int64_t i = static_cast<int64_t>(h) * a.n_tokens + t;
    a.dd[i] = acc;
    a.lse2[i] = a.lse[i] * 1.44269504088896341f;
  }
}

// The dQ and dK / dV bodies below stream their tiles with the forward's direct-to-LDS loads into
// the swizzled [64][128] layout (tile_chunk): 16-byte row reads give the operands taken row by
// row, and the transposing reads (read_tr_operand_untracked) give K^T, Q^T and dO^T straight
// from the same tiles, so no transposed copy is written. A two-slot ring, one tile ahead; the
// loop is unrolled by two so every slot address is a compile-time offset.
constexpr int kBwdSlot = 2 * kTileBytes + 2048;  // two tiles (+ per-wavefront lse / Dd rows: dK / dV)
constexpr int kBwdLds = 2 * kBwdSlot;

// Runs body(tile, slot) for tile = 0 .. n - 1 in ring slot tile & 1, after issue(tile + 1, slot)
// put the next tile in flight into the other slot. Each tile's loads are waited for (this
// wavefront's, then the barrier for everyone's) right before its body, and the barrier also
// retires the slot the previous body read. Unrolled by two, so every slot address is a
// compile-time offset. (A third slot, two tiles in flight, measured slower.)
template <class Issue, class Body>
__device__ __forceinline__ void ring2(int n, Issue&& issue, Body&& body) {
  issue(0, 0);
  for (int t = 0; t < n; t += 2) {
    wait_vmcnt<0>();
    lds_barrier();
    if (t + 1 < n) issue(t + 1, 1);
    body(t, 0);
    if (t + 1 >= n) break;
    wait_vmcnt<0>();
    lds_barrier();
    if (t + 2 < n) issue(t + 2, 0);
    body(t + 1, 1);
  }
}

// dQ: the forward's structure, one query row per lane (S^T = K Q^T, dP^T = V dO^T, then
// dQ^T += K^T dS^T with K^T read transposed from the K tile); `tile` is the 32W-row query tile.
template <int W>
__device__ __forceinline__ void attn_bwd_dq(const BwdArgs& a, int tile, unsigned char* smem) {
  constexpr int kRows = 32 * W;
  const int seq = blockIdx.y, head = blockIdx.x;
  const int s0 = a.cu[seq], len = a.cu[seq + 1] - s0;
  const int q0 = tile * kRows;
  if (q0 >= len) return;
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int hh = lane >> 5, l32 = lane & 31;
  const int kvh = head / a.group;
  const int qrow = q0 + 32 * wave + l32;
  const int qr = min(qrow, len - 1);
  half8_t qf[kD / 16], df[kD / 16];
  {
    const uint16_t* qp = a.q + static_cast<int64_t>(s0 + qr) * a.q_tok + head * a.q_head + 8 * hh;
    const uint16_t* dp = a.dout + static_cast<int64_t>(s0 + qr) * a.do_tok + head * a.do_head + 8 * hh;
#pragma unroll
    for (int s = 0; s < kD / 16; ++s) {
      qf[s] = *reinterpret_cast<const half8_t*>(qp + 16 * s);
      df[s] = *reinterpret_cast<const half8_t*>(dp + 16 * s);
    }
  }
  const float lse2 = a.lse2[static_cast<int64_t>(head) * a.n_tokens + s0 + qr];
  const float ddr = a.dd[static_cast<int64_t>(head) * a.n_tokens + s0 + qr];
  const int wq0 = q0 + 32 * wave;  // the wavefront's first query row

  const int kend = min(len, q0 + kRows);
  const int n_kt = (kend + kKeys - 1) / kKeys;
  const uint16_t* kbase = a.k + static_cast<int64_t>(s0) * a.k_tok + kvh * a.k_head;
  const uint16_t* vbase = a.v + static_cast<int64_t>(s0) * a.v_tok + kvh * a.v_head;
  auto issue = [&](int kt, int slot) {
    unsigned char* dst = smem + slot * kBwdSlot;
    const int r0 = kt * kKeys;
    dma_tile<W>(kbase + static_cast<int64_t>(r0) * a.k_tok, a.k_tok, len - r0, dst, wave, lane);
    dma_tile<W>(vbase + static_cast<int64_t>(r0) * a.v_tok, a.v_tok, len - r0, dst + kTileBytes,
                wave, lane);
  };

  f32x16 acc[kD / 32];
#pragma unroll
  for (int j = 0; j < kD / 32; ++j)
#pragma unroll
    for (int v = 0; v < 16; ++v) acc[j][v] = 0.f;

  auto body = [&](int kt, int slot) {
    const unsigned char* ks = smem + slot * kBwdSlot;
    const uint4* k16 = reinterpret_cast<const uint4*>(ks);
    const uint4* v16 = reinterpret_cast<const uint4*>(ks + kTileBytes);
    const int k0 = kt * kKeys;
    if (k0 > wq0 + 31) return;  // every key of the tile is after every row of the wavefront
    f32x16 st[2], dpt[2];
#pragma unroll
    for (int b = 0; b < 2; ++b) {
#pragma unroll
      for (int v = 0; v < 16; ++v) st[b][v] = dpt[b][v] = 0.f;
      // the block's 16 operand reads issued before its MFMAs
      half8_t ka[kD / 16], va[kD / 16];
#pragma unroll
      for (int s = 0; s < kD / 16; ++s) {
        ka[s] = __builtin_bit_cast(half8_t, k16[tile_chunk(32 * b + l32, 2 * s + hh)]);
        va[s] = __builtin_bit_cast(half8_t, v16[tile_chunk(32 * b + l32, 2 * s + hh)]);
      }
      __builtin_amdgcn_sched_group_barrier(0x100, 16, 0);
      __builtin_amdgcn_sched_group_barrier(0x008, 16, 0);
#pragma unroll
      for (int s = 0; s < kD / 16; ++s) {
        st[b] = __builtin_amdgcn_mfma_f32_32x32x16_f16(ka[s], qf[s], st[b], 0, 0, 0);
        dpt[b] = __builtin_amdgcn_mfma_f32_32x32x16_f16(va[s], df[s], dpt[b], 0, 0, 0);
      }
    }
    // K^T operands of the first 16-key group, read while the scores are turned into dS^T
    half4_t kt_[2][8];
    auto read_k = [&](int g16, int buf) {
#pragma unroll
      for (int j = 0; j < kD / 32; ++j)
        read_tr_operand_untracked(ks, 16 * g16, 32 * j, lane, kt_[buf][2 * j], kt_[buf][2 * j + 1]);
    };
    read_k(0, 0);
    // dS^T = P^T (dP^T - Dd), P^T = exp2(S^T scale log2e - lse2); 0 where masked (only on a tile
    // that reaches past the wavefront's first row or past the sequence: a uniform branch)
    if (k0 + kKeys - 1 > wq0 || k0 + kKeys > len) {
      asm volatile("");
#pragma unroll
      for (int b = 0; b < 2; ++b)
#pragma unroll
        for (int v = 0; v < 16; ++v) {
          const int key = k0 + 32 * b + 8 * (v >> 2) + 4 * hh + (v & 3);
          const float p = (key <= qrow && key < len) ? exp2_(st[b][v] * a.scale_log2 - lse2) : 0.f;
          st[b][v] = p * (dpt[b][v] - ddr);
        }
    } else {
#pragma unroll
      for (int b = 0; b < 2; ++b)
#pragma unroll
        for (int v = 0; v < 16; ++v)
          st[b][v] = exp2_(st[b][v] * a.scale_log2 - lse2) * (dpt[b][v] - ddr);
    }
    // dQ^T[d][q] += K^T[d][key] dS^T[key][q], 16 keys per step in the accumulator's key order
#pragma unroll
    for (int g16 = 0; g16 < 4; ++g16) {
      const int b = g16 >> 1, h = g16 & 1, buf = g16 & 1;
      lgkm_wait8(kt_[buf]);
      if (g16 < 3) read_k(g16 + 1, buf ^ 1);
      half8_t sb;
#pragma unroll
      for (int e = 0; e < 8; ++e) sb[e] = static_cast<_Float16>(st[b][8 * h + e]);
#pragma unroll
      for (int j = 0; j < kD / 32; ++j)
        acc[j] = __builtin_amdgcn_mfma_f32_32x32x16_f16(
            __builtin_bit_cast(half8_t, __builtin_shufflevector(kt_[buf][2 * j], kt_[buf][2 * j + 1],
                                                                0, 1, 2, 3, 4, 5, 6, 7)),
            sb, acc[j], 0, 0, 0);
    }
  };
  ring2(n_kt, issue, body);

  __syncthreads();  // every wavefront is done with the ring: it becomes the output staging
  uint16_t* os = reinterpret_cast<uint16_t*>(smem) + wave * 32 * kKS;
  // dQ = scale * the accumulated sum; rows d = 32 j + 8 g + 4 hh + e of block j pair with the
  // same (g, e) of block j + 2 (d + 64): with cos / sin the rotary backward is applied in fp32
  // here, before the one rounding to fp16 (row qr: rows past the sequence are not stored)
  float dqv[kD / 32][16];
#pragma unroll
  for (int j = 0; j < kD / 32; ++j)
#pragma unroll
    for (int v = 0; v < 16; ++v) dqv[j][v] = acc[j][v] * a.scale;
  if (a.cos) {
    const float* cr = a.cos + static_cast<int64_t>(s0 + qr) * a.cs_tok;
    const float* sr = a.sin + static_cast<int64_t>(s0 + qr) * a.cs_tok;
#pragma unroll
    for (int j = 0; j < kD / 64; ++j)
#pragma unroll
      for (int g = 0; g < 4; ++g) {
        float x[4], y[4];
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          x[e] = dqv[j][4 * g + e];
          y[e] = dqv[j + 2][4 * g + e];
        }
        rope_back4(x, y, cr, sr, 32 * j + 8 * g + 4 * hh);
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          dqv[j][4 * g + e] = x[e];
          dqv[j + 2][4 * g + e] = y[e];
        }
      }
  }
#pragma unroll
  for (int j = 0; j < kD / 32; ++j)
#pragma unroll
    for (int g = 0; g < 4; ++g) {
      const int d0 = 32 * j + 8 * g + 4 * hh;
      uint2 w;
      w.x = pack2(dqv[j][4 * g], dqv[j][4 * g + 1]);
      w.y = pack2(dqv[j][4 * g + 2], dqv[j][4 * g + 3]);
      *reinterpret_cast<uint2*>(&os[l32 * kKS + d0]) = w;
    }
  // the wavefront reads back its own staging rows: its LDS writes complete first
  asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
  constexpr int kOut = (32 * kD / 8) / 64;  // 16-byte chunks per lane
  u32x4 ov[kOut];
#pragma unroll
  for (int it = 0; it < kOut; ++it) {
    const int c = it * 64 + lane, r = c / (kD / 8), cc = c % (kD / 8);
    ov[it] = *reinterpret_cast<const u32x4*>(&os[r * kKS + 8 * cc]);
  }
  const __amdgpu_buffer_rsrc_t ors =
      store_rsrc(a.dq + static_cast<int64_t>(s0 + wq0) * a.dq_tok + head * a.dq_head);
#pragma unroll
  for (int it = 0; it < kOut; ++it) {
    const int c = it * 64 + lane, r = c / (kD / 8), cc = c % (kD / 8);
    store16(ors, wq0 + r < len ? static_cast<uint32_t>((r * a.dq_tok + 8 * cc) * 2) : kOob, ov[it]);
  }
}

// dK / dV partials of one query head; `tile` is the 32W-key tile, each lane owns one key (S and
// dP untransposed: keys are accumulator columns), looping over 64-row query tiles: dV^T += dO^T P
// and dK^T += Q^T dS with Q^T and dO^T read transposed from the row-major tiles. Each slot holds
// the Q tile, the dO tile, then each wavefront's copy of the tile's 64 lse and 64 Dd values.
template <int W>
__device__ __forceinline__ void attn_bwd_dkdv(const BwdArgs& a, int tile, unsigned char* smem) {
  constexpr int kCols = 32 * W;  // keys per workgroup
  constexpr int kRowsT = kKeys;  // query rows per tile
  const int seq = blockIdx.y, head = blockIdx.x;
  const int s0 = a.cu[seq], len = a.cu[seq + 1] - s0;
  const int k0 = tile * kCols;
  if (k0 >= len) return;
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int hh = lane >> 5, l32 = lane & 31;
  const int kvh = head / a.group;
  const int key = k0 + 32 * wave + l32;
  const int kr_ = min(key, len - 1);
  const int wk0 = k0 + 32 * wave;  // the wavefront's first key
  half8_t kf[kD / 16], vf[kD / 16];
  {
    const uint16_t* kp = a.k + static_cast<int64_t>(s0 + kr_) * a.k_tok + kvh * a.k_head + 8 * hh;
    const uint16_t* vp = a.v + static_cast<int64_t>(s0 + kr_) * a.v_tok + kvh * a.v_head + 8 * hh;
#pragma unroll
    for (int s = 0; s < kD / 16; ++s) {
      kf[s] = *reinterpret_cast<const half8_t*>(kp + 16 * s);
      vf[s] = *reinterpret_cast<const half8_t*>(vp + 16 * s);
    }
  }
  const int qstart = k0;  // causal: rows below k0 see no key here (k0 is a multiple of 64)
  const int n_qt = (len - qstart + kRowsT - 1) / kRowsT;
  const uint16_t* qbase = a.q + static_cast<int64_t>(s0) * a.q_tok + head * a.q_head;
  const uint16_t* dbase = a.dout + static_cast<int64_t>(s0) * a.do_tok + head * a.do_head;
  const __amdgpu_buffer_rsrc_t lrs = __builtin_amdgcn_make_buffer_rsrc(
      a.lse2 + static_cast<int64_t>(head) * a.n_tokens + s0, 0, len * 4, 0x00020000);
  const __amdgpu_buffer_rsrc_t drs = __builtin_amdgcn_make_buffer_rsrc(
      a.dd + static_cast<int64_t>(head) * a.n_tokens + s0, 0, len * 4, 0x00020000);
  auto issue = [&](int qt, int slot) {
    unsigned char* dst = smem + slot * kBwdSlot;
    const int r0 = qstart + qt * kRowsT;
    dma_tile<W>(qbase + static_cast<int64_t>(r0) * a.q_tok, a.q_tok, len - r0, dst, wave, lane);
    dma_tile<W>(dbase + static_cast<int64_t>(r0) * a.do_tok, a.do_tok, len - r0, dst + kTileBytes,
                wave, lane);
    // the tile's 64 lse and 64 Dd values, one 4-byte load per lane (rows past len read 0), into
    // this wavefront's own copy (read by it alone)
    const uint32_t off = static_cast<uint32_t>((r0 + lane) * 4);
    unsigned char* st = dst + 2 * kTileBytes + wave * 512;
    __builtin_amdgcn_raw_ptr_buffer_load_lds(lrs, (lds_ptr_t)(st), 4, off, 0, 0, 0);
    __builtin_amdgcn_raw_ptr_buffer_load_lds(drs, (lds_ptr_t)(st + 256), 4, off, 0, 0, 0);
  };

  f32x16 dka[kD / 32], dva[kD / 32];
#pragma unroll
  for (int j = 0; j < kD / 32; ++j)
#pragma unroll
    for (int v = 0; v < 16; ++v) dka[j][v] = dva[j][v] = 0.f;

  auto body = [&](int qt, int slot) {
    const unsigned char* qs = smem + slot * kBwdSlot;
    const unsigned char* ds = qs + kTileBytes;
    const uint4* q16 = reinterpret_cast<const uint4*>(qs);
    const uint4* d16 = reinterpret_cast<const uint4*>(ds);
    const float* ls = reinterpret_cast<const float*>(qs + 2 * kTileBytes + wave * 512);
    const float* dds = ls + 64;
    const int r0 = qstart + qt * kRowsT;
    if (r0 + kRowsT - 1 < wk0) return;  // every row of the tile is before every key of the wavefront
    // S[q][key], dP[q][key] for the tile's 32-row blocks: rows q = 32 blk + 8 (v / 4) + 4 hh + v % 4
    f32x16 sc[2], dp[2];
#pragma unroll
    for (int blk = 0; blk < 2; ++blk) {
#pragma unroll
      for (int v = 0; v < 16; ++v) sc[blk][v] = dp[blk][v] = 0.f;
      // the block's 16 operand reads issued before its MFMAs (one LDS round trip, not one per
      // MFMA pair)
      half8_t qa[kD / 16], da[kD / 16];
#pragma unroll
      for (int s = 0; s < kD / 16; ++s) {
        qa[s] = __builtin_bit_cast(half8_t, q16[tile_chunk(32 * blk + l32, 2 * s + hh)]);
        da[s] = __builtin_bit_cast(half8_t, d16[tile_chunk(32 * blk + l32, 2 * s + hh)]);
      }
      __builtin_amdgcn_sched_group_barrier(0x100, 16, 0);  // the 16 LDS reads first
      __builtin_amdgcn_sched_group_barrier(0x008, 16, 0);  // then the 16 MFMAs
#pragma unroll
      for (int s = 0; s < kD / 16; ++s) {
        sc[blk] = __builtin_amdgcn_mfma_f32_32x32x16_f16(qa[s], kf[s], sc[blk], 0, 0, 0);
        dp[blk] = __builtin_amdgcn_mfma_f32_32x32x16_f16(da[s], vf[s], dp[blk], 0, 0, 0);
      }
    }
    // dO^T and Q^T operands of the first 16-row group, read while P and dS are formed
    half4_t tr[2][2][8];  // [buf][dO, Q][4 j x 2 halves]
    auto read_t = [&](int g16, int buf) {
#pragma unroll
      for (int j = 0; j < kD / 32; ++j) {
        read_tr_operand_untracked(ds, 16 * g16, 32 * j, lane, tr[buf][0][2 * j], tr[buf][0][2 * j + 1]);
        read_tr_operand_untracked(qs, 16 * g16, 32 * j, lane, tr[buf][1][2 * j], tr[buf][1][2 * j + 1]);
      }
    };
    read_t(0, 0);
    // P and dS, 0 where masked (query row < key or past the sequence, key past the sequence: only
    // on a tile with a row before the wavefront's last key or reaching past the sequence, a
    // uniform branch); the rows' lse and Dd come from the slot with untracked reads as well
    const bool edge = r0 < wk0 + 31 || r0 + kRowsT > len || wk0 + 32 > len;
#pragma unroll
    for (int blk = 0; blk < 2; ++blk) {
      f32x4_t l4[4], d4[4];
#pragma unroll
      for (int g = 0; g < 4; ++g) {
        l4[g] = read_f4_untracked(&ls[32 * blk + 8 * g + 4 * hh]);
        d4[g] = read_f4_untracked(&dds[32 * blk + 8 * g + 4 * hh]);
      }
      lgkm_wait_f4(l4);
      lgkm_wait_f4(d4);
      if (edge) {
        asm volatile("");
#pragma unroll
        for (int g = 0; g < 4; ++g)
#pragma unroll
          for (int e = 0; e < 4; ++e) {
            const int v = 4 * g + e, q = r0 + 32 * blk + 8 * g + 4 * hh + e;
            const bool valid = q >= key && q < len && key < len;
            const float p = valid ? exp2_(sc[blk][v] * a.scale_log2 - l4[g][e]) : 0.f;
            sc[blk][v] = p;
            dp[blk][v] = p * (dp[blk][v] - d4[g][e]);
          }
      } else {
#pragma unroll
        for (int g = 0; g < 4; ++g)
#pragma unroll
          for (int e = 0; e < 4; ++e) {
            const int v = 4 * g + e;
            const float p = exp2_(sc[blk][v] * a.scale_log2 - l4[g][e]);
            sc[blk][v] = p;
            dp[blk][v] = p * (dp[blk][v] - d4[g][e]);
          }
      }
    }
    // dV^T[d][key] += dO^T[d][q] P[q][key];  dK^T[d][key] += Q^T[d][q] dS[q][key]
#pragma unroll
    for (int g16 = 0; g16 < 4; ++g16) {
      const int blk = g16 >> 1, h = g16 & 1, buf = g16 & 1;
      lgkm_wait8(tr[buf][0]);
      lgkm_wait8(tr[buf][1]);
      if (g16 < 3) read_t(g16 + 1, buf ^ 1);
      half8_t pb, sb;
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        pb[e] = static_cast<_Float16>(sc[blk][8 * h + e]);
        sb[e] = static_cast<_Float16>(dp[blk][8 * h + e]);
      }
#pragma unroll
      for (int j = 0; j < kD / 32; ++j) {
        dva[j] = __builtin_amdgcn_mfma_f32_32x32x16_f16(
            __builtin_bit_cast(half8_t, __builtin_shufflevector(tr[buf][0][2 * j], tr[buf][0][2 * j + 1],
                                                                0, 1, 2, 3, 4, 5, 6, 7)),
            pb, dva[j], 0, 0, 0);
        dka[j] = __builtin_amdgcn_mfma_f32_32x32x16_f16(
            __builtin_bit_cast(half8_t, __builtin_shufflevector(tr[buf][1][2 * j], tr[buf][1][2 * j + 1],
                                                                0, 1, 2, 3, 4, 5, 6, 7)),
            sb, dka[j], 0, 0, 0);
      }
    }
  };
  ring2(n_qt, issue, body);

  // fp32 partials [head][token][d]. A lane holds its key's column of the accumulators (rows
  // d = 32 j + 8 (v / 4) + 4 hh + v % 4): stored as they are, every store instruction would touch
  // 64 rows 16 bytes each. Each wavefront stages its 32 keys x 128 columns in its own part of the
  // ring instead (rows of 132 floats: the 16 lanes of a write phase meet 16 distinct bank groups)
  // and stores whole rows, two per instruction.
  __syncthreads();  // every wavefront is done with the ring
  constexpr int kStageLd = kD + 4;
  float* stage = reinterpret_cast<float*>(smem) + wave * 32 * kStageLd;
  auto store_rows = [&](const f32x16 (&acc)[kD / 32], float mul, float* part) {
#pragma unroll
    for (int j = 0; j < kD / 32; ++j)
#pragma unroll
      for (int g = 0; g < 4; ++g)
        *reinterpret_cast<float4*>(&stage[l32 * kStageLd + 32 * j + 8 * g + 4 * hh]) =
            make_float4(acc[j][4 * g] * mul, acc[j][4 * g + 1] * mul, acc[j][4 * g + 2] * mul,
                        acc[j][4 * g + 3] * mul);
    // the wavefront reads back its own rows: its LDS writes complete first
    asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
    u32x4 x[16];
#pragma unroll
    for (int it = 0; it < 16; ++it) {
      const int r = 2 * it + (lane >> 5), c = lane & 31;
      x[it] = *reinterpret_cast<const u32x4*>(&stage[r * kStageLd + 4 * c]);
    }
    const __amdgpu_buffer_rsrc_t prs =
        store_rsrc(part + (static_cast<int64_t>(head) * a.n_tokens + s0 + wk0) * kD);
#pragma unroll
    for (int it = 0; it < 16; ++it) {
      const int r = 2 * it + (lane >> 5), c = lane & 31;
      store16(prs, wk0 + r < len ? static_cast<uint32_t>((r * kD + 4 * c) * 4) : kOob, x[it]);
    }
    // the next call overwrites the rows: every read above has returned first
    asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
  };
  store_rows(dka, a.scale, a.dk_part);
  store_rows(dva, 1.f, a.dv_part);
}

// dQ and the dK / dV partials in one launch: they read the same inputs and write disjoint
// outputs, and each alone has fewer workgroups than the chip has CUs (its time is its longest
// workgroup's), so side by side they share the chip. The grid is (query head, sequence,
// 2 x rank): every sequence's longest work is dispatched first, rank by rank, so the workgroups
// that wait for a free CU are the shortest ones. Rank r of a sequence of n tiles is dQ query tile
// n - 1 - r (even z) and dK / dV key tile r (odd z); ranks past n exit at once.
template <int W>
__global__ __launch_bounds__(64 * W, 1) void attn_bwd_kernel(BwdArgs a) {
  __shared__ __attribute__((aligned(1024))) unsigned char smem[kBwdLds];
  const int rank = static_cast<int>(blockIdx.z) >> 1;
  const int len = a.cu[blockIdx.y + 1] - a.cu[blockIdx.y];
  const int n_own = (len + 32 * W - 1) / (32 * W);
  if (rank >= n_own) return;  // the whole workgroup, before any barrier
  if ((blockIdx.z & 1) == 0)
    attn_bwd_dq<W>(a, n_own - 1 - rank, smem);
  else
    attn_bwd_dkdv<W>(a, rank, smem);
}

// dK / dV fp16 [token][kv head][d] = sum over the KV head's query heads, in head order. A
// thread takes 4 columns d and, with the rotary backward (a.cos), also their partners d + 64:
// dK's pairs are rotated back in fp32 before the rounding.
// dK / dV partials of the KV head's query heads at columns d_c .. d_c + 3 (c < C), summed in head
// order; every load of eight heads is in flight before their adds.
template <int C>
__device__ __forceinline__ void sum_heads4(const BwdArgs& a, int kvh, int64_t t, const int (&d)[C],
                                           float (&k)[C][4], float (&v)[C][4]) {
#pragma unroll
  for (int c = 0; c < C; ++c)
#pragma unroll
    for (int e = 0; e < 4; ++e) k[c][e] = v[c][e] = 0.f;
  const int64_t head_stride = a.n_tokens * kD;
  const int64_t off0 = (static_cast<int64_t>(kvh) * a.group * a.n_tokens + t) * kD;
  for (int g0 = 0; g0 < a.group; g0 += 8) {
    float4 xk[8][C], xv[8][C];
#pragma unroll
    for (int j = 0; j < 8; ++j)
#pragma unroll
      for (int c = 0; c < C; ++c) {
        const int64_t off = off0 + (g0 + j < a.group ? g0 + j : 0) * head_stride + d[c];
        xk[j][c] = *reinterpret_cast<const float4*>(a.dk_part + off);
        xv[j][c] = *reinterpret_cast<const float4*>(a.dv_part + off);
      }
    // selects, not a branch: a branch between the loads and the adds would let the compiler sink
    // each load to its add, one round trip per head (heads past the group add +0)
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      const bool in = g0 + j < a.group;
#pragma unroll
      for (int c = 0; c < C; ++c) {
        k[c][0] += in ? xk[j][c].x : 0.f; k[c][1] += in ? xk[j][c].y : 0.f;
        k[c][2] += in ? xk[j][c].z : 0.f; k[c][3] += in ? xk[j][c].w : 0.f;
        v[c][0] += in ? xv[j][c].x : 0.f; v[c][1] += in ? xv[j][c].y : 0.f;
        v[c][2] += in ? xv[j][c].z : 0.f; v[c][3] += in ? xv[j][c].w : 0.f;
      }
    }
  }
}

template <bool kRope>
__global__ __launch_bounds__(256) void attn_bwd_reduce_kernel(BwdArgs a) {
  constexpr int kGroups = kRope ? kD / 8 : kD / 4;  // threads per (token, KV head)
  const int64_t idx = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x;
  const int64_t total = a.n_tokens * a.n_kv_heads * kGroups;
  if (idx >= total) return;
  const int c4 = static_cast<int>(idx % kGroups);
  const int64_t tk = idx / kGroups;
  const int kvh = static_cast<int>(tk % a.n_kv_heads);
  const int64_t t = tk / a.n_kv_heads;
  uint16_t* dk = a.dk + t * a.dk_tok + kvh * a.dk_head;
  uint16_t* dv = a.dv + t * a.dv_tok + kvh * a.dv_head;
  constexpr int C = kRope ? 2 : 1;  // with the rotary backward: the (d, d + 64) column pairs
  int d[C];
  d[0] = 4 * c4;
  if constexpr (kRope) d[C - 1] = 4 * c4 + kD / 2;
  float kk[C][4], vv[C][4];
  sum_heads4<C>(a, kvh, t, d, kk, vv);
  float(&k1)[4] = kk[0];
  float(&v1)[4] = vv[0];
  if constexpr (kRope) {
    float(&k2)[4] = kk[C - 1];
    float(&v2)[4] = vv[C - 1];
    rope_back4(k1, k2, a.cos + t * a.cs_tok, a.sin + t * a.cs_tok, 4 * c4);
    *reinterpret_cast<uint2*>(dk + 4 * c4 + kD / 2) = make_uint2(pack2(k2[0], k2[1]), pack2(k2[2], k2[3]));
    *reinterpret_cast<uint2*>(dv + 4 * c4 + kD / 2) = make_uint2(pack2(v2[0], v2[1]), pack2(v2[2], v2[3]));
  }
  *reinterpret_cast<uint2*>(dk + 4 * c4) = make_uint2(pack2(k1[0], k1[1]), pack2(k1[2], k1[3]));
  *reinterpret_cast<uint2*>(dv + 4 * c4) = make_uint2(pack2(v1[0], v1[1]), pack2(v1[2], v1[3]));
}

}  // namespace
}  // namespace talm

using namespace talm;

TALM_API int talm_attn_fwd(const uint16_t* q, int64_t q_stride_tok, int64_t q_stride_head,
                           const uint16_t* k, int64_t k_stride_tok, int64_t k_stride_head,
                           const uint16_t* v, int64_t v_stride_tok, int64_t v_stride_head,
                           const int32_t* cu_seqlens, int32_t n_seqs, int32_t max_seqlen,
                           int64_t n_tokens, int32_t n_q_heads, int32_t n_kv_heads,
                           int32_t head_dim, float scale, uint16_t* out, int64_t o_stride_tok,
                           int64_t o_stride_head, float* lse, void* stream) {
  if (head_dim != kD)
    return fail(TALM_EINVAL, "attn_fwd: head_dim %d (only %d)", head_dim, kD);
  if (n_seqs < 0 || max_seqlen < 0 || n_tokens < 0 || n_q_heads < 1 || n_kv_heads < 1 ||
      n_q_heads % n_kv_heads || n_tokens >= (int64_t{1} << 31))
    return fail(TALM_EINVAL, "attn_fwd: bad shape (seqs %d, max_seqlen %d, tokens %lld, heads %d/%d)",
                n_seqs, max_seqlen, (long long)n_tokens, n_q_heads, n_kv_heads);
  for (int64_t s : {q_stride_tok, q_stride_head, k_stride_tok, k_stride_head, v_stride_tok,
                    v_stride_head, o_stride_tok, o_stride_head})
    if (s < 0 || s % 8)
      return fail(TALM_EINVAL, "attn_fwd: strides must be non-negative multiples of 8 elements");
  if (k_stride_tok >= (int64_t{1} << 23) || v_stride_tok >= (int64_t{1} << 23) ||
      o_stride_tok >= (int64_t{1} << 23))
    return fail(TALM_EINVAL, "attn_fwd: k / v / out token strides must be below 2^23 elements");
  if (n_seqs == 0 || max_seqlen == 0 || n_tokens == 0) return ok();
  if (!q || !k || !v || !cu_seqlens || !out || !lse) return fail(TALM_EINVAL, "attn_fwd: null pointer");
  if (!aligned(q, 16) || !aligned(k, 16) || !aligned(v, 16) || !aligned(out, 16))
    return fail(TALM_EINVAL, "attn_fwd: q, k, v and out must be 16-byte aligned");
  const int group = n_q_heads / n_kv_heads;
  // query heads per workgroup: the largest of 4, 3, 2, 1 that divides the group; two groups
  // of wavefronts split each workgroup's key tiles
  int w = 1;
  for (int cand : {4, 3, 2})
    if (group % cand == 0) { w = cand; break; }
  FwdArgs a{};
  a.q = q; a.q_tok = q_stride_tok; a.q_head = q_stride_head;
  a.k = k; a.k_tok = k_stride_tok; a.k_head = k_stride_head;
  a.v = v; a.v_tok = v_stride_tok; a.v_head = v_stride_head;
  a.cu = cu_seqlens; a.group = group; a.head_chunks = group / w;
  a.n_tiles = (max_seqlen + 31) / 32;
  a.scale_log2 = scale * 1.44269504088896341f;
  a.out = out; a.o_tok = o_stride_tok; a.o_head = o_stride_head;
  a.lse = lse; a.n_tokens = n_tokens;
  const dim3 grid(static_cast<unsigned>(a.n_tiles), static_cast<unsigned>(n_kv_heads * a.head_chunks),
                  static_cast<unsigned>(n_seqs));
  const hipStream_t s = as_stream(stream);
  switch (w) {
    case 4: hipLaunchKernelGGL((attn_fwd_kernel<4, 2>), grid, dim3(512), 0, s, a); break;
    case 3: hipLaunchKernelGGL((attn_fwd_kernel<3, 2>), grid, dim3(384), 0, s, a); break;
    case 2: hipLaunchKernelGGL((attn_fwd_kernel<2, 2>), grid, dim3(256), 0, s, a); break;
    default: hipLaunchKernelGGL((attn_fwd_kernel<1, 2>), grid, dim3(128), 0, s, a); break;
  }
  return check_launch("attn_fwd");
}

TALM_API int64_t talm_attn_bwd_workspace(int64_t n_tokens, int32_t n_q_heads) {
  if (n_tokens < 0 || n_q_heads < 1) return -1;
  // Dd and lse2 [Hq, N] f32, then the dK and dV partials [Hq, N, D] f32 each (256-byte aligned
  // parts)
  const int64_t dd = (n_tokens * n_q_heads * 4 + 255) / 256 * 256;
  return 2 * dd + 2 * n_tokens * n_q_heads * kD * 4;
}

namespace talm {
namespace {

int attn_bwd_impl(const uint16_t* q, int64_t q_stride_tok, int64_t q_stride_head,
                  const uint16_t* k, int64_t k_stride_tok, int64_t k_stride_head,
                  const uint16_t* v, int64_t v_stride_tok, int64_t v_stride_head,
                  const uint16_t* out, int64_t o_stride_tok, int64_t o_stride_head,
                  const uint16_t* dout, int64_t do_stride_tok, int64_t do_stride_head,
                  const float* lse, const int32_t* cu_seqlens, int32_t n_seqs,
                  int32_t max_seqlen, int64_t n_tokens, int32_t n_q_heads, int32_t n_kv_heads,
                  int32_t head_dim, float scale, const float* cos, const float* sin,
                  int64_t cs_stride, uint16_t* dq, int64_t dq_stride_tok,
                  int64_t dq_stride_head, uint16_t* dk, int64_t dk_stride_tok,
                  int64_t dk_stride_head, uint16_t* dv, int64_t dv_stride_tok,
                  int64_t dv_stride_head, void* workspace, int64_t workspace_bytes,
                  void* stream) {
  if (head_dim != kD)
    return fail(TALM_EINVAL, "attn_bwd: head_dim %d (only %d)", head_dim, kD);
  if (n_seqs < 0 || max_seqlen < 0 || n_tokens < 0 || n_q_heads < 1 || n_kv_heads < 1 ||
      n_q_heads % n_kv_heads || n_tokens >= (int64_t{1} << 31))
    return fail(TALM_EINVAL, "attn_bwd: bad shape (seqs %d, max_seqlen %d, tokens %lld, heads %d/%d)",
                n_seqs, max_seqlen, (long long)n_tokens, n_q_heads, n_kv_heads);
  for (int64_t s : {q_stride_tok, q_stride_head, k_stride_tok, k_stride_head, v_stride_tok,
                    v_stride_head, o_stride_tok, o_stride_head, do_stride_tok, do_stride_head,
                    dq_stride_tok, dq_stride_head, dk_stride_tok, dk_stride_head, dv_stride_tok,
                    dv_stride_head})
    if (s < 0 || s % 8)
      return fail(TALM_EINVAL, "attn_bwd: strides must be non-negative multiples of 8 elements");
  if (q_stride_tok >= (int64_t{1} << 23) || k_stride_tok >= (int64_t{1} << 23) ||
      v_stride_tok >= (int64_t{1} << 23) || do_stride_tok >= (int64_t{1} << 23) ||
      dq_stride_tok >= (int64_t{1} << 23))
    return fail(TALM_EINVAL, "attn_bwd: q / k / v / dout / dq token strides must be below 2^23 elements");
  if (n_seqs > 65535 || (max_seqlen + 127) / 128 > 32767)
    return fail(TALM_EINVAL, "attn_bwd: at most 65535 sequences of at most 4194176 tokens");
  const int64_t need = talm_attn_bwd_workspace(n_tokens, n_q_heads);
  if (workspace_bytes < need)
    return fail(TALM_EINVAL, "attn_bwd: workspace of %lld bytes, %lld needed",
                (long long)workspace_bytes, (long long)need);
  const bool rope = cos != nullptr || sin != nullptr;
  if (rope && (cs_stride < kD || cs_stride % 4 || cs_stride >= (int64_t{1} << 24)))
    return fail(TALM_EINVAL, "attn_bwd: cos / sin row stride %lld (at least %d, a multiple of 4)",
                (long long)cs_stride, kD);
  if (n_seqs == 0 || max_seqlen == 0 || n_tokens == 0) return ok();
  if (!q || !k || !v || !out || !dout || !lse || !cu_seqlens || !dq || !dk || !dv || !workspace)
    return fail(TALM_EINVAL, "attn_bwd: null pointer");
  if (rope && (!cos || !sin || !aligned(cos, 16) || !aligned(sin, 16)))
    return fail(TALM_EINVAL, "attn_bwd: cos and sin both given, 16-byte aligned");
  if (!aligned(q, 16) || !aligned(k, 16) || !aligned(v, 16) || !aligned(out, 16) ||
      !aligned(dout, 16) || !aligned(dq, 16) || !aligned(dk, 8) || !aligned(dv, 8) ||
      !aligned(workspace, 256))
    return fail(TALM_EINVAL, "attn_bwd: operands 16-byte aligned (dk, dv 8), workspace 256");
  constexpr int W = 4;
  BwdArgs a{};
  a.q = q; a.q_tok = q_stride_tok; a.q_head = q_stride_head;
  a.k = k; a.k_tok = k_stride_tok; a.k_head = k_stride_head;
  a.v = v; a.v_tok = v_stride_tok; a.v_head = v_stride_head;
  a.o = out; a.o_tok = o_stride_tok; a.o_head = o_stride_head;
  a.dout = dout; a.do_tok = do_stride_tok; a.do_head = do_stride_head;
  a.lse = lse; a.cu = cu_seqlens;
  a.group = n_q_heads / n_kv_heads; a.n_q_heads = n_q_heads; a.n_kv_heads = n_kv_heads;
  a.n_tiles = (max_seqlen + 32 * W - 1) / (32 * W);
  a.scale = scale; a.scale_log2 = scale * 1.44269504088896341f;
  a.n_tokens = n_tokens;
  unsigned char* ws = static_cast<unsigned char*>(workspace);
  const int64_t dd_bytes = (n_tokens * n_q_heads * 4 + 255) / 256 * 256;
  a.dd = reinterpret_cast<float*>(ws);
  a.lse2 = reinterpret_cast<float*>(ws + dd_bytes);
  a.dk_part = reinterpret_cast<float*>(ws + 2 * dd_bytes);
  a.dv_part = a.dk_part + n_tokens * n_q_heads * kD;
  a.dq = dq; a.dq_tok = dq_stride_tok; a.dq_head = dq_stride_head;
  a.dk = dk; a.dk_tok = dk_stride_tok; a.dk_head = dk_stride_head;
  a.dv = dv; a.dv_tok = dv_stride_tok; a.dv_head = dv_stride_head;
  a.cos = rope ? cos : nullptr; a.sin = rope ? sin : nullptr; a.cs_tok = cs_stride;
  const hipStream_t s = as_stream(stream);
  const int64_t rows = n_tokens * n_q_heads;
  hipLaunchKernelGGL(attn_bwd_dot_kernel, dim3(static_cast<unsigned>((rows * 16 + 255) / 256)),
                     dim3(256), 0, s, a);
  const dim3 grid(static_cast<unsigned>(n_q_heads), static_cast<unsigned>(n_seqs),
                  static_cast<unsigned>(2 * a.n_tiles));
  hipLaunchKernelGGL((attn_bwd_kernel<W>), grid, dim3(64 * W), 0, s, a);
  const int64_t red = n_tokens * n_kv_heads * (rope ? kD / 8 : kD / 4);
  if (rope)
    hipLaunchKernelGGL(attn_bwd_reduce_kernel<true>, dim3(static_cast<unsigned>((red + 255) / 256)),
                       dim3(256), 0, s, a);
  else
    hipLaunchKernelGGL(attn_bwd_reduce_kernel<false>, dim3(static_cast<unsigned>((red + 255) / 256)),
                       dim3(256), 0, s, a);
  return check_launch("attn_bwd");
}

}  // namespace
}  // namespace talm

TALM_API int talm_attn_bwd(const uint16_t* q, int64_t q_stride_tok, int64_t q_stride_head,
                           const uint16_t* k, int64_t k_stride_tok, int64_t k_stride_head,
                           const uint16_t* v, int64_t v_stride_tok, int64_t v_stride_head,
                           const uint16_t* out, int64_t o_stride_tok, int64_t o_stride_head,
                           const uint16_t* dout, int64_t do_stride_tok, int64_t do_stride_head,
                           const float* lse, const int32_t* cu_seqlens, int32_t n_seqs,
                           int32_t max_seqlen, int64_t n_tokens, int32_t n_q_heads,
                           int32_t n_kv_heads, int32_t head_dim, float scale, uint16_t* dq,
                           int64_t dq_stride_tok, int64_t dq_stride_head, uint16_t* dk,
                           int64_t dk_stride_tok, int64_t dk_stride_head, uint16_t* dv,
                           int64_t dv_stride_tok, int64_t dv_stride_head, void* workspace,
                           int64_t workspace_bytes, void* stream) {
  return attn_bwd_impl(q, q_stride_tok, q_stride_head, k, k_stride_tok, k_stride_head, v,
                       v_stride_tok, v_stride_head, out, o_stride_tok, o_stride_head, dout,
                       do_stride_tok, do_stride_head, lse, cu_seqlens, n_seqs, max_seqlen,
                       n_tokens, n_q_heads, n_kv_heads, head_dim, scale, nullptr, nullptr, 0, dq,
                       dq_stride_tok, dq_stride_head, dk, dk_stride_tok, dk_stride_head, dv,
                       dv_stride_tok, dv_stride_head, workspace, workspace_bytes, stream);
}

TALM_API int talm_attn_bwd_rope(const uint16_t* q, int64_t q_stride_tok, int64_t q_stride_head,
                                const uint16_t* k, int64_t k_stride_tok, int64_t k_stride_head,
                                const uint16_t* v, int64_t v_stride_tok, int64_t v_stride_head,
                                const uint16_t* out, int64_t o_stride_tok, int64_t o_stride_head,
                                const uint16_t* dout, int64_t do_stride_tok,
                                int64_t do_stride_head, const float* lse,
                                const int32_t* cu_seqlens, int32_t n_seqs, int32_t max_seqlen,
                                int64_t n_tokens, int32_t n_q_heads, int32_t n_kv_heads,
                                int32_t head_dim, float scale, const float* cos, const float* sin,
                                int64_t cs_stride, uint16_t* dq, int64_t dq_stride_tok,
                                int64_t dq_stride_head, uint16_t* dk, int64_t dk_stride_tok,
                                int64_t dk_stride_head, uint16_t* dv, int64_t dv_stride_tok,
                                int64_t dv_stride_head, void* workspace, int64_t workspace_bytes,
                                void* stream) {
  if (!cos || !sin) return fail(TALM_EINVAL, "attn_bwd_rope: cos and sin are required");
  return attn_bwd_impl(q, q_stride_tok, q_stride_head, k, k_stride_tok, k_stride_head, v,
                       v_stride_tok, v_stride_head, out, o_stride_tok, o_stride_head, dout,
                       do_stride_tok, do_stride_head, lse, cu_seqlens, n_seqs, max_seqlen,
                       n_tokens, n_q_heads, n_kv_heads, head_dim, scale, cos, sin, cs_stride, dq,
                       dq_stride_tok, dq_stride_head, dk, dk_stride_tok, dk_stride_head, dv,
                       dv_stride_tok, dv_stride_head, workspace, workspace_bytes, stream);
}
