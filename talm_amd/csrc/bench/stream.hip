// Streaming probes for bench.py (not part of libtalm.so): the HBM rate this chip reaches for the
// read / write mixes of the bandwidth-bound kernels, written the way those kernels are (16-byte
// accesses, 64 consecutive 16-byte items per wavefront and iteration, two iterations in flight),
// with ordinary or non-temporal loads and stores (both ordinary, both non-temporal, or
// non-temporal loads with ordinary stores: the kind the package's bandwidth kernels use). Each mix moves R reads and W * WR writes of 16
// bytes per item:
//   (0, 1, 1)  fill                          (1, 1, 1)  copy
//   (1, 1, 4)  the grouped NF4 dequant's mix (a 16-byte read, 64 bytes written)
//   (2, 1, 1)  the SwiGLU forward's mix      (3, 2, 1)  the SwiGLU backward's mix
//   (2, 3, 1)  the add+RMSNorm forward's mix
// The values written are the reads combined with XOR (so that no load is dead).
#include <hip/hip_runtime.h>
#include <stdint.h>

#define TALM_BENCH_API extern "C" __attribute__((visibility("default")))

namespace {

typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

template <bool kNt>
__device__ __forceinline__ u32x4 ld(const u32x4* p) {
  if constexpr (kNt) return __builtin_nontemporal_load(p);
  else return *p;
}

template <bool kNt>
__device__ __forceinline__ void st(u32x4* p, u32x4 v) {
  if constexpr (kNt) __builtin_nontemporal_store(v, p);
  else *p = v;
}

// 16 bytes stored with a buffer store carrying the cache-policy bits `kAux` (gfx950: 1 sc0,
// 2 nt, 16 sc1) at byte offset `off` of the range that starts at `base`.
template <int kAux>
__device__ __forceinline__ void st_aux(void* base, int64_t item, u32x4 v) {
  const __amdgpu_buffer_rsrc_t r = __builtin_amdgcn_make_buffer_rsrc(base, 0, 0x7fffffff, 0x00020000);
  __builtin_amdgcn_raw_buffer_store_b128(v, r, static_cast<uint32_t>(item * 16), 0, kAux);
}

struct StreamArgs {
  const u32x4* src[3];
  u32x4* dst[3];
  int64_t n;  // items (16 bytes of each read stream)
};

// kAux >= 0: the stores are buffer stores with those cache-policy bits (kNtStore unused)
template <int R, int W, int WR, bool kNtLoad, bool kNtStore, int kAux = -1>
__global__ __launch_bounds__(256) void stream_kernel(StreamArgs a) {
  const int lane = threadIdx.x & 63;
  const int64_t wave = (static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x) >> 6;
  const int64_t waves = (static_cast<int64_t>(gridDim.x) * 256) >> 6;
  for (int64_t base = wave * 128; base < a.n; base += waves * 128) {
    u32x4 v[2];
#pragma unroll
    for (int u = 0; u < 2; ++u) {
      const int64_t i = base + u * 64 + lane;
      u32x4 x = {static_cast<uint32_t>(i), 1u, 2u, 3u};
      if (i < a.n) {
#pragma unroll
        for (int r = 0; r < R; ++r) x ^= ld<kNtLoad>(a.src[r] + i);
      }
      v[u] = x;
    }
#pragma unroll
    for (int u = 0; u < 2; ++u) {
      const int64_t i0 = base + u * 64;
      if (i0 + lane >= a.n) continue;
#pragma unroll
      for (int w = 0; w < W; ++w)
#pragma unroll
        for (int j = 0; j < WR; ++j)
          if constexpr (kAux >= 0)
            st_aux<kAux>(a.dst[w], i0 * WR + j * 64 + lane, v[u] ^ static_cast<uint32_t>(j + w));
          else
            st<kNtStore>(a.dst[w] + i0 * WR + j * 64 + lane, v[u] ^ static_cast<uint32_t>(j + w));
    }
  }
}

// nt: 0 ordinary loads and stores, 1 both non-temporal, 2 non-temporal loads, ordinary stores;
// 3 .. 10 non-temporal loads and buffer stores with the cache-policy bits kStoreAux[nt - 3]
constexpr int kStoreAux[8] = {0, 2, 16, 18, 1, 3, 17, 19};
template <int R, int W, int WR>
void launch(const StreamArgs& a, int nt, int grid, hipStream_t s) {
#define TALM_AUX(I)                                                                            \
  if (nt == 3 + I) {                                                                           \
    hipLaunchKernelGGL((stream_kernel<R, W, WR, true, false, kStoreAux[I]>), dim3(grid),       \
                       dim3(256), 0, s, a);                                                    \
    return;                                                                                    \
  }
  TALM_AUX(0) TALM_AUX(1) TALM_AUX(2) TALM_AUX(3) TALM_AUX(4) TALM_AUX(5) TALM_AUX(6) TALM_AUX(7)
#undef TALM_AUX
  if (nt == 1)
    hipLaunchKernelGGL((stream_kernel<R, W, WR, true, true>), dim3(grid), dim3(256), 0, s, a);
  else if (nt == 2)
    hipLaunchKernelGGL((stream_kernel<R, W, WR, true, false>), dim3(grid), dim3(256), 0, s, a);
  else
    hipLaunchKernelGGL((stream_kernel<R, W, WR, false, false>), dim3(grid), dim3(256), 0, s, a);
}

}  // namespace

// Runs one mix (nt: the access kinds, see launch) over n_items 16-byte items (a multiple of 128; every pointer 16-byte aligned, the
// read streams n_items * 16 bytes each, the write streams n_items * 16 * wr bytes each). grid 0:
// one 128-item group per wavefront (no grid-stride loop). Returns 0, 1 for an unsupported mix or
// bad arguments, 2 for a launch error.
TALM_BENCH_API int talm_bench_stream(int reads, int writes, int wr, int nt, const void* s0,
                                     const void* s1, const void* s2, void* d0, void* d1, void* d2,
                                     int64_t n_items, int grid, void* stream) {
  if (n_items <= 0 || n_items % 128 || grid < 0 || nt < 0 || nt > 10) return 1;
  for (int w = 0; nt >= 3 && w < writes; ++w)
    if (n_items * 16 * wr > 0x7fffffff) return 1;  // buffer-store offsets are 32-bit
  StreamArgs a{};
  const void* src[3] = {s0, s1, s2};
  void* dst[3] = {d0, d1, d2};
  for (int r = 0; r < reads; ++r) {
    if (!src[r] || reinterpret_cast<uintptr_t>(src[r]) % 16) return 1;
    a.src[r] = static_cast<const u32x4*>(src[r]);
  }
  for (int w = 0; w < writes; ++w) {
    if (!dst[w] || reinterpret_cast<uintptr_t>(dst[w]) % 16) return 1;
    a.dst[w] = static_cast<u32x4*>(dst[w]);
  }
  a.n = n_items;
  const int64_t groups = n_items / 128;  // 128 items per wavefront and iteration
  const int g = grid > 0 ? grid : static_cast<int>((groups + 3) / 4);
  const hipStream_t s = reinterpret_cast<hipStream_t>(stream);
  const int t = nt;
  if (reads == 0 && writes == 1 && wr == 1) launch<0, 1, 1>(a, t, g, s);
  else if (reads == 1 && writes == 1 && wr == 1) launch<1, 1, 1>(a, t, g, s);
  else if (reads == 1 && writes == 1 && wr == 4) launch<1, 1, 4>(a, t, g, s);
  else if (reads == 2 && writes == 1 && wr == 1) launch<2, 1, 1>(a, t, g, s);
  else if (reads == 3 && writes == 2 && wr == 1) launch<3, 2, 1>(a, t, g, s);
  else if (reads == 2 && writes == 3 && wr == 1) launch<2, 3, 1>(a, t, g, s);
  else return 1;
  return hipGetLastError() == hipSuccess ? 0 : 2;
}
