// Split-K fp16 GEMM on gfx950 for the decoder's long-reduction products: out [M, N] fp16 =
// A [M, K] B [N, K]^T with fp32 accumulation, both operands k-contiguous (the forward's product
// form). It serves the MLP's down projection (K = 8960) and its input gradient on the transposed
// gate|up weight (K = 17920) at training token counts, where the output has few 256 x 256 tiles
// (36 at 1300 tokens) and each needs a long reduction: the library's kernels reach about 0.6 of
// MFMA peak there.
//
// Each workgroup computes one 256 x 256 output tile over one part of K with the tile core of
// mfma_tile.h (8 wavefronts of 128 x 64, 64-deep steps through a two-slot buffer-load-to-LDS
// ring), and writes it as an fp32 partial; the K parts are chosen so that the tiles x parts fill
// the chip in one round. A second kernel sums the partials of each element in part order
// (deterministic) and rounds to fp16 once.
#include "mfma_tile.h"
#include "splitk.h"

namespace talm {
namespace {

using SplitShape = TileShape<256, 256, 64, 2, 2, 4>;

struct SplitArgs {
  const uint16_t* A;
  int64_t lda;
  const uint16_t* B;
  int64_t ldb;
  float* part;  // [parts][M][N]
  int M, N, K;
  int steps_per_part;
  int n_mtiles, n_ntiles, n_tiles;
};

template <class S>
__global__ __launch_bounds__(S::kThreads, S::kPerCu) void gemm_splitk_kernel(SplitArgs a) {
  __shared__ __attribute__((aligned(1024))) unsigned char smem[S::kRing];
  // row tiles vary fastest, then column tiles, then K parts: the tiles in flight on one XCD share
  // the B panel of their column tile and K part in its L2
  const uint32_t tile = xcd_tile(blockIdx.x, static_cast<uint32_t>(a.n_tiles));
  const int mt = static_cast<int>(tile % a.n_mtiles);
  const int rest = static_cast<int>(tile / a.n_mtiles);
  const int nt = rest % a.n_ntiles, kp = rest / a.n_ntiles;
  const int m0 = mt * S::kBM, n0 = nt * S::kBN;
  const int k0 = kp * a.steps_per_part * S::kBK;
  const int kn = max(0, min(a.K - k0, a.steps_per_part * S::kBK));
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int wm = wave / S::kWavesN, wn = wave % S::kWavesN;

  Loader<S, S::kBM> la;
  Loader<S, S::kBN> lb;
  la.init(a.A + static_cast<int64_t>(m0) * a.lda + k0, a.lda, a.M - m0, kn, wave, lane);
  lb.init(a.B + static_cast<int64_t>(n0) * a.ldb + k0, a.ldb, a.N - n0, kn, wave, lane);
  Acc<S> acc;
  ring_gemm<S>(
      smem, (kn + S::kBK - 1) / S::kBK,
      [&](unsigned char* slot, int kt) {
        la.issue(slot, kt * S::kBK, wave);
        lb.issue(slot + S::kAChunks * 16, kt * S::kBK, wave);
      },
      acc, lane, wave);

  float* P = a.part + static_cast<int64_t>(kp) * a.M * a.N;
#pragma unroll
  for (int i = 0; i < S::kFragM; ++i)
#pragma unroll
    for (int j = 0; j < S::kFragN; ++j)
#pragma unroll
      for (int v = 0; v < 16; ++v) {
        const int gr = m0 + acc_row<S>(wm, i, v, lane);
        const int gc = n0 + acc_col<S>(wn, j, lane);
        if (gr < a.M && gc < a.N) P[static_cast<int64_t>(gr) * a.N + gc] = acc[i][j][v];
      }
}

bool splitk_shape_ok(int64_t m, int64_t n, int64_t k) {
  return m >= 1 && n >= 8 && k >= 8 && n % 8 == 0 && k % 8 == 0 && m <= (1 << 24) &&
         n <= (1 << 24) && k <= (1 << 24);
}

}  // namespace
}  // namespace talm

using namespace talm;

TALM_API int64_t talm_gemm_splitk_workspace(int64_t m, int64_t n, int64_t k) {
  if (!splitk_shape_ok(m, n, k)) return -1;
  return static_cast<int64_t>(plan_split(m, n, k, SplitShape::kBM, SplitShape::kBN, SplitShape::kBK).parts) * m * n * 4;
}

namespace talm {
namespace {

// out == nullptr: the fp32 partials stay in the workspace for the caller's next launch.
int splitk_impl(const char* what, const uint16_t* a, int64_t lda, const uint16_t* b, int64_t ldb,
                uint16_t* out, int64_t ldo, int64_t m, int64_t n, int64_t k, void* workspace,
                int64_t workspace_bytes, hipStream_t s) {
  if (!splitk_shape_ok(m, n, k) || lda < k || ldb < k || (out && (ldo < n || ldo % 8)) ||
      lda % 8 || ldb % 8 || lda > (1 << 22) || ldb > (1 << 22))
    return fail(TALM_EINVAL,
                "%s: bad shape (m %lld, n %lld, k %lld, lda %lld, ldb %lld, ldo %lld): "
                "n, k and the strides multiples of 8, strides at least k (a, b) and n (out), "
                "a / b strides below 2^22",
                what, (long long)m, (long long)n, (long long)k, (long long)lda, (long long)ldb,
                (long long)ldo);
  if (!a || !b || !workspace) return fail(TALM_EINVAL, "%s: null pointer", what);
  if (!aligned(a, 16) || !aligned(b, 16) || !aligned(out, 16) || !aligned(workspace, 16))
    return fail(TALM_EINVAL, "%s: operands and workspace must be 16-byte aligned", what);
  const SplitPlan p = plan_split(m, n, k, SplitShape::kBM, SplitShape::kBN, SplitShape::kBK);
  const int64_t need = static_cast<int64_t>(p.parts) * m * n * 4;
  if (workspace_bytes < need)
    return fail(TALM_EINVAL, "%s: workspace of %lld bytes, %lld needed", what,
                (long long)workspace_bytes, (long long)need);
  SplitArgs args{};
  args.A = a; args.lda = lda; args.B = b; args.ldb = ldb;
  args.part = static_cast<float*>(workspace);
  args.M = static_cast<int>(m); args.N = static_cast<int>(n); args.K = static_cast<int>(k);
  args.steps_per_part = p.steps_per_part;
  args.n_mtiles = p.n_mtiles; args.n_ntiles = p.n_ntiles;
  args.n_tiles = p.n_mtiles * p.n_ntiles * p.parts;
  hipLaunchKernelGGL((gemm_splitk_kernel<SplitShape>), dim3(static_cast<unsigned>(args.n_tiles)),
                     dim3(SplitShape::kThreads), 0, s, args);
  if (out) launch_splitk_reduce(static_cast<const float*>(workspace), p.parts, m, n, out, ldo, s);
  return check_launch(what);
}

}  // namespace
}  // namespace talm

TALM_API int talm_gemm_splitk(const uint16_t* a, int64_t lda, const uint16_t* b, int64_t ldb,
                              uint16_t* out, int64_t ldo, int64_t m, int64_t n, int64_t k,
                              void* workspace, int64_t workspace_bytes, void* stream) {
  if (!out) return fail(TALM_EINVAL, "gemm_splitk: null pointer");
  return splitk_impl("gemm_splitk", a, lda, b, ldb, out, ldo, m, n, k, workspace,
                     workspace_bytes, as_stream(stream));
}

TALM_API int64_t talm_gemm_splitk_parts(int64_t m, int64_t n, int64_t k) {
  if (!splitk_shape_ok(m, n, k)) return -1;
  return plan_split(m, n, k, SplitShape::kBM, SplitShape::kBN, SplitShape::kBK).parts;
}

TALM_API int talm_gemm_splitk_partials(const uint16_t* a, int64_t lda, const uint16_t* b,
                                       int64_t ldb, int64_t m, int64_t n, int64_t k,
                                       float* partials, int64_t partials_bytes, void* stream) {
  return splitk_impl("gemm_splitk_partials", a, lda, b, ldb, nullptr, 0, m, n, k, partials,
                     partials_bytes, as_stream(stream));
}
