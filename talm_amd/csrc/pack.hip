// The small per-step kernels around the decoder of the packed causal-LM step: the batch's
// packing into a fixed row count, the next batch's row statistics, the loss and per-token
// metrics after the LM head and the head backward's scaling. Each replaces a chain of PyTorch
// launches of a few microseconds each (5 to 25 per call); in a step replayed from a HIP graph
// that glue is launch-bound, not bandwidth-bound.
//
// The batch kernels are integer work on a few thousand tokens: one workgroup each, so the row
// offsets they compute are visible to the per-token work after a workgroup barrier.
#include "common.h"

namespace talm {
namespace {

constexpr int kBlock = 1024;
constexpr int kMaxRows = 8192;  // rows of a batch whose offsets one workgroup keeps in LDS

// Sum over the workgroup, one value per thread; every thread receives the total. The 16
// wavefront sums are added in wavefront order: the result does not depend on timing.
template <typename T>
__device__ T block_sum(T v, T* red) {
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) v += __shfl_xor(v, off, kWave);
  const int w = threadIdx.x >> 6, lane = threadIdx.x & 63;
  __syncthreads();  // the previous call's readers are done with `red`
  if (lane == 0) red[w] = v;
  __syncthreads();
  T total = red[0];
#pragma unroll
  for (int i = 1; i < kBlock / kWave; ++i) total += red[i];
  return total;
}

// Fixed-shape packing (solution/unpad.py:66-92, restated for a fixed row count): row b of the
// right-padded [batch, seq] batch holds len_b = sum_t mask[b][t] real tokens (clamped to
// [0, seq]); they go to flat rows [cu[b], cu[b + 1]) with cu[k] = min(len_0 + .. + len_{k-1},
// n_tokens), and flat rows [cu[batch], n_tokens) form one more sequence (cu[batch + 1] =
// n_tokens) that reads the pad slot batch * seq: id 0, target -100. Per flat row j: its row
// (the number of cu[1..batch] <= j), its position j - cu[row], its source index and its
// shifted target (labels[b][p + 1], -100 at a row's last position).
__global__ __launch_bounds__(kBlock) void pack_rows_kernel(
    const int64_t* __restrict__ ids, const int64_t* __restrict__ mask,
    const int64_t* __restrict__ labels, int batch, int seq, int n_tokens,
    int64_t* __restrict__ ids_out, int64_t* __restrict__ pos_out, int32_t* __restrict__ cu_out,
    int64_t* __restrict__ tgt_out, int64_t* __restrict__ src_out) {
  extern __shared__ int32_t cu[];  // [batch + 2]
  __shared__ int64_t red[kBlock / kWave];
  int64_t run = 0;
  for (int b = 0; b < batch; ++b) {
    int64_t s = 0;
    for (int t = threadIdx.x; t < seq; t += kBlock) s += mask[static_cast<int64_t>(b) * seq + t];
    const int64_t len = block_sum(s, red);
    run += len < 0 ? 0 : (len > seq ? seq : len);
    if (threadIdx.x == 0) cu[b + 1] = static_cast<int32_t>(run < n_tokens ? run : n_tokens);
  }
  if (threadIdx.x == 0) {
    cu[0] = 0;
    cu[batch + 1] = n_tokens;
  }
  __syncthreads();
  for (int k = threadIdx.x; k < batch + 2; k += kBlock) cu_out[k] = cu[k];
  for (int j = threadIdx.x; j < n_tokens; j += kBlock) {
    int lo = 0, hi = batch;  // the count of cu[1..batch] <= j (cu is non-decreasing)
    while (lo < hi) {
      const int mid = (lo + hi) >> 1;
      if (cu[mid + 1] <= j) lo = mid + 1; else hi = mid;
    }
    const int pos = j - cu[lo];
    const bool real = lo < batch;
    const int64_t src = real ? static_cast<int64_t>(lo) * seq + pos : static_cast<int64_t>(batch) * seq;
    ids_out[j] = real ? ids[src] : 0;
    tgt_out[j] = real && pos + 1 < seq ? labels[src + 1] : -100;
    pos_out[j] = pos;
    src_out[j] = src;
  }
}

// stats[b] = sum_t mask[b][t]; stats[batch] = labelled positions among each row's first
// stats[b] positions; stats[batch + 1] = labelled positions overall; position t of row b is
// labelled when t + 1 < seq and labels[b][t + 1] >= 0 (the shifted labels).
__global__ __launch_bounds__(kBlock) void row_stats_kernel(const int64_t* __restrict__ mask,
                                                           const int64_t* __restrict__ labels,
                                                           int batch, int seq,
                                                           int64_t* __restrict__ stats) {
  __shared__ int64_t red[kBlock / kWave];
  int64_t in_rows = 0, all = 0;
  for (int b = 0; b < batch; ++b) {
    const int64_t* mrow = mask + static_cast<int64_t>(b) * seq;
    const int64_t* lrow = labels + static_cast<int64_t>(b) * seq;
    int64_t s = 0;
    for (int t = threadIdx.x; t < seq; t += kBlock) s += mrow[t];
    const int64_t len = block_sum(s, red);
    if (threadIdx.x == 0) stats[b] = len;
    int64_t in = 0, any = 0;
    for (int t = threadIdx.x; t + 1 < seq; t += kBlock) {
      const int64_t lab = lrow[t + 1] >= 0;
      any += lab;
      in += lab && t < len;
    }
    in_rows += block_sum(in, red);
    all += block_sum(any, red);
  }
  if (threadIdx.x == 0) {
    stats[batch] = in_rows;
    stats[batch + 1] = all;
  }
}

// loss = sum_i token_loss[i] / denom, denom = the labelled count clamped to >= 1 (mode 0), the
// device scalar *num_items (mode 1) or num_items_value (mode 2); correct_bool[i] = correct[i] != 0
// (solution/fused_head.py:53-58, :272-277).
__global__ __launch_bounds__(kBlock) void head_loss_kernel(
    const float* __restrict__ token_loss, const int32_t* __restrict__ correct,
    const int64_t* __restrict__ targets, int64_t n, const float* __restrict__ num_items,
    float num_items_value, int mode, float* __restrict__ loss, float* __restrict__ denom,
    uint8_t* __restrict__ correct_bool) {
  __shared__ float redf[kBlock / kWave];
  __shared__ int64_t redi[kBlock / kWave];
  float s = 0.f;
  int64_t lab = 0;
  for (int64_t i = threadIdx.x; i < n; i += kBlock) {
    s += token_loss[i];
    lab += targets[i] >= 0;
    correct_bool[i] = correct[i] != 0;
  }
  const float total = block_sum(s, redf);
  const int64_t labelled = block_sum(lab, redi);
  if (threadIdx.x == 0) {
    const float d = mode == 0 ? static_cast<float>(labelled > 1 ? labelled : 1)
                    : mode == 1 ? *num_items : num_items_value;
    *denom = d;
    *loss = total / d;
  }
}

// The per-token loss and entropy back to the batch layout: full[k] = 0, then full[src[i]] =
// value[i] (rows sharing a slot: one of them, the pad slot's value is not used); stats = (the
// count of correct rows, the count of rows with target >= 0).
__global__ __launch_bounds__(kBlock) void scatter_rows_kernel(
    const float* __restrict__ token_loss, const float* __restrict__ entropy,
    const uint8_t* __restrict__ correct, const int64_t* __restrict__ targets,
    const int64_t* __restrict__ src, int64_t n, int64_t out_len, float* __restrict__ full_loss,
    float* __restrict__ full_entropy, int64_t* __restrict__ stats) {
  __shared__ int64_t red[kBlock / kWave];
  for (int64_t k = threadIdx.x; k < out_len; k += kBlock) {
    full_loss[k] = 0.f;
    full_entropy[k] = 0.f;
  }
  __syncthreads();  // every zero is written before a row's value lands on its slot
  int64_t c = 0, lab = 0;
  for (int64_t i = threadIdx.x; i < n; i += kBlock) {
    const int64_t k = src[i];
    if (k >= 0 && k < out_len) {
      full_loss[k] = token_loss[i];
      full_entropy[k] = entropy[i];
    }
    c += correct[i] != 0;
    lab += targets[i] >= 0;
  }
  const int64_t n_correct = block_sum(c, red);
  const int64_t n_labelled = block_sum(lab, red);
  if (threadIdx.x == 0) {
    stats[0] = n_correct;
    stats[1] = n_labelled;
  }
}

// out = fp16(fp32(g) * s), s = grad_loss / denom (0 when denom is 0), eight values per thread
// (solution/fused_head.py:280-287). The product is rounded to fp32 and then to fp16, as the
// reference's two ops do (mul_f32: not one v_fma_mix rounding straight to fp16).
__global__ __launch_bounds__(256) void scale_rows_kernel(const uint16_t* __restrict__ g,
                                                         int64_t n_vec, int64_t n,
                                                         const float* __restrict__ grad_loss,
                                                         const float* __restrict__ denom,
                                                         uint16_t* __restrict__ out) {
  const float d = *denom;
  const float s = d != 0.f ? *grad_loss / d : 0.f;
  const int64_t stride = static_cast<int64_t>(gridDim.x) * blockDim.x;
  for (int64_t v = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x; v < n_vec;
       v += stride) {
    const uint4 x = reinterpret_cast<const uint4*>(g)[v];
    uint4 y;
    y.x = pack2(mul_f32(lo_f(x.x), s), mul_f32(hi_f(x.x), s));
    y.y = pack2(mul_f32(lo_f(x.y), s), mul_f32(hi_f(x.y), s));
    y.z = pack2(mul_f32(lo_f(x.z), s), mul_f32(hi_f(x.z), s));
    y.w = pack2(mul_f32(lo_f(x.w), s), mul_f32(hi_f(x.w), s));
    reinterpret_cast<uint4*>(out)[v] = y;
  }
  for (int64_t i = 8 * n_vec + static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x; i < n;
       i += stride)
    out[i] = f2h(mul_f32(h2f(g[i]), s));
}

}  // namespace
}  // namespace talm

using namespace talm;

TALM_API int talm_pack_rows(const int64_t* input_ids, const int64_t* mask, const int64_t* labels,
                            int32_t batch, int32_t seq, int64_t n_tokens, int64_t* ids,
                            int64_t* positions, int32_t* cu_seqlens, int64_t* targets,
                            int64_t* src, void* stream) {
  if (batch < 1 || batch > kMaxRows || seq < 1 || n_tokens < 1 || n_tokens > (1 << 30) ||
      static_cast<int64_t>(batch) * seq >= (int64_t{1} << 40))
    return fail(TALM_EINVAL, "pack_rows: bad shape (batch %d, seq %d, rows %lld): batch 1-%d",
                batch, seq, (long long)n_tokens, kMaxRows);
  if (!input_ids || !mask || !labels || !ids || !positions || !cu_seqlens || !targets || !src)
    return fail(TALM_EINVAL, "pack_rows: null pointer");
  hipLaunchKernelGGL(pack_rows_kernel, dim3(1), dim3(kBlock), (batch + 2) * sizeof(int32_t),
                     as_stream(stream), input_ids, mask, labels, batch, seq,
                     static_cast<int>(n_tokens), ids, positions, cu_seqlens, targets, src);
  return check_launch("pack_rows");
}

TALM_API int talm_row_stats(const int64_t* mask, const int64_t* labels, int32_t batch, int32_t seq,
                            int64_t* stats, void* stream) {
  if (batch < 1 || seq < 1 || static_cast<int64_t>(batch) * seq >= (int64_t{1} << 40))
    return fail(TALM_EINVAL, "row_stats: bad shape (batch %d, seq %d)", batch, seq);
  if (!mask || !labels || !stats) return fail(TALM_EINVAL, "row_stats: null pointer");
  hipLaunchKernelGGL(row_stats_kernel, dim3(1), dim3(kBlock), 0, as_stream(stream), mask, labels,
                     batch, seq, stats);
  return check_launch("row_stats");
}

TALM_API int talm_head_loss(const float* token_loss, const int32_t* correct,
                            const int64_t* targets, int64_t n, const float* num_items,
                            float num_items_value, int32_t mode, float* loss, float* denom,
                            uint8_t* correct_bool, void* stream) {
  if (n < 0 || mode < 0 || mode > 2 || (mode == 1 && !num_items))
    return fail(TALM_EINVAL, "head_loss: bad arguments (rows %lld, mode %d)", (long long)n, mode);
  if (!loss || !denom || (n > 0 && (!token_loss || !correct || !targets || !correct_bool)))
    return fail(TALM_EINVAL, "head_loss: null pointer");
  hipLaunchKernelGGL(head_loss_kernel, dim3(1), dim3(kBlock), 0, as_stream(stream), token_loss,
                     correct, targets, n, num_items, num_items_value, mode, loss, denom,
                     correct_bool);
  return check_launch("head_loss");
}

TALM_API int talm_scatter_rows(const float* token_loss, const float* entropy,
                               const uint8_t* correct, const int64_t* targets,
                               const int64_t* src, int64_t n, int64_t out_len, float* full_loss,
                               float* full_entropy, int64_t* stats, void* stream) {
  if (n < 0 || out_len < 0)
    return fail(TALM_EINVAL, "scatter_rows: bad sizes (rows %lld, slots %lld)", (long long)n,
                (long long)out_len);
  if (!stats || (out_len > 0 && (!full_loss || !full_entropy)) ||
      (n > 0 && (!token_loss || !entropy || !correct || !targets || !src)))
    return fail(TALM_EINVAL, "scatter_rows: null pointer");
  hipLaunchKernelGGL(scatter_rows_kernel, dim3(1), dim3(kBlock), 0, as_stream(stream), token_loss,
                     entropy, correct, targets, src, n, out_len, full_loss, full_entropy, stats);
  return check_launch("scatter_rows");
}

TALM_API int talm_scale_rows(const uint16_t* g, int64_t n, const float* grad_loss,
                             const float* denom, uint16_t* out, void* stream) {
  if (n < 0) return fail(TALM_EINVAL, "scale_rows: %lld elements", (long long)n);
  if (n == 0) return ok();
  if (!g || !grad_loss || !denom || !out) return fail(TALM_EINVAL, "scale_rows: null pointer");
  if (!aligned(g, 16) || !aligned(out, 16))
    return fail(TALM_EINVAL, "scale_rows: g and out must be 16-byte aligned");
  const int64_t n_vec = n / 8;
  const int64_t blocks = (n_vec + 255) / 256;
  const int cap = 4 * device_cus();
  hipLaunchKernelGGL(scale_rows_kernel,
                     dim3(static_cast<unsigned>(blocks < 1 ? 1 : (blocks < cap ? blocks : cap))),
                     dim3(256), 0, as_stream(stream), g, n_vec, n, grad_loss, denom, out);
  return check_launch("scale_rows");
}
