/*
 * talm.h — the C-ABI of libtalm.so, the MI355X (gfx950) QLoRA kernel set.
 *
 * Every entry point:
 *   - takes plain device pointers, sizes and an explicit stream (a hipStream_t passed as void*;
 *     NULL is the legacy default stream);
 *   - only enqueues work on that stream: it never synchronizes and never allocates device
 *     memory (every buffer, workspaces included, is owned by the caller);
 *   - returns TALM_OK (0) or a nonzero status, with a message for the calling thread in
 *     talm_last_error(). TALM_EINVAL means the arguments were rejected before anything was
 *     launched (the Python layer raises ValueError), TALM_EHIP a HIP launch error (RuntimeError).
 *   - is reentrant: no state is kept between calls (forward launches come from the Python main
 *     thread, backward launches from the autograd device thread).
 *
 * fp16 tensors are passed as uint16_t* / void* holding IEEE binary16 bit patterns.
 * Reference citations are paths inside otarernazar-eng/Talm.
 */
#ifndef TALM_H
#define TALM_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define TALM_OK 0
#define TALM_EINVAL 1
#define TALM_EHIP 2

/* Element types of the tensors whose dtype is a runtime argument. */
#define TALM_F32 0
#define TALM_F16 1

/* Message of the last failed call on this thread ("" after a success). */
const char* talm_last_error(void);

/* ABI version: bumped whenever a signature below changes. */
int talm_abi_version(void);

/*
 * Grouped NF4 dequantization of the seven projections of one decoder layer in one launch.
 * Replaces qgroup.launch / nf4_group_dequant_kernel (solution/qgroup.py:72-99).
 *   packed   u8  [n_rows * qblock / 2]   two NF4 codes per byte, the high nibble is the even element
 *   absmax8  u8  [n_rows]                index into `code` of each block's absmax
 *   code     f32 [256]                   second-level code table (bitsandbytes state2.code)
 *   absmax2  f32 [n_rows / qblock2]      second-level scale of every qblock2 blocks
 *   offset2  f32 [n_rows / qblock2]      the offset of the projection each block belongs to
 *   out      f16 [n_rows * qblock]
 * Per element e of block r: scale = fl32(fl32(code[absmax8[r]] * absmax2[r/qblock2]) +
 * offset2[r/qblock2]); out[e] = f16_rne(fl32(NF4[nibble] * scale)) (no fused multiply-add).
 * qblock: even power of two >= 8; qblock2 >= 1. Pointers 4-byte (packed) / 16-byte (out) aligned.
 */
int talm_nf4_group_dequant(const uint8_t* packed, const uint8_t* absmax8, const float* code,
                           const float* absmax2, const float* offset2, uint16_t* out,
                           int64_t n_rows, int32_t qblock, int32_t qblock2, void* stream);

/*
 * talm_nf4_group_dequant with non-temporal stores: the same arguments and the same values, bit
 * for bit, for an output that is not read again soon (a layer dequantized ahead of its use, or
 * on its own), so that it does not displace the last-level cache's contents. The training step
 * uses talm_nf4_group_dequant instead: its GEMMs read the layer right after it is written, from
 * the last-level cache the ordinary stores fill. Replaces the same reference launch
 * (solution/qgroup.py:72-99); the reference has one store kind.
 */
int talm_nf4_group_dequant_streaming(const uint8_t* packed, const uint8_t* absmax8,
                                     const float* code, const float* absmax2,
                                     const float* offset2, uint16_t* out, int64_t n_rows,
                                     int32_t qblock, int32_t qblock2, void* stream);

/*
 * The same grouped dequantization written transposed, for the backward's input-gradient GEMMs
 * (dX = dY W reads W^T as the k-contiguous operand). No counterpart of its own in the reference,
 * whose backward multiplies by the row-major weight of qgroup.launch (solution/qgroup.py:72-99,
 * :346-355); the values are talm_nf4_group_dequant's, bit for bit.
 *   segs  i64 [n_seg][5]: for each projection W [rows, cols]: the element index of its first
 *         weight in packed / absmax8 (a multiple of qblock), rows, cols, the element offset of
 *         W^T in `out` and the row stride of W^T (so projections with the same cols can sit
 *         side by side in one W^T: q|k|v, gate|up);
 *   out   f16 [out_numel]: out[dst + c * ld + r] = W[r][c].
 * qblock: power of two >= 64; rows a multiple of 8, cols of 64; ld >= rows, ld and dst multiples
 * of 8; n_seg <= 8. packed and out 16-byte aligned.
 */
int talm_nf4_group_dequant_t(const uint8_t* packed, const uint8_t* absmax8, const float* code,
                             const float* absmax2, const float* offset2, const int64_t* segs,
                             int32_t n_seg, int32_t qblock, int32_t qblock2, uint16_t* out,
                             int64_t out_numel, void* stream);

/*
 * Split-K fp16 GEMM: out [m, n] = f16(a [m, k] b [n, k]^T), fp32 accumulation, both operands
 * k-contiguous. No counterpart of its own: it replaces the library GEMM (cuBLAS in the reference,
 * GroupLinear / F.linear, solution/qgroup.py:346-355) for the MLP's long-reduction products
 * (down projection, input gradient on the transposed gate|up weight). The workspace holds one
 * fp32 partial [m, n] per K part (talm_gemm_splitk_workspace bytes, -1 for an unsupported
 * shape); the partials are summed in part order (deterministic).
 * n, k, lda, ldb, ldo multiples of 8; lda, ldb >= k, below 2^22; ldo >= n; 16-byte aligned.
 */
int64_t talm_gemm_splitk_workspace(int64_t m, int64_t n, int64_t k);
int talm_gemm_splitk(const uint16_t* a, int64_t lda, const uint16_t* b, int64_t ldb,
                     uint16_t* out, int64_t ldo, int64_t m, int64_t n, int64_t k, void* workspace,
                     int64_t workspace_bytes, void* stream);
/*
 * The same product leaving its fp32 partials [parts][m][n] in `partials` (no reduction, no fp16
 * output), for a caller whose next launch sums them (talm_splitk_add_rmsnorm,
 * talm_splitk_rmsnorm_bwd); talm_gemm_splitk_parts gives the part count (-1 for an unsupported
 * shape), partials_bytes >= parts * m * n * 4.
 */
int64_t talm_gemm_splitk_parts(int64_t m, int64_t n, int64_t k);
int talm_gemm_splitk_partials(const uint16_t* a, int64_t lda, const uint16_t* b, int64_t ldb,
                              int64_t m, int64_t n, int64_t k, float* partials,
                              int64_t partials_bytes, void* stream);

/*
 * Per-projection NF4 dequantization with an fp32 absmax per block (bitsandbytes'
 * dequantize_blockwise + offset already applied).
 * Replaces nf4_dequant.nf4_dequantize / nf4_dequant_pairs_kernel (solution/nf4_dequant.py:38-91).
 *   packed u8 [n / 2], absmax f32 [ceil(n / blocksize)], out f16 [n]; n even, blocksize even.
 */
int talm_nf4_dequant(const uint8_t* packed, const float* absmax, uint16_t* out, int64_t n,
                     int32_t blocksize, void* stream);

/*
 * Fused (residual-add +) RMSNorm, forward or backward, one launch.
 * Replaces rmsnorm.launch / rmsnorm_kernel (solution/rmsnorm.py:58-118).
 * Every [n_rows, n_cols] operand is contiguous (row stride n_cols).
 *   a, q: x_dtype;  h, xhat, p: out_dtype;  weight: w_dtype [n_cols];  rstd: f32 [n_rows].
 * backward == 0: x = a (+ p when add); writes q = x (when add), h = w * xhat, xhat = x * rstd,
 *                rstd = rsqrt(mean(x^2) + eps).
 * backward != 0: reads dy = h, xhat, rstd; dx = rstd * (g - xhat * mean(g * xhat)), g = dy * w;
 *                with add, dx += q and dx is also written to p; dx is written to a. A NULL q
 *                with add stands for ds = 0 (the sum's gradient is not used).
 * p and q are ignored (may be NULL) when add == 0.
 */
int talm_rmsnorm(void* a, void* q, void* h, void* xhat, void* p, const void* weight, float* rstd,
                 int64_t n_rows, int64_t n_cols, int32_t x_dtype, int32_t out_dtype,
                 int32_t w_dtype, float eps, int32_t backward, int32_t add, void* stream);

/*
 * talm_rmsnorm's residual-add forward and backward with the branch (forward) or dy (backward)
 * given as a split-K product's fp32 partials [parts][n_rows][n_cols] (talm_gemm_splitk_partials,
 * talm_nf4_gemm_partials): the partials are summed in part order and rounded to fp16, exactly the
 * values the product's own reduction would write, and the norm then runs as talm_rmsnorm does on
 * them (bit-identical to the two launches). x fp32, outputs fp16, weight w_dtype (f32 / f16);
 * n_cols a multiple of 8, at most 2048; 16-byte aligned rows.
 *   talm_splitk_add_rmsnorm: x = resid + branch -> sum_out, h = w * xhat, xhat, rstd.
 *   talm_splitk_rmsnorm_bwd: dx = rstd (g - xhat mean(g xhat)) (+ ds; NULL: 0), g = dy * w, to dx
 *                            (fp32) and dbranch (fp16).
 * No counterpart of its own: they fuse the K-part reduction of the MLP's long products with the
 * residual add and RMSNorm that follow (solution/rmsnorm.py:335-404) or precede them.
 */
int talm_splitk_add_rmsnorm(const float* partials, int32_t parts, const float* resid,
                            const void* weight, int32_t w_dtype, float eps, int64_t n_rows,
                            int64_t n_cols, float* sum_out, uint16_t* h, uint16_t* xhat,
                            float* rstd, void* stream);
int talm_splitk_rmsnorm_bwd(const float* partials, int32_t parts, const uint16_t* xhat,
                            const float* rstd, const void* weight, int32_t w_dtype, const float* ds,
                            int64_t n_rows, int64_t n_cols, float* dx, uint16_t* dbranch,
                            void* stream);

/*
 * Rotary position embedding of q and k, forward or backward, fp16 with fp32 math.
 * Replaces rope._launch / rope_kernel (solution/rope.py:64-134). In place when the output
 * pointers equal the input pointers (every thread reads its elements before writing them).
 * Element (token t, head h, column d) of q is at q[t * q_stride_tok + h * q_stride_head + d];
 * k, out_q, out_k alike; cos/sin f32 at [t * cs_stride_tok + d], d < head_dim.
 *   forward:  y1 = x1 c1 - x2 s1,  y2 = x2 c2 + x1 s2
 *   backward: y1 = x1 c1 + x2 s2,  y2 = x2 c2 - x1 s1      (x1/x2: first/second half of d)
 * head_dim even, <= 512; strides in elements.
 */
int talm_rope(const uint16_t* q, const uint16_t* k, const float* cos, const float* sin,
              uint16_t* out_q, uint16_t* out_k, int64_t n_tokens, int32_t n_q_heads,
              int32_t n_k_heads, int32_t head_dim, int64_t q_stride_tok, int64_t q_stride_head,
              int64_t k_stride_tok, int64_t k_stride_head, int64_t out_q_stride_tok,
              int64_t out_q_stride_head, int64_t out_k_stride_tok, int64_t out_k_stride_head,
              int64_t cs_stride_tok, int32_t backward, void* stream);

/*
 * The rotary tables of transformers' rotary embedding (Qwen2RotaryEmbedding.forward, default
 * and statically scaled types): for token t and j < half, angle = fl32(inv_freq[j] *
 * fl32(positions[t])), cos[t][j] = cos[t][j + half] = fl32(cosf(angle) * scaling), sin likewise;
 * positions int64 [n_tokens], cos / sin f32 [n_tokens, 2 half] row-major. One launch instead of
 * the position cast, the K = 1 product, the concatenation and the four elementwise ops; the
 * tables feed the rotation the reference fuses (solution/rope.py:64-134).
 */
int talm_rope_table(const int64_t* positions, int64_t n_tokens, const float* inv_freq,
                    int32_t half, float scaling, float* cos, float* sin, void* stream);

/*
 * SwiGLU forward: out = silu(gate) * up in fp32, written as fp16. n elements, contiguous.
 * Replaces example_swiglu_fwd_kernel (solution/swiglu.py:23-30); `out` may alias `gate`
 * (the save-up node, solution/mlp_save_up.py:63).
 */
int talm_swiglu_fwd(const uint16_t* gate, const uint16_t* up, uint16_t* out, int64_t n,
                    void* stream);

/*
 * SwiGLU backward: sig = sigmoid(gate); dup = grad * gate * sig;
 * dgate = grad * up * sig * (1 + gate * (1 - sig)), fp16 in and out, fp32 math.
 * Replaces example_swiglu_bwd_kernel (solution/swiglu.py:33-45); dgate may alias gate and dup
 * may alias up (the in-place backward, solution/swiglu_inplace.py:40).
 */
int talm_swiglu_bwd(const uint16_t* grad, const uint16_t* gate, const uint16_t* up,
                    uint16_t* dgate, uint16_t* dup, int64_t n, void* stream);

/*
 * The same two SwiGLU passes on [rows, cols] fp16 views with row strides (elements): gate and up
 * may be the two halves of one [rows, 2 cols] buffer (the fused MLP's gate|up GEMM output,
 * solution/fused_proj.py:241-287, where the reference runs the flat kernels on a transposed
 * buffer). cols and every row stride multiples of 8, pointers 16-byte aligned, rows <= 65535;
 * outputs may alias inputs element for element.
 */
int talm_swiglu_fwd_rows(const uint16_t* gate, int64_t ld_gate, const uint16_t* up, int64_t ld_up,
                         uint16_t* out, int64_t ld_out, int64_t rows, int64_t cols, void* stream);
int talm_swiglu_bwd_rows(const uint16_t* grad, int64_t ld_grad, const uint16_t* gate,
                         int64_t ld_gate, const uint16_t* up, int64_t ld_up, uint16_t* dgate,
                         int64_t ld_dgate, uint16_t* dup, int64_t ld_dup, int64_t rows,
                         int64_t cols, void* stream);

/*
 * Bytes of workspace talm_head_ce needs (-1 for arguments it would reject). `group` vocabulary
 * slices are processed per step: the workspace holds their fp16 logits [n_rows, group * vchunk],
 * the per-tile statistics and the fp32 gradient partials [group, n_grad, hidden].
 */
int64_t talm_head_ce_workspace(int64_t n_rows, int64_t hidden, int64_t vocab, int64_t vchunk,
                               int64_t n_grad, int32_t group);

/*
 * A weight's transpose: weight_t[h][v] = weight[v][h] for v < vocab, 0 for vocab <= v < ldwt (row
 * stride ldwt >= vocab, a multiple of 8); 64 x 64 blocks through LDS. Used for the q|k|v layer's
 * W^T of talm_qkv_lora_bwd_dx when no transposed dequantization of the layer is at hand.
 */
int talm_head_weight_t(const uint16_t* weight, int64_t ldw, int64_t vocab, int64_t hidden,
                       uint16_t* weight_t, int64_t ldwt, void* stream);

/*
 * Fused LM head + cross-entropy over the vocabulary in slices of `vchunk` columns (a multiple of
 * 128), forward and gradient in one call; the [n_rows, vocab] logits never exist.
 * Replaces FusedHeadLossVocab.forward's slice loop with torch.mm, launch_vocab /
 * fused_head_vocab_kernel and the accumulator addmm (solution/fused_head.py:88-182, :236-251,
 * :356-383).
 *   hidden_states f16 [n_rows, hidden] (row stride ldh), weight f16 [vocab, hidden] (row
 *   stride ldw), targets i64 [n_rows] (-100 = ignore). Rows [0, n_grad) are the gradient
 *   rows: every labelled row must be among them (the caller orders rows labelled-first,
 *   solution/fused_head.py:290-299, or passes n_grad = n_rows); an ignored row among them
 *   costs gradient work and gets a zero gradient.
 *   The gradient GEMM reads the weight's rows as they lie (no transposed copy); with the
 *   gradient, group * vchunk * ldw * 2 stays below 2^31.
 * Writes per row: token_loss f32 (log s + m - z_target, 0 unlabelled), entropy f32
 * (lse - t / s), best_idx i32 (first argmax of the fp16 logits), correct i32 (labelled and
 * best_idx == target); and, when grad_hidden is not NULL, grad_hidden f16 [n_rows, hidden]
 * (row stride hidden): dH = acc / s - W[target] for labelled rows, 0 for the others, with
 * acc = sum over slices of the reference's rescaled fp16(e^{z - m}) W products.
 * `workspace` (256-byte aligned) holds talm_head_ce_workspace(...) bytes.
 */
int talm_head_ce(const uint16_t* hidden_states, int64_t ldh, const uint16_t* weight, int64_t ldw,
                 const int64_t* targets, int64_t n_rows,
                 int64_t hidden, int64_t vocab, int64_t vchunk, int64_t n_grad, int32_t group,
                 float* token_loss, float* entropy, int32_t* best_idx, int32_t* correct,
                 uint16_t* grad_hidden, void* workspace, int64_t workspace_bytes, void* stream);

/*
 * LoRA down-projection of the q|k|v node, rank 16 per adapter (1 or 2 adapters): adapter g
 * reduces x's columns [xcol_g, xcol_g + k_g) against A_g f16 [16, k_g] (contiguous):
 * t[:, 16g:16g+16] = fp16(sum) and ts[:, 16g:16g+16] = fp16(scaling_g * sum), fp32 sums.
 * x f16 [n_tokens, ldx], t and ts f16 [n_tokens, ldt], k_g multiples of 32.
 * Forward (xcol 0, k = hidden): the adapters' t = drop(x) A^T without dropout
 * (solution/fused_proj.py:139-153, solution/lora.py:183-186); t is what the backward keeps.
 * Backward (x = the node's output gradient over the adapter's own output columns, A_g = B_g^T
 * given as B_g [k_g, 16] with a_kmajor = 1, scaling as in the forward): ts = u = (scaling dy) B
 * (solution/fused_proj.py:200-201, solution/lora.py:218-219).
 */
int talm_lora_down(const uint16_t* x, int64_t ldx, int64_t n_tokens, int64_t k0, int64_t k1,
                   int64_t xcol0, int64_t xcol1, const uint16_t* a0, const uint16_t* a1,
                   int32_t n_adapters, int32_t a_kmajor, float scaling0, float scaling1,
                   uint16_t* t, uint16_t* ts, int64_t ldt, void* stream);

/*
 * The fused q|k|v projection forward: out = x W^T + bias + sum_g (ts_g B_g^T on adapter g's
 * columns), then the rotary embedding on the heads of 128 columns in [0, rope_cols), in one MFMA
 * GEMM (the adapter term is one more reduction step: rounded once with the base product).
 *   x f16 [n_tokens, hidden] (ldx); weight f16 [n_out, hidden] (ldw; the layer group's q|k|v
 *   rows); bias f16 [n_out] or NULL; ts from talm_lora_down (ldt); adapter g: B_g f16
 *   [seg_end - seg_begin, 16] contiguous on output columns [seg_begin, seg_end) (whole
 *   128-column tiles); cos/sin f32 [n_tokens, cs_stride >= 128] or NULL (no rotation);
 *   out f16 [n_tokens, ldo].
 * Replaces FusedProjections.forward's base GEMM, the adapters' branch GEMMs and adds, and the
 * RoPE launch on q and k (solution/fused_proj.py:88-218, solution/rope.py:64-134).
 */
int talm_qkv_lora_fwd(const uint16_t* x, int64_t ldx, int64_t n_tokens, int64_t hidden,
                      const uint16_t* weight, int64_t ldw, int64_t n_out, const uint16_t* bias,
                      const uint16_t* ts, int64_t ldt, int32_t n_adapters, const uint16_t* b0,
                      int64_t seg0_begin, int64_t seg0_end, const uint16_t* b1,
                      int64_t seg1_begin, int64_t seg1_end, const float* cos, const float* sin,
                      int64_t cs_stride, int64_t rope_cols, uint16_t* out, int64_t ldo,
                      void* stream);

/*
 * talm_qkv_lora_fwd with the adapters' down-projection inside the same GEMM: A_g f16 [16, hidden]
 * (row stride lda) for adapter g; every output tile of an adapter's columns accumulates
 * t = x A_g^T over its rows during the main product and adds fp16(scaling_g t) B_g^T after it (in
 * fp32, before the bias and the one rounding). t f16 [n_tokens, 16 * n_adapters] (row stride ldt,
 * adapter g in columns 16 g ..) is written for the backward. Replaces the same reference code as
 * talm_qkv_lora_fwd together with the adapters' down projection x A^T (solution/lora.py:
 * 151-231, solution/fused_proj.py:118-140), in one launch instead of talm_lora_down + it.
 */
int talm_qkv_lora_fwd_down(const uint16_t* x, int64_t ldx, int64_t n_tokens, int64_t hidden,
                           const uint16_t* weight, int64_t ldw, int64_t n_out, const uint16_t* bias,
                           int32_t n_adapters, const uint16_t* a0, const uint16_t* a1, int64_t lda,
                           float scaling0, float scaling1, const uint16_t* b0, int64_t seg0_begin,
                           int64_t seg0_end, const uint16_t* b1, int64_t seg1_begin,
                           int64_t seg1_end, const float* cos, const float* sin, int64_t cs_stride,
                           int64_t rope_cols, uint16_t* t, int64_t ldt, uint16_t* out, int64_t ldo,
                           void* stream);

/*
 * The q|k|v node's backward operand: dcat f16 [n_tokens, q + k + v] (row stride ldc) =
 * [rope_back(dq) | rope_back(dk) | dv] with dx1 = dy1 c1 + dy2 s2, dx2 = dy2 c2 - dy1 s1 on the
 * (j, j + 64) pairs of each 128-column head (no rotation when cos is NULL). Replaces the
 * backward's gradient concatenation and its RoPE launch (solution/fused_proj.py:165-175,
 * solution/rope.py:145-157).
 */
int talm_qkv_bwd_prep(const uint16_t* dq, int64_t ldq, const uint16_t* dk, int64_t ldk,
                      const uint16_t* dv, int64_t ldv, int64_t n_tokens, int64_t q_cols,
                      int64_t k_cols, int64_t v_cols, const float* cos, const float* sin,
                      int64_t cs_stride, uint16_t* dcat, int64_t ldc, void* stream);

/*
 * The q|k|v node's input gradient on MFMA: dx f16 [n_tokens, hidden] = dcat W + u A, with
 * dcat f16 [n_tokens, n_out] (ldc), weight_t = W^T f16 [hidden, ldwt >= n_out] (W the layer
 * group's q|k|v rows), u f16 [n_tokens, rank] (ldu; the adapters' u side by side) and
 * a_t = A^T f16 [hidden, ldat] (the adapters' A side by side, transposed), rank <= 64 a
 * multiple of 8 (0: no adapter term). One fp32 accumulation, one rounding. Replaces the
 * backward's dX GEMM (K = n_out) and the adapters' u A GEMMs and adds
 * (solution/fused_proj.py:172-184, :202-209, solution/lora.py:221-222).
 */
int talm_qkv_lora_bwd_dx(const uint16_t* dcat, int64_t ldc, int64_t n_tokens, int64_t n_out,
                         const uint16_t* weight_t, int64_t ldwt, int64_t hidden, const uint16_t* u,
                         int64_t ldu, int64_t rank, const uint16_t* a_t, int64_t ldat,
                         uint16_t* dx, int64_t lddx, void* stream);

/*
 * The adapters' weight gradients in fp32 (both adapters, one call, two launches):
 * dA_g [16, hidden] = u[:, 16g:16g+16]^T x and dB_g [seg_g, 16] = scaling_g dy[:, lo_g:lo_g+seg_g]^T
 * t[:, 16g:16g+16], summed over the tokens in fixed-size chunks and then over the chunks in
 * order (deterministic). x f16 [n_tokens, ldx], dy f16 [n_tokens, ldy] (the node's output
 * gradient after the RoPE backward), u and t f16 [n_tokens, 16 per adapter]. `workspace` holds
 * talm_lora_wgrad_workspace(...) bytes. Replaces the adapters' dA / dB GEMMs, their fp32 casts
 * and the scaling of g (solution/fused_proj.py:199-215, solution/lora.py:218, :229-230).
 */
int64_t talm_lora_wgrad_workspace(int64_t n_tokens, int64_t hidden, int64_t seg0, int64_t seg1);
int talm_lora_wgrad(const uint16_t* x, int64_t ldx, const uint16_t* dy, int64_t ldy,
                    const uint16_t* u, int64_t ldu, const uint16_t* t, int64_t ldt,
                    int64_t n_tokens, int64_t hidden, int32_t n_adapters, int64_t lo0,
                    int64_t seg0, float scaling0, float* da0, float* db0, int64_t lo1,
                    int64_t seg1, float scaling1, float* da1, float* db1, void* workspace,
                    int64_t workspace_bytes, void* stream);

/*
 * talm_lora_wgrad without a workspace argument, for callers that cannot allocate device memory
 * (code under HIP graph capture, tight serving loops, harnesses that forbid hipMalloc). It has
 * no counterpart in the reference. Same arguments, kernels and results as talm_lora_wgrad; the
 * fp32 partials live in a fixed array of TALM_LORA_WGRAD_SCRATCH_BYTES in the library's device
 * memory, one per GPU (held until the process ends), whose address is looked up on the first
 * call on each device. Calls whose partials need more than that (talm_lora_wgrad_workspace(...)
 * > TALM_LORA_WGRAD_SCRATCH_BYTES: about 4992 tokens with hidden 1536 and adapters on 1536 +
 * 256 columns) are rejected with TALM_EINVAL. It calls no allocator. The stream must belong to
 * the current device. Every call on one GPU shares that GPU's array: calls that overlap on one
 * GPU (concurrent streams, or threads) race and must be serialized by the caller.
 */
#define TALM_LORA_WGRAD_SCRATCH_BYTES (32ll << 20)
int talm_lora_wgrad_noalloc(const uint16_t* x, int64_t ldx, const uint16_t* dy, int64_t ldy,
                            const uint16_t* u, int64_t ldu, const uint16_t* t, int64_t ldt,
                            int64_t n_tokens, int64_t hidden, int32_t n_adapters, int64_t lo0,
                            int64_t seg0, float scaling0, float* da0, float* db0, int64_t lo1,
                            int64_t seg1, float scaling1, float* da1, float* db1, void* stream);

/*
 * Variable-length causal attention with grouped KV heads, forward. Sequence s holds the packed
 * rows [cu_seqlens[s], cu_seqlens[s+1]) (int32, device); row i attends to keys j <= i of its own
 * sequence; query head h reads KV head h / (n_q_heads / n_kv_heads). q f16 [n_tokens, n_q_heads,
 * head_dim], k / v f16 [n_tokens, n_kv_heads, head_dim] at element strides (token, head), unit
 * column stride; out likewise [n_tokens, n_q_heads, head_dim]; lse f32 [n_q_heads, n_tokens] =
 * log sum_j exp(scale q.k_j) per row. head_dim 128; strides multiples of 8, the token strides of
 * k, v and out below 2^23 elements; max_seqlen >= the longest sequence. Replaces the reference's per-KV-head memory-efficient attention launches
 * (solution/unpad.py:199-294) with per-row causal SDPA semantics (solution/unpad.py:121-134).
 */
int talm_attn_fwd(const uint16_t* q, int64_t q_stride_tok, int64_t q_stride_head,
                  const uint16_t* k, int64_t k_stride_tok, int64_t k_stride_head,
                  const uint16_t* v, int64_t v_stride_tok, int64_t v_stride_head,
                  const int32_t* cu_seqlens, int32_t n_seqs, int32_t max_seqlen,
                  int64_t n_tokens, int32_t n_q_heads, int32_t n_kv_heads, int32_t head_dim,
                  float scale, uint16_t* out, int64_t o_stride_tok, int64_t o_stride_head,
                  float* lse, void* stream);

/*
 * Its backward: dq f16 [n_tokens, n_q_heads, head_dim], dk / dv f16 [n_tokens, n_kv_heads,
 * head_dim] (any strides as above; the token strides of q, k, v, dout and dq below 2^23
 * elements) from q, k, v, the forward's out and lse, and dout. dk / dv of
 * a KV head sum its query heads' contributions in head order (deterministic). `workspace`
 * (256-byte aligned) holds talm_attn_bwd_workspace(n_tokens, n_q_heads) bytes: rowsum(dout *
 * out), lse in base-2 units and fp32 dk / dv partials per query head. Replaces the backward of the same launches
 * (solution/unpad.py:199-294).
 */
int64_t talm_attn_bwd_workspace(int64_t n_tokens, int32_t n_q_heads);
int talm_attn_bwd(const uint16_t* q, int64_t q_stride_tok, int64_t q_stride_head,
                  const uint16_t* k, int64_t k_stride_tok, int64_t k_stride_head,
                  const uint16_t* v, int64_t v_stride_tok, int64_t v_stride_head,
                  const uint16_t* out, int64_t o_stride_tok, int64_t o_stride_head,
                  const uint16_t* dout, int64_t do_stride_tok, int64_t do_stride_head,
                  const float* lse, const int32_t* cu_seqlens, int32_t n_seqs,
                  int32_t max_seqlen, int64_t n_tokens, int32_t n_q_heads, int32_t n_kv_heads,
                  int32_t head_dim, float scale, uint16_t* dq, int64_t dq_stride_tok,
                  int64_t dq_stride_head, uint16_t* dk, int64_t dk_stride_tok,
                  int64_t dk_stride_head, uint16_t* dv, int64_t dv_stride_tok,
                  int64_t dv_stride_head, void* workspace, int64_t workspace_bytes,
                  void* stream);

/*
 * talm_attn_bwd with the rotary embedding's backward folded into its outputs: q and k are the
 * rotated projections the forward attended over, and dq / dk come out as the gradients of the
 * projections BEFORE the rotation, each 128-wide head rotated back on its (d, d + 64) pairs:
 * dx1 = dy1 c1 + dy2 s2, dx2 = dy2 c2 - dy1 s1 with c / s the token's cos / sin rows (f32
 * [n_tokens] rows of cs_stride >= 128 elements, a multiple of 4; 16-byte aligned), in fp32
 * before the one rounding to fp16. dv as talm_attn_bwd. Replaces the attention backward
 * followed by the rotary backward of q and k (solution/unpad.py:199-294, solution/rope.py:
 * 145-157).
 */
int talm_attn_bwd_rope(const uint16_t* q, int64_t q_stride_tok, int64_t q_stride_head,
                       const uint16_t* k, int64_t k_stride_tok, int64_t k_stride_head,
                       const uint16_t* v, int64_t v_stride_tok, int64_t v_stride_head,
                       const uint16_t* out, int64_t o_stride_tok, int64_t o_stride_head,
                       const uint16_t* dout, int64_t do_stride_tok, int64_t do_stride_head,
                       const float* lse, const int32_t* cu_seqlens, int32_t n_seqs,
                       int32_t max_seqlen, int64_t n_tokens, int32_t n_q_heads,
                       int32_t n_kv_heads, int32_t head_dim, float scale, const float* cos,
                       const float* sin, int64_t cs_stride, uint16_t* dq, int64_t dq_stride_tok,
                       int64_t dq_stride_head, uint16_t* dk, int64_t dk_stride_tok,
                       int64_t dk_stride_head, uint16_t* dv, int64_t dv_stride_tok,
                       int64_t dv_stride_head, void* workspace, int64_t workspace_bytes,
                       void* stream);

/*
 * fp16 copies of the LoRA adapters' fp32 weights, every adapter in one launch. `table` (device
 * memory, int64, 8-byte aligned) holds 9 entries per tensor: the fp32 weight's address (a
 * row-major contiguous [rows, cols] matrix), its element count, its column count, the element
 * offset of its fp16 copy in `out` (-1: none), the element offset of a transposed fp16 copy in
 * `out` (-1: none; out[t_off + c * ld_t + r] = fp16(w[r, c])), that copy's row stride ld_t, and
 * three optimizer addresses (gradient, first and second moment, fp32, same layout as the weight;
 * unused here). Conversions round to nearest even (as .to(float16)). max_numel bounds every
 * element count; n_tensors <= 65535. Replaces the adapters' fp16 casts, one foreach copy per
 * refresh (solution/lora.py:57-137), and the q|k|v backward's concatenation and transposition of
 * the two A matrices (solution/fused_proj.py:202-209 forms u A per adapter instead).
 */
int talm_lora_mirror(const int64_t* table, int32_t n_tensors, int64_t max_numel, uint16_t* out,
                     void* stream);

/*
 * One AdamW step (decoupled weight decay, bias-corrected moments: w -= lr*wd*w; m = b1 m +
 * (1-b1) g; v = b2 v + (1-b2) g^2; w -= lr/(1-b1^t) * m / (sqrt(v)/sqrt(1-b2^t) + eps)) of every
 * tensor in `table` (layout above, optimizer addresses required), then the same fp16 copies as
 * talm_lora_mirror of the updated weights. t = *step_in + 1 (device fp32); one thread writes
 * *step_out (a different address): t, or *step_in when *found_inf is nonzero — then no weight or
 * moment changes (the copies are still written). grad_scale (device fp32, may be NULL) divides
 * the gradients; found_inf may be NULL. Replaces torch.optim.AdamW(fused=True) on the LoRA
 * parameters plus the next forward's fp16 casts (solution/lora.py:57-137): the scale and inf
 * flag of torch.amp.GradScaler are taken on the device, as by PyTorch's fused optimizers.
 */
int talm_lora_adamw(const int64_t* table, int32_t n_tensors, int64_t max_numel, float lr,
                    float beta1, float beta2, float eps, float weight_decay, const float* step_in,
                    float* step_out, const float* grad_scale, const float* found_inf,
                    uint16_t* out, void* stream);

/*
 * GradScaler.unscale_ + clip_grad_norm_ + the AdamW step without rewriting the gradients:
 * talm_lora_grad_norm computes, over every gradient of the table (entry column 6), u =
 * fl32(g * inv_scale) with inv_scale = fl32(1 / (double) *scale) (unscale_'s reciprocal) and
 * writes stats f32 [4] = {found_inf (1 when any u or the norm is not finite), inv_scale,
 * min(max_norm / (norm + 1e-6), 1) (NaN kept), norm = sqrt(sum of u^2)}: two launches, the
 * workgroup sums added in a fixed order (talm_lora_grad_norm_workspace bytes of workspace).
 * talm_lora_adamw_clipped is talm_lora_adamw with each gradient taken as fl32(fl32(g *
 * grad_mul[0]) * grad_mul[1]) (pass stats + 1: the unscaled, then clipped value the two in-place
 * ops would leave) and found_inf = stats. Replaces the unscale, norm and clip launches before the
 * optimizer step (solution/lora.py:57-137's optimizer, under the trainer's GradScaler and
 * gradient clipping).
 */
int64_t talm_lora_grad_norm_workspace(int32_t n_tensors, int64_t max_numel);
int talm_lora_grad_norm(const int64_t* table, int32_t n_tensors, int64_t max_numel,
                        const float* scale, float max_norm, void* workspace,
                        int64_t workspace_bytes, float* stats, void* stream);
int talm_lora_adamw_clipped(const int64_t* table, int32_t n_tensors, int64_t max_numel, float lr,
                            float beta1, float beta2, float eps, float weight_decay,
                            const float* step_in, float* step_out, const float* found_inf,
                            const float* grad_mul, uint16_t* out, void* stream);

/*
 * The decoded absmax of NF4 blocks: out[b] = fl32(fl32(code[absmax8[b]] * absmax2[b / qblock2])
 * + offset2[b / qblock2]) for b < n_blocks, the scale talm_nf4_group_dequant multiplies block b's
 * levels by (solution/qgroup.py:82-83, decoded once instead of per element; the frozen base
 * weights need it once). For talm_nf4_gemm.
 */
int talm_nf4_block_scales(const uint8_t* absmax8, const float* code, const float* absmax2,
                          const float* offset2, int64_t n_blocks, int32_t qblock2, float* out,
                          void* stream);

/*
 * A product on a weight W [rows, cols] held in NF4 form, dequantized inside the GEMM (never
 * written out): packed [rows * cols / 2] (two weights per byte, high nibble first) and scale
 * f32 [rows * cols / 64] (each 64-weight block's decoded absmax, talm_nf4_block_scales), both
 * starting at the weight's first element.
 *   transpose == 0: out [n_tokens, rows] = x [n_tokens, cols] W^T  (a projection's forward)
 *   transpose != 0: out [n_tokens, cols] = x [n_tokens, rows] W    (its input gradient)
 * x and out fp16 with row strides ldx / ldo (multiples of 8). The fp16 weights are bit-identical
 * to talm_nf4_group_dequant's; fp32 accumulation. blocksize 64 only; cols a multiple of 64, rows
 * a multiple of 8 (64 with transpose), rows * cols whole 16384-weight groups below 2^31;
 * x / packed / out 16-byte aligned. When the output has too few tiles to fill the chip the
 * reduction is split: the workspace (talm_nf4_gemm_workspace bytes, 0 when none is needed, -1
 * for an unsupported shape) holds the fp32 partials, summed in a fixed order (deterministic).
 * Replaces the dequantization of the layer's weights plus the projection GEMM on them
 * (solution/qgroup.py:72-99, :346-355; GroupLinear's forward and input gradient) for a
 * projection it serves.
 */
int64_t talm_nf4_gemm_workspace(int64_t n_tokens, int64_t rows, int64_t cols, int32_t transpose);
int talm_nf4_gemm(const uint16_t* x, int64_t ldx, int64_t n_tokens, const uint8_t* packed,
                  const float* scale, int64_t rows, int64_t cols, int32_t transpose,
                  int32_t blocksize, uint16_t* out, int64_t ldo, void* workspace,
                  int64_t workspace_bytes, void* stream);
/*
 * talm_nf4_gemm leaving fp32 partials [parts][n_tokens][n] (n = rows, or cols with transpose)
 * in `partials`, also when the plan has one part (talm_nf4_gemm_parts; -1 for an unsupported
 * shape); partials_bytes >= parts * n_tokens * n * 4. For the same callers as
 * talm_gemm_splitk_partials.
 */
int64_t talm_nf4_gemm_parts(int64_t n_tokens, int64_t rows, int64_t cols, int32_t transpose);
int talm_nf4_gemm_partials(const uint16_t* x, int64_t ldx, int64_t n_tokens, const uint8_t* packed,
                           const float* scale, int64_t rows, int64_t cols, int32_t transpose,
                           int32_t blocksize, float* partials, int64_t partials_bytes,
                           void* stream);

/*
 * The packed causal-LM step's per-step glue (each one launch of one workgroup for the batch
 * work). int64 tensors are contiguous; the batch is right-padded [batch, seq] (row-major).
 *
 * talm_pack_rows: the batch packed into exactly n_tokens rows (a step captured in a HIP graph).
 * Row b holds len_b = sum_t mask[b][t] real tokens (clamped to [0, seq]); they go to flat rows
 * [cu[b], cu[b+1]) with cu[0] = 0, cu[k] = min(len_0 + .. + len_{k-1}, n_tokens), and flat rows
 * [cu[batch], n_tokens) form one more sequence (cu[batch+1] = n_tokens, int32 [batch + 2]) that
 * reads the pad slot batch * seq. Per flat row j of row r at position p: src[j] = r * seq + p
 * (batch * seq for the pad sequence), ids[j] = input_ids at src (0 for the pad sequence),
 * positions[j] = p, targets[j] = labels[r][p + 1] (-100 at a row's last position and in the
 * pad sequence). batch <= 8192. Replaces the label shift and packing of the fused forward
 * (solution/patches.py:173-260 with solution/unpad.py:66-92's gather), restated for a fixed row
 * count.
 *
 * talm_row_stats: stats int64 [batch + 2] = the row lengths sum_t mask[b][t], then the number of
 * labelled positions among each row's first length positions and among all positions (position
 * t of row b is labelled when t + 1 < seq and labels[b][t + 1] >= 0). Replaces the one host
 * copy's device side of solution/unpad.py:66-92.
 *
 * talm_head_loss: loss f32 [1] = sum_i token_loss[i] / denom with denom f32 [1] = max(#i with
 * targets[i] >= 0, 1) (mode 0), *num_items (mode 1, device f32) or num_items_value (mode 2);
 * correct_bool[i] = correct[i] != 0 (bytes 0 / 1). Replaces the loss and denominator of the
 * fused head (solution/fused_head.py:272-277, :386).
 *
 * talm_scatter_rows: full_loss, full_entropy f32 [out_len] zeroed, then full[src[i]] = the row's
 * value (src outside [0, out_len) skipped; rows sharing a slot leave one of their values);
 * stats int64 [2] = (#i with correct[i] != 0 (bytes), #i with targets[i] >= 0). Replaces the scatter of
 * the per-token outputs and the step's metric sums (solution/patches.py:244-253).
 *
 * talm_scale_rows: out[i] = fp16(fp32(g[i]) * s), s = *grad_loss / *denom (0 when *denom is 0),
 * fp16 [n], 16-byte aligned. Replaces the head's backward (solution/fused_head.py:280-287).
 */
int talm_pack_rows(const int64_t* input_ids, const int64_t* mask, const int64_t* labels,
                   int32_t batch, int32_t seq, int64_t n_tokens, int64_t* ids, int64_t* positions,
                   int32_t* cu_seqlens, int64_t* targets, int64_t* src, void* stream);
int talm_row_stats(const int64_t* mask, const int64_t* labels, int32_t batch, int32_t seq,
                   int64_t* stats, void* stream);
int talm_head_loss(const float* token_loss, const int32_t* correct, const int64_t* targets,
                   int64_t n, const float* num_items, float num_items_value, int32_t mode,
                   float* loss, float* denom, uint8_t* correct_bool, void* stream);
int talm_scatter_rows(const float* token_loss, const float* entropy, const uint8_t* correct,
                      const int64_t* targets, const int64_t* src, int64_t n, int64_t out_len,
                      float* full_loss, float* full_entropy, int64_t* stats, void* stream);
int talm_scale_rows(const uint16_t* g, int64_t n, const float* grad_loss, const float* denom,
                    uint16_t* out, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* TALM_H */
