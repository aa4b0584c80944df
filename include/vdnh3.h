/*
 * vdnh3.h - C ABI of libvdnh3.so, the MI355X (gfx950) VDN-H3 hybrid attention hot path.
 *
 * Conventions (every entry point):
 *   - plain pointers and sizes only; device buffers are caller-owned, nothing is
 *     allocated inside a compute entry point;
 *   - bf16 tensors are passed as uint16_t bit patterns, fp8 as uint8_t (OCP e4m3fn);
 *   - strides are in elements; the innermost (head_dim / K) dimension is contiguous;
 *   - `stream` is a hipStream_t (NULL = the default stream); work is enqueued
 *     asynchronously on it, like every op of the reference runs on the caller's
 *     current CUDA stream;
 *   - the return value is a VDNH3_* status; on failure vdnh3_last_error() returns a
 *     thread-local message. The Python layer maps VDNH3_ERR_INVALID to ValueError,
 *     VDNH3_ERR_RUNTIME to RuntimeError and VDNH3_ERR_LINALG to
 *     torch.linalg.LinAlgError, as the reference raises them.
 */
#ifndef VDNH3_H
#define VDNH3_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define VDNH3_OK 0
#define VDNH3_ERR_INVALID 1 /* geometry / shape / argument error (ValueError)    */
#define VDNH3_ERR_RUNTIME 2 /* HIP launch or device failure (RuntimeError)       */
#define VDNH3_ERR_LINALG 3  /* non-SPD factor reported by a host check            */

/* Anchor-frame modes, in the order of ANCHOR_FRAME_MODES (vdn_h3/window.py:18). */
#define VDNH3_ANCHOR_NONE 0
#define VDNH3_ANCHOR_COLUMNS 1
#define VDNH3_ANCHOR_ROWS 2
#define VDNH3_ANCHOR_BOTH 3

/* Thread-local message of the last failing call ("" if none). */
const char *vdnh3_last_error(void);

/* ABI version of this library (major * 100 + minor). */
int vdnh3_abi_version(void);

/* ------------------------------------------------------------------------------
 * Window attention (local-window softmax, reference vdn_h3/window.py)
 * ------------------------------------------------------------------------------ */

/*
 * Block-sparse tile plan of the window mask. Host-only, no device access.
 * Replaces the key-set construction of vdn_h3/window.py:248-270 (_window_runs),
 * :233-245 (_select_keys) and the mask of :327-344 (_window_mask_mod), and the
 * geometry validation of :162-178 (_validate_layout).
 *
 * `bounds` holds num_frames (lo, hi) pairs (window_bounds, vdn_h3/window.py:141-153).
 * The plan is a list of work items, one per (<= block_m query rows of one run):
 *   items[4*i + 0..3] = { q_start, q_end, tile_offset, tile_count }
 * and a list of key tiles of block_n keys:
 *   tiles[2*j + 0..1] = { key_start (multiple of block_n), valid_lo | valid_hi << 16 }
 * Items are sorted by descending tile_count (longest work first).
 * vdnh3_window_plan_size returns the two lengths and the number of allowed
 * (query, key) pairs per head (the FLOP model's sum_i |A(i)|).
 */
int vdnh3_window_plan_size(int seq, int video_start, int video_end, int num_frames,
                           int tokens_per_frame, const int32_t *bounds, int anchor_mode,
                           int block_m, int block_n, int32_t *n_items, int32_t *n_tiles,
                           int64_t *pairs_per_head);
int vdnh3_window_plan_build(int seq, int video_start, int video_end, int num_frames,
                            int tokens_per_frame, const int32_t *bounds, int anchor_mode,
                            int block_m, int block_n, int32_t *items, int32_t n_items,
                            int32_t *tiles, int32_t n_tiles);

/* Query/key tile sizes the attention kernel was built for. */
int vdnh3_window_block_m(void);
int vdnh3_window_block_n(void);

/* Device workspace (bytes) for vdnh3_window_attn_fwd: the V^T copy, per head one contiguous image per
 * 96-key tile in the attention kernel's LDS order (seq rounded up to 192 rows per head). */
size_t vdnh3_window_workspace_bytes(int seq, int heads, int head_dim);

/*
 * Exact local-window softmax attention, bf16 in / bf16 out, fp32 softmax and
 * accumulation. Replaces window_softmax_grouped / _flex / _flash2 / _decomposed
 * (vdn_h3/window.py:277-313, :694-723, :811-861) and the dense exact path
 * (vdn_h3/hybrid.py:295-302, a plan whose every row is dense).
 *   q, k, v  : [seq, heads, head_dim] views, element (s, h, d) at p[s*row + h*head + d]
 *   out      : [seq, heads, head_dim], same addressing
 *   gate     : optional bf16 [seq, heads] (element (s, h) at gate[s*gate_row + h]);
 *              when given, out = bf16(bf16(O) * gate), the per-head softmax gate of
 *              vdn_h3/hybrid.py:518-529 / vdn_h3/softmax_kernels.py:8-9 fused into
 *              the epilogue.
 *   items/tiles : the plan above (device copies), built with vdnh3_window_block_m/_n.
 * head_dim must be 64 or 128.
 */
int vdnh3_window_attn_fwd(const uint16_t *q, int64_t q_row, int64_t q_head,
                          const uint16_t *k, int64_t k_row, int64_t k_head,
                          const uint16_t *v, int64_t v_row, int64_t v_head,
                          uint16_t *out, int64_t o_row, int64_t o_head,
                          const uint16_t *gate, int64_t gate_row,
                          int seq, int heads, int head_dim, float scale,
                          const int32_t *items, int32_t n_items, const int32_t *tiles,
                          void *workspace, size_t workspace_bytes, void *stream);

/*
 * The two phases of vdnh3_window_attn_fwd, for callers that time or reuse them:
 * vdnh3_window_vt_prepass writes the V^T tile images into `workspace`;
 * vdnh3_window_attn_prepared runs the attention from q, k and that copy.
 */
int vdnh3_window_vt_prepass(const uint16_t *v, int64_t v_row, int64_t v_head, int seq, int heads,
                            int head_dim, void *workspace, size_t workspace_bytes, void *stream);
int vdnh3_window_attn_prepared(const uint16_t *q, int64_t q_row, int64_t q_head,
                               const uint16_t *k, int64_t k_row, int64_t k_head,
                               uint16_t *out, int64_t o_row, int64_t o_head,
                               const uint16_t *gate, int64_t gate_row,
                               int seq, int heads, int head_dim, float scale,
                               const int32_t *items, int32_t n_items, const int32_t *tiles,
                               const void *workspace, size_t workspace_bytes, void *stream);

/*
 * The attention with the block's q_norm / k_norm fused in (vdn_h3/hybrid.py:271-292 followed by
 * the window softmax of vdn_h3/hybrid.py:295-302): q and k are passed raw, as the qkv projection
 * wrote them, and normalised with the arithmetic of vdnh3_qk_rmsnorm / vdnh3_qk_rmsnorm_rope, so
 * that the result has the same bits as those calls followed by vdnh3_window_attn_prepared.
 * The workspace holds up to three regions of vdnh3_window_workspace_bytes(seq, heads, head_dim)
 * bytes each, all [heads][seq rounded up to 192][head_dim] bf16: 0 the V^T tile images, 1 the
 * normalised keys, 2 the normalised queries (zero rows past seq).
 *   vdnh3_window_norm_workspace_bytes: 2 regions, 3 with_queries; 16-byte aligned.
 *   vdnh3_window_qkv_prepass: writes regions 0 and 1 (keys: k_weight / k_eps) and, when q is not
 *     NULL, region 2 (queries: q_weight / q_eps). With freqs (the RoPE table of
 *     vdnh3_qk_rmsnorm_rope, or NULL) the normalised vectors are rotated; the reference then uses
 *     the q_norm epsilon for both: pass k_eps = q_eps.
 *   vdnh3_window_attn_qnorm: the attention from raw q, normalised as the kernel loads it (q_weight,
 *     q_eps), against regions 0 and 1 (a pre-pass with q = NULL and no freqs). With RoPE, run the
 *     pre-pass with q and pass regions 2 and 1 as q and k to vdnh3_window_attn_prepared (q_row =
 *     k_row = head_dim, q_head = k_head = seq rounded up to 192 times head_dim): a rotation in the
 *     attention kernel would re-read the table for every head and query block.
 */
size_t vdnh3_window_norm_workspace_bytes(int seq, int heads, int head_dim, int with_queries);
int vdnh3_window_qkv_prepass(const uint16_t *q, int64_t q_row, int64_t q_head, const uint16_t *q_weight, float q_eps,
                             const uint16_t *k, int64_t k_row, int64_t k_head, const uint16_t *k_weight, float k_eps,
                             const uint16_t *v, int64_t v_row, int64_t v_head, const float *freqs,
                             int64_t freqs_row, int rot_dim, int seq, int heads, int head_dim, void *workspace,
                             size_t workspace_bytes, void *stream);
int vdnh3_window_attn_qnorm(const uint16_t *q, int64_t q_row, int64_t q_head, const uint16_t *q_weight, float q_eps,
                            uint16_t *out, int64_t o_row, int64_t o_head, const uint16_t *gate, int64_t gate_row,
                            int seq, int heads, int head_dim, float scale, const int32_t *items, int32_t n_items,
                            const int32_t *tiles, const void *workspace, size_t workspace_bytes, void *stream);

/* ------------------------------------------------------------------------------
 * Projections (reference vdn_h3/projection.py, vdn_h3/fp8.py, the block's qkv/out GEMMs)
 * ------------------------------------------------------------------------------ */

#define VDNH3_GEMM_BF16 0 /* bf16 x bf16, fp32 accumulate                         */
#define VDNH3_GEMM_I8 1   /* int8 x int8, int32 accumulate                         */
#define VDNH3_GEMM_F8 2   /* fp8 e4m3fn x fp8 e4m3fn, fp32 accumulate             */
#define VDNH3_OUT_BF16 0
#define VDNH3_OUT_F32 1
#define VDNH3_OUT_I32 2   /* raw int32 accumulators (int8 operands only)           */

/*
 * C[m][n] = act( acc[m][n] * a_scale[m] * alpha * b_scale[n] + bias[n] ),  acc = sum_k A[m][k] B[n][k]
 * A: [M, K] row-major (lda), B: [N, K] row-major (ldb) - the nn.Linear weight layout - so C = A B^T.
 * a_scale / b_scale: fp32, NULL, or with 1 or M (N) entries; bias: fp32 or bf16 [N] or NULL;
 * act: 0 none, 1 sigmoid, 2 c + 1 (0 < c <= N) sigmoid on columns n < c only, the others plain
 * (two projections of the same rows in one pass, e.g. beta and the output-gate down-projection);
 * accumulate: C = bf16(C + bf16(result)) (bf16 out) or C += result (not together with the sigmoid).
 * round_linear (bf16 out): round the linear result to bf16 before the activation, as
 * torch.sigmoid(F.linear(x, W, b)) does in bf16. K * element size must be a multiple of 128 bytes.
 * Replaces F.linear (vdn_h3/projection.py:259-261, vdn_h3/branch.py:736, :754-758,
 * vdn_h3/hybrid.py:520-522), torch._scaled_mm (vdn_h3/fp8.py:254-262), comfy-kitchen
 * ck.int8_linear (vdn_h3/projection.py:243-256, without ConvRot) and the ComfyUI qkv_proj /
 * out_proj GEMMs (vdn_h3/hybrid.py:263, :535).
 */
int vdnh3_gemm(int kind, const void *A, int64_t lda, const void *B, int64_t ldb, void *C, int64_t ldc,
               int M, int N, int K, const float *a_scale, int a_scale_n, const float *b_scale,
               int b_scale_n, float alpha, const void *bias, int bias_bf16, int act, int out_type,
               int accumulate, int round_linear, void *stream);

/*
 * Row-wise symmetric quantisation of a bf16 [M, K] matrix: kind 1 = int8 (scale amax/127,
 * round half to even, clamp +-127), kind 2 = fp8 e4m3fn (scale amax/448, clamp +-448,
 * vdn_h3/fp8.py:41-54 and :99-105). scale[m] = max(amax_m / qmax, 1e-12).
 */
int vdnh3_quant_rows(int kind, const uint16_t *x, int64_t ldx, int M, int K, uint8_t *q, int64_t ldq,
                     float *scale, void *stream);

/*
 * Per-tensor fp8 quantisation of n contiguous bf16 values (vdn_h3/fp8.py:56-71, :114-126):
 * amax by a grid reduction into amax_workspace[0] (cleared by the call), then the cast;
 * scale[0] = max(amax / 448, 1e-12).
 */
int vdnh3_quant_tensor_f8(const uint16_t *x, int64_t n, uint8_t *q, float *scale, float *amax_workspace,
                          void *stream);

/*
 * No counterpart in the reference: vdnh3_quant_tensor_f8 for callers that cannot allocate device
 * memory (code under HIP graph capture, tight serving loops, harnesses that forbid hipMalloc). Same
 * codes and scale as vdnh3_quant_tensor_f8, with no workspace argument: the amax is reduced through
 * a fixed 64 KiB device array inside the library (one per GPU, held until the process ends), one
 * partial maximum per 16,384 elements, so n may not exceed
 * vdnh3_quant_tensor_f8_noalloc_max_elements() (268,435,456); larger n returns VDNH3_ERR_INVALID.
 * Allocates nothing and needs no clearing between calls; calls that overlap on one GPU race.
 */
int vdnh3_quant_tensor_f8_noalloc(const uint16_t *x, int64_t n, uint8_t *q, float *scale, void *stream);
size_t vdnh3_quant_tensor_f8_noalloc_max_elements(void);

/* ------------------------------------------------------------------------------
 * Video Delta Attention branch (reference vdn_h3/branch.py, vdn_h3/runtime.py)
 * All head_dim arguments must be 64 or 128. fp32 matrices are [n][D][D] row-major.
 * ------------------------------------------------------------------------------ */

/*
 * Frame statistics with the feature map fused in: for frame f and head h (tokens t of the
 * frame at rows f*tokens + t; element d of k at k[row*k_row + h*k_head + d], of v likewise):
 *   k~ = L2(SiLU(k)), v~ = SiLU(v) (vdn_h3/kernels.py:47-51), b = beta[row*beta_row + h] (bf16),
 *   A[f][h] = 0.5 (S + S^T), S = (k~ b)^T k~ in fp32        (vdn_h3/branch.py:197-241)
 *   B[f][h] = bf16((v~ * b)^T k~)                             (vdn_h3/branch.py:242)
 * `features` bit 0: k already holds k~; bit 1: v already holds v~ (the outputs of
 * vdnh3_short_conv, vdn_h3/runtime.py:319-341), so the feature map is not applied to it;
 * bit 2: S = bf16(bf16(k~ b)^T k~), the reference's a_fp32=False statistics
 * (vdn_h3/branch.py:238-240), instead of the fp32 product.
 * A and B are [frames][heads][D][D] fp32.
 */
int vdnh3_frame_stats(const uint16_t *k, int64_t k_row, int64_t k_head, const uint16_t *v, int64_t v_row,
                      int64_t v_head, int features, const uint16_t *beta, int64_t beta_row, int frames,
                      int tokens, int heads, int head_dim, float *A, float *B, void *stream);

/*
 * K/V (or Q) short convolutions of the branch features (vdn_h3/runtime.py:319-341,
 * vdn_h3/branch.py:443-480, vdn_h3/kernels.py:100-129). x holds frames * grid_h * grid_w rows
 * (frame-major, then row-major over the grid), element (r, h, d) at x[r*x_row + h*x_head + d]:
 *   s = bf16(depthwise kernel_h x kernel_w spatial conv per frame, zero padded)   (F.conv2d, groups=C)
 *   a = depthwise kernel_t-tap temporal conv of s over frames, zero padded, fp32 (temporal kernel)
 *   out = bf16(SiLU(a) / max(||SiLU(a)||_head, 1e-6)) with l2norm, else bf16(SiLU(a))
 * w_spatial: bf16 [heads*head_dim][kernel_h*kernel_w] (the [C,1,kh,kw] Conv2d weight);
 * w_temporal: bf16 [heads*head_dim][kernel_t] (the [C,1,kt] weight). Supported: 3x3 or 5x5 and
 * 3 or 5 taps. out: element (r, h, d) at out[r*out_row + h*out_head + d], 8-byte aligned.
 */
int vdnh3_short_conv(const uint16_t *x, int64_t x_row, int64_t x_head, const uint16_t *w_spatial, int kernel_h,
                     int kernel_w, const uint16_t *w_temporal, int kernel_t, int frames, int grid_h, int grid_w,
                     int heads, int head_dim, int l2norm, uint16_t *out, int64_t out_row, int64_t out_head,
                     void *stream);

/*
 * Several short convolutions over the same frame grid and kernel sizes in one launch (the
 * reference convolves k and v one after the other, vdn_h3/runtime.py:319-341): 1 to 4 jobs, each
 * with the operands and meaning of vdnh3_short_conv.
 */
typedef struct vdnh3_short_conv_job {
  const uint16_t *x;
  int64_t x_row, x_head;
  const uint16_t *w_spatial, *w_temporal;
  int l2norm;
  uint16_t *out;
  int64_t out_row, out_head;
} vdnh3_short_conv_job;
int vdnh3_short_conv_batch(const vdnh3_short_conv_job *jobs, int n_jobs, int kernel_h, int kernel_w, int kernel_t,
                           int frames, int grid_h, int grid_w, int heads, int head_dim, void *stream);

/*
 * VdnDelta.factor_apply (vdn_h3/branch.py:148-160) over n matrices with the status of
 * torch.linalg.cholesky_ex (vdn_h3/branch.py:62-71): L = chol(I + A), M = L^-T L^-1,
 * phi = alpha[i] * M[i][j] (phi may be NULL; alpha NULL means ones), jay = jay_scale * (B M),
 * info[i] = 0 or the order of the first non-positive leading minor.
 */
int vdnh3_delta_factor(const float *A, const float *B, const float *alpha, float *phi, float *jay,
                       float jay_scale, int32_t *info, int n, int head_dim, void *stream);

/* SanaDelta.factor_apply (vdn_h3/branch.py:163-177): phi = alpha (I - A/T), jay = jay_scale * (B / sqrt(T)),
 * each fp32 product / difference rounded on its own as the reference's tensor ops do; alpha NULL
 * means ones, phi may be NULL (not written). */
int vdnh3_sana_factor(const float *A, const float *B, const float *alpha, float *phi, float *jay,
                      float jay_scale, int tokens_per_frame, int n, int head_dim, void *stream);

/*
 * Bidirectional scans (vdn_h3/runtime.py:118-131, vdn_h3/branch.py:315-333) over
 * phi/jay [frames][heads][D][D]: prefix[f] = jay[f] + prefix[f-1] phi[f] (prefix[-1] = init),
 * suffix[f] = jay[f] + suffix[f+1] phi[f] (suffix[frames] = init); init [heads][D][D] or NULL (zeros).
 */
int vdnh3_delta_scan(const float *phi, const float *jay, const float *init, float *prefix, float *suffix,
                     int frames, int heads, int head_dim, void *stream);

/*
 * Running sums of the log decay over frames (vdn_h3/branch.py:372-396, the cumulative
 * log(alpha) of the bridge): out[i][h][d] = sum_{j<i} log(max(alpha[j][h][d], 1e-12)), i = 0..frames,
 * summed in frame order. alpha: [frames][heads][D] fp32; out: [frames+1][heads][D] fp32.
 */
int vdnh3_alpha_logsum(const float *alpha, int frames, int heads, int head_dim, float *out, void *stream);

/*
 * Gather + readout + epilogue (vdn_h3/branch.py:372-396, vdn_h3/runtime.py:406-419,
 * vdn_h3/branch.py:494-505), q~ = L2(SiLU(q)) fused in (q_features = 1: q already holds q~,
 * the output of vdnh3_short_conv). For frame f with bounds
 * lo = max(bounds[2f], 0), hi = min(bounds[2f+1], frames-1):
 *   L_f = bf16(before * decay_b + after * decay_a)  (before = prefix[lo-1] or text_state or 0,
 *         after = suffix[hi+1] or text_state or 0; when use_alpha, decay_b = exp(S[f+1] - S[lo])
 *         and decay_a = exp(S[hi+1] - S[f]) with S = alpha_logsum)
 *   r = bf16(q~ L_f^T);  out[row][h*D + v] = bf16(RMSNorm(r)[v] * norm_w[v]) * gate[row][h*D + v]
 * alpha_logsum: [frames+1][heads][D] fp32 from vdnh3_alpha_logsum (may be NULL without use_alpha);
 * out and gate: [frame_count*tokens, heads*D] bf16 with 16-byte aligned rows; prefix, suffix and
 * text_state 16-byte aligned.
 * Frame range (the reference's frame-tiled gather, vdn_h3/runtime.py:513-517, _gather_range over
 * [start, stop)): the call reads out frames first_frame .. first_frame + frame_count - 1 of the
 * `frames` frames that prefix, suffix, alpha_logsum and bounds describe; q, gate and out hold only
 * that range's rows (row 0 = the first token of frame first_frame). first_frame = 0 and
 * frame_count = frames read out every frame.
 */
int vdnh3_readout(const uint16_t *q, int64_t q_row, int64_t q_head, int q_features, const float *prefix,
                  const float *suffix, const float *alpha_logsum, const float *text_state, const int32_t *bounds,
                  int use_alpha, const uint16_t *norm_w, const uint16_t *gate, int64_t gate_row,
                  uint16_t *out, int64_t out_row, int frames, int first_frame, int frame_count, int tokens,
                  int heads, int head_dim, void *stream);

/*
 * vdnh3_readout with the output gate computed inside (vdn_h3/branch.py:754-758): for head h,
 *   gate[row][h*D + v] = bf16(sigmoid(bf16(sum_j gate_hidden[row][j] * gate_up_w[h*D + v][j] + gate_up_b[h*D + v])))
 * with gate_hidden = x W_down^T ([frame_count*tokens, D] bf16, row stride hidden_row, 16-byte aligned),
 * gate_up_w [heads*D, D] bf16 and gate_up_b [heads*D] bf16 or NULL. The same values as
 * vdnh3_gemm's sigmoid epilogue followed by vdnh3_readout, without the [rows, heads*D] gate in
 * memory. out: 8-byte aligned rows.
 */
int vdnh3_readout_fused_gate(const uint16_t *q, int64_t q_row, int64_t q_head, int q_features, const float *prefix,
                             const float *suffix, const float *alpha_logsum, const float *text_state,
                             const int32_t *bounds, int use_alpha, const uint16_t *norm_w,
                             const uint16_t *gate_hidden, int64_t hidden_row, const uint16_t *gate_up_w,
                             const uint16_t *gate_up_b, uint16_t *out, int64_t out_row, int frames,
                             int first_frame, int frame_count, int tokens, int heads, int head_dim, void *stream);

/* Per-frame mean over tokens in fp32: out[f][c] = mean_t x[(f*tokens + t)*x_row + c]
 * (vdn_h3/branch.py:743-745). */
int vdnh3_frame_mean(const uint16_t *x, int64_t x_row, int frames, int tokens, int hidden, float *out,
                     void *stream);

/* fp32 F.linear for the small alpha projections: out = x W^T (+ bias); W fp32 or bf16
 * (vdn_h3/branch.py:485-486). */
int vdnh3_linear_f32(const float *x, int64_t x_row, const void *w, int w_bf16, int64_t w_row,
                     const float *bias, float *out, int64_t out_row, int M, int N, int K, void *stream);

/* alpha = exp(-exp(a_log[h]) * softplus(delta)) over [frames][heads][D] (vdn_h3/branch.py:489-491). */
int vdnh3_alpha_decay(const float *delta, const float *a_log, float *alpha, int frames, int heads,
                      int head_dim, void *stream);

/* ------------------------------------------------------------------------------
 * Hybrid block pointwise passes (reference vdn_h3/hybrid.py, vdn_h3/softmax_kernels.py)
 * ------------------------------------------------------------------------------ */

/*
 * q_norm / k_norm of the block (vdn_h3/hybrid.py:271-273, rope_freqs=None: the attention's
 * RMSNorm modules over the head dim): y = bf16(x * rsqrt(mean(x^2) + eps) * w), fp32 statistics,
 * with q_eps for q (attn.q_norm.eps) and k_eps for k (attn.k_norm.eps).
 * q / k are [seq, heads, head_dim] views (element (s, h, d) at p[s*row + h*head + d]); the
 * results go to separate views q_out / k_out (the raw q / k stay intact for the VDN branch).
 * Weights are bf16 [head_dim]. All pointers 16-byte aligned, strides multiples of 8.
 */
int vdnh3_qk_rmsnorm(const uint16_t *q, int64_t q_row, int64_t q_head, const uint16_t *k, int64_t k_row,
                     int64_t k_head, const uint16_t *q_weight, const uint16_t *k_weight, float q_eps,
                     float k_eps, uint16_t *q_out, int64_t qo_row, int64_t qo_head, uint16_t *k_out, int64_t ko_row,
                     int64_t ko_head, int seq, int heads, int head_dim, void *stream);

/*
 * The same with RoPE (vdn_h3/hybrid.py:274-292: the fused RMSNorm + split-half rotary embedding
 * the reference runs when rope_freqs is given, comfy-kitchen rms_rope_split_half_ with
 * rot_dim = 2 * rope_freqs.shape[-3] and the q_norm epsilon for both). After the RMSNorm and
 * weight (fp32, not rounded), for i < rot_dim / 2 the pair (y_i, y_{i + rot_dim/2}) is replaced
 * by F (y_i, y_{i + rot_dim/2}) with F the 2x2 matrix of (row, i): element (r, c) at
 * freqs[row*freqs_row + 4*i + 2*r + c] (fp32, 16-byte aligned, freqs_row a multiple of 4; freqs_row = 0
 * shares one set across rows);
 * channels >= rot_dim pass unchanged; one bf16 rounding at the end. rot_dim: a multiple of 16,
 * at most head_dim.
 */
int vdnh3_qk_rmsnorm_rope(const uint16_t *q, int64_t q_row, int64_t q_head, const uint16_t *k, int64_t k_row,
                          int64_t k_head, const uint16_t *q_weight, const uint16_t *k_weight, float eps,
                          const float *freqs, int64_t freqs_row, int rot_dim, uint16_t *q_out, int64_t qo_row,
                          int64_t qo_head, uint16_t *k_out, int64_t ko_row, int64_t ko_head, int seq, int heads,
                          int head_dim, void *stream);

/*
 * apply_softmax_gate (vdn_h3/softmax_kernels.py:8-9): out[s][h*D + d] = bf16(O[s][h][d] * gate[s][h])
 * with O a [seq, heads, head_dim] bf16 view and gate bf16 (element (s, h) at gate[s*gate_row + h]).
 * The window attention kernel fuses the same gate into its epilogue; this is the standalone op.
 */
int vdnh3_head_gate(const uint16_t *o, int64_t o_row, int64_t o_head, const uint16_t *gate, int64_t gate_row,
                    uint16_t *out, int64_t out_row, int seq, int heads, int head_dim, void *stream);

/* ------------------------------------------------------------------------------
 * Token-level chunked Gated DeltaNet (chunk 64). No counterpart in the reference, whose Video
 * Delta Attention solves its delta rule per frame (vdn_h3/branch.py:148-160): this is the
 * published Gated DeltaNet recurrence in chunk (WY) form, per head with an fp32 state S (dv x dk):
 *   S_t = a_t S_{t-1} (I - b_t k_t k_t^T) + b_t v_t k_t^T,  o_t = S_t q_t,  a_t = exp(log_decay_t)
 * q, k, v: [tokens, heads, 128] bf16 views (element (t, h, d) at p[t*row + h*head + d]);
 * beta, log_decay: fp32 (element (t, h) at p[t*row + h]); out: bf16 like q; initial_state /
 * final_state: fp32 [heads][128][128] (dv rows, dk columns) or NULL (zero start / not written).
 * workspace: vdnh3_gdn_workspace_bytes(tokens, heads, 128) bytes, 16-byte aligned: one or two segment
 * buffers of at most ~1 GiB each and the fp32 state carried between segments. A call runs in
 * vdnh3_gdn_segments(tokens, heads, 128) segments (one below 64 chunks, else about 8 of at least 32
 * chunks); segment i's prep (vdnh3_gdn_prep) fills buffer i % 2 from q, k, v, beta and the log-decay,
 * and its scan (vdnh3_gdn_scan) reads that buffer and carries the state from segment i - 1 (the
 * initial_state for i = 0) to segment i + 1 (final_state for the last one) while writing out.
 * vdnh3_gdn_chunk_fwd runs prep 0, scan 0, prep 1, scan 1, ... on `stream`. A caller may instead
 * overlap them on two streams (the faster path, vdn_h3_amd.gdn): prep i after scan i - 2 (its buffer's
 * last reader), scan i after prep i and scan i - 1. The library holds no state: no streams, events
 * or allocations of its own; all buffers are the caller's.
 * ------------------------------------------------------------------------------ */
size_t vdnh3_gdn_workspace_bytes(int tokens, int heads, int head_dim);
int vdnh3_gdn_chunk_fwd(const uint16_t *q, int64_t q_row, int64_t q_head, const uint16_t *k, int64_t k_row,
                        int64_t k_head, const uint16_t *v, int64_t v_row, int64_t v_head, const float *beta,
                        int64_t beta_row, const float *log_decay, int64_t decay_row, const float *initial_state,
                        float *final_state, uint16_t *out, int64_t o_row, int64_t o_head, int tokens, int heads,
                        int head_dim, void *workspace, size_t workspace_bytes, void *stream);
int vdnh3_gdn_segments(int tokens, int heads, int head_dim);
int vdnh3_gdn_prep(const uint16_t *q, int64_t q_row, int64_t q_head, const uint16_t *k, int64_t k_row,
                   int64_t k_head, const uint16_t *v, int64_t v_row, int64_t v_head, const float *beta,
                   int64_t beta_row, const float *log_decay, int64_t decay_row, int tokens, int heads, int head_dim,
                   int segment, void *workspace, size_t workspace_bytes, void *stream);
int vdnh3_gdn_scan(const float *initial_state, float *final_state, uint16_t *out, int64_t o_row, int64_t o_head,
                   int tokens, int heads, int head_dim, int segment, void *workspace, size_t workspace_bytes,
                   void *stream);

/* ------------------------------------------------------------------------------
 * DiT block pointwise passes around attention and the MLP (reference vdn_h3/block_kernels.py)
 * Every op rounds to bf16 where the reference's torch op returns a bf16 tensor. `idx[row]`
 * (int32) selects the modulation row of each token (BlockPointwiseCache.indices,
 * vdn_h3/block_kernels.py:25-82); modulation tables are [n, hidden], fp32 (rounded to bf16 on
 * load, the reference's .to(bf16)) or bf16 (mod_bf16 / gate_bf16 = 1), row stride mod_row.
 * hidden is a multiple of 8; bf16 rows and tables are 16-byte aligned. `table_rows` is the
 * number of rows of the modulation table: a token whose idx lies outside [0, table_rows)
 * reads no table memory and its output row is NaN (the host layer raises ValueError for
 * indices it can check without a device round trip).
 * ------------------------------------------------------------------------------ */

/* _pre_body (vdn_h3/block_kernels.py:85-89): out = bf16(bf16(n * bf16(1 + scale[idx])) +
 * shift[idx]) with n = F.rms_norm(x, weight, eps) (fp32 statistics, one rounding); hidden <= 8192. */
int vdnh3_rmsnorm_modulate(const uint16_t *x, int64_t x_row, const uint16_t *weight, float eps, const void *scale,
                           const void *shift, int64_t mod_row, int mod_bf16, const int32_t *idx, int table_rows,
                           uint16_t *out, int64_t out_row, int rows, int hidden, void *stream);

/* _post_body (vdn_h3/block_kernels.py:92-93): out = bf16(x + bf16(gate[idx] * branch)); out may be x. */
int vdnh3_gated_residual(const uint16_t *x, int64_t x_row, const void *gate, int64_t gate_row, int gate_bf16,
                         const int32_t *idx, int table_rows, const uint16_t *branch, int64_t branch_row,
                         uint16_t *out, int64_t out_row, int rows, int hidden, void *stream);

/* _swiglu_body (vdn_h3/block_kernels.py:113-116): with h = [gate | up] ([rows, 2 ffn]),
 * out = bf16(bf16(silu(gate)) * up). */
int vdnh3_swiglu(const uint16_t *h, int64_t h_row, int rows, int ffn, uint16_t *out, int64_t out_row, void *stream);

/* The SwiGLU output quantised row-wise for a W8A8 fc2 (kind 1 int8, 2 fp8 e4m3fn), equal to
 * vdnh3_quant_rows(kind, swiglu(h)) without materialising the bf16 activation. */
int vdnh3_swiglu_quant_rows(int kind, const uint16_t *h, int64_t h_row, int rows, int ffn, uint8_t *q, int64_t q_row,
                            float *scale, void *stream);

/* Fill rows x cols of a bf16 matrix with a constant (anchor-frame rows of the branch output). */
int vdnh3_fill_rows_bf16(uint16_t *p, int64_t ld, int rows, int cols, float value, void *stream);

/* ------------------------------------------------------------------------------
 * Calibration (no counterpart in the reference): the sustained MFMA rate of the part on
 * caller-supplied operand bits, the ceiling the kernels' rates are read against besides the
 * datasheet peak (the part is power-limited, so the rate depends on how many bits toggle).
 * ------------------------------------------------------------------------------ */

/* Runs `blocks` workgroups of 4 wavefronts, each issuing iters x 8 independent MFMAs of `kind`
 * (0 bf16 32x32x16, 1 int8 32x32x32, 2 fp8 e4m3 32x32x64) on register-resident fragments:
 * a and b hold 8 x 64 lanes x 32 bytes each (32-byte aligned; bf16 and int8 use the first 16
 * bytes of each lane's 32). out receives blocks x 256 floats (a checksum that keeps the work live). */
int vdnh3_mfma_peak(int kind, const void *a, const void *b, int iters, int blocks, float *out, void *stream);

/* Operations (2 per multiply-add) one vdnh3_mfma_peak call performs. */
double vdnh3_mfma_peak_ops(int kind, int iters, int blocks);

#ifdef __cplusplus
}
#endif

#endif /* VDNH3_H */
