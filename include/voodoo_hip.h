/*
 * voodoo_hip.h - C ABI of libvoodoo_hip.so, the MI355X (gfx950) kernels of the
 * gated-mixture Linear:
 *
 *     W_eff = sum_k softmax(g / T)_k * W_k        (K GGUF-packed candidates)
 *     Y     = X . W_eff^T
 *     dX    = dY . W_eff,   dL/dp_k = <dY^T X, W_k>
 *
 * Conventions
 *   - Matrices are row-major.  bf16 values travel as uint16_t bit patterns.
 *   - qtype is the ggml type id: 8 Q8_0, 10 Q2_K, 11 Q3_K, 12 Q4_K, 13 Q5_K,
 *     14 Q6_K, 16 IQ2_XXS, 17 IQ2_XS, 18 IQ3_XXS, 19 IQ1_S, 21 IQ3_S, 22 IQ2_S,
 *     23 IQ4_XS, 29 IQ1_M (the reference's quant registry, voodoo_quant/
 *     ggml.py:51-66, less the ternary TQ1_0/TQ2_0).  A candidate is the ggml byte stream of an [N][D_pad] weight
 *     (rows back to back, D_pad a multiple of 256 as in the reference's
 *     256-padding of in_features, voodoo_quant/layers.py:973-997).
 *   - Every pointer except `stream` and the host arrays `qtypes`/`qbytes` is a
 *     device pointer.  The caller owns all memory; the library allocates none.
 *   - Calls are asynchronous on `stream` (a hipStream_t; NULL = the default
 *     stream) and never synchronise the host.
 *   - Return value: VQ_OK or a VQ_ERR_* code; vq_last_error_string() gives the
 *     message of the calling thread's last failure.  Validation errors mirror
 *     the reference's ValueError cases (ggml.py:195-198, 242-253).
 */
#ifndef VOODOO_HIP_H
#define VOODOO_HIP_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define VQ_OK 0
#define VQ_ERR_QTYPE 1       /* unsupported quant type */
#define VQ_ERR_ALIGN 2       /* block or vector alignment violated */
#define VQ_ERR_NULL 3        /* a required pointer is NULL */
#define VQ_ERR_SHAPE 4       /* inconsistent or unsupported sizes */
#define VQ_ERR_HIP 5         /* a HIP runtime call failed */
#define VQ_ERR_WORKSPACE 6   /* workspace missing or too small */

/* Library ABI version (major * 100 + minor). */
int vq_version(void);

/* Message of the calling thread's most recent failed call ("" if none). */
const char *vq_last_error_string(void);

/* Bytes of one 256-weight group of `qtype` (Q8_0: eight 34-byte blocks = 272),
 * 0 when the type is unsupported.  Replaces QuantTypeInfo.block_bytes /
 * block_size arithmetic of voodoo_quant/ggml.py:30-48 for the six formats. */
int64_t vq_group_bytes(int qtype);

/* Packed size of an [nrows][ncols] tensor, or -1 when ncols is not a multiple
 * of the type's block size (the reference's ValueError, ggml.py:195-198). */
int64_t vq_qbytes_size(int qtype, int64_t nrows, int64_t ncols);

/* Host-side checks of a candidate set (no GPU work): supported types, D_pad a
 * multiple of 256, D <= D_pad, N and D multiples of 8, 1 <= ncand <= 16. */
int vq_validate_candidates(int ncand, const int *qtypes, int64_t n, int64_t d, int64_t d_pad);

/* out[nrows*ncols] fp32 = ggml dequantize_row_<qtype>(qbytes) bit for bit.
 * Replaces dequantize_tensor_gpu (voodoo_quant/layers.py:298-319) and the
 * per-type torch decoders (layers.py:62-213). */
int vq_dequant(int qtype, const void *qbytes, float *out, int64_t nrows, int64_t ncols, void *stream);

/* out[nrows*ncols] bf16 = bf16(ggml dequantize_row_<qtype>(qbytes)) with torch's
 * rounding: the source-dtype candidate the reference's lazy path decodes
 * (voodoo_quant/layers.py:298-319, 514-556). */
int vq_dequant_bf16(int qtype, const void *qbytes, uint16_t *out, int64_t nrows, int64_t ncols, void *stream);

/* w_eff[n][d_pad] bf16 = bf16(sum_k probs[k] * dequant(qbytes[k])), mixed in
 * fp32 in k order with separately rounded products and sums.  Replaces
 * _MixedWeightFunction.forward (voodoo_quant/layers.py:336-352). */
int vq_mix_weight(int ncand, const int *qtypes, const void *const *qbytes, const float *probs, int64_t n,
                  int64_t d_pad, uint16_t *w_eff, void *stream);

/* Workspace bytes vq_gated_linear_fwd can use: fp32 partial tiles for the
 * K-split parts of the GEMM's last tiles (0 when the shape needs none). */
int64_t vq_gated_linear_fwd_workspace(int64_t m, int64_t n, int64_t d);

/* y[m][n] = x[m][d] . w^T for a bf16 weight w[n][ldw] already in memory (the
 * forward GEMM of vq_gated_linear_fwd without the mix).  `workspace` is
 * optional as there (vq_gated_linear_fwd_workspace bytes).  Replaces the
 * F.linear of Q8Linear.forward over its decoded weight
 * (voodoo_quant/training/q8_teacher.py:121-122). */
int vq_linear_fwd(const uint16_t *x, int64_t m, int64_t n, int64_t d, const uint16_t *w, int64_t ldw, uint16_t *y,
                  void *workspace, int64_t ws_bytes, void *stream);

/* Forward of the gated Linear: mixes W_eff into `w_eff` ([n][d_pad] bf16,
 * caller-owned, kept for the backward) and writes y[m][n] = x[m][d] . W_eff^T.
 * `workspace` (optional, ws_bytes >= vq_gated_linear_fwd_workspace) lets the
 * GEMM split its last round of tiles along K; NULL runs them whole.  With
 * m == 0 it only mixes (x and y may then be NULL).
 * Replaces get_mixed_weight + F.linear in MixedQuantLinear.forward
 * (voodoo_quant/layers.py:1729-1731). */
int vq_gated_linear_fwd(const uint16_t *x, int64_t m, int64_t n, int64_t d, int64_t d_pad, int ncand,
                        const int *qtypes, const void *const *qbytes, const float *probs, uint16_t *w_eff,
                        uint16_t *y, void *workspace, int64_t ws_bytes, void *stream);

/* Workspace bytes of vq_gated_linear_fwd_fused (dx == 0) or
 * vq_gated_linear_dx_fused (dx != 0): fp32 parts of the reduction, split
 * across workgroups when the output alone gives too few (0: no split). */
int64_t vq_gated_linear_fused_workspace(int64_t m, int64_t n, int64_t d, int dx);

/* The gated Linear's products for few tokens with W_eff never in memory: each
 * workgroup decodes the K candidates' packed bytes for its 32-row x 256-weight
 * tiles into LDS, mixes them with probs in fp32 (fma(p_k dl, u, acc): within
 * a bf16 ulp of vq_mix_weight's W_eff, not bit-identical) and multiplies them
 * there.  The tiles are decoded again for every 32 tokens, so the caller
 * picks these below a measured token count and the materialising entry
 * points above it.
 *   vq_gated_linear_fwd_fused: y[m][n] = x[m][d] . W_eff^T
 *     (replaces get_mixed_weight + F.linear, voodoo_quant/layers.py:1729-1731);
 *   vq_gated_linear_dx_fused: dx[m][d] = dy[m][n] . W_eff
 *     (the dX half of the backward, voodoo_quant/layers.py:354-363 via
 *     F.linear's autograd; dL/dp comes from vq_gated_linear_bwd with dx NULL,
 *     whose gate product never needs W_eff).
 * workspace: vq_gated_linear_fused_workspace bytes. */
int vq_gated_linear_fwd_fused(const uint16_t *x, int64_t m, int64_t n, int64_t d, int64_t d_pad, int ncand,
                              const int *qtypes, const void *const *qbytes, const float *probs, uint16_t *y,
                              void *workspace, int64_t ws_bytes, void *stream);
int vq_gated_linear_dx_fused(const uint16_t *dy, int64_t m, int64_t n, int64_t d, int64_t d_pad, int ncand,
                             const int *qtypes, const void *const *qbytes, const float *probs, uint16_t *dx,
                             void *workspace, int64_t ws_bytes, void *stream);

/* Per-token quant routing (PTQR) forward: y[t] = x[t] . W_{k(t)}^T, every
 * token through ONE candidate.  perm (device int32 [m]) lists the tokens
 * grouped by candidate, group_off (device int32 [ncand + 1]) the group bounds
 * in perm (group_off[0] = 0, group_off[ncand] = m); cand_bf16[k] (device
 * [n][d_pad]) is candidate k decoded by vq_dequant_bf16.  Entries outside
 * [0, m) are skipped.  Requires m * d_pad * 2 < 2^31.  Replaces
 * _RoutedMixedLinear.forward (voodoo_quant/layers.py:383-406); its backward is
 * vq_gated_linear_bwd (layers.py:408-429 computes the same dX and dL/dp). */
int vq_routed_linear_fwd(const uint16_t *x, int64_t m, int64_t n, int64_t d, int64_t d_pad, int ncand,
                         const uint16_t *const *cand_bf16, const int32_t *perm, const int32_t *group_off,
                         uint16_t *y, void *stream);

/* Embedding rows of the packed candidates (vocabulary [num_embeddings][d_pad],
 * every candidate's rows stored as d_pad/256 consecutive groups):
 *   routing == NULL: out[r][0:dim] = row ids[r] of
 *       sum_k probs[k] * dequant(qbytes[k]) mixed in fp32 in k order with
 *       separately rounded products and sums; as bf16 it is bit-identical to
 *       the same row of vq_mix_weight's W_eff;
 *   routing != NULL (device int64 [nids], PTQR): out[r] = row ids[r] of
 *       candidate routing[r] (probs unused): ggml's value, bf16-rounded as
 *       vq_dequant_bf16 does or exact in fp32.
 * ids: device int64 [nids].  An id outside [0, num_embeddings), or a route
 * outside [0, ncand), gives a zero row.  dim % 8 == 0; out is [nids][dim],
 * bf16 (out_f32 == 0) or fp32 (out_f32 != 0), 16-byte aligned.
 * Replaces the row-select lookup of _MixedEmbeddingRowFunctionLazy.forward
 * (voodoo_quant/layers.py:684-728), _RoutedEmbeddingRowFunction.forward
 * (layers.py:764-779) and, with one Q8_0 candidate and probs = {1},
 * Q8Embedding.forward (voodoo_quant/training/q8_teacher.py:156-173). */
int vq_embedding_rows_fwd(int ncand, const int *qtypes, const void *const *qbytes, const float *probs,
                          const int64_t *routing, const int64_t *ids, int64_t nids, int64_t num_embeddings,
                          int64_t dim, int64_t d_pad, void *out, int out_f32, void *stream);

/* Workspace bytes vq_embedding_rows_bwd needs (one fp32 partial per
 * workgroup and candidate). */
int64_t vq_embedding_rows_bwd_workspace(int64_t nids, int64_t dim, int ncand);

/* dprobs[k] = sum_r <grad[r][0:dim], W_k[ids[r]][0:dim]> (fp32 [ncand]; the
 * candidates decoded exactly, partials reduced in a fixed order in fp64).
 * grad: device [nids][dim], bf16 (grad_f32 == 0) or fp32.  Replaces _MixedEmbeddingRowFunctionLazy.backward
 * (voodoo_quant/layers.py:730-750) and _RoutedEmbeddingRowFunction.backward
 * (layers.py:781-790). */
int vq_embedding_rows_bwd(int ncand, const int *qtypes, const void *const *qbytes, const int64_t *ids,
                          int64_t nids, int64_t num_embeddings, int64_t dim, int64_t d_pad, const void *grad,
                          int grad_f32, float *dprobs, void *workspace, int64_t ws_bytes, void *stream);

/* Gated tensors that read the same input (q/k/v, gate/up), stacked along N:
 * member i has n[i] rows (a multiple of 256 when nmembers > 1), ncand[i]
 * candidates whose types and byte pointers follow the previous members' in
 * qtypes/qbytes, and probs[i] (device fp32 [ncand[i]]).  Mixes every member
 * into its rows of w_eff ([sum n][d_pad] bf16) and runs ONE GEMM:
 * y[m][sum n] = x . w_eff^T (member i's outputs are columns
 * [n[0] + ... + n[i-1], ... + n[i]) of y).  1 <= nmembers <= 4; with m == 0
 * only the mixes run (x and y may be NULL).  Replaces the
 * separate forwards of MixedQuantLinear (voodoo_quant/layers.py:1729-1731)
 * for projections of one input; no counterpart entry in the reference. */
int vq_gated_linear_group_fwd(const uint16_t *x, int64_t m, int64_t d, int64_t d_pad, int nmembers, const int64_t *n,
                              const int *ncand, const int *qtypes, const void *const *qbytes,
                              const float *const *probs, uint16_t *w_eff, uint16_t *y, void *workspace,
                              int64_t ws_bytes, void *stream);

/* Workspace bytes of vq_gated_linear_group_bwd (gate partials of every member
 * and dX's split tail tiles). */
int64_t vq_gated_linear_group_bwd_workspace(int64_t m, int64_t d, int nmembers, const int64_t *n, const int *ncand);

/* Backward of the stacked group: dx = dy . w_eff (one GEMM over the stacked
 * rows, which also sums the members' input gradients) and, for each member,
 * dprobs[i][k] = <dy_i^T x, W_ik> (device fp32 [ncand[i]]), all in one
 * launch.  dy: [m][sum n] bf16; w_eff: the forward's.  dprobs may be NULL
 * (no gate gradients), dx may be NULL.  Replaces the members' F.linear
 * backwards and _MixedWeightFunction.backward (voodoo_quant/layers.py:354-363). */
int vq_gated_linear_group_bwd(const uint16_t *dy, const uint16_t *x, int64_t m, int64_t d, int64_t d_pad, int nmembers,
                              const int64_t *n, const int *ncand, const int *qtypes, const void *const *qbytes,
                              const uint16_t *w_eff, uint16_t *dx, float *const *dprobs, void *workspace,
                              int64_t ws_bytes, void *stream);

/* vq_gated_linear_group_bwd with the gate gradients finished on `gate_stream`:
 * the products run on `stream`; the dot pass over dW parts (where the shape
 * takes it) and the fixed-order reduce into dprobs run on `gate_stream`,
 * after an event fence on `stream`.  The caller keeps the workspace and
 * dprobs alive until `gate_stream` has passed them, and makes its readers of
 * dprobs wait for `gate_stream`.  Values are bit-identical to
 * vq_gated_linear_group_bwd's.  No counterpart in the reference (its gate
 * gradients come from autograd in stream order, layers.py:354-363). */
int vq_gated_linear_group_bwd_gate_stream(const uint16_t *dy, const uint16_t *x, int64_t m, int64_t d, int64_t d_pad,
                                          int nmembers, const int64_t *n, const int *ncand, const int *qtypes,
                                          const void *const *qbytes, const uint16_t *w_eff, uint16_t *dx,
                                          float *const *dprobs, void *workspace, int64_t ws_bytes, void *stream,
                                          void *gate_stream);

/* Decoder-layer glue of the gate-training step (the model the trainer runs
 * around the gated projections; no counterpart in voodoo_quant itself).
 * vq_rope_qkv_fwd: qkv [B*S][(Hq + 2 Hkv) D] bf16 (stacked q/k/v projection
 * output) -> q [B*S][Hq][D] and k, v [B*S][kv_heads_out][D] bf16: rotary
 * embedding on q and k (y = x cos + [-x2, x1] sin with cos/sin fp32 [S][D]);
 * kv_heads_out = Hq repeats each K/V head Hq / Hkv times, kv_heads_out = Hkv
 * keeps them as they are (for vq_attention_fwd/_bwd, which read K/V head
 * h / (Hq/Hkv) themselves).  D % 16 == 0, Hq % Hkv == 0. */
int vq_rope_qkv_fwd(const uint16_t *qkv, int64_t B, int64_t S, int Hq, int Hkv, int kv_heads_out, int D,
                    const float *cosb, const float *sinb, uint16_t *q, uint16_t *k, uint16_t *v, void *stream);

/* Backward of vq_rope_qkv_fwd: dq, dk, dv [B][Hq][S][D] with element strides
 * (stride_b, stride_h, stride_s; multiples of 8; unit stride along D) ->
 * dqkv [B*S][(Hq + 2 Hkv) D] (inverse rotation, repeated heads summed). */
int vq_rope_qkv_bwd(const uint16_t *dq, const uint16_t *dk, const uint16_t *dv, int64_t stride_b, int64_t stride_h,
                    int64_t stride_s, int64_t B, int64_t S, int Hq, int Hkv, int D, const float *cosb,
                    const float *sinb, uint16_t *dqkv, void *stream);

/* out [tokens][F] = silu(gu[:, :F]) * gu[:, F:] for the stacked gate/up
 * projection output gu [tokens][2F] (F % 8 == 0), and its backward
 * dgu [tokens][2F] from dy [tokens][F]. */
int vq_swiglu_fwd(const uint16_t *gu, int64_t tokens, int64_t F, uint16_t *out, void *stream);
int vq_swiglu_bwd(const uint16_t *gu, const uint16_t *dy, int64_t tokens, int64_t F, uint16_t *dgu, void *stream);

/* Residual add + RMSNorm in one pass over rows of dim bf16 (dim % 8 == 0):
 * s = h + a (bf16, torch's add; a may be NULL: a plain RMSNorm of h, s_out
 * unused), n = s * rstd * w with rstd = 1 / sqrt(mean(s^2) + eps) in fp32
 * and one bf16 rounding (F.rms_norm).  rstd_out (fp32 [rows]) and s_out may
 * be NULL when no backward follows.  vq_rmsnorm_bwd: dh = ds + rstd (dn w -
 * s rstd mean(dn w s rstd)), the gradient of both h and a (ds may be NULL);
 * the norm weight's gradient is not formed (the trainer freezes it). */
int vq_add_rmsnorm_fwd(const uint16_t *h, const uint16_t *a, const uint16_t *w, int64_t rows, int64_t dim, float eps,
                       uint16_t *s_out, uint16_t *n_out, float *rstd_out, void *stream);
int vq_rmsnorm_bwd(const uint16_t *dn, const uint16_t *ds, const uint16_t *s, const uint16_t *w, const float *rstd,
                   int64_t rows, int64_t dim, uint16_t *dh, void *stream);

/* Causal self-attention forward of the decoder step: per (batch b, query
 * head h), o[i] = sum_{j <= i} softmax_j(scale q[i].k[j]) v[j] over positions
 * 0 .. S-1 (torch's scaled_dot_product_attention with is_causal=True), key/
 * value head h / (Hq / Hk).  q, o: bf16 [B][S][Hq][64]-indexed through
 * element strides {batch, position, head} (q_strides, o_strides), k, v
 * likewise with Hk heads; unit stride along the head dim, strides multiples
 * of 8 (k/v position strides at most 2^22), pointers 16-byte aligned.
 * Scores and softmax in fp32, probabilities
 * rounded to bf16 for the value product.  lse (fp32 [B][Hq][S], natural-log
 * log-sum-exp of the scaled scores per query; may be NULL) is the saved
 * state torch's memory-efficient attention backward reads.  Only head dim 64.
 * No counterpart in voodoo_quant (the step's attention is outside the gated
 * path); it replaces F.scaled_dot_product_attention's forward in the step. */
int vq_attention_fwd(const uint16_t *q, const uint16_t *k, const uint16_t *v, uint16_t *o, float *lse, int64_t B,
                     int64_t S, int Hq, int Hk, int D, const int64_t *q_strides, const int64_t *k_strides,
                     const int64_t *v_strides, const int64_t *o_strides, float scale, void *stream);

/* Backward of vq_attention_fwd: dq, dk, dv (bf16, softmax scale `scale`)
 * from dout and the forward's o and lse.  q, o, dout, dq, dk, dv have Hq
 * heads, k and v Hk (Hq % Hk == 0; query head h reads K/V head h / (Hq/Hk)).
 * dk and dv are per query head, [B][S][Hq][D]: the gradients of K and V with
 * each head repeated Hq/Hk times, so at Hk < Hq the gradient of K/V head j is
 * the sum of query heads j (Hq/Hk) .. (j+1) (Hq/Hk) - 1 (the decoder step's
 * vq_rope_qkv_bwd forms it).  strides: 24 int64, the {batch, position, head}
 * element strides of q, k, v, o, dout, dq, dk, dv (multiples of 8; unit
 * stride along the head dim; q/k/v/dout position strides at most 2^22).  Two launches, no atomics: dq (which also writes
 * lse log2 e and -D, D = rowsum(dout o o), per query into the workspace,
 * padded to a multiple of 128 queries), then dk and dv; deterministic.
 * workspace: vq_attention_bwd_workspace(B, S, Hq) bytes, 16-byte aligned,
 * device memory.
 * Only head dim 64.  No counterpart in voodoo_quant; it replaces the
 * memory-efficient attention backward of the step. */
int64_t vq_attention_bwd_workspace(int64_t B, int64_t S, int Hq);
int vq_attention_bwd(const uint16_t *q, const uint16_t *k, const uint16_t *v, const uint16_t *o, const uint16_t *dout,
                     const float *lse, uint16_t *dq, uint16_t *dk, uint16_t *dv, int64_t B, int64_t S, int Hq, int Hk,
                     int D, const int64_t *strides, float scale, void *workspace, int64_t ws_bytes, void *stream);

/* Workspace bytes of the distillation loss (per-row log-sum-exps and losses;
 * written by vq_distill_loss_fwd, read by vq_distill_loss_bwd). */
int64_t vq_distill_loss_workspace(int64_t rows);

/* out[0] = mean over rows with labels != -100 of cross-entropy(logits, labels);
 * out[1] = mean over rows of T^2 KL(softmax(teacher / T) || softmax(logits / T)).
 * logits, teacher_logits: device bf16 [rows][vocab], vocab % 8 == 0; labels:
 * device int64 [rows] (a label outside [0, vocab) other than -100 gives a NaN
 * cross-entropy).  Sums run in fp64 in a fixed order.  Replaces the
 * full-logits losses of the trainer (voodoo_quant/training/trainer.py:2566-2575:
 * F.cross_entropy, F.log_softmax, F.softmax, F.kl_div ... .sum(-1) * T^2, .mean()). */
int vq_distill_loss_fwd(const uint16_t *logits, const uint16_t *teacher_logits, const int64_t *labels, int64_t rows,
                        int64_t vocab, float temperature, float *out, void *workspace, int64_t ws_bytes, void *stream);

/* grad_logits (bf16 [rows][vocab]) = grad_out[0] d out[0] / d logits + grad_out[1] d out[1] / d logits,
 * with grad_out a device fp32 [2] and the forward's workspace.  Replaces the
 * autograd backward of those losses. */
int vq_distill_loss_bwd(const uint16_t *logits, const uint16_t *teacher_logits, const int64_t *labels, int64_t rows,
                        int64_t vocab, float temperature, const float *grad_out, uint16_t *grad_logits,
                        const void *workspace, int64_t ws_bytes, void *stream);

/* Workspace bytes vq_gated_linear_bwd needs (gate partials; plus the W_eff
 * buffer when it will be called with w_eff == NULL and dx != NULL). */
int64_t vq_gated_linear_bwd_workspace(int64_t m, int64_t n, int64_t d, int64_t d_pad, int ncand, int need_w_eff);

/* Backward of the gated Linear.  dx (nullable) = dy . W_eff;
 * dprobs (nullable) [ncand] fp32 = <dy^T x, W_k> with the dW tiles kept on
 * chip (registers and LDS) and the candidates decoded exactly; at shapes with
 * few dW tiles (the plan splits each along m 4 ways or more) the tiles' fp32
 * parts go through the workspace (at most 64 MiB) and one pass takes the
 * dots.  `w_eff` is
 * the forward's buffer, or NULL to re-mix into the workspace.  Replaces the
 * F.linear autograd backward and _MixedWeightFunction.backward
 * (voodoo_quant/layers.py:354-363). */
int vq_gated_linear_bwd(const uint16_t *dy, const uint16_t *x, int64_t m, int64_t n, int64_t d, int64_t d_pad,
                        int ncand, const int *qtypes, const void *const *qbytes, const float *probs,
                        const uint16_t *w_eff, uint16_t *dx, float *dprobs, void *workspace, int64_t ws_bytes,
                        void *stream);

/* vq_gated_linear_bwd with the gate gradient finished on `gate_stream` (the
 * dot pass over dW parts where the shape takes it, and the fixed-order
 * reduce into dprobs), after an event fence on `stream`, where the products
 * run.  The caller keeps the workspace and dprobs alive until `gate_stream`
 * has passed them and makes readers of dprobs wait for `gate_stream`.
 * Values are bit-identical to vq_gated_linear_bwd's.  No counterpart in the
 * reference (layers.py:354-363 finishes the gate gradient in stream order). */
int vq_gated_linear_bwd_gate_stream(const uint16_t *dy, const uint16_t *x, int64_t m, int64_t n, int64_t d,
                                    int64_t d_pad, int ncand, const int *qtypes, const void *const *qbytes,
                                    const float *probs, const uint16_t *w_eff, uint16_t *dx, float *dprobs,
                                    void *workspace, int64_t ws_bytes, void *stream, void *gate_stream);

/* Bytes of the library's static scratch (per device, held until the process
 * ends) behind vq_gated_linear_bwd_static. */
#define VQ_STATIC_SCRATCH_BYTES (4 << 20)

/* vq_gated_linear_bwd with no workspace and no allocation of any kind: the
 * gate partials live in a static device array of VQ_STATIC_SCRATCH_BYTES,
 * dX runs whole tiles (no split tail: its partials would need 16 MiB or
 * more), and dx needs the forward's w_eff (no re-mix).  Sizes whose gate
 * partials exceed the scratch return VQ_ERR_WORKSPACE.  Every call on a
 * device shares that device's scratch: calls that overlap on one device
 * (concurrent streams, threads) race and must be serialised by the caller.
 * dprobs is bit-identical to vq_gated_linear_bwd's; dx is bit-identical to
 * vq_gated_linear_bwd's when that one runs without a workspace.
 * No counterpart in the reference: this entry point is for callers that
 * cannot allocate (code under HIP graph capture, tight serving loops,
 * harnesses that forbid hipMalloc). */
int vq_gated_linear_bwd_static(const uint16_t *dy, const uint16_t *x, int64_t m, int64_t n, int64_t d, int64_t d_pad,
                               int ncand, const int *qtypes, const void *const *qbytes, const uint16_t *w_eff,
                               uint16_t *dx, float *dprobs, void *stream);

#ifdef __cplusplus
}
#endif

#endif /* VOODOO_HIP_H */
