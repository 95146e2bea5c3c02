// Internal launch interface between the C-ABI (vq_capi.hip) and the kernels.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "vq_common.h"

namespace vq {

// Workgroup geometry of the streaming kernels: 256 threads, each decoding
// kRunsPerThread runs of 8 weights, so one workgroup covers
// kGroupsPerBlock groups of 256 weights.
constexpr int kStreamThreads = 256;
constexpr int kRunsPerThread = 2;
constexpr int kGroupsPerBlock = kStreamThreads * 8 * kRunsPerThread / 256;  // 16

// Lets `kern` take `lds` bytes of dynamic LDS: above 64 KiB a kernel needs
// the opt-in attribute (raised per kernel as larger sizes are asked for).
hipError_t allow_dynamic_lds(const void* kern, size_t lds);

hipError_t launch_dequant(int qtype, const uint8_t* q, float* out, int64_t ngroups, hipStream_t s);
hipError_t launch_dequant_bf16(int qtype, const uint8_t* q, bf16_t* out, int64_t ngroups, hipStream_t s);
hipError_t launch_mix(const CandSet& cs, const float* probs, bf16_t* w_eff, int64_t ngroups, hipStream_t s);
// Mixes of up to kMaxSets tensors in one launch (set i: ngroups[i] groups into out[i]).
hipError_t launch_mix_sets(int nsets, const CandSet* sets, const float* const* probs, bf16_t* const* out,
                           const int64_t* ngroups, hipStream_t s);

// Gated-Linear GEMMs (vq_gemm.hip).  All matrices are row-major bf16.
//   fwd:  Y[M][N]  = X[M][D] . W[N][D]^T          (W row stride ldw)
//   dx:   dX[M][D] = dY[M][N] . W[N][D]
//   gate: part[t][k] = sum over tile t of (dY^T X)[n][d] * W_k[n][d]
// tail_ws: fwd_tail_bytes(M, N, D) of fp32 workspace (NULL: no K-split tail tiles)
hipError_t launch_gemm_fwd(const bf16_t* X, const bf16_t* W, int64_t ldw, bf16_t* Y, int M, int N, int D,
                           float* tail_ws, hipStream_t s);
int64_t fwd_tail_bytes(int M, int N, int D);      // forward split-tail workspace bytes
// tail_ws: dx_tail_bytes(M, N, D) of fp32 workspace (NULL: no K-split tail tiles)
hipError_t launch_gemm_dx(const bf16_t* dY, const bf16_t* W, int64_t ldw, bf16_t* dX, int M, int N, int D,
                          float* tail_ws, hipStream_t s);
int device_cus();
// Makes stream `to` wait for everything queued on `from` so far (no-op when
// they are the same stream).  The events come from a small per-thread,
// per-device ring: hipStreamWaitEvent takes an event's state when it is
// called, so an event may be recorded again after it has been waited on.
hipError_t stream_fence(hipStream_t from, hipStream_t to);
int64_t gate_partial_count(int M, int N, int D);  // gate partials per candidate (one per grid block)
int64_t dx_tail_bytes(int M, int N, int D);       // dX split-tail workspace bytes
// Where the gate reduce writes dL/dp: member i's candidate k from partial
// slot i * kstride + k.
struct GateReduceOut {
    float* dprobs[kMaxSets];
    int ncand[kMaxSets];
    int kstride;
};
// Most parts per tile of a gate product that writes dW parts.
constexpr int kMaxGateParts = 8;
// Gate products at sizes whose tiles split along M 4 ways or more: parts per
// tile when the product writes fp32 dW parts and one pass takes the candidate
// dots (0: the fused epilogue), and that parts buffer's bytes.
int gate_parts(int M, int N, int D);
int64_t gate_parts_bytes(int M, int N, int D);
// Gate partials of the parts path: one per dot block, sum over members of
// ceil(n_i * row_groups / 16).
int64_t gate_dot_blocks(int nsets, const int64_t* n, int64_t row_groups);
// dwp: NULL for the fused epilogue (partials: gate_partial_count blocks),
// else gate_parts_bytes of workspace for the parts path (partials:
// gate_dot_blocks blocks); either way launch_gate_reduce* sums the partials.
// ds: the stream the parts path's dot pass runs on, after a fence on s.
hipError_t launch_gemm_gate(const bf16_t* dY, const bf16_t* X, const CandGroup& cg, float* partials, int M, int N,
                            int D, float* dwp, hipStream_t s, hipStream_t ds);
hipError_t launch_gemm_dx_gate(const bf16_t* dY, const bf16_t* W, int64_t ldw, bf16_t* dX, const bf16_t* X,
                               const CandGroup& cg, float* partials, int M, int N, int D, float* tail_ws,
                               float* dwp, hipStream_t s, hipStream_t ds);
// partials[block][nsets * kstride] = sum over the block's weights of
// dW[n][d] * W_k[n][d], dW the sum of the parts dwp in part order
hipError_t launch_gate_dot(const CandGroup& cg, int N, int D, const float* dwp, int parts, float* partials,
                           hipStream_t s);
// PTQR: Y[perm[r]] = X[perm[r]] . W_g^T for r in [group_off[g], group_off[g+1])
hipError_t launch_routed_fwd(const bf16_t* X, int M, int D, const bf16_t* const* cand_bf16, int64_t ldw, int N,
                             int ncand, const int* perm, const int* group_off, bf16_t* Y, hipStream_t s);
hipError_t launch_gate_reduce(const float* partials, int64_t ntiles, int ncand, float* dprobs, hipStream_t s);
// dprobs[k] = sum_t partials[t * stride + k], k < ncand
hipError_t launch_gate_reduce_group(const float* partials, int64_t ntiles, int stride, const GateReduceOut& out,
                                    int nmembers, hipStream_t s);
hipError_t launch_gate_reduce_strided(const float* partials, int64_t ntiles, int stride, int ncand, float* dprobs,
                                      hipStream_t s);

// Fused decode + mix GEMMs for few tokens (vq_fused.hip): W_eff is built in
// LDS tile by tile from the packed candidates and never written.
//   forward (dx = false): out = Y[M][N] = act . W_eff^T, act = X [M][D]
//   dx      (dx = true):  out = dX[M][D] = act . W_eff,  act = dY [M][N]
// ws: fused_plan(...).ws_bytes of fp32 parts (NULL when 0).
struct FusedPlan {
    int splits, per_split, grid_x, grid_z;
    int64_t ws_bytes;
};
FusedPlan fused_plan(bool dx, int M, int N, int D);
hipError_t launch_fused(bool dx, const bf16_t* act, const CandSet& cs, const float* probs, int M, int N, int D,
                        bf16_t* out, float* ws, hipStream_t s);

// Embedding rows (vq_embed.hip): one workgroup per (requested row, segment of
// at most kGroupsPerBlock groups); gused = groups covering dim.
struct EmbedPlan {
    int gused, nseg, seg;
    int64_t blocks;  // nids * nseg; also the backward's partials per candidate
};
EmbedPlan embed_plan(int64_t nids, int64_t dim);
// out[r][0:dim] (bf16, or fp32 when out_f32) = row ids[r] of the mixture
// (routing NULL) or of candidate routing[r]
hipError_t launch_embed_rows(const CandSet& cs, const float* probs, const int64_t* routing, const int64_t* ids,
                             int64_t nids, int64_t vocab, int64_t dim, void* out, bool out_f32, hipStream_t s);
// dprobs[k] = sum_r <grad[r][0:dim], W_k[ids[r]][0:dim]> (grad bf16, or fp32
// when grad_f32); partials: embed_plan(...).blocks * ncand floats
hipError_t launch_embed_rows_bwd(const CandSet& cs, const int64_t* ids, int64_t nids, int64_t vocab, int64_t dim,
                                 const void* grad, bool grad_f32, float* partials, float* dprobs, hipStream_t s);

// Decoder glue (vq_decoder.hip).
hipError_t launch_rope_qkv_fwd(const bf16_t* qkv, int64_t tokens, int S, int Hq, int Hkv, int kv_out, int D,
                               const float* cosb, const float* sinb, bf16_t* q, bf16_t* k, bf16_t* v, hipStream_t s);
hipError_t launch_rope_qkv_bwd(const bf16_t* dq, const bf16_t* dk, const bf16_t* dv, int64_t sb, int64_t sh,
                               int64_t ss, int64_t tokens, int S, int Hq, int Hkv, int D, const float* cosb,
                               const float* sinb, bf16_t* dqkv, hipStream_t s);
hipError_t launch_swiglu_fwd(const bf16_t* gu, int64_t tokens, int F, bf16_t* out, hipStream_t s);
hipError_t launch_add_rmsnorm_fwd(const bf16_t* h, const bf16_t* a, const bf16_t* w, int64_t rows, int dim, float eps,
                                 bf16_t* s_out, bf16_t* n_out, float* rstd_out, hipStream_t s);
hipError_t launch_rmsnorm_bwd(const bf16_t* dn, const bf16_t* ds, const bf16_t* x, const bf16_t* w, const float* rstd,
                              int64_t rows, int dim, bf16_t* dh, hipStream_t s);
hipError_t launch_swiglu_bwd(const bf16_t* gu, const bf16_t* dy, int64_t tokens, int F, bf16_t* dgu, hipStream_t s);

// Causal self-attention forward, head dim 64 (vq_attention.hip).  Strides are
// element strides (batch, position, head) of q, k, v, o; lse [B][H][S] fp32
// (natural log) or NULL; kv head of query head h is h / (H / Hk).
hipError_t launch_attention_fwd(const bf16_t* q, const bf16_t* k, const bf16_t* v, bf16_t* o, float* lse, int B,
                                int S, int H, int Hk, const int64_t* qs, const int64_t* ks, const int64_t* vs,
                                const int64_t* os, float scale, hipStream_t s);

// Its backward: dq, dk, dv (softmax scale `scale`) from dout, the forward's
// o and lse; strides: 8 x {batch, position, head} for q, k, v, o, dout, dq,
// dk, dv; q, o, dout, dq, dk, dv have H heads, k and v Hk (kv head of query
// head h is h / (H / Hk)); dk and dv are per query head, unsummed.  stats:
// attention_bwd_workspace(B, S, H) bytes.
int64_t attention_bwd_workspace(int B, int S, int H);
hipError_t launch_attention_bwd(const bf16_t* q, const bf16_t* k, const bf16_t* v, const bf16_t* o,
                                const bf16_t* dout, const float* lse, bf16_t* dq, bf16_t* dk, bf16_t* dv, int B,
                                int S, int H, int Hk, const int64_t* strides, float scale, float* stats,
                                hipStream_t s);

// Distillation loss over full logits (vq_loss.hip).  ws: 5 * rows + 2 floats
// (per-row log-sum-exps and losses, then 1/N_ce and 1/N), written by the
// forward and read by the backward.
hipError_t launch_distill_fwd(const bf16_t* S, const bf16_t* T, const int64_t* labels, int64_t rows, int64_t V,
                              float temperature, float* out, float* ws, hipStream_t s);
hipError_t launch_distill_bwd(const bf16_t* S, const bf16_t* T, const int64_t* labels, int64_t rows, int64_t V,
                              float temperature, const float* grad_out, bf16_t* dS, const float* ws, hipStream_t s);

}  // namespace vq
