// Fused distillation loss over full logits: token cross-entropy against the
// labels plus KL(teacher || student) of the temperature-softened
// distributions, and its gradient with respect to the student logits
// (reference training/trainer.py:2566-2575: F.cross_entropy, F.log_softmax,
// F.softmax and F.kl_div over [tokens, vocab] logits, then autograd).
//
// Forward: one workgroup per token row streams the student and teacher rows
// once (16-byte loads) and keeps per-lane online log-sum-exps of s, s/T and
// t/T, plus A = sum exp(t/T - m_t) (t - s), so that
//   CE_r = lse(s) - s[y_r]
//   KL_r = T^2 (A / Z_t / T - lse(t/T) + lse(s/T))     (= T^2 sum p (log p - log q))
// and stores the three log-sum-exps of the row for the backward.  A fixed-
// order fp64 reduction gives the means (labels equal to -100 are ignored by
// the cross-entropy, as F.cross_entropy's default ignore_index).
// Backward: one more pass writes
//   dS = g_ce / N_ce (softmax(s) - onehot(y)) + g_kl T / N (softmax(s/T) - softmax(t/T)).
// At T = 1 (the trainer's default) s/T is s: both passes then take one
// exponential of s per logit instead of two (UNIT).
#include <cfloat>

#include "vq_internal.h"

namespace vq {

namespace {

constexpr int kLossThreads = 256;
constexpr float kLog2e = 1.4426950408889634f;
constexpr float kLn2 = 0.6931471805599453f;

// e^x through the hardware base-2 exponential, v_exp_f32 alone: results
// below 2^-126 flush to zero (exp2f would rescale its input around them, four
// more instructions per exponential).  Such terms sit more than 87 nats below
// the row maximum's, whose term is 1 in every sum, and the gradient elements
// they would give are below 2^-126 times the loss weights.
__device__ __forceinline__ float fexp(float x) { return __builtin_amdgcn_exp2f(x * kLog2e); }

__device__ __forceinline__ void load8_bf16(const bf16_t* p, float (&v)[8]) {
    const uint4 q = *reinterpret_cast<const uint4*>(p);
    const uint32_t w[4] = {q.x, q.y, q.z, q.w};
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        v[2 * i] = __uint_as_float(w[i] << 16);
        v[2 * i + 1] = __uint_as_float(w[i] & 0xffff0000u);
    }
}

// (m, z): z = sum exp(x - m).  Merge b into a.
__device__ __forceinline__ void lse_merge(float& ma, float& za, float mb, float zb) {
    const float m = fmaxf(ma, mb);
    za = za * fexp(ma - m) + zb * fexp(mb - m);
    ma = m;
}

struct RowAcc {
    float ms, zs;      // s
    float mq, zq;      // s / T
    float mt, zt, at;  // t / T, and sum exp(t/T - mt) (t - s)
};

__device__ __forceinline__ void acc_merge(RowAcc& a, const RowAcc& b) {
    lse_merge(a.ms, a.zs, b.ms, b.zs);
    lse_merge(a.mq, a.zq, b.mq, b.zq);
    const float m = fmaxf(a.mt, b.mt);
    const float fa = fexp(a.mt - m), fb = fexp(b.mt - m);
    a.zt = a.zt * fa + b.zt * fb;
    a.at = a.at * fa + b.at * fb;
    a.mt = m;
}

__device__ __forceinline__ RowAcc shfl_acc(const RowAcc& a, int lane) {
    RowAcc b;
    b.ms = __shfl(a.ms, lane, 64);
    b.zs = __shfl(a.zs, lane, 64);
    b.mq = __shfl(a.mq, lane, 64);
    b.zq = __shfl(a.zq, lane, 64);
    b.mt = __shfl(a.mt, lane, 64);
    b.zt = __shfl(a.zt, lane, 64);
    b.at = __shfl(a.at, lane, 64);
    return b;
}

}  // namespace

template <bool UNIT>
__global__ __launch_bounds__(kLossThreads) void distill_fwd_kernel(const bf16_t* __restrict__ S,
                                                                   const bf16_t* __restrict__ Tl,
                                                                   const int64_t* __restrict__ labels, int64_t V,
                                                                   float inv_tau, float tau2,
                                                                   float* __restrict__ stats,
                                                                   float* __restrict__ row_loss) {
    __shared__ RowAcc part[kLossThreads / 64];
    const int64_t r = blockIdx.x;
    const bf16_t* s = S + r * V;
    const bf16_t* t = Tl + r * V;
    RowAcc a{-FLT_MAX, 0.f, -FLT_MAX, 0.f, -FLT_MAX, 0.f, 0.f};
    for (int64_t i = (int64_t)threadIdx.x * 8; i < V; i += kLossThreads * 8) {
        float sv[8], tv[8];
        load8_bf16(s + i, sv);
        load8_bf16(t + i, tv);
        float cs = sv[0], ct = tv[0];
#pragma unroll
        for (int j = 1; j < 8; ++j) {
            cs = fmaxf(cs, sv[j]);
            ct = fmaxf(ct, tv[j]);
        }
        // rescale the running sums once per 8 values
        const float ns = fmaxf(a.ms, cs), nt = fmaxf(a.mt, UNIT ? ct : ct * inv_tau);
        a.zs *= fexp(a.ms - ns);
        const float ft = fexp(a.mt - nt);
        a.zt *= ft;
        a.at *= ft;
        a.ms = ns;
        a.mt = nt;
        if constexpr (!UNIT) {
            const float nq = fmaxf(a.mq, cs * inv_tau);
            a.zq *= fexp(a.mq - nq);
            a.mq = nq;
        }
#pragma unroll
        for (int j = 0; j < 8; ++j) {
            a.zs += fexp(sv[j] - ns);
            if constexpr (!UNIT) a.zq += fexp(sv[j] * inv_tau - a.mq);
            const float e = fexp((UNIT ? tv[j] : tv[j] * inv_tau) - nt);
            a.zt += e;
            a.at += e > 0.f ? e * (tv[j] - sv[j]) : 0.f;
        }
    }
    if constexpr (UNIT) {
        a.mq = a.ms;
        a.zq = a.zs;
    }
    // wave then workgroup reduction (fixed order)
#pragma unroll
    for (int off = 32; off >= 1; off >>= 1) {
        const RowAcc b = shfl_acc(a, (int)(threadIdx.x ^ off) & 63);
        acc_merge(a, b);
    }
    if ((threadIdx.x & 63) == 0) part[threadIdx.x >> 6] = a;
    __syncthreads();
    if (threadIdx.x == 0) {
        RowAcc w = part[0];
#pragma unroll
        for (int k = 1; k < kLossThreads / 64; ++k) acc_merge(w, part[k]);
        const float lse_s = w.ms + __log2f(w.zs) * kLn2;
        const float lse_q = w.mq + __log2f(w.zq) * kLn2;
        const float lse_t = w.mt + __log2f(w.zt) * kLn2;
        const int64_t y = labels[r];
        float ce = 0.f;
        if (y != -100) ce = (y >= 0 && y < V) ? lse_s - __uint_as_float((uint32_t)s[y] << 16) : __int_as_float(0x7fc00000);
        const float kl = tau2 * (w.at / w.zt * inv_tau - lse_t + lse_q);
        stats[3 * r] = lse_s;
        stats[3 * r + 1] = lse_q;
        stats[3 * r + 2] = lse_t;
        row_loss[2 * r] = ce;
        row_loss[2 * r + 1] = kl;
    }
}

// out = {CE mean over labelled rows, KL mean over all rows}; aux = {1/N_ce, 1/N}
__global__ __launch_bounds__(256) void distill_reduce_kernel(const float* __restrict__ row_loss,
                                                             const int64_t* __restrict__ labels, int64_t rows,
                                                             float* __restrict__ out, float* __restrict__ aux) {
    __shared__ double sh[3][256];
    double ce = 0.0, kl = 0.0, n = 0.0;
    for (int64_t r = threadIdx.x; r < rows; r += 256) {
        ce += (double)row_loss[2 * r];
        kl += (double)row_loss[2 * r + 1];
        n += labels[r] != -100 ? 1.0 : 0.0;
    }
    sh[0][threadIdx.x] = ce;
    sh[1][threadIdx.x] = kl;
    sh[2][threadIdx.x] = n;
    __syncthreads();
    for (int w = 128; w >= 1; w >>= 1) {
        if ((int)threadIdx.x < w) {
            sh[0][threadIdx.x] += sh[0][threadIdx.x + w];
            sh[1][threadIdx.x] += sh[1][threadIdx.x + w];
            sh[2][threadIdx.x] += sh[2][threadIdx.x + w];
        }
        __syncthreads();
    }
    if (threadIdx.x == 0) {
        out[0] = (float)(sh[0][0] / sh[2][0]);  // 0/0 = NaN with no labelled row, as torch's mean
        out[1] = (float)(sh[1][0] / (double)rows);
        aux[0] = (float)(1.0 / sh[2][0]);
        aux[1] = (float)(1.0 / (double)rows);
    }
}

template <bool UNIT>
__global__ __launch_bounds__(kLossThreads) void distill_bwd_kernel(const bf16_t* __restrict__ S,
                                                                   const bf16_t* __restrict__ Tl,
                                                                   const int64_t* __restrict__ labels, int64_t V,
                                                                   float inv_tau, float tau,
                                                                   const float* __restrict__ stats,
                                                                   const float* __restrict__ aux,
                                                                   const float* __restrict__ grad_out,
                                                                   bf16_t* __restrict__ dS) {
    const int64_t r = blockIdx.x;
    const bf16_t* s = S + r * V;
    const bf16_t* t = Tl + r * V;
    bf16_t* d = dS + r * V;
    const float lse_s = stats[3 * r], lse_q = stats[3 * r + 1], lse_t = stats[3 * r + 2];
    const int64_t y = labels[r];
    const float a = y != -100 ? grad_out[0] * aux[0] : 0.f;  // dL/dCE_mean / N_ce
    const float b = grad_out[1] * tau * aux[1];              // dL/dKL_mean * T^2 / T / N
    for (int64_t i = (int64_t)threadIdx.x * 8; i < V; i += kLossThreads * 8) {
        float sv[8], tv[8], g[8];
        load8_bf16(s + i, sv);
        load8_bf16(t + i, tv);
#pragma unroll
        for (int j = 0; j < 8; ++j) {
            const float es = fexp(sv[j] - lse_s);
            const float ps = es - ((i + j) == y ? 1.f : 0.f);
            const float dq = UNIT ? es - fexp(tv[j] - lse_t)
                                  : fexp(sv[j] * inv_tau - lse_q) - fexp(tv[j] * inv_tau - lse_t);
            g[j] = a * ps + b * dq;
        }
        uint4 q;
        q.x = f2bf2(g[0], g[1]);
        q.y = f2bf2(g[2], g[3]);
        q.z = f2bf2(g[4], g[5]);
        q.w = f2bf2(g[6], g[7]);
        *reinterpret_cast<uint4*>(d + i) = q;
    }
}

hipError_t launch_distill_fwd(const bf16_t* S, const bf16_t* T, const int64_t* labels, int64_t rows, int64_t V,
                              float temperature, float* out, float* ws, hipStream_t s) {
    float* stats = ws;
    float* row_loss = ws + 3 * rows;
    float* aux = ws + 5 * rows;
    if (temperature == 1.0f)
        distill_fwd_kernel<true><<<dim3((unsigned)rows), kLossThreads, 0, s>>>(S, T, labels, V, 1.0f, 1.0f, stats,
                                                                            row_loss);
    else
        distill_fwd_kernel<false><<<dim3((unsigned)rows), kLossThreads, 0, s>>>(
            S, T, labels, V, 1.0f / temperature, temperature * temperature, stats, row_loss);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return e;
    distill_reduce_kernel<<<1, 256, 0, s>>>(row_loss, labels, rows, out, aux);
    return hipGetLastError();
}

hipError_t launch_distill_bwd(const bf16_t* S, const bf16_t* T, const int64_t* labels, int64_t rows, int64_t V,
                              float temperature, const float* grad_out, bf16_t* dS, const float* ws, hipStream_t s) {
    if (temperature == 1.0f)
        distill_bwd_kernel<true><<<dim3((unsigned)rows), kLossThreads, 0, s>>>(S, T, labels, V, 1.0f, 1.0f, ws,
                                                                            ws + 5 * rows, grad_out, dS);
    else
        distill_bwd_kernel<false><<<dim3((unsigned)rows), kLossThreads, 0, s>>>(
            S, T, labels, V, 1.0f / temperature, temperature, ws, ws + 5 * rows, grad_out, dS);
    return hipGetLastError();
}

}  // namespace vq
