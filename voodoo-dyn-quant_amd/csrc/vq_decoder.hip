// Decoder-layer glue around the gated projections, fused so the step does not
// pay a dozen elementwise passes per layer:
//   rope_qkv:  the stacked q/k/v projection output [tokens][(Hq + 2 Hkv) D]
//              -> q, k, v as [tokens][Hq][D] (the [B, S, H, D] memory layout),
//              rotary embedding applied to q and k (rotate-half form:
//              y = x cos + [-x2, x1] sin), K/V heads repeated Hq / Hkv times
//              for grouped-query attention; the backward undoes all three
//              (inverse rotation, sum over the repeated heads, back into the
//              stacked layout the grouped backward reads).
//   swiglu:    the stacked gate/up output [tokens][2F] -> silu(g) * u [tokens][F],
//              and its gradient back into [tokens][2F].
//   add_rmsnorm: the residual add and the RMSNorm that follows it, one pass:
//              s = h + a (bf16, as torch's add), n = s * rstd * w with
//              rstd = 1 / sqrt(mean(s^2) + eps); its backward
//              dh = ds + rstd (dn w - s rstd mean(dn w s rstd)) is also the
//              gradient of a (the add passes it to both).
// Arithmetic in fp32, one bf16 rounding per output (torch's separate bf16
// ops round after each op).
#include "vq_internal.h"

namespace vq {

namespace {

__device__ __forceinline__ void ld8(const bf16_t* p, float (&v)[8]) {
    const uint4 q = *reinterpret_cast<const uint4*>(p);
    const uint32_t w[4] = {q.x, q.y, q.z, q.w};
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        v[2 * i] = __uint_as_float(w[i] << 16);
        v[2 * i + 1] = __uint_as_float(w[i] & 0xffff0000u);
    }
}

__device__ __forceinline__ void st8(bf16_t* p, const float (&v)[8]) {
    uint4 q;
    q.x = f2bf2(v[0], v[1]);
    q.y = f2bf2(v[2], v[3]);
    q.z = f2bf2(v[4], v[5]);
    q.w = f2bf2(v[6], v[7]);
    *reinterpret_cast<uint4*>(p) = q;
}

__device__ __forceinline__ void ld8f(const float* p, float (&v)[8]) {
    const float4 a = reinterpret_cast<const float4*>(p)[0];
    const float4 b = reinterpret_cast<const float4*>(p)[1];
    v[0] = a.x; v[1] = a.y; v[2] = a.z; v[3] = a.w;
    v[4] = b.x; v[5] = b.y; v[6] = b.z; v[7] = b.w;
}

}  // namespace

// One thread: 8 weights of the first half of one head and the matching 8 of
// the second half, for one token.  Items per token: (Hq + 2 Hkv) * D / 16.
__global__ __launch_bounds__(256) void rope_qkv_fwd_kernel(const bf16_t* __restrict__ qkv, int64_t tokens, int S,
                                                           int Hq, int Hkv, int kv_out, int D,
                                                           const float* __restrict__ cosb,
                                                           const float* __restrict__ sinb, bf16_t* __restrict__ q,
                                                           bf16_t* __restrict__ k, bf16_t* __restrict__ v) {
    const int per_head = D / 16;
    const int heads = Hq + 2 * Hkv;
    const int64_t item = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (item >= tokens * heads * per_head) return;
    const int64_t m = item / (heads * per_head);
    const int rem = (int)(item - m * heads * per_head);
    const int hh = rem / per_head, c = rem % per_head;
    const int s = (int)(m % S);
    const int half = D / 2, d0 = 8 * c;
    const bf16_t* src = qkv + m * (int64_t)heads * D + (int64_t)hh * D;
    float x1[8], x2[8];
    ld8(src + d0, x1);
    ld8(src + half + d0, x2);
    const int rep = kv_out / Hkv;  // copies of each K/V head: Hq / Hkv, or 1
    if (hh >= Hq + Hkv) {  // v: copied into its rep output head slots
        const int kv = hh - Hq - Hkv;
        for (int r = 0; r < rep; ++r) {
            bf16_t* dst = v + (m * kv_out + (int64_t)kv * rep + r) * D;
            st8(dst + d0, x1);
            st8(dst + half + d0, x2);
        }
        return;
    }
    float c1[8], c2[8], s1[8], s2[8], y1[8], y2[8];
    ld8f(cosb + (int64_t)s * D + d0, c1);
    ld8f(cosb + (int64_t)s * D + half + d0, c2);
    ld8f(sinb + (int64_t)s * D + d0, s1);
    ld8f(sinb + (int64_t)s * D + half + d0, s2);
#pragma unroll
    for (int i = 0; i < 8; ++i) {
        y1[i] = x1[i] * c1[i] - x2[i] * s1[i];
        y2[i] = x2[i] * c2[i] + x1[i] * s2[i];
    }
    if (hh < Hq) {
        bf16_t* dst = q + (m * Hq + hh) * D;
        st8(dst + d0, y1);
        st8(dst + half + d0, y2);
    } else {
        const int kv = hh - Hq;
        for (int r = 0; r < rep; ++r) {
            bf16_t* dst = k + (m * kv_out + (int64_t)kv * rep + r) * D;
            st8(dst + d0, y1);
            st8(dst + half + d0, y2);
        }
    }
}

// Gradients of q, k, v ([B, Hq, S, D] with element strides sb, sh, ss; unit
// stride along D) back into the stacked layout [tokens][(Hq + 2 Hkv) D]:
// dx1 = dy1 cos1 + dy2 sin2, dx2 = dy2 cos2 - dy1 sin1, K/V summed over their
// repeated heads.
__global__ __launch_bounds__(256) void rope_qkv_bwd_kernel(const bf16_t* __restrict__ dq, const bf16_t* __restrict__ dk,
                                                           const bf16_t* __restrict__ dv, int64_t sb, int64_t sh,
                                                           int64_t ss, int64_t tokens, int S, int Hq, int Hkv, int D,
                                                           const float* __restrict__ cosb,
                                                           const float* __restrict__ sinb,
                                                           bf16_t* __restrict__ dqkv) {
    const int per_head = D / 16;
    const int heads = Hq + 2 * Hkv;
    const int64_t item = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (item >= tokens * heads * per_head) return;
    const int64_t m = item / (heads * per_head);
    const int rem = (int)(item - m * heads * per_head);
    const int hh = rem / per_head, c = rem % per_head;
    const int64_t b = m / S;
    const int s = (int)(m % S);
    const int half = D / 2, d0 = 8 * c;
    const int rep = Hq / Hkv;
    float g1[8], g2[8];
    const bf16_t* base;
    int h0, nh;
    if (hh < Hq) {
        base = dq; h0 = hh; nh = 1;
    } else if (hh < Hq + Hkv) {
        base = dk; h0 = (hh - Hq) * rep; nh = rep;
    } else {
        base = dv; h0 = (hh - Hq - Hkv) * rep; nh = rep;
    }
#pragma unroll
    for (int i = 0; i < 8; ++i) g1[i] = g2[i] = 0.0f;
    for (int r = 0; r < nh; ++r) {
        const bf16_t* p = base + b * sb + (int64_t)(h0 + r) * sh + (int64_t)s * ss;
        float a1[8], a2[8];
        ld8(p + d0, a1);
        ld8(p + half + d0, a2);
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            g1[i] += a1[i];
            g2[i] += a2[i];
        }
    }
    float o1[8], o2[8];
    if (hh < Hq + Hkv) {
        float c1[8], c2[8], s1[8], s2[8];
        ld8f(cosb + (int64_t)s * D + d0, c1);
        ld8f(cosb + (int64_t)s * D + half + d0, c2);
        ld8f(sinb + (int64_t)s * D + d0, s1);
        ld8f(sinb + (int64_t)s * D + half + d0, s2);
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            o1[i] = g1[i] * c1[i] + g2[i] * s2[i];
            o2[i] = g2[i] * c2[i] - g1[i] * s1[i];
        }
    } else {
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            o1[i] = g1[i];
            o2[i] = g2[i];
        }
    }
    bf16_t* dst = dqkv + m * (int64_t)heads * D + (int64_t)hh * D;
    st8(dst + d0, o1);
    st8(dst + half + d0, o2);
}

// One wave per row, 8 consecutive elements per lane and step.
constexpr int kNormWaves = 4;

__device__ __forceinline__ float bf16_round(float x) { return __uint_as_float((uint32_t)f2bf(x) << 16); }

__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
    for (int off = 32; off >= 1; off >>= 1) v += __shfl_xor(v, off, 64);
    return v;
}

// NIT > 0 (dim <= 512 NIT): each lane keeps its 8 NIT values in registers
// between the reduction and the second sweep, so a row is read once; NIT = 0:
// two sweeps over any dim.  Same arithmetic in the same order either way.
template <int NIT>
__global__ __launch_bounds__(64 * kNormWaves) void add_rmsnorm_fwd_kernel(
    const bf16_t* __restrict__ h, const bf16_t* __restrict__ a, const bf16_t* __restrict__ w, int64_t rows, int dim,
    float eps, bf16_t* __restrict__ s_out, bf16_t* __restrict__ n_out, float* __restrict__ rstd_out) {
    const int lane = threadIdx.x & 63;
    const int64_t r = (int64_t)blockIdx.x * kNormWaves + (threadIdx.x >> 6);
    if (r >= rows) return;
    const int64_t base = r * dim;
    if constexpr (NIT > 0) {
        float x[NIT][8];
        float ss = 0.0f;
#pragma unroll
        for (int it = 0; it < NIT; ++it) {
            const int c = 8 * lane + 512 * it;
            if (c < dim) {
                ld8(h + base + c, x[it]);
                if (a) {
                    float y[8];
                    ld8(a + base + c, y);
#pragma unroll
                    for (int j = 0; j < 8; ++j) x[it][j] = bf16_round(x[it][j] + y[j]);
                    if (s_out) st8(s_out + base + c, x[it]);
                }
#pragma unroll
                for (int j = 0; j < 8; ++j) ss += x[it][j] * x[it][j];
            }
        }
        const float rstd = rsqrtf(wave_sum(ss) / (float)dim + eps);
        if (rstd_out && lane == 0) rstd_out[r] = rstd;
#pragma unroll
        for (int it = 0; it < NIT; ++it) {
            const int c = 8 * lane + 512 * it;
            if (c < dim) {
                float wv[8];
                ld8(w + c, wv);
#pragma unroll
                for (int j = 0; j < 8; ++j) x[it][j] = x[it][j] * rstd * wv[j];
                st8(n_out + base + c, x[it]);
            }
        }
        return;
    }
    float ss = 0.0f;
    for (int c = 8 * lane; c < dim; c += 512) {
        float x[8];
        ld8(h + base + c, x);
        if (a) {
            float y[8];
            ld8(a + base + c, y);
#pragma unroll
            for (int j = 0; j < 8; ++j) x[j] = bf16_round(x[j] + y[j]);
            if (s_out) st8(s_out + base + c, x);
        }
#pragma unroll
        for (int j = 0; j < 8; ++j) ss += x[j] * x[j];
    }
    const float rstd = rsqrtf(wave_sum(ss) / (float)dim + eps);
    if (rstd_out && lane == 0) rstd_out[r] = rstd;
    for (int c = 8 * lane; c < dim; c += 512) {
        float x[8], wv[8];
        if (a && s_out) {
            ld8(s_out + base + c, x);  // this lane's own stores
        } else {
            ld8(h + base + c, x);
            if (a) {
                float y[8];
                ld8(a + base + c, y);
#pragma unroll
                for (int j = 0; j < 8; ++j) x[j] = bf16_round(x[j] + y[j]);
            }
        }
        ld8(w + c, wv);
#pragma unroll
        for (int j = 0; j < 8; ++j) x[j] = x[j] * rstd * wv[j];
        st8(n_out + base + c, x);
    }
}

// NIT as in add_rmsnorm_fwd_kernel: dn and s stay in registers between the
// dot product and the second sweep.
template <int NIT>
__global__ __launch_bounds__(64 * kNormWaves) void rmsnorm_bwd_kernel(
    const bf16_t* __restrict__ dn, const bf16_t* __restrict__ ds, const bf16_t* __restrict__ s,
    const bf16_t* __restrict__ w, const float* __restrict__ rstd_in, int64_t rows, int dim, bf16_t* __restrict__ dh) {
    const int lane = threadIdx.x & 63;
    const int64_t r = (int64_t)blockIdx.x * kNormWaves + (threadIdx.x >> 6);
    if (r >= rows) return;
    const int64_t base = r * dim;
    const float rstd = rstd_in[r];
    if constexpr (NIT > 0) {
        float g[NIT][8], x[NIT][8];
        float dot = 0.0f;  // sum dn w s
#pragma unroll
        for (int it = 0; it < NIT; ++it) {
            const int c = 8 * lane + 512 * it;
            if (c < dim) {
                float wv[8];
                ld8(dn + base + c, g[it]);
                ld8(s + base + c, x[it]);
                ld8(w + c, wv);
#pragma unroll
                for (int j = 0; j < 8; ++j) dot += g[it][j] * wv[j] * x[it][j];
            }
        }
        const float k = wave_sum(dot) * rstd * rstd / (float)dim;
#pragma unroll
        for (int it = 0; it < NIT; ++it) {
            const int c = 8 * lane + 512 * it;
            if (c < dim) {
                float wv[8], o[8];
                ld8(w + c, wv);
#pragma unroll
                for (int j = 0; j < 8; ++j) o[j] = rstd * (g[it][j] * wv[j] - x[it][j] * k);
                if (ds) {
                    float d[8];
                    ld8(ds + base + c, d);
#pragma unroll
                    for (int j = 0; j < 8; ++j) o[j] += d[j];
                }
                st8(dh + base + c, o);
            }
        }
        return;
    }
    float dot = 0.0f;  // sum dn w s
    for (int c = 8 * lane; c < dim; c += 512) {
        float g[8], x[8], wv[8];
        ld8(dn + base + c, g);
        ld8(s + base + c, x);
        ld8(w + c, wv);
#pragma unroll
        for (int j = 0; j < 8; ++j) dot += g[j] * wv[j] * x[j];
    }
    // mean(g xhat) with xhat = s rstd, times rstd once more for the xhat term
    const float k = wave_sum(dot) * rstd * rstd / (float)dim;
    for (int c = 8 * lane; c < dim; c += 512) {
        float g[8], x[8], wv[8];
        ld8(dn + base + c, g);
        ld8(s + base + c, x);
        ld8(w + c, wv);
        float o[8];
#pragma unroll
        for (int j = 0; j < 8; ++j) o[j] = rstd * (g[j] * wv[j] - x[j] * k);
        if (ds) {
            float d[8];
            ld8(ds + base + c, d);
#pragma unroll
            for (int j = 0; j < 8; ++j) o[j] += d[j];
        }
        st8(dh + base + c, o);
    }
}

__device__ __forceinline__ float sigmoidf_(float x) { return 1.0f / (1.0f + __expf(-x)); }

// out[m][j] = silu(gu[m][j]) * gu[m][F + j]; one thread per 8 outputs.
__global__ __launch_bounds__(256) void swiglu_fwd_kernel(const bf16_t* __restrict__ gu, int64_t tokens, int F,
                                                         bf16_t* __restrict__ out) {
    const int per_row = F / 8;
    const int64_t item = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (item >= tokens * per_row) return;
    const int64_t m = item / per_row;
    const int j = 8 * (int)(item - m * per_row);
    float g[8], u[8], y[8];
    ld8(gu + m * 2 * (int64_t)F + j, g);
    ld8(gu + m * 2 * (int64_t)F + F + j, u);
#pragma unroll
    for (int i = 0; i < 8; ++i) y[i] = g[i] * sigmoidf_(g[i]) * u[i];
    st8(out + m * (int64_t)F + j, y);
}

// dgu[m][j] = dy u silu'(g), dgu[m][F + j] = dy silu(g), with
// silu'(g) = s (1 + g (1 - s)) and s = sigmoid(g).
__global__ __launch_bounds__(256) void swiglu_bwd_kernel(const bf16_t* __restrict__ gu, const bf16_t* __restrict__ dy,
                                                         int64_t tokens, int F, bf16_t* __restrict__ dgu) {
    const int per_row = F / 8;
    const int64_t item = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (item >= tokens * per_row) return;
    const int64_t m = item / per_row;
    const int j = 8 * (int)(item - m * per_row);
    float g[8], u[8], d[8], dg[8], du[8];
    ld8(gu + m * 2 * (int64_t)F + j, g);
    ld8(gu + m * 2 * (int64_t)F + F + j, u);
    ld8(dy + m * (int64_t)F + j, d);
#pragma unroll
    for (int i = 0; i < 8; ++i) {
        const float sg = sigmoidf_(g[i]);
        du[i] = d[i] * g[i] * sg;
        dg[i] = d[i] * u[i] * sg * (1.0f + g[i] * (1.0f - sg));
    }
    st8(dgu + m * 2 * (int64_t)F + j, dg);
    st8(dgu + m * 2 * (int64_t)F + F + j, du);
}

static unsigned blocks_for(int64_t items) { return (unsigned)((items + 255) / 256); }

hipError_t launch_rope_qkv_fwd(const bf16_t* qkv, int64_t tokens, int S, int Hq, int Hkv, int kv_out, int D,
                               const float* cosb, const float* sinb, bf16_t* q, bf16_t* k, bf16_t* v, hipStream_t s) {
    const int64_t items = tokens * (Hq + 2 * Hkv) * (D / 16);
    if (items == 0) return hipSuccess;
    rope_qkv_fwd_kernel<<<blocks_for(items), 256, 0, s>>>(qkv, tokens, S, Hq, Hkv, kv_out, D, cosb, sinb, q, k, v);
    return hipGetLastError();
}

hipError_t launch_rope_qkv_bwd(const bf16_t* dq, const bf16_t* dk, const bf16_t* dv, int64_t sb, int64_t sh,
                               int64_t ss, int64_t tokens, int S, int Hq, int Hkv, int D, const float* cosb,
                               const float* sinb, bf16_t* dqkv, hipStream_t s) {
    const int64_t items = tokens * (Hq + 2 * Hkv) * (D / 16);
    if (items == 0) return hipSuccess;
    rope_qkv_bwd_kernel<<<blocks_for(items), 256, 0, s>>>(dq, dk, dv, sb, sh, ss, tokens, S, Hq, Hkv, D, cosb, sinb,
                                                          dqkv);
    return hipGetLastError();
}

hipError_t launch_add_rmsnorm_fwd(const bf16_t* h, const bf16_t* a, const bf16_t* w, int64_t rows, int dim, float eps,
                                 bf16_t* s_out, bf16_t* n_out, float* rstd_out, hipStream_t s) {
    if (rows == 0) return hipSuccess;
    const dim3 grid((unsigned)((rows + kNormWaves - 1) / kNormWaves));
    switch ((dim + 511) / 512) {  // row sweeps of 512 per wave: kept in registers up to 4
        case 1: add_rmsnorm_fwd_kernel<1><<<grid, 64 * kNormWaves, 0, s>>>(h, a, w, rows, dim, eps, s_out, n_out, rstd_out); break;
        case 2: add_rmsnorm_fwd_kernel<2><<<grid, 64 * kNormWaves, 0, s>>>(h, a, w, rows, dim, eps, s_out, n_out, rstd_out); break;
        case 3: add_rmsnorm_fwd_kernel<3><<<grid, 64 * kNormWaves, 0, s>>>(h, a, w, rows, dim, eps, s_out, n_out, rstd_out); break;
        case 4: add_rmsnorm_fwd_kernel<4><<<grid, 64 * kNormWaves, 0, s>>>(h, a, w, rows, dim, eps, s_out, n_out, rstd_out); break;
        default: add_rmsnorm_fwd_kernel<0><<<grid, 64 * kNormWaves, 0, s>>>(h, a, w, rows, dim, eps, s_out, n_out, rstd_out);
    }
    return hipGetLastError();
}

hipError_t launch_rmsnorm_bwd(const bf16_t* dn, const bf16_t* ds, const bf16_t* x, const bf16_t* w, const float* rstd,
                              int64_t rows, int dim, bf16_t* dh, hipStream_t s) {
    if (rows == 0) return hipSuccess;
    const dim3 grid((unsigned)((rows + kNormWaves - 1) / kNormWaves));
    switch ((dim + 511) / 512) {
        case 1: rmsnorm_bwd_kernel<1><<<grid, 64 * kNormWaves, 0, s>>>(dn, ds, x, w, rstd, rows, dim, dh); break;
        case 2: rmsnorm_bwd_kernel<2><<<grid, 64 * kNormWaves, 0, s>>>(dn, ds, x, w, rstd, rows, dim, dh); break;
        case 3: rmsnorm_bwd_kernel<3><<<grid, 64 * kNormWaves, 0, s>>>(dn, ds, x, w, rstd, rows, dim, dh); break;
        case 4: rmsnorm_bwd_kernel<4><<<grid, 64 * kNormWaves, 0, s>>>(dn, ds, x, w, rstd, rows, dim, dh); break;
        default: rmsnorm_bwd_kernel<0><<<grid, 64 * kNormWaves, 0, s>>>(dn, ds, x, w, rstd, rows, dim, dh);
    }
    return hipGetLastError();
}

hipError_t launch_swiglu_fwd(const bf16_t* gu, int64_t tokens, int F, bf16_t* out, hipStream_t s) {
    const int64_t items = tokens * (F / 8);
    if (items == 0) return hipSuccess;
    swiglu_fwd_kernel<<<blocks_for(items), 256, 0, s>>>(gu, tokens, F, out);
    return hipGetLastError();
}

hipError_t launch_swiglu_bwd(const bf16_t* gu, const bf16_t* dy, int64_t tokens, int F, bf16_t* dgu, hipStream_t s) {
    const int64_t items = tokens * (F / 8);
    if (items == 0) return hipSuccess;
    swiglu_bwd_kernel<<<blocks_for(items), 256, 0, s>>>(gu, dy, tokens, F, dgu);
    return hipGetLastError();
}

}  // namespace vq
