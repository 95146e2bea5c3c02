// Shared device helpers for libvoodoo_hip: GGUF block geometry, exact fp16
// widening, torch-compatible bf16 rounding and the per-run block decoders.
//
// Block layouts follow the public GGUF format (llama.cpp ggml-common.h); for
// Q8_0/Q4_K/Q5_K/Q6_K they are the layouts the reference decodes in
// voodoo_quant/layers.py:62-213.  Every decoder reproduces ggml's float
// expression for a weight: the products d*sc*q are exact in fp32, so the one
// rounding (the subtraction of dmin*m, where present) is the same whether or
// not the compiler contracts it into an FMA.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace vq {

// ggml type ids (ggml.h), the only ones this library decodes
enum QType : int { Q8_0 = 8, Q2_K = 10, Q3_K = 11, Q4_K = 12, Q5_K = 13, Q6_K = 14 };

// Bytes per 256 weights.  Q8_0 is handled as groups of eight 34-byte blocks, so
// every format advances in 256-weight "groups" along a row.
__host__ __device__ constexpr int group_bytes(int qt) {
    return qt == Q8_0 ? 272 : qt == Q2_K ? 84 : qt == Q3_K ? 110 : qt == Q4_K ? 144 : qt == Q5_K ? 176
         : qt == Q6_K ? 210 : 0;
}

__host__ __device__ constexpr bool qtype_supported(int qt) { return group_bytes(qt) != 0; }

typedef uint16_t bf16_t;
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

// Exact fp16 -> fp32 (normals by re-biasing, subnormals as man * 2^-24).
__device__ __forceinline__ float h2f(uint32_t h) {
    const uint32_t sign = (h & 0x8000u) << 16;
    const uint32_t em = h & 0x7fffu;
    if (em >= 0x0400u) {
        const uint32_t bits = em >= 0x7c00u ? (0x7f800000u | ((em & 0x3ffu) << 13)) : ((em << 13) + 0x38000000u);
        return __uint_as_float(bits | sign);
    }
    return __uint_as_float(sign | __float_as_uint((float)em * 5.9604644775390625e-8f));
}

// fp32 -> bf16 exactly as torch's Float->BFloat16 cast: NaN -> 0x7FC0, else
// round to nearest, ties to even.
__device__ __forceinline__ bf16_t f2bf(float f) {
    const uint32_t u = __float_as_uint(f);
    if ((u & 0x7fffffffu) > 0x7f800000u) return 0x7fc0;
    return (bf16_t)((u + (((u >> 16) & 1u) + 0x7fffu)) >> 16);
}

__device__ __forceinline__ float bf2f(bf16_t b) { return __uint_as_float((uint32_t)b << 16); }

__device__ __forceinline__ uint32_t rd_u8(const uint8_t* p) { return p[0]; }
__device__ __forceinline__ uint32_t rd_u16(const uint8_t* p) { return (uint32_t)p[0] | ((uint32_t)p[1] << 8); }

// ---------------------------------------------------------------------------
// decode_run<QT, R>(g, p, y): weights p .. p+R-1 of the 256-weight group whose
// bytes start at g.  R is 4 or 8 and p is a multiple of R, so the run never
// crosses a 16-weight sub-block.  g may point into LDS or global memory.
// ---------------------------------------------------------------------------
template <int QT, int R>
__device__ __forceinline__ void decode_run(const uint8_t* __restrict__ g, int p, float* __restrict__ y);

template <int R>
__device__ __forceinline__ void decode_q8_0(const uint8_t* __restrict__ g, int p, float* __restrict__ y) {
    const uint8_t* b = g + 34 * (p >> 5);
    const float d = h2f(rd_u16(b));
    const int o = 2 + (p & 31);
#pragma unroll
    for (int r = 0; r < R; ++r) y[r] = (float)(int8_t)b[o + r] * d;
}

// 6-bit scale/min pair j of the 12-byte Q4_K/Q5_K scale array
__device__ __forceinline__ void scale_min_k4(const uint8_t* __restrict__ s, int j, uint32_t& sc, uint32_t& m) {
    if (j < 4) {
        sc = s[j] & 63u;
        m = s[j + 4] & 63u;
    } else {
        sc = (s[j + 4] & 0xFu) | ((uint32_t)(s[j - 4] >> 6) << 4);
        m = (s[j + 4] >> 4) | ((uint32_t)(s[j] >> 6) << 4);
    }
}

template <int R, bool FIVE>
__device__ __forceinline__ void decode_q45_K(const uint8_t* __restrict__ g, int p, float* __restrict__ y) {
    const float d = h2f(rd_u16(g)), dmin = h2f(rd_u16(g + 2));
    const int c = p >> 6, h = (p >> 5) & 1, l = p & 31;
    uint32_t sc, m;
    scale_min_k4(g + 4, 2 * c + h, sc, m);
    const float dl = d * (float)sc, ml = dmin * (float)m;
    const uint8_t* qs = g + (FIVE ? 48 : 16) + 32 * c + l;
#pragma unroll
    for (int r = 0; r < R; ++r) {
        uint32_t q = (qs[r] >> (4 * h)) & 0xFu;
        if (FIVE) q += ((g[16 + l + r] >> (2 * c + h)) & 1u) << 4;
        y[r] = dl * (float)q - ml;
    }
}

template <int R>
__device__ __forceinline__ void decode_q6_K(const uint8_t* __restrict__ g, int p, float* __restrict__ y) {
    const float d = h2f(rd_u16(g + 208));
    const int n = p >> 7, t = (p >> 5) & 3, l = p & 31;
    const float dl = d * (float)(int8_t)g[192 + 8 * n + (l >> 4) + 2 * t];
    const uint8_t* ql = g + 64 * n + l + 32 * (t & 1);
    const uint8_t* qh = g + 128 + 32 * n + l;
    const int ls = 4 * (t >> 1), hs = 2 * t;
#pragma unroll
    for (int r = 0; r < R; ++r) {
        const int q = (int)(((ql[r] >> ls) & 0xFu) | (((qh[r] >> hs) & 3u) << 4)) - 32;
        y[r] = dl * (float)q;
    }
}

template <int R>
__device__ __forceinline__ void decode_q3_K(const uint8_t* __restrict__ g, int p, float* __restrict__ y) {
    const float d = h2f(rd_u16(g + 108));
    const int n = p >> 7, j = (p >> 5) & 3, half = (p >> 4) & 1, l = p & 15;
    const int is = 8 * n + 2 * j + half;
    const uint8_t* s = g + 96;
    const uint32_t lo4 = is < 8 ? (s[is] & 0xFu) : (uint32_t)(s[is - 8] >> 4);
    const uint32_t hi2 = (s[8 + (is & 3)] >> (2 * (is >> 2))) & 3u;
    const float dl = d * (float)((int)(lo4 | (hi2 << 4)) - 32);
    const uint8_t* qs = g + 32 + 32 * n + 16 * half + l;
    const uint8_t* hm = g + 16 * half + l;
    const int hb = 4 * n + j;
#pragma unroll
    for (int r = 0; r < R; ++r) {
        const int q = (int)((qs[r] >> (2 * j)) & 3u) - (((hm[r] >> hb) & 1u) ? 0 : 4);
        y[r] = dl * (float)q;
    }
}

template <int R>
__device__ __forceinline__ void decode_q2_K(const uint8_t* __restrict__ g, int p, float* __restrict__ y) {
    const float d = h2f(rd_u16(g + 80)), dmin = h2f(rd_u16(g + 82));
    const int n = p >> 7, j = (p >> 5) & 3, half = (p >> 4) & 1, l = p & 15;
    const uint32_t s = g[8 * n + 2 * j + half];
    const float dl = d * (float)(s & 0xFu), ml = dmin * (float)(s >> 4);
    const uint8_t* qs = g + 16 + 32 * n + 16 * half + l;
#pragma unroll
    for (int r = 0; r < R; ++r) y[r] = dl * (float)((qs[r] >> (2 * j)) & 3u) - ml;
}

template <int QT, int R>
__device__ __forceinline__ void decode_run(const uint8_t* __restrict__ g, int p, float* __restrict__ y) {
    if constexpr (QT == Q8_0) decode_q8_0<R>(g, p, y);
    else if constexpr (QT == Q4_K) decode_q45_K<R, false>(g, p, y);
    else if constexpr (QT == Q5_K) decode_q45_K<R, true>(g, p, y);
    else if constexpr (QT == Q6_K) decode_q6_K<R>(g, p, y);
    else if constexpr (QT == Q3_K) decode_q3_K<R>(g, p, y);
    else if constexpr (QT == Q2_K) decode_q2_K<R>(g, p, y);
}

// Runtime-type dispatch (the type is uniform across a wave).
template <int R>
__device__ __forceinline__ void decode_run_rt(int qt, const uint8_t* __restrict__ g, int p, float* __restrict__ y) {
    switch (qt) {
    case Q8_0: decode_run<Q8_0, R>(g, p, y); break;
    case Q2_K: decode_run<Q2_K, R>(g, p, y); break;
    case Q3_K: decode_run<Q3_K, R>(g, p, y); break;
    case Q4_K: decode_run<Q4_K, R>(g, p, y); break;
    case Q5_K: decode_run<Q5_K, R>(g, p, y); break;
    default: decode_run<Q6_K, R>(g, p, y); break;
    }
}

// Up to this many candidates per gated tensor (the reference's widest menus
// are 12 types, its training recipes use 4-8).
constexpr int kMaxCand = 12;

struct CandSet {
    const uint8_t* qbytes[kMaxCand];  // packed rows [N][D_pad/256 groups]
    int qtype[kMaxCand];
    int ncand;
    int64_t row_groups;  // D_pad / 256
};

}  // namespace vq
