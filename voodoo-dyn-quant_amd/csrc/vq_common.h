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
enum QType : int {
    Q8_0 = 8, Q2_K = 10, Q3_K = 11, Q4_K = 12, Q5_K = 13, Q6_K = 14,
    IQ2_XXS = 16, IQ2_XS = 17, IQ3_XXS = 18, IQ1_S = 19, IQ3_S = 21, IQ2_S = 22, IQ4_XS = 23, IQ1_M = 29
};

// Bytes per 256 weights.  Q8_0 is handled as groups of eight 34-byte blocks, so
// every format advances in 256-weight "groups" along a row.  Every size is
// even, so a group starts on a 2-byte boundary whatever its index.
__host__ __device__ constexpr int group_bytes(int qt) {
    return qt == Q8_0 ? 272 : qt == Q2_K ? 84 : qt == Q3_K ? 110 : qt == Q4_K ? 144 : qt == Q5_K ? 176
         : qt == Q6_K ? 210 : qt == IQ2_XXS ? 66 : qt == IQ2_XS ? 74 : qt == IQ3_XXS ? 98 : qt == IQ1_S ? 50
         : qt == IQ3_S ? 110 : qt == IQ2_S ? 82 : qt == IQ4_XS ? 136 : qt == IQ1_M ? 56 : 0;
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

// Hardware fp16 -> fp32 (v_cvt_f32_f16): exact for normals, subnormals and
// infinities; a NaN stays a NaN but its payload may be quieted, so only paths
// whose output does not carry NaN payloads (the bf16 mixture) use it.
__device__ __forceinline__ float h2f_hw(uint32_t h) {
    return (float)__builtin_bit_cast(_Float16, (uint16_t)h);
}

// fp32 -> bf16 exactly as torch's Float->BFloat16 cast: NaN -> 0x7FC0, else
// round to nearest, ties to even.
__device__ __forceinline__ bf16_t f2bf(float f) {
    const uint32_t u = __float_as_uint(f);
    if ((u & 0x7fffffffu) > 0x7f800000u) return 0x7fc0;
    return (bf16_t)((u + (((u >> 16) & 1u) + 0x7fffu)) >> 16);
}

// Two values -> packed bf16 pair (a in the low half), the same bits as f2bf:
// gfx950's v_cvt_pk_bf16_f32 rounds to nearest even; NaNs become 0x7fc0.
__device__ __forceinline__ uint32_t f2bf2(float a, float b) {
    typedef __bf16 bf2_t __attribute__((ext_vector_type(2)));
    typedef float f2_t __attribute__((ext_vector_type(2)));
    const f2_t v = {a, b};
    uint32_t r = __builtin_bit_cast(uint32_t, __builtin_convertvector(v, bf2_t));
    if (a != a) r = (r & 0xffff0000u) | 0x7fc0u;
    if (b != b) r = (r & 0x0000ffffu) | 0x7fc00000u;
    return r;
}

// Two values -> packed bf16 pair by v_cvt_pk_bf16_f32 alone: f2bf2's bits for
// every non-NaN value; a NaN comes out as some quiet NaN.
__device__ __forceinline__ uint32_t pk_bf16(float a, float b) {
    typedef __bf16 bf2_t __attribute__((ext_vector_type(2)));
    typedef float f2_t __attribute__((ext_vector_type(2)));
    const f2_t v = {a, b};
    return __builtin_bit_cast(uint32_t, __builtin_convertvector(v, bf2_t));
}

__device__ __forceinline__ float bf2f(bf16_t b) { return __uint_as_float((uint32_t)b << 16); }

__device__ __forceinline__ uint32_t rd_u8(const uint8_t* p) { return p[0]; }
__device__ __forceinline__ uint32_t rd_u16(const uint8_t* p) { return (uint32_t)p[0] | ((uint32_t)p[1] << 8); }

}  // namespace vq

#include "vq_iq.h"

namespace vq {

// ---------------------------------------------------------------------------
// Block decoders.  decode_codes<QT, R>(g, p, q, dl, ml) reads weights
// p .. p+R-1 of the 256-weight group whose bytes start at g (R is 4 or 8, p a
// multiple of R, so the run never crosses a 16-weight sub-block) as integer
// codes q (held in floats) and the run's scale dl and offset ml:
//     weight = dl * q - ml          (ml = 0 for the formats without mins)
// dl * q is exact in fp32 for every format, so decode_run's single rounding is
// ggml's.  g may point into LDS or global memory.
// ---------------------------------------------------------------------------
template <int QT>
struct HasMin {
    static constexpr bool value = (QT == Q4_K || QT == Q5_K || QT == Q2_K);
};

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

// Load R (4, 8 or 16) consecutive bytes whose address is a multiple of ALIGN
// (a property of the format's layout: group bases are 16-byte aligned in
// memory and in LDS, so field offsets fix the alignment), with the widest
// loads that alignment allows.  Byte r is (w[r / 4] >> (8 * (r % 4))) & 0xff.
template <int ALIGN, int R>
__device__ __forceinline__ void load_run(const uint8_t* __restrict__ p, uint32_t (&w)[R / 4]) {
    if constexpr (ALIGN >= 8 && R % 8 == 0) {
#pragma unroll
        for (int i = 0; i < R / 8; ++i) {
            const uint2 v = *reinterpret_cast<const uint2*>(p + 8 * i);
            w[2 * i] = v.x;
            w[2 * i + 1] = v.y;
        }
    } else if constexpr (ALIGN >= 4) {
#pragma unroll
        for (int i = 0; i < R / 4; ++i) w[i] = *reinterpret_cast<const uint32_t*>(p + 4 * i);
    } else {
        const uint16_t* h = reinterpret_cast<const uint16_t*>(p);
#pragma unroll
        for (int i = 0; i < R / 4; ++i) w[i] = (uint32_t)h[2 * i] | ((uint32_t)h[2 * i + 1] << 16);
    }
}

// The code words as opaque values: without this the compiler folds a word's
// mask and each byte's shift into one v_bfe_u32 per weight (Q4_K, Q2_K)
// instead of letting v_cvt_f32_ubyteN read the byte: 16 extra VALU
// instructions per run of 16.
template <int W>
__device__ __forceinline__ void opaque_words(uint32_t (&uw)[W]) {
#pragma unroll
    for (int i = 0; i < W; ++i) asm volatile("" : "+v"(uw[i]));
}

template <int R>
__device__ __forceinline__ uint32_t run_byte(const uint32_t (&w)[R / 4], int r) {
    return (w[r >> 2] >> (8 * (r & 3))) & 0xffu;
}

template <int QT, int R>
__device__ __forceinline__ void decode_codes(const uint8_t* __restrict__ g, int p, float* __restrict__ q, float& dl,
                                             float& ml) {
    if constexpr (QT == Q8_0) {
        // blocks of 34 bytes: codes start 2 bytes into a block -> 2-byte aligned
        const uint8_t* b = g + 34 * (p >> 5);
        dl = h2f(*reinterpret_cast<const uint16_t*>(b));
        ml = 0.0f;
        uint32_t w[R / 4];
        load_run<2, R>(b + 2 + (p & 31), w);
#pragma unroll
        for (int r = 0; r < R; ++r) q[r] = (float)(int8_t)run_byte<R>(w, r);
    } else if constexpr (QT == Q4_K || QT == Q5_K) {
        // 144- and 176-byte groups keep 16-byte alignment; code runs are 8-aligned
        constexpr bool FIVE = QT == Q5_K;
        const uint32_t dd = *reinterpret_cast<const uint32_t*>(g);
        const float d = h2f(dd & 0xffffu), dmin = h2f(dd >> 16);
        const int c = p >> 6, h = (p >> 5) & 1, l = p & 31;
        uint32_t sc, m;
        scale_min_k4(g + 4, 2 * c + h, sc, m);
        dl = d * (float)sc;
        ml = dmin * (float)m;
        uint32_t w[R / 4];
        load_run<8, R>(g + (FIVE ? 48 : 16) + 32 * c + l, w);
        uint32_t hw[R / 4];
        if (FIVE) load_run<8, R>(g + 16 + l, hw);
#pragma unroll
        for (int r = 0; r < R; ++r) {
            uint32_t v = (run_byte<R>(w, r) >> (4 * h)) & 0xFu;
            if (FIVE) v += ((run_byte<R>(hw, r) >> (2 * c + h)) & 1u) << 4;
            q[r] = (float)v;
        }
    } else if constexpr (QT == Q6_K) {
        // 210-byte groups: 2-byte alignment only
        const float d = h2f(*reinterpret_cast<const uint16_t*>(g + 208));
        const int n = p >> 7, t = (p >> 5) & 3, l = p & 31;
        dl = d * (float)(int8_t)g[192 + 8 * n + (l >> 4) + 2 * t];
        ml = 0.0f;
        uint32_t lw[R / 4], hw[R / 4];
        load_run<2, R>(g + 64 * n + l + 32 * (t & 1), lw);
        load_run<2, R>(g + 128 + 32 * n + l, hw);
        const int ls = 4 * (t >> 1), hs = 2 * t;
#pragma unroll
        for (int r = 0; r < R; ++r)
            q[r] = (float)((int)(((run_byte<R>(lw, r) >> ls) & 0xFu) | (((run_byte<R>(hw, r) >> hs) & 3u) << 4)) - 32);
    } else if constexpr (QT == Q3_K) {
        // 110-byte groups: 2-byte alignment only
        const float d = h2f(*reinterpret_cast<const uint16_t*>(g + 108));
        const int n = p >> 7, j = (p >> 5) & 3, half = (p >> 4) & 1, l = p & 15;
        const int is = 8 * n + 2 * j + half;
        const uint8_t* s = g + 96;
        const uint32_t lo4 = is < 8 ? (s[is] & 0xFu) : (uint32_t)(s[is - 8] >> 4);
        const uint32_t hi2 = (s[8 + (is & 3)] >> (2 * (is >> 2))) & 3u;
        dl = d * (float)((int)(lo4 | (hi2 << 4)) - 32);
        ml = 0.0f;
        uint32_t qw[R / 4], mw[R / 4];
        load_run<2, R>(g + 32 + 32 * n + 16 * half + l, qw);
        load_run<2, R>(g + 16 * half + l, mw);
        const int hb = 4 * n + j;
#pragma unroll
        for (int r = 0; r < R; ++r)
            q[r] = (float)((int)((run_byte<R>(qw, r) >> (2 * j)) & 3u) - (((run_byte<R>(mw, r) >> hb) & 1u) ? 0 : 4));
    } else {  // Q2_K: 84-byte groups keep 4-byte alignment
        const uint32_t dd = *reinterpret_cast<const uint32_t*>(g + 80);
        const float d = h2f(dd & 0xffffu), dmin = h2f(dd >> 16);
        const int n = p >> 7, j = (p >> 5) & 3, half = (p >> 4) & 1, l = p & 15;
        const uint32_t s = g[8 * n + 2 * j + half];
        dl = d * (float)(s & 0xFu);
        ml = dmin * (float)(s >> 4);
        uint32_t w[R / 4];
        load_run<4, R>(g + 16 + 32 * n + 16 * half + l, w);
#pragma unroll
        for (int r = 0; r < R; ++r) q[r] = (float)((run_byte<R>(w, r) >> (2 * j)) & 3u);
    }
}

// Exact fp32 weights (ggml's dequantize_row_* values, signed zeros included).
template <int QT, int R>
__device__ __forceinline__ void decode_run(const uint8_t* __restrict__ g, int p, float* __restrict__ y) {
    float q[R], dl, ml;
    decode_codes<QT, R>(g, p, q, dl, ml);
    if constexpr (QT == Q8_0) {
#pragma unroll
        for (int r = 0; r < R; ++r) y[r] = q[r] * dl;  // ggml: qs * d
    } else if constexpr (HasMin<QT>::value) {
#pragma unroll
        for (int r = 0; r < R; ++r) y[r] = dl * q[r] - ml;
    } else {
#pragma unroll
        for (int r = 0; r < R; ++r) y[r] = dl * q[r];
    }
}

// <v, W> over one run: sum_r v[r] * (dl * q[r] - ml) = dl * sum(v q) - ml * sum(v)
template <int QT, int R>
__device__ __forceinline__ float dot_run(const uint8_t* __restrict__ g, int p, const float* __restrict__ v) {
    float q[R], dl, ml;
    decode_codes<QT, R>(g, p, q, dl, ml);
    float s1 = 0.0f, s0 = 0.0f;
#pragma unroll
    for (int r = 0; r < R; ++r) {
        s1 = fmaf(v[r], q[r], s1);
        if constexpr (HasMin<QT>::value) s0 += v[r];
    }
    if constexpr (HasMin<QT>::value) return dl * s1 - ml * s0;
    return dl * s1;
}

// <v, W> over the 16 consecutive weights p .. p + 15 (p a multiple of 16) of
// the group at g, with v[r] the value of weight p + r: the per-lane footprint
// of a 32x32 MFMA accumulator block whose rows are permuted so that each lane
// holds 16 consecutive rows.  sv is the sum of v; it is the same for every
// candidate, so the caller computes it once.  The 16 weights share one scale
// (K-quant scales cover 16 or 32 weights, a Q8_0 block 32).  Codes are
// unpacked four at a time (one shift and mask per 32-bit word, then
// v_cvt_f32_ubyteN per weight) as unsigned values u; a format's constant
// offset o (Q8_0's sign via u = q ^ 0x80, Q6_K's -32, Q3_K's -4) and the
// K-quant min are applied once through sv:
//   sum v (dl (u - o) - ml) = dl (sum v u - o sv) - ml sv.
// Field offsets follow the layouts decode_codes reads (reference
// layers.py:62-213 for Q8_0, Q4_K, Q5_K, Q6_K; the GGUF block layouts for
// Q2_K and Q3_K).
template <int QT>
__device__ __forceinline__ float dot_sub16(const uint8_t* __restrict__ g, int p, const float* __restrict__ v, float sv) {
    uint32_t uw[4];  // four unsigned code bytes per word: weights p + 4 u .. p + 4 u + 3
    float dl, ml = 0.0f, off = 0.0f;
    const int l = p & 16;  // first weight within the 32-weight run
    if constexpr (QT == Q8_0) {
        const uint8_t* b = g + 34 * (p >> 5);
        dl = h2f(*reinterpret_cast<const uint16_t*>(b));
        const uint16_t* q = reinterpret_cast<const uint16_t*>(b + 2 + l);  // 2-byte aligned
#pragma unroll
        for (int u = 0; u < 4; ++u) uw[u] = ((uint32_t)q[2 * u] | ((uint32_t)q[2 * u + 1] << 16)) ^ 0x80808080u;
        off = 128.0f;
    } else if constexpr (QT == Q4_K || QT == Q5_K) {
        const uint32_t dd = *reinterpret_cast<const uint32_t*>(g);
        const int c = p >> 6, nib = (p >> 5) & 1;
        uint32_t sc, m;
        scale_min_k4(g + 4, 2 * c + nib, sc, m);
        dl = h2f(dd & 0xffffu) * (float)sc;
        ml = h2f(dd >> 16) * (float)m;
        // 144- and 176-byte groups keep 16-byte alignment
        const u32x4 w = *reinterpret_cast<const u32x4*>(g + (QT == Q5_K ? 48 : 16) + 32 * c + l);
#pragma unroll
        for (int u = 0; u < 4; ++u) uw[u] = (w[u] >> (4 * nib)) & 0x0F0F0F0Fu;
        if constexpr (QT == Q5_K) {
            const u32x4 x = *reinterpret_cast<const u32x4*>(g + 16 + l);
            const int xs = 2 * c + nib;
#pragma unroll
            for (int u = 0; u < 4; ++u) uw[u] |= ((x[u] >> xs) & 0x01010101u) << 4;
        }
    } else if constexpr (QT == Q6_K) {
        const float d = h2f(*reinterpret_cast<const uint16_t*>(g + 208));
        const int n = p >> 7, t4 = (p >> 5) & 3;
        dl = d * (float)(int8_t)g[192 + 8 * n + 2 * t4 + (l >> 4)];
        const uint16_t* a = reinterpret_cast<const uint16_t*>(g + 64 * n + 32 * (t4 & 1) + l);  // 2-byte aligned
        const uint16_t* b = reinterpret_cast<const uint16_t*>(g + 128 + 32 * n + l);
#pragma unroll
        for (int u = 0; u < 4; ++u) {
            const uint32_t lw = (uint32_t)a[2 * u] | ((uint32_t)a[2 * u + 1] << 16);
            const uint32_t hw = (uint32_t)b[2 * u] | ((uint32_t)b[2 * u + 1] << 16);
            uw[u] = ((lw >> (4 * (t4 >> 1))) & 0x0F0F0F0Fu) | (((hw >> (2 * t4)) & 0x03030303u) << 4);
        }
        off = 32.0f;
    } else if constexpr (QT == Q3_K) {
        const float d = h2f(*reinterpret_cast<const uint16_t*>(g + 108));
        const int n = p >> 7, j = (p >> 5) & 3;
        const uint8_t* sb = g + 96;
        const int is = 8 * n + 2 * j + (l >> 4);
        const uint32_t lo4 = is < 8 ? (sb[is] & 0xFu) : (uint32_t)(sb[is - 8] >> 4);
        const uint32_t hi2 = (sb[8 + (is & 3)] >> (2 * (is >> 2))) & 3u;
        dl = d * (float)((int)(lo4 | (hi2 << 4)) - 32);
        const uint16_t* a = reinterpret_cast<const uint16_t*>(g + 32 + 32 * n + l);  // 2-byte aligned
        const uint16_t* b = reinterpret_cast<const uint16_t*>(g + l);
        const int xs = 4 * n + j;
#pragma unroll
        for (int u = 0; u < 4; ++u) {
            const uint32_t lw = (uint32_t)a[2 * u] | ((uint32_t)a[2 * u + 1] << 16);
            const uint32_t hw = (uint32_t)b[2 * u] | ((uint32_t)b[2 * u + 1] << 16);
            // q = low2 - (hmask bit ? 0 : 4) = (low2 | bit << 2) - 4
            uw[u] = ((lw >> (2 * j)) & 0x03030303u) | (((hw >> xs) & 0x01010101u) << 2);
        }
        off = 4.0f;
    } else {  // Q2_K: 84-byte groups keep 4-byte alignment
        const uint32_t dd = *reinterpret_cast<const uint32_t*>(g + 80);
        const int n = p >> 7, j = (p >> 5) & 3;
        const uint32_t sc = g[8 * n + 2 * j + (l >> 4)];
        dl = h2f(dd & 0xffffu) * (float)(sc & 0xFu);
        ml = h2f(dd >> 16) * (float)(sc >> 4);
        const uint32_t* q = reinterpret_cast<const uint32_t*>(g + 16 + 32 * n + l);
#pragma unroll
        for (int u = 0; u < 4; ++u) uw[u] = (q[u] >> (2 * j)) & 0x03030303u;
    }
    opaque_words(uw);
    // two partial sums shorten the dependent fma chain
    float s1[2] = {0.0f, 0.0f};
#pragma unroll
    for (int u = 0; u < 4; ++u)
#pragma unroll
        for (int t = 0; t < 4; ++t) s1[u & 1] = fmaf(v[4 * u + t], (float)((uw[u] >> (8 * t)) & 0xffu), s1[u & 1]);
    float r = dl * ((s1[0] + s1[1]) - off * sv);
    if constexpr (HasMin<QT>::value) r -= ml * sv;
    return r;
}

// Exact values of the R (8 or 16) weights p .. p + R - 1 (p a multiple of R)
// of a group, for the mixture: the same real numbers as ggml's
// dequantize_row_*, computed as y = dl * u + c with u the unsigned code
// (unpacked four per 32-bit word and converted by v_cvt_f32_ubyteN) and c
// folding the format's offset and min.  dl * u is exact and each y is rounded
// once, like ggml's; only the sign of a zero may differ, which the mixture
// cannot see (+0 + (+-0) = +0).  A run of 16 never crosses a 16-weight scale
// block, so each run decodes one scale.
//
// decode_affine gives the run's unsigned codes (four per word: weight
// p + 4 i + t is byte t of uw[i]) and its affine map, weight = dl * u + c;
// decode_mix applies it.
template <int QT, int R>
__device__ __forceinline__ void decode_affine(const uint8_t* __restrict__ g, int p, uint32_t (&uw)[R / 4], float& dl,
                                              float& c) {
    static_assert(R == 8 || R == 16, "runs of 8 or 16 weights");
    constexpr int W = R / 4;
    if constexpr (QT == Q8_0) {
        const uint8_t* b = g + 34 * (p >> 5);
        const float d = h2f_hw(*reinterpret_cast<const uint16_t*>(b));
        load_run<2, R>(b + 2 + (p & 31), uw);
#pragma unroll
        for (int i = 0; i < W; ++i) uw[i] ^= 0x80808080u;  // q + 128
        dl = d;
        c = -128.0f * d;
    } else if constexpr (QT == Q4_K || QT == Q5_K) {
        const uint32_t dd = *reinterpret_cast<const uint32_t*>(g);
        const int ch = p >> 6, hi = (p >> 5) & 1;
        uint32_t sc, m;
        scale_min_k4(g + 4, 2 * ch + hi, sc, m);
        dl = h2f_hw(dd & 0xffffu) * (float)sc;
        c = -(h2f_hw(dd >> 16) * (float)m);
        load_run<8, R>(g + (QT == Q5_K ? 48 : 16) + 32 * ch + (p & 31), uw);
#pragma unroll
        for (int i = 0; i < W; ++i) uw[i] = (uw[i] >> (4 * hi)) & 0x0F0F0F0Fu;
        if constexpr (QT == Q5_K) {
            uint32_t xw[W];
            load_run<8, R>(g + 16 + (p & 31), xw);
            const int xs = 2 * ch + hi;
#pragma unroll
            for (int i = 0; i < W; ++i) uw[i] |= ((xw[i] >> xs) & 0x01010101u) << 4;
        }
    } else if constexpr (QT == Q6_K) {
        const float d = h2f_hw(*reinterpret_cast<const uint16_t*>(g + 208));
        const int n = p >> 7, t = (p >> 5) & 3, l = p & 31;
        dl = d * (float)(int8_t)g[192 + 8 * n + (l >> 4) + 2 * t];
        c = -32.0f * dl;
        uint32_t hw[W];
        load_run<2, R>(g + 64 * n + 32 * (t & 1) + l, uw);
        load_run<2, R>(g + 128 + 32 * n + l, hw);
#pragma unroll
        for (int i = 0; i < W; ++i)
            uw[i] = ((uw[i] >> (4 * (t >> 1))) & 0x0F0F0F0Fu) | (((hw[i] >> (2 * t)) & 0x03030303u) << 4);
    } else if constexpr (QT == Q3_K) {
        const float d = h2f_hw(*reinterpret_cast<const uint16_t*>(g + 108));
        const int n = p >> 7, j = (p >> 5) & 3, half = (p >> 4) & 1, l = p & 15;
        const int is = 8 * n + 2 * j + half;
        const uint8_t* sb = g + 96;
        const uint32_t lo4 = is < 8 ? (sb[is] & 0xFu) : (uint32_t)(sb[is - 8] >> 4);
        const uint32_t hi2 = (sb[8 + (is & 3)] >> (2 * (is >> 2))) & 3u;
        dl = d * (float)((int)(lo4 | (hi2 << 4)) - 32);
        c = -4.0f * dl;
        uint32_t hw[W];
        load_run<2, R>(g + 32 + 32 * n + 16 * half + l, uw);
        load_run<2, R>(g + 16 * half + l, hw);
        const int xs = 4 * n + j;
#pragma unroll
        for (int i = 0; i < W; ++i)
            uw[i] = ((uw[i] >> (2 * j)) & 0x03030303u) | (((hw[i] >> xs) & 0x01010101u) << 2);
    } else {  // Q2_K
        const uint32_t dd = *reinterpret_cast<const uint32_t*>(g + 80);
        const int n = p >> 7, j = (p >> 5) & 3, half = (p >> 4) & 1, l = p & 15;
        const uint32_t sc = g[8 * n + 2 * j + half];
        dl = h2f_hw(dd & 0xffffu) * (float)(sc & 0xFu);
        c = -(h2f_hw(dd >> 16) * (float)(sc >> 4));
        load_run<4, R>(g + 16 + 32 * n + 16 * half + l, uw);
#pragma unroll
        for (int i = 0; i < W; ++i) uw[i] = (uw[i] >> (2 * j)) & 0x03030303u;
    }
}

template <int QT, int R = 8>
__device__ __forceinline__ void decode_mix(const uint8_t* __restrict__ g, int p, float (&y)[R]) {
    uint32_t uw[R / 4];
    float dl, c;
    decode_affine<QT, R>(g, p, uw, dl, c);
    opaque_words(uw);
#pragma unroll
    for (int r = 0; r < R; ++r) y[r] = fmaf(dl, (float)((uw[r >> 2] >> (8 * (r & 3))) & 0xffu), c);
}

template <int QT>
__device__ __forceinline__ void decode8_mix(const uint8_t* __restrict__ g, int p, float (&y)[8]) {
    decode_mix<QT, 8>(g, p, y);
}

// ---------------------------------------------------------------------------
// The IQ formats, one runtime-dispatched path (their decode is table lookups,
// not shifts, so one instantiation per consumer serves all eight): the same
// four operations as the K-quant templates above, on iq_affine's codes.
// ---------------------------------------------------------------------------
template <int R, class Books = GlobalBooks>
__device__ __forceinline__ void decode_run_iq(int qt, const uint8_t* __restrict__ g, int p, float* __restrict__ y,
                                              const Books& bk = Books()) {
    uint32_t uw[R / 4];
    float dl;
    iq_affine<R>(qt, g, p, uw, dl, bk);
#pragma unroll
    for (int r = 0; r < R; ++r) y[r] = dl * ((float)((uw[r >> 2] >> (8 * (r & 3))) & 0xffu) - 128.0f);
}

template <int R>
__device__ __forceinline__ void decode_affine_iq(int qt, const uint8_t* __restrict__ g, int p, uint32_t (&uw)[R / 4],
                                                 float& dl, float& c) {
    iq_affine<R>(qt, g, p, uw, dl);
    c = -128.0f * dl;
}

template <int R>
__device__ __forceinline__ void decode_mix_iq(int qt, const uint8_t* __restrict__ g, int p, float (&y)[R]) {
    uint32_t uw[R / 4];
    float dl, c;
    decode_affine_iq<R>(qt, g, p, uw, dl, c);
#pragma unroll
    for (int r = 0; r < R; ++r) y[r] = fmaf(dl, (float)((uw[r >> 2] >> (8 * (r & 3))) & 0xffu), c);
}

template <int R>
__device__ __forceinline__ float dot_run_iq(int qt, const uint8_t* __restrict__ g, int p, const float* __restrict__ v) {
    uint32_t uw[R / 4];
    float dl;
    iq_affine<R>(qt, g, p, uw, dl);
    float s1 = 0.0f, s0 = 0.0f;
#pragma unroll
    for (int r = 0; r < R; ++r) {
        s1 = fmaf(v[r], (float)((uw[r >> 2] >> (8 * (r & 3))) & 0xffu), s1);
        s0 += v[r];
    }
    return dl * (s1 - 128.0f * s0);
}

// dot_sub16 for the IQ formats: sum v (dl (u - 128)) = dl (sum v u - 128 sv)
__device__ __forceinline__ float dot_sub16_iq(int qt, const uint8_t* __restrict__ g, int p, const float* __restrict__ v,
                                              float sv) {
    uint32_t uw[4];
    float dl;
    iq_affine<16>(qt, g, p, uw, dl);
    float s1[2] = {0.0f, 0.0f};
#pragma unroll
    for (int u = 0; u < 4; ++u)
#pragma unroll
        for (int t = 0; t < 4; ++t) s1[u & 1] = fmaf(v[4 * u + t], (float)((uw[u] >> (8 * t)) & 0xffu), s1[u & 1]);
    return dl * ((s1[0] + s1[1]) - 128.0f * sv);
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
    case Q6_K: decode_run<Q6_K, R>(g, p, y); break;
    default: decode_run_iq<R>(qt, g, p, y); break;
    }
}

// Up to this many candidates per gated tensor: every format this library
// decodes (the reference's default menu, list_quant_types(), has 14 types
// of which 12 decode here; its training recipes use 4-8).
constexpr int kMaxCand = 16;

struct CandSet {
    const uint8_t* qbytes[kMaxCand];  // packed rows [N][D_pad/256 groups]
    int qtype[kMaxCand];
    int ncand;
    int64_t row_groups;  // D_pad / 256
};

// Whether a launch must take the instantiation that decodes IQ formats.
inline bool any_iq(const CandSet& cs) {
    for (int k = 0; k < cs.ncand; ++k)
        if (is_iq(cs.qtype[k])) return true;
    return false;
}

// Gated tensors that share one input, stacked along N: set g owns rows
// [set_j0[g], set_j0[g + 1]) of the stacked weight (boundaries on 256-row
// tiles).  Gate partials are [grid block][nsets * kstride], set g's candidate
// k at g * kstride + k.
constexpr int kMaxSets = 4;
struct CandGroup {
    int nsets;
    int kstride;
    int set_j0[kMaxSets + 1];
    CandSet sets[kMaxSets];
};

inline bool any_iq(const CandGroup& cg) {
    for (int i = 0; i < cg.nsets; ++i)
        if (any_iq(cg.sets[i])) return true;
    return false;
}

}  // namespace vq
