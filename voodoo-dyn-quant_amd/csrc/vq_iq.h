// GGUF i-quant ("IQ") decoders, included by vq_common.h after its helpers.
//
// Every IQ weight is a sub-block scale times a small signed value taken from
// a code book (the grids of vq_iq_grids.inc) or, for IQ4_XS, from a 16-entry
// non-linear table.  The byte layouts and float expressions are those of the
// reference's decoders (voodoo_quant/quants/gpu_dequant.py:53-519, which
// follow ggml's dequantize_row_iq*):
//
//   IQ2_XXS {d; u16 qs[32]}                       db = d (0.5 + s) / 4, 7 sign bits + parity
//   IQ2_XS  {d; u16 qs[32]; scales[8]}            9-bit grid index, 7 sign bits + parity
//   IQ2_S   {d; qs[32]; signs[32]; qh[8]; sc[8]}  10-bit grid index, 8 stored signs
//   IQ3_XXS {d; qs[64]; u32 scale+signs[8]}       two 4-value grids per 8 weights
//   IQ3_S   {d; qs[64]; qh[8]; signs[32]; sc[4]}  db = d (1 + 2 s)
//   IQ1_S   {d; qs[32]; u16 qh[8]}                dl (g + delta), g in {-1, 0, 1}, delta = +-1/8
//   IQ1_M   {qs[32]; qh[16]; u16 sc[4]}           d spread over the sc top nibbles
//   IQ4_XS  {d; u16 sh; sl[4]; qs[128]}           dl = d (ls - 32), 4-bit codes into the table
//
// iq_affine gives a run of R (8 or 16) weights in the form decode_affine uses:
// unsigned byte codes u (four per word) and a scale dl with
//     weight = dl * (u - 128).
// Each weight is exact in fp32 (scales carry at most 16 significant bits and
// grid values at most 8), so any evaluation of dl * (u - 128), including an
// FMA, gives ggml's value.  IQ1 values g + delta are carried as 8 g +- 1 with
// dl / 8 (exact), which is the same real product.  A run never crosses a scale:
// runs of 16 start at multiples of 16, and every IQ sub-block scale covers 16
// or 32 weights.
#pragma once

namespace vq {

// 16-byte aligned, so a kernel can copy a table to LDS with direct-to-LDS loads
#define VQ_IQ_TABLE(type, name, n) static __device__ const type name[n] __attribute__((aligned(16)))
#include "vq_iq_grids.inc"
#undef VQ_IQ_TABLE

// Where the code-book lookups of a decode read from.  GlobalBooks: the tables
// in global memory (every decode site; the lookups go through L1).  LdsBook:
// a kernel that decodes one IQ format has copied that format's table to LDS
// (iq_book_bytes / iq_book_src) and reads it there.
struct GlobalBooks {
    __device__ __forceinline__ uint64_t q2xxs(uint32_t i) const { return iq2xxs_grid[i]; }
    __device__ __forceinline__ uint64_t q2xs(uint32_t i) const { return iq2xs_grid[i]; }
    __device__ __forceinline__ uint64_t q2s(uint32_t i) const { return iq2s_grid[i]; }
    __device__ __forceinline__ uint32_t q3xxs(uint32_t i) const { return iq3xxs_grid[i]; }
    __device__ __forceinline__ uint32_t q3s(uint32_t i) const { return iq3s_grid[i]; }
    __device__ __forceinline__ uint64_t q1s(uint32_t i) const { return iq1s_grid[i]; }
};

struct LdsBook {
    const __attribute__((address_space(3))) uint8_t* p;
    __device__ __forceinline__ uint64_t u64(uint32_t i) const {
        return reinterpret_cast<const __attribute__((address_space(3))) uint64_t*>(p)[i];
    }
    __device__ __forceinline__ uint32_t u32(uint32_t i) const {
        return reinterpret_cast<const __attribute__((address_space(3))) uint32_t*>(p)[i];
    }
    __device__ __forceinline__ uint64_t q2xxs(uint32_t i) const { return u64(i); }
    __device__ __forceinline__ uint64_t q2xs(uint32_t i) const { return u64(i); }
    __device__ __forceinline__ uint64_t q2s(uint32_t i) const { return u64(i); }
    __device__ __forceinline__ uint32_t q3xxs(uint32_t i) const { return u32(i); }
    __device__ __forceinline__ uint32_t q3s(uint32_t i) const { return u32(i); }
    __device__ __forceinline__ uint64_t q1s(uint32_t i) const { return u64(i); }
};

// Bytes of the code book a format's decode reads (0: none, IQ4_XS's 16
// values sit in registers), and its address in global memory.
__host__ __device__ constexpr int iq_book_bytes(int qt) {
    return qt == IQ2_XXS ? 256 * 8 : qt == IQ2_XS ? 512 * 8 : qt == IQ2_S ? 1024 * 8 : qt == IQ3_XXS ? 256 * 4
         : qt == IQ3_S ? 512 * 4 : (qt == IQ1_S || qt == IQ1_M) ? 2048 * 8 : 0;
}

__device__ __forceinline__ const uint8_t* iq_book_src(int qt) {
    switch (qt) {
    case IQ2_XXS: return reinterpret_cast<const uint8_t*>(iq2xxs_grid);
    case IQ2_XS: return reinterpret_cast<const uint8_t*>(iq2xs_grid);
    case IQ2_S: return reinterpret_cast<const uint8_t*>(iq2s_grid);
    case IQ3_XXS: return reinterpret_cast<const uint8_t*>(iq3xxs_grid);
    case IQ3_S: return reinterpret_cast<const uint8_t*>(iq3s_grid);
    default: return reinterpret_cast<const uint8_t*>(iq1s_grid);
    }
}

__host__ __device__ constexpr bool is_iq(int qt) {
    return qt == IQ2_XXS || qt == IQ2_XS || qt == IQ3_XXS || qt == IQ1_S || qt == IQ3_S || qt == IQ2_S ||
           qt == IQ4_XS || qt == IQ1_M;
}

__device__ __forceinline__ uint32_t rd_u32(const uint8_t* p) { return rd_u16(p) | (rd_u16(p + 2) << 16); }

// bit j of s (j < 4) -> byte j all ones
__device__ __forceinline__ uint32_t nibble_mask(uint32_t s) { return ((s & 15u) * 0x00204081u & 0x01010101u) * 0xFFu; }

// 7 stored sign bits -> 8, the eighth making the count of negatives even
__device__ __forceinline__ uint32_t parity_signs(uint32_t i7) { return i7 | ((uint32_t)(__builtin_popcount(i7) & 1) << 7); }

// Four grid bytes b (1..127) and their sign bits -> bytes 128 + b or 128 - b.
// Negating a byte as (b ^ 0xff) + 1 cannot carry for b >= 1, and 256 - b then
// has its top bit set, so XOR 0x80 turns both cases into the biased code.
__device__ __forceinline__ uint32_t signed_grid(uint32_t g4, uint32_t s4) {
    const uint32_t m = nibble_mask(s4);
    return ((g4 ^ m) + (m & 0x01010101u)) ^ 0x80808080u;
}

// Four IQ1 grid bytes (int8 -1, 0, 1) and delta sign -> bytes 128 + 8 g +- 1:
// g ^ 0x80 = 128 + g, minus 112 is 16 + g (no borrow), times 8 stays below 256.
__device__ __forceinline__ uint32_t iq1_codes(uint32_t g4, bool neg) {
    const uint32_t e = (((g4 ^ 0x80808080u) - 0x70707070u) << 3);
    return neg ? e - 0x01010101u : e + 0x01010101u;
}

// Eight consecutive weights 8 l .. 8 l + 7 of sub-block ib (32 weights), as
// biased codes in two words.  g may point into LDS or global memory; IQ
// groups are only 2-byte aligned, so every multi-byte field is read in halves.
template <class Books = GlobalBooks>
__device__ __forceinline__ void iq_group8(int qt, const uint8_t* __restrict__ g, int ib, int l, uint32_t& w0,
                                          uint32_t& w1, const Books& bk = Books()) {
    switch (qt) {
    case IQ2_XXS: {
        const uint8_t* q = g + 2 + 8 * ib;
        const uint64_t gr = bk.q2xxs(q[l]);
        const uint32_t s = parity_signs((rd_u32(q + 4) >> (7 * l)) & 127u);
        w0 = signed_grid((uint32_t)gr, s);
        w1 = signed_grid((uint32_t)(gr >> 32), s >> 4);
        break;
    }
    case IQ2_XS: {
        const uint32_t q = rd_u16(g + 2 + 2 * (4 * ib + l));
        const uint64_t gr = bk.q2xs(q & 511u);
        const uint32_t s = parity_signs(q >> 9);
        w0 = signed_grid((uint32_t)gr, s);
        w1 = signed_grid((uint32_t)(gr >> 32), s >> 4);
        break;
    }
    case IQ2_S: {
        const uint32_t idx = g[2 + 4 * ib + l] | (((uint32_t)g[66 + ib] << (8 - 2 * l)) & 0x300u);
        const uint64_t gr = bk.q2s(idx);
        const uint32_t s = g[34 + 4 * ib + l];
        w0 = signed_grid((uint32_t)gr, s);
        w1 = signed_grid((uint32_t)(gr >> 32), s >> 4);
        break;
    }
    case IQ3_XXS: {
        const uint32_t s = parity_signs((rd_u32(g + 66 + 4 * ib) >> (7 * l)) & 127u);
        w0 = signed_grid(bk.q3xxs(g[2 + 8 * ib + 2 * l]), s);
        w1 = signed_grid(bk.q3xxs(g[2 + 8 * ib + 2 * l + 1]), s >> 4);
        break;
    }
    case IQ3_S: {
        const uint32_t h = g[66 + ib];
        const uint32_t s = g[74 + 4 * ib + l];
        w0 = signed_grid(bk.q3s(g[2 + 8 * ib + 2 * l] | ((h << (8 - 2 * l)) & 256u)), s);
        w1 = signed_grid(bk.q3s(g[2 + 8 * ib + 2 * l + 1] | ((h << (7 - 2 * l)) & 256u)), s >> 4);
        break;
    }
    case IQ1_S: {
        const uint32_t qh = rd_u16(g + 34 + 2 * ib);
        const uint64_t gr = bk.q1s(g[2 + 4 * ib + l] | (((qh >> (3 * l)) & 7u) << 8));
        const bool neg = (qh & 0x8000u) != 0;
        w0 = iq1_codes((uint32_t)gr, neg);
        w1 = iq1_codes((uint32_t)(gr >> 32), neg);
        break;
    }
    case IQ1_M: {
        const uint32_t h = g[32 + 2 * ib + (l >> 1)];
        const uint32_t idx = g[4 * ib + l] | ((h << ((l & 1) ? 4 : 8)) & 0x700u);
        const uint64_t gr = bk.q1s(idx);
        const bool neg = (h & ((l & 1) ? 0x80u : 0x08u)) != 0;
        w0 = iq1_codes((uint32_t)gr, neg);
        w1 = iq1_codes((uint32_t)(gr >> 32), neg);
        break;
    }
    default: {  // IQ4_XS: weight j of the sub-block is the low nibble of qs[16 ib + j] (j < 16), else the high
        // the table biased by 128, four entries per word
        uint32_t k[4];
#pragma unroll
        for (int t = 0; t < 4; ++t)
            k[t] = (uint32_t)(uint8_t)(iq4nl_values[4 * t] + 128) |
                   ((uint32_t)(uint8_t)(iq4nl_values[4 * t + 1] + 128) << 8) |
                   ((uint32_t)(uint8_t)(iq4nl_values[4 * t + 2] + 128) << 16) |
                   ((uint32_t)(uint8_t)(iq4nl_values[4 * t + 3] + 128) << 24);
        const uint8_t* q = g + 8 + 16 * ib + 8 * (l & 1);
        const int sh = 4 * (l >> 1);
        uint32_t w[2];
#pragma unroll
        for (int h = 0; h < 2; ++h) {
            const uint32_t n = (rd_u32(q + 4 * h) >> sh) & 0x0F0F0F0Fu;  // four 4-bit codes
            const uint32_t lo = __builtin_amdgcn_perm(k[1], k[0], n & 0x07070707u);
            const uint32_t hi = __builtin_amdgcn_perm(k[3], k[2], n & 0x07070707u);
            const uint32_t m = ((n >> 3) & 0x01010101u) * 0xFFu;
            w[h] = (lo & ~m) | (hi & m);
        }
        w0 = w[0];
        w1 = w[1];
        break;
    }
    }
}

// The scale of weights 8 l .. 8 l + 7 of sub-block ib, in ggml's float
// expression (IQ1: divided by 8 for the 8 g +- 1 codes).
__device__ __forceinline__ float iq_scale(int qt, const uint8_t* __restrict__ g, int ib, int l) {
    if (qt == IQ1_M) {
        const uint32_t s0 = rd_u16(g + 48), s1 = rd_u16(g + 50), s2 = rd_u16(g + 52), s3 = rd_u16(g + 54);
        const float d = h2f((s0 >> 12) | ((s1 >> 8) & 0x00f0u) | ((s2 >> 4) & 0x0f00u) | (s3 & 0xf000u));
        const uint32_t s = rd_u16(g + 48 + 2 * (ib >> 1));
        return d * (float)(2 * ((s >> (6 * (ib & 1) + 3 * (l >> 1))) & 7u) + 1) * 0.125f;
    }
    const float d = h2f(rd_u16(g));
    switch (qt) {
    case IQ2_XXS: return d * (0.5f + (float)(rd_u16(g + 2 + 8 * ib + 6) >> 12)) * 0.25f;
    case IQ2_XS: {
        const uint32_t sc = g[66 + ib];
        return d * (0.5f + (float)(l < 2 ? sc & 15u : sc >> 4)) * 0.25f;
    }
    case IQ2_S: {
        const uint32_t sc = g[74 + ib];
        return d * (0.5f + (float)(l < 2 ? sc & 15u : sc >> 4)) * 0.25f;
    }
    case IQ3_XXS: return d * (0.5f + (float)(rd_u16(g + 66 + 4 * ib + 2) >> 12)) * 0.5f;
    case IQ3_S: {
        const uint32_t sc = g[106 + (ib >> 1)];
        return d * (float)(1 + 2 * (int)((ib & 1) ? sc >> 4 : sc & 15u));
    }
    case IQ1_S: return d * (float)(2 * ((rd_u16(g + 34 + 2 * ib) >> 12) & 7u) + 1) * 0.125f;
    default: {  // IQ4_XS
        const uint32_t sh = rd_u16(g + 2);
        const int ls = (int)(((g[4 + (ib >> 1)] >> (4 * (ib & 1))) & 15u) | (((sh >> (2 * ib)) & 3u) << 4));
        return d * ((float)ls - 32.0f);
    }
    }
}

// Weights p .. p + R - 1 (p a multiple of R) of the 256-weight group at g.
template <int R, class Books = GlobalBooks>
__device__ __forceinline__ void iq_affine(int qt, const uint8_t* __restrict__ g, int p, uint32_t (&uw)[R / 4],
                                          float& dl, const Books& bk = Books()) {
    static_assert(R == 8 || R == 16, "runs of 8 or 16 weights");
    const int ib = p >> 5, l = (p >> 3) & 3;
    dl = iq_scale(qt, g, ib, l);
#pragma unroll
    for (int h = 0; h < R / 8; ++h) iq_group8(qt, g, ib, l + h, uw[2 * h], uw[2 * h + 1], bk);
}

}  // namespace vq
