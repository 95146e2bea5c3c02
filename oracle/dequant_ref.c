/*
 * ORACLE — test infrastructure only.  Nothing in the product links this file;
 * only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg load it,
 * and only as the checker.
 *
 * Scalar CPU restatement of GGUF block dequantisation (ggml's
 * dequantize_row_<type>) for the six formats on the gated-Linear path.  Each
 * routine walks a block in the order ggml's own loops do, so the float
 * expressions (and therefore every rounding and every signed zero) are the
 * same as ggml's:
 *
 *   Q8_0  voodoo_quant/layers.py:62-75    y = qs[j] * d
 *   Q4_K  voodoo_quant/layers.py:78-122   y = (d*sc) * q - (dmin*m),  6-bit scale/min unpack :91-105
 *   Q5_K  voodoo_quant/layers.py:125-179  as Q4_K with a 5th bit from qh (bit 2j / 2j+1)
 *   Q6_K  voodoo_quant/layers.py:182-213  y = (d*sc) * (q - 32), d stored last
 *   Q3_K  not in the reference: public GGUF layout (llama.cpp ggml-common.h /
 *         ggml-quants.c, MIT), block {hmask[32]; qs[64]; scales[12]; d}
 *   Q2_K  not in the reference: public GGUF layout, block {scales[16]; qs[64]; d; dmin}
 *
 * Q3_K and Q2_K are pinned only by the structured packer round trip in
 * oracle/blocks.py and by the closed-form checks in tests/ — against ggml's own
 * decoder they are "parity unpinned" (no libggml and no reference text exists
 * for them in this environment).
 *
 * fp16 -> fp32 is an exact bit-level widening (subnormals, infinities, NaNs).
 */
#include <stdint.h>
#include <string.h>

static float oracle_fp16_to_fp32(uint16_t h) {
    uint32_t sign = (uint32_t)(h >> 15) << 31;
    uint32_t exp = (h >> 10) & 0x1f;
    uint32_t man = h & 0x3ff;
    uint32_t bits;
    if (exp == 0) {
        if (man == 0) {
            bits = sign;
        } else {
            /* subnormal half: value = man * 2^-24, exact in fp32 */
            int e = -1;
            do { man <<= 1; e++; } while ((man & 0x400) == 0);
            man &= 0x3ff;
            bits = sign | ((uint32_t)(127 - 15 - e) << 23) | (man << 13);
        }
    } else if (exp == 0x1f) {
        bits = sign | 0x7f800000u | (man << 13);
    } else {
        bits = sign | ((exp + (127 - 15)) << 23) | (man << 13);
    }
    float f;
    memcpy(&f, &bits, 4);
    return f;
}

static uint16_t rd16(const uint8_t *p) { return (uint16_t)(p[0] | (p[1] << 8)); }

float oracle_half_to_float(uint16_t h) { return oracle_fp16_to_fp32(h); }

/* Q8_0: 34-byte blocks {fp16 d; int8 qs[32]} */
void oracle_dequant_q8_0(const uint8_t *x, float *y, int64_t k) {
    const int64_t nb = k / 32;
    for (int64_t i = 0; i < nb; i++) {
        const uint8_t *b = x + i * 34;
        const float d = oracle_fp16_to_fp32(rd16(b));
        const int8_t *qs = (const int8_t *)(b + 2);
        for (int j = 0; j < 32; ++j) y[i * 32 + j] = qs[j] * d;
    }
}

/* 6-bit scale/min pair j of a Q4_K/Q5_K 12-byte scales array */
static void oracle_scale_min_k4(int j, const uint8_t *q, uint8_t *d, uint8_t *m) {
    if (j < 4) {
        *d = q[j] & 63;
        *m = q[j + 4] & 63;
    } else {
        *d = (q[j + 4] & 0xF) | ((q[j - 4] >> 6) << 4);
        *m = (q[j + 4] >> 4) | ((q[j] >> 6) << 4);
    }
}

/* Q4_K: 144-byte blocks {fp16 d; fp16 dmin; scales[12]; qs[128]} */
void oracle_dequant_q4_K(const uint8_t *x, float *y, int64_t k) {
    const int64_t nb = k / 256;
    for (int64_t i = 0; i < nb; i++) {
        const uint8_t *b = x + i * 144;
        const float d = oracle_fp16_to_fp32(rd16(b));
        const float min = oracle_fp16_to_fp32(rd16(b + 2));
        const uint8_t *scales = b + 4;
        const uint8_t *q = b + 16;
        int is = 0;
        uint8_t sc, m;
        for (int j = 0; j < 256; j += 64) {
            oracle_scale_min_k4(is + 0, scales, &sc, &m);
            const float d1 = d * sc, m1 = min * m;
            oracle_scale_min_k4(is + 1, scales, &sc, &m);
            const float d2 = d * sc, m2 = min * m;
            for (int l = 0; l < 32; ++l) *y++ = d1 * (q[l] & 0xF) - m1;
            for (int l = 0; l < 32; ++l) *y++ = d2 * (q[l] >> 4) - m2;
            q += 32;
            is += 2;
        }
    }
}

/* Q5_K: 176-byte blocks {fp16 d; fp16 dmin; scales[12]; qh[32]; qs[128]} */
void oracle_dequant_q5_K(const uint8_t *x, float *y, int64_t k) {
    const int64_t nb = k / 256;
    for (int64_t i = 0; i < nb; i++) {
        const uint8_t *b = x + i * 176;
        const float d = oracle_fp16_to_fp32(rd16(b));
        const float min = oracle_fp16_to_fp32(rd16(b + 2));
        const uint8_t *scales = b + 4;
        const uint8_t *qh = b + 16;
        const uint8_t *ql = b + 48;
        int is = 0;
        uint8_t sc, m;
        uint8_t u1 = 1, u2 = 2;
        for (int j = 0; j < 256; j += 64) {
            oracle_scale_min_k4(is + 0, scales, &sc, &m);
            const float d1 = d * sc, m1 = min * m;
            oracle_scale_min_k4(is + 1, scales, &sc, &m);
            const float d2 = d * sc, m2 = min * m;
            for (int l = 0; l < 32; ++l) *y++ = d1 * ((ql[l] & 0xF) + (qh[l] & u1 ? 16 : 0)) - m1;
            for (int l = 0; l < 32; ++l) *y++ = d2 * ((ql[l] >> 4) + (qh[l] & u2 ? 16 : 0)) - m2;
            ql += 32;
            is += 2;
            u1 <<= 2;
            u2 <<= 2;
        }
    }
}

/* Q6_K: 210-byte blocks {ql[128]; qh[64]; int8 scales[16]; fp16 d} */
void oracle_dequant_q6_K(const uint8_t *x, float *y, int64_t k) {
    const int64_t nb = k / 256;
    for (int64_t i = 0; i < nb; i++) {
        const uint8_t *b = x + i * 210;
        const float d = oracle_fp16_to_fp32(rd16(b + 208));
        const uint8_t *ql = b;
        const uint8_t *qh = b + 128;
        const int8_t *sc = (const int8_t *)(b + 192);
        for (int n = 0; n < 256; n += 128) {
            for (int l = 0; l < 32; ++l) {
                const int is = l / 16;
                const int8_t q1 = (int8_t)((ql[l + 0] & 0xF) | (((qh[l] >> 0) & 3) << 4)) - 32;
                const int8_t q2 = (int8_t)((ql[l + 32] & 0xF) | (((qh[l] >> 2) & 3) << 4)) - 32;
                const int8_t q3 = (int8_t)((ql[l + 0] >> 4) | (((qh[l] >> 4) & 3) << 4)) - 32;
                const int8_t q4 = (int8_t)((ql[l + 32] >> 4) | (((qh[l] >> 6) & 3) << 4)) - 32;
                y[l + 0] = d * sc[is + 0] * q1;
                y[l + 32] = d * sc[is + 2] * q2;
                y[l + 64] = d * sc[is + 4] * q3;
                y[l + 96] = d * sc[is + 6] * q4;
            }
            y += 128;
            ql += 64;
            qh += 32;
            sc += 8;
        }
    }
}

/*
 * The Q3_K and Q2_K routines below follow llama.cpp's dequantize_row_q3_K and
 * dequantize_row_q2_K (ggml/src/ggml-quants.c) step for step, so that the
 * oracle reproduces ggml's arithmetic; that code is under the MIT License:
 *
 *   Copyright (c) 2023-2024 The ggml authors
 *
 *   Permission is hereby granted, free of charge, to any person obtaining a
 *   copy of this software and associated documentation files (the
 *   "Software"), to deal in the Software without restriction, including
 *   without limitation the rights to use, copy, modify, merge, publish,
 *   distribute, sublicense, and/or sell copies of the Software, and to permit
 *   persons to whom the Software is furnished to do so, subject to the
 *   following conditions:
 *
 *   The above copyright notice and this permission notice shall be included
 *   in all copies or substantial portions of the Software.
 *
 *   THE SOFTWARE IS PROVIDED "AS IS", WITHOUT WARRANTY OF ANY KIND, EXPRESS
 *   OR IMPLIED, INCLUDING BUT NOT LIMITED TO THE WARRANTIES OF
 *   MERCHANTABILITY, FITNESS FOR A PARTICULAR PURPOSE AND NONINFRINGEMENT. IN
 *   NO EVENT SHALL THE AUTHORS OR COPYRIGHT HOLDERS BE LIABLE FOR ANY CLAIM,
 *   DAMAGES OR OTHER LIABILITY, WHETHER IN AN ACTION OF CONTRACT, TORT OR
 *   OTHERWISE, ARISING FROM, OUT OF OR IN CONNECTION WITH THE SOFTWARE OR THE
 *   USE OR OTHER DEALINGS IN THE SOFTWARE.
 */

/* Q3_K: 110-byte blocks {hmask[32]; qs[64]; scales[12]; fp16 d} */
void oracle_dequant_q3_K(const uint8_t *x, float *y, int64_t k) {
    const int64_t nb = k / 256;
    const uint32_t kmask1 = 0x03030303u, kmask2 = 0x0f0f0f0fu;
    uint32_t aux[4];
    const int8_t *scales = (const int8_t *)aux;
    for (int64_t i = 0; i < nb; i++) {
        const uint8_t *b = x + i * 110;
        const float d_all = oracle_fp16_to_fp32(rd16(b + 108));
        const uint8_t *q = b + 32;
        const uint8_t *hm = b;
        uint8_t m = 1;
        memcpy(aux, b + 96, 12);
        const uint32_t tmp = aux[2];
        aux[2] = ((aux[0] >> 4) & kmask2) | (((tmp >> 4) & kmask1) << 4);
        aux[3] = ((aux[1] >> 4) & kmask2) | (((tmp >> 6) & kmask1) << 4);
        aux[0] = (aux[0] & kmask2) | (((tmp >> 0) & kmask1) << 4);
        aux[1] = (aux[1] & kmask2) | (((tmp >> 2) & kmask1) << 4);
        int is = 0;
        float dl;
        for (int n = 0; n < 256; n += 128) {
            int shift = 0;
            for (int j = 0; j < 4; ++j) {
                dl = d_all * (scales[is++] - 32);
                for (int l = 0; l < 16; ++l)
                    *y++ = dl * ((int8_t)((q[l + 0] >> shift) & 3) - ((hm[l + 0] & m) ? 0 : 4));
                dl = d_all * (scales[is++] - 32);
                for (int l = 0; l < 16; ++l)
                    *y++ = dl * ((int8_t)((q[l + 16] >> shift) & 3) - ((hm[l + 16] & m) ? 0 : 4));
                shift += 2;
                m <<= 1;
            }
            q += 32;
        }
    }
}

/* Q2_K: 84-byte blocks {scales[16]; qs[64]; fp16 d; fp16 dmin} */
void oracle_dequant_q2_K(const uint8_t *x, float *y, int64_t k) {
    const int64_t nb = k / 256;
    for (int64_t i = 0; i < nb; i++) {
        const uint8_t *b = x + i * 84;
        const float d = oracle_fp16_to_fp32(rd16(b + 80));
        const float min = oracle_fp16_to_fp32(rd16(b + 82));
        const uint8_t *sc_arr = b;
        const uint8_t *q = b + 16;
        int is = 0;
        float dl, ml;
        for (int n = 0; n < 256; n += 128) {
            int shift = 0;
            for (int j = 0; j < 4; ++j) {
                uint8_t sc = sc_arr[is++];
                dl = d * (sc & 0xF);
                ml = min * (sc >> 4);
                for (int l = 0; l < 16; ++l) *y++ = dl * ((int8_t)((q[l] >> shift) & 3)) - ml;
                sc = sc_arr[is++];
                dl = d * (sc & 0xF);
                ml = min * (sc >> 4);
                for (int l = 0; l < 16; ++l) *y++ = dl * ((int8_t)((q[l + 16] >> shift) & 3)) - ml;
                shift += 2;
            }
            q += 32;
        }
    }
}

/* ---------------------------------------------------------------------------
 * IQ formats: restatement of the reference's decoders in
 * voodoo_quant/quants/gpu_dequant.py (line numbers below), which follow
 * ggml's dequantize_row_iq*.  Every weight is a product of an fp16-derived
 * sub-block scale and a grid value (sign applied last), in the reference's
 * order of float operations.  The grids are the GGUF code books, carried as
 * data in voodoo-dyn-quant_amd/csrc/vq_iq_grids.inc; the sign byte of a 7-bit
 * index is its even-parity completion.
 * ------------------------------------------------------------------------- */
#define VQ_IQ_TABLE(type, name, n) static const type name[n]
#include "../voodoo-dyn-quant_amd/csrc/vq_iq_grids.inc"
#undef VQ_IQ_TABLE

static uint32_t rd32(const uint8_t *p) {
    return (uint32_t)p[0] | ((uint32_t)p[1] << 8) | ((uint32_t)p[2] << 16) | ((uint32_t)p[3] << 24);
}

static uint8_t parity_signs(uint32_t i7) { /* ksigns_iq2xs[i7] */
    return (uint8_t)(i7 | ((uint32_t)__builtin_parity(i7) << 7));
}

static float sgn(uint32_t signs, int j) { return (signs >> j) & 1u ? -1.f : 1.f; }

/* IQ2_XXS, 66-byte blocks {fp16 d; u16 qs[32]}: gpu_dequant.py:53-114 */
void oracle_dequant_iq2_xxs(const uint8_t *x, float *y, int64_t k) {
    for (int64_t i = 0; i < k / 256; i++) {
        const uint8_t *b = x + i * 66;
        const float d = oracle_fp16_to_fp32(rd16(b));
        for (int ib32 = 0; ib32 < 8; ++ib32) {
            const uint8_t *q = b + 2 + 8 * ib32;
            const uint32_t aux1 = rd32(q + 4);
            const float db = d * (0.5f + (float)(aux1 >> 28)) * 0.25f;
            for (int l = 0; l < 4; ++l) {
                const uint8_t *grid = (const uint8_t *)&iq2xxs_grid[q[l]];
                const uint32_t signs = parity_signs((aux1 >> (7 * l)) & 127u);
                for (int j = 0; j < 8; ++j) *y++ = db * (float)grid[j] * sgn(signs, j);
            }
        }
    }
}

/* IQ2_XS, 74-byte blocks {fp16 d; u16 qs[32]; scales[8]}: gpu_dequant.py:121-166 */
void oracle_dequant_iq2_xs(const uint8_t *x, float *y, int64_t k) {
    for (int64_t i = 0; i < k / 256; i++) {
        const uint8_t *b = x + i * 74;
        const float d = oracle_fp16_to_fp32(rd16(b));
        for (int ib32 = 0; ib32 < 8; ++ib32) {
            const uint8_t sc = b[66 + ib32];
            const float db0 = d * (0.5f + (float)(sc & 0xf)) * 0.25f;
            const float db1 = d * (0.5f + (float)(sc >> 4)) * 0.25f;
            for (int l = 0; l < 4; ++l) {
                const uint32_t q = rd16(b + 2 + 2 * (4 * ib32 + l));
                const uint8_t *grid = (const uint8_t *)&iq2xs_grid[q & 511u];
                const uint32_t signs = parity_signs(q >> 9);
                const float db = l < 2 ? db0 : db1;
                for (int j = 0; j < 8; ++j) *y++ = db * (float)grid[j] * sgn(signs, j);
            }
        }
    }
}

/* IQ2_S, 82-byte blocks {fp16 d; qs[32] + signs[32]; qh[8]; scales[8]}: gpu_dequant.py:173-217 */
void oracle_dequant_iq2_s(const uint8_t *x, float *y, int64_t k) {
    for (int64_t i = 0; i < k / 256; i++) {
        const uint8_t *b = x + i * 82;
        const float d = oracle_fp16_to_fp32(rd16(b));
        const uint8_t *qs = b + 2, *qh = b + 66, *scales = b + 74;
        for (int ib32 = 0; ib32 < 8; ++ib32) {
            const float db0 = d * (0.5f + (float)(scales[ib32] & 0xf)) * 0.25f;
            const float db1 = d * (0.5f + (float)(scales[ib32] >> 4)) * 0.25f;
            for (int l = 0; l < 4; ++l) {
                const uint32_t idx = qs[4 * ib32 + l] | (((uint32_t)qh[ib32] << (8 - 2 * l)) & 0x300u);
                const uint8_t *grid = (const uint8_t *)&iq2s_grid[idx];
                const uint32_t signs = qs[32 + 4 * ib32 + l];
                const float db = l < 2 ? db0 : db1;
                for (int j = 0; j < 8; ++j) *y++ = db * (float)grid[j] * sgn(signs, j);
            }
        }
    }
}

/* IQ3_XXS, 98-byte blocks {fp16 d; qs[64]; u32 scales_and_signs[8]}: gpu_dequant.py:224-265 */
void oracle_dequant_iq3_xxs(const uint8_t *x, float *y, int64_t k) {
    for (int64_t i = 0; i < k / 256; i++) {
        const uint8_t *b = x + i * 98;
        const float d = oracle_fp16_to_fp32(rd16(b));
        const uint8_t *qs = b + 2;
        for (int ib32 = 0; ib32 < 8; ++ib32) {
            const uint32_t aux = rd32(qs + 64 + 4 * ib32);
            const float db = d * (0.5f + (float)(aux >> 28)) * 0.5f;
            for (int l = 0; l < 4; ++l) {
                const uint32_t signs = parity_signs((aux >> (7 * l)) & 127u);
                const uint8_t *g1 = (const uint8_t *)&iq3xxs_grid[qs[8 * ib32 + 2 * l]];
                const uint8_t *g2 = (const uint8_t *)&iq3xxs_grid[qs[8 * ib32 + 2 * l + 1]];
                for (int j = 0; j < 4; ++j) y[j] = db * (float)g1[j] * sgn(signs, j);
                for (int j = 0; j < 4; ++j) y[j + 4] = db * (float)g2[j] * sgn(signs, j + 4);
                y += 8;
            }
        }
    }
}

/* IQ3_S, 110-byte blocks {fp16 d; qs[64]; qh[8]; signs[32]; scales[4]}: gpu_dequant.py:272-349 */
void oracle_dequant_iq3_s(const uint8_t *x, float *y, int64_t k) {
    for (int64_t i = 0; i < k / 256; i++) {
        const uint8_t *b = x + i * 110;
        const float d = oracle_fp16_to_fp32(rd16(b));
        const uint8_t *qs = b + 2, *qh = b + 66, *sg = b + 74, *scales = b + 106;
        for (int ib32 = 0; ib32 < 8; ++ib32) {
            const uint32_t s4 = ib32 & 1 ? (uint32_t)scales[ib32 / 2] >> 4 : scales[ib32 / 2] & 0xfu;
            const float db = d * (float)(1 + 2 * (int)s4);
            const uint32_t h = qh[ib32];
            for (int l = 0; l < 4; ++l) {
                const uint8_t *g1 = (const uint8_t *)&iq3s_grid[qs[8 * ib32 + 2 * l] | ((h << (8 - 2 * l)) & 256u)];
                const uint8_t *g2 = (const uint8_t *)&iq3s_grid[qs[8 * ib32 + 2 * l + 1] | ((h << (7 - 2 * l)) & 256u)];
                const uint32_t signs = sg[4 * ib32 + l];
                for (int j = 0; j < 4; ++j) y[j] = db * (float)g1[j] * sgn(signs, j);
                for (int j = 0; j < 4; ++j) y[j + 4] = db * (float)g2[j] * sgn(signs, j + 4);
                y += 8;
            }
        }
    }
}

#define IQ1S_DELTA 0.125f

/* IQ1_S, 50-byte blocks {fp16 d; qs[32]; u16 qh[8]}: gpu_dequant.py:356-383 */
void oracle_dequant_iq1_s(const uint8_t *x, float *y, int64_t k) {
    for (int64_t i = 0; i < k / 256; i++) {
        const uint8_t *b = x + i * 50;
        const float d = oracle_fp16_to_fp32(rd16(b));
        for (int ib = 0; ib < 8; ++ib) {
            const uint32_t qh = rd16(b + 34 + 2 * ib);
            const float dl = d * (float)(2 * ((qh >> 12) & 7) + 1);
            const float delta = qh & 0x8000 ? -IQ1S_DELTA : IQ1S_DELTA;
            for (int l = 0; l < 4; ++l) {
                const int8_t *grid = (const int8_t *)&iq1s_grid[b[2 + 4 * ib + l] | (((qh >> (3 * l)) & 7) << 8)];
                for (int j = 0; j < 8; ++j) *y++ = dl * ((float)grid[j] + delta);
            }
        }
    }
}

/* IQ1_M, 56-byte blocks {qs[32]; qh[16]; u16 scales[4]} with the fp16 super-block
 * scale spread over the top nibbles of the four scale words: gpu_dequant.py:390-450 */
void oracle_dequant_iq1_m(const uint8_t *x, float *y, int64_t k) {
    for (int64_t i = 0; i < k / 256; i++) {
        const uint8_t *b = x + i * 56;
        const uint8_t *qs = b, *qh = b + 32;
        uint32_t sc[4];
        for (int t = 0; t < 4; ++t) sc[t] = rd16(b + 48 + 2 * t);
        const uint16_t dh = (uint16_t)((sc[0] >> 12) | ((sc[1] >> 8) & 0x00f0u) | ((sc[2] >> 4) & 0x0f00u) | (sc[3] & 0xf000u));
        const float d = oracle_fp16_to_fp32(dh);
        for (int ib = 0; ib < 8; ++ib) {
            const uint32_t s = sc[ib / 2];
            const float dl1 = d * (float)(2 * ((s >> (6 * (ib % 2) + 0)) & 7) + 1);
            const float dl2 = d * (float)(2 * ((s >> (6 * (ib % 2) + 3)) & 7) + 1);
            const uint32_t h0 = qh[2 * ib], h1 = qh[2 * ib + 1];
            const uint32_t idx[4] = {qs[4 * ib + 0] | ((h0 << 8) & 0x700u), qs[4 * ib + 1] | ((h0 << 4) & 0x700u),
                                     qs[4 * ib + 2] | ((h1 << 8) & 0x700u), qs[4 * ib + 3] | ((h1 << 4) & 0x700u)};
            const float delta[4] = {h0 & 0x08 ? -IQ1S_DELTA : IQ1S_DELTA, h0 & 0x80 ? -IQ1S_DELTA : IQ1S_DELTA,
                                    h1 & 0x08 ? -IQ1S_DELTA : IQ1S_DELTA, h1 & 0x80 ? -IQ1S_DELTA : IQ1S_DELTA};
            for (int l = 0; l < 4; ++l) {
                const int8_t *grid = (const int8_t *)&iq1s_grid[idx[l]];
                const float dl = l < 2 ? dl1 : dl2;
                for (int j = 0; j < 8; ++j) *y++ = dl * ((float)grid[j] + delta[l]);
            }
        }
    }
}

/* IQ4_XS, 136-byte blocks {fp16 d; u16 scales_h; scales_l[4]; qs[128]}: gpu_dequant.py:457-519 */
void oracle_dequant_iq4_xs(const uint8_t *x, float *y, int64_t k) {
    for (int64_t i = 0; i < k / 256; i++) {
        const uint8_t *b = x + i * 136;
        const float d = oracle_fp16_to_fp32(rd16(b));
        const uint32_t sh = rd16(b + 2);
        const uint8_t *sl = b + 4, *qs = b + 8;
        for (int ib = 0; ib < 8; ++ib) {
            const int ls = (int)(((sl[ib / 2] >> (4 * (ib % 2))) & 0xf) | (((sh >> (2 * ib)) & 3) << 4));
            const float dl = d * ((float)ls - 32.0f);
            for (int j = 0; j < 16; ++j) {
                y[j] = dl * (float)iq4nl_values[qs[16 * ib + j] & 0xf];
                y[j + 16] = dl * (float)iq4nl_values[qs[16 * ib + j] >> 4];
            }
            y += 32;
        }
    }
}

/* Dispatch by ggml type id (8 Q8_0, 10 Q2_K, 11 Q3_K, 12 Q4_K, 13 Q5_K, 14 Q6_K,
 * 16 IQ2_XXS, 17 IQ2_XS, 18 IQ3_XXS, 19 IQ1_S, 21 IQ3_S, 22 IQ2_S, 23 IQ4_XS, 29 IQ1_M).
 * Returns 0 on success, -1 for an unknown type. */
int oracle_dequant(int ggml_type, const uint8_t *x, float *y, int64_t k) {
    switch (ggml_type) {
    case 8: oracle_dequant_q8_0(x, y, k); return 0;
    case 10: oracle_dequant_q2_K(x, y, k); return 0;
    case 11: oracle_dequant_q3_K(x, y, k); return 0;
    case 12: oracle_dequant_q4_K(x, y, k); return 0;
    case 13: oracle_dequant_q5_K(x, y, k); return 0;
    case 14: oracle_dequant_q6_K(x, y, k); return 0;
    case 16: oracle_dequant_iq2_xxs(x, y, k); return 0;
    case 17: oracle_dequant_iq2_xs(x, y, k); return 0;
    case 18: oracle_dequant_iq3_xxs(x, y, k); return 0;
    case 19: oracle_dequant_iq1_s(x, y, k); return 0;
    case 21: oracle_dequant_iq3_s(x, y, k); return 0;
    case 22: oracle_dequant_iq2_s(x, y, k); return 0;
    case 23: oracle_dequant_iq4_xs(x, y, k); return 0;
    case 29: oracle_dequant_iq1_m(x, y, k); return 0;
    default: return -1;
    }
}

/* Multi-threaded driver for the CPU baseline: blocks are independent, so the
 * tensor is split into contiguous runs of 256-weight groups. */
#ifdef _OPENMP
#include <omp.h>
#endif
int oracle_dequant_parallel(int ggml_type, const uint8_t *x, float *y, int64_t k, int nthreads) {
    int64_t bb;
    switch (ggml_type) {
    case 8: bb = 272; break; /* eight 34-byte Q8_0 blocks per 256 weights */
    case 10: bb = 84; break;
    case 11: bb = 110; break;
    case 12: bb = 144; break;
    case 13: bb = 176; break;
    case 14: bb = 210; break;
    case 16: bb = 66; break;
    case 17: bb = 74; break;
    case 18: bb = 98; break;
    case 19: bb = 50; break;
    case 21: bb = 110; break;
    case 22: bb = 82; break;
    case 23: bb = 136; break;
    case 29: bb = 56; break;
    default: return -1;
    }
    const int64_t ngroups = k / 256;
    const int64_t per = 1024; /* groups per task */
    const int64_t ntasks = (ngroups + per - 1) / per;
    int rc = 0;
#ifdef _OPENMP
    if (nthreads > 0) omp_set_num_threads(nthreads);
#pragma omp parallel for schedule(static)
#endif
    for (int64_t t = 0; t < ntasks; t++) {
        const int64_t g0 = t * per;
        const int64_t g1 = g0 + per < ngroups ? g0 + per : ngroups;
        if (oracle_dequant(ggml_type, x + g0 * bb, y + g0 * 256, (g1 - g0) * 256) != 0) rc = -1;
    }
    return rc;
}
