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

/* Dispatch by ggml type id (8 Q8_0, 10 Q2_K, 11 Q3_K, 12 Q4_K, 13 Q5_K, 14 Q6_K).
 * Returns 0 on success, -1 for an unknown type. */
int oracle_dequant(int ggml_type, const uint8_t *x, float *y, int64_t k) {
    switch (ggml_type) {
    case 8: oracle_dequant_q8_0(x, y, k); return 0;
    case 10: oracle_dequant_q2_K(x, y, k); return 0;
    case 11: oracle_dequant_q3_K(x, y, k); return 0;
    case 12: oracle_dequant_q4_K(x, y, k); return 0;
    case 13: oracle_dequant_q5_K(x, y, k); return 0;
    case 14: oracle_dequant_q6_K(x, y, k); return 0;
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
