/*
 * TEST-ONLY STAND-IN FOR libggml-base.  This is NOT llama.cpp and its bytes are
 * NOT llama.cpp's quantizer output.
 *
 * It exists so that the CPU tests can drive voodoo_quant/ggml.py's ctypes
 * bridge (library discovery through $VOODOO_GGML_LIB, argument types, the
 * all-ones importance-matrix default, the returned-size check, the decode
 * call) and the gated layers' "ggml" candidate branch on a machine without
 * llama.cpp.  It exports the part of ggml's C ABI the bridge binds:
 *
 *   void   ggml_quantize_init(enum ggml_type type);
 *   size_t quantize_q8_0(const float *src, void *dst, int64_t nrows, int64_t n_per_row, const float *imatrix);
 *   size_t quantize_q4_K(...same...);
 *   void   dequantize_row_<t>(const void *x, float *y, int64_t k);   for the 14 decoded formats
 *
 * quantize_q8_0 is ggml's round-to-nearest Q8_0 (amax / 127 scale, roundf
 * codes, fp16 scale rounded to nearest even), which is also what
 * voodoo_quant/rtn.py writes.  quantize_q4_K is the same min/scale
 * round-to-nearest as rtn.py's Q4_K (not llama.cpp's search).  The decoders
 * are the oracle's (oracle/dequant_ref.c, linked into the same library).
 *
 * Probe functions (stand_in_*) report what the last call received, so a test
 * can check the arguments the bridge passed.
 */
#include <math.h>
#include <stddef.h>
#include <stdint.h>
#include <string.h>

/* the oracle's decoders (oracle/dequant_ref.c) */
void oracle_dequant_q8_0(const uint8_t *x, float *y, int64_t k);
void oracle_dequant_q2_K(const uint8_t *x, float *y, int64_t k);
void oracle_dequant_q3_K(const uint8_t *x, float *y, int64_t k);
void oracle_dequant_q4_K(const uint8_t *x, float *y, int64_t k);
void oracle_dequant_q5_K(const uint8_t *x, float *y, int64_t k);
void oracle_dequant_q6_K(const uint8_t *x, float *y, int64_t k);
void oracle_dequant_iq2_xxs(const uint8_t *x, float *y, int64_t k);
void oracle_dequant_iq2_xs(const uint8_t *x, float *y, int64_t k);
void oracle_dequant_iq2_s(const uint8_t *x, float *y, int64_t k);
void oracle_dequant_iq3_xxs(const uint8_t *x, float *y, int64_t k);
void oracle_dequant_iq3_s(const uint8_t *x, float *y, int64_t k);
void oracle_dequant_iq1_s(const uint8_t *x, float *y, int64_t k);
void oracle_dequant_iq1_m(const uint8_t *x, float *y, int64_t k);
void oracle_dequant_iq4_xs(const uint8_t *x, float *y, int64_t k);

/* ------------------------------------------------------------ probes */
static int g_init_type = -1;
static int g_init_calls = 0;
static int64_t g_rows = -1, g_cols = -1;
static int g_imatrix_null = -1;
static double g_imatrix_sum = 0.0;
static int64_t g_size_skew = 0;

int stand_in_init_type(void) { return g_init_type; }
int stand_in_init_calls(void) { return g_init_calls; }
int64_t stand_in_rows(void) { return g_rows; }
int64_t stand_in_cols(void) { return g_cols; }
int stand_in_imatrix_null(void) { return g_imatrix_null; }
double stand_in_imatrix_sum(void) { return g_imatrix_sum; }
/* a non-zero skew makes every quantize_* report that many bytes more than it wrote */
void stand_in_set_size_skew(int64_t skew) { g_size_skew = skew; }
void stand_in_reset(void) {
    g_init_type = -1;
    g_init_calls = 0;
    g_rows = g_cols = -1;
    g_imatrix_null = -1;
    g_imatrix_sum = 0.0;
    g_size_skew = 0;
}

static void record(int64_t nrows, int64_t n_per_row, const float *imatrix) {
    g_rows = nrows;
    g_cols = n_per_row;
    g_imatrix_null = imatrix == NULL;
    g_imatrix_sum = 0.0;
    if (imatrix)
        for (int64_t i = 0; i < n_per_row; i++) g_imatrix_sum += imatrix[i];
}

void ggml_quantize_init(int type) {
    g_init_type = type;
    g_init_calls++;
}

/* ------------------------------------------------------------ helpers */
/* fp32 -> fp16, round to nearest even (what F16C's _cvtss_sh(x, 0) gives) */
static uint16_t to_half(float f) {
    uint32_t x;
    memcpy(&x, &f, 4);
    const uint16_t sign = (uint16_t)((x >> 16) & 0x8000u);
    const int exp = (int)((x >> 23) & 0xff);
    uint32_t mant = x & 0x7fffffu;
    if (exp == 0xff) return sign | 0x7c00u | (mant ? 0x200u : 0u);
    const int e = exp - 127 + 15;
    if (e >= 31) return sign | 0x7c00u;
    if (e <= 0) {
        if (e < -11) return sign;
        mant |= 0x800000u;
        const int shift = 14 - e;
        const uint32_t half = 1u << (shift - 1);
        uint32_t r = mant >> shift;
        const uint32_t rem = mant & ((1u << shift) - 1u);
        if (rem > half || (rem == half && (r & 1u))) r++;
        return sign | (uint16_t)r;
    }
    uint32_t r = ((uint32_t)e << 10) | (mant >> 13);
    const uint32_t rem = mant & 0x1fffu;
    if (rem > 0x1000u || (rem == 0x1000u && (r & 1u))) r++;
    return sign | (uint16_t)r;
}

static float from_half(uint16_t h) {
    const uint32_t sign = (uint32_t)(h & 0x8000u) << 16;
    int exp = (h >> 10) & 0x1f;
    uint32_t mant = h & 0x3ffu, x;
    if (exp == 0x1f) {
        x = sign | 0x7f800000u | (mant << 13);
    } else if (exp == 0) {
        if (mant == 0) {
            x = sign;
        } else {
            exp = 1;
            while (!(mant & 0x400u)) {
                mant <<= 1;
                exp--;
            }
            x = sign | ((uint32_t)(exp + 112) << 23) | ((mant & 0x3ffu) << 13);
        }
    } else {
        x = sign | ((uint32_t)(exp + 112) << 23) | (mant << 13);
    }
    float f;
    memcpy(&f, &x, 4);
    return f;
}

static void put_half(uint8_t *p, uint16_t h) {
    p[0] = (uint8_t)(h & 0xff);
    p[1] = (uint8_t)(h >> 8);
}

static float div0(float a, float b) { return b != 0.0f ? a / b : 0.0f; }

static int clampi(float v, int lo, int hi) { return v < (float)lo ? lo : v > (float)hi ? hi : (int)v; }

/* ------------------------------------------------------------ Q8_0 */
size_t quantize_q8_0(const float *src, void *dst, int64_t nrows, int64_t n_per_row, const float *imatrix) {
    record(nrows, n_per_row, imatrix);
    if (n_per_row % 32) return 0;
    uint8_t *out = (uint8_t *)dst;
    const int64_t nblocks = nrows * (n_per_row / 32);
    for (int64_t b = 0; b < nblocks; b++) {
        const float *x = src + 32 * b;
        float amax = 0.0f;
        for (int j = 0; j < 32; j++) amax = fabsf(x[j]) > amax ? fabsf(x[j]) : amax;
        const float d = amax / 127.0f;
        const float id = d != 0.0f ? 1.0f / d : 0.0f;
        uint8_t *o = out + 34 * b;
        put_half(o, to_half(d));
        for (int j = 0; j < 32; j++) o[2 + j] = (uint8_t)(int8_t)roundf(x[j] * id);
    }
    return (size_t)(nblocks * 34 + g_size_skew);
}

/* ------------------------------------------------------------ Q4_K */
/* Per 256-weight super-block: eight 32-weight sub-blocks, each with a scale
 * (max - min) / 15 and a min -min (min clamped to at most 0); the super-block
 * scales d = max scale / 63 and dmin = max min / 63 go to fp16, the 6-bit
 * sub-block scales and mins are round(scale / d) and round(min / dmin), and
 * each code is round((x + dmin m) / (d sc)) clamped to 0..15. */
size_t quantize_q4_K(const float *src, void *dst, int64_t nrows, int64_t n_per_row, const float *imatrix) {
    record(nrows, n_per_row, imatrix);
    if (n_per_row % 256) return 0;
    uint8_t *out = (uint8_t *)dst;
    const int64_t nblocks = nrows * (n_per_row / 256);
    for (int64_t b = 0; b < nblocks; b++) {
        const float *x = src + 256 * b;
        uint8_t *o = out + 144 * b;
        float scale[8], mn[8], smax = 0.0f, mmax = 0.0f;
        for (int s = 0; s < 8; s++) {
            float lo = x[32 * s], hi = x[32 * s];
            for (int j = 1; j < 32; j++) {
                lo = x[32 * s + j] < lo ? x[32 * s + j] : lo;
                hi = x[32 * s + j] > hi ? x[32 * s + j] : hi;
            }
            lo = lo < 0.0f ? lo : 0.0f;
            scale[s] = (hi - lo) / 15.0f;
            mn[s] = -lo;
            smax = scale[s] > smax ? scale[s] : smax;
            mmax = mn[s] > mmax ? mn[s] : mmax;
        }
        const uint16_t dh = to_half(smax / 63.0f), mh = to_half(mmax / 63.0f);
        const float df = from_half(dh), mf = from_half(mh);
        int sc[8], m[8];
        for (int s = 0; s < 8; s++) {
            sc[s] = clampi(roundf(div0(scale[s], df)), 0, 63);
            m[s] = clampi(roundf(div0(mn[s], mf)), 0, 63);
        }
        put_half(o, dh);
        put_half(o + 2, mh);
        for (int j = 0; j < 4; j++) {
            o[4 + j] = (uint8_t)(sc[j] | ((sc[j + 4] >> 4) << 6));
            o[8 + j] = (uint8_t)(m[j] | ((m[j + 4] >> 4) << 6));
            o[12 + j] = (uint8_t)((sc[j + 4] & 0xf) | ((m[j + 4] & 0xf) << 4));
        }
        memset(o + 16, 0, 128);
        for (int i = 0; i < 256; i++) {
            const int s = i / 32;
            const float dl = df * (float)sc[s], ml = mf * (float)m[s];
            const int q = clampi(roundf(div0(x[i] + ml, dl)), 0, 15);
            o[16 + 32 * (i / 64) + (i % 32)] |= (uint8_t)(q << (4 * ((i % 64) / 32)));
        }
    }
    return (size_t)(nblocks * 144 + g_size_skew);
}

/* ------------------------------------------------------------ decoders */
#define ROW(name, fn) \
    void dequantize_row_##name(const void *x, float *y, int64_t k) { fn((const uint8_t *)x, y, k); }
ROW(q8_0, oracle_dequant_q8_0)
ROW(q2_K, oracle_dequant_q2_K)
ROW(q3_K, oracle_dequant_q3_K)
ROW(q4_K, oracle_dequant_q4_K)
ROW(q5_K, oracle_dequant_q5_K)
ROW(q6_K, oracle_dequant_q6_K)
ROW(iq2_xxs, oracle_dequant_iq2_xxs)
ROW(iq2_xs, oracle_dequant_iq2_xs)
ROW(iq2_s, oracle_dequant_iq2_s)
ROW(iq3_xxs, oracle_dequant_iq3_xxs)
ROW(iq3_s, oracle_dequant_iq3_s)
ROW(iq1_s, oracle_dequant_iq1_s)
ROW(iq1_m, oracle_dequant_iq1_m)
ROW(iq4_xs, oracle_dequant_iq4_xs)
