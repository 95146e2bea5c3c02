// Causal self-attention forward of the decoder step (torch's
// scaled_dot_product_attention with is_causal=True and equal query/key
// lengths: key j is visible to query i when j <= i), head dim 64, bf16 q/k/v
// and output, fp32 scores and softmax, on gfx950 MFMA (v_mfma_f32_32x32x16_bf16).
//
// One workgroup takes 128 queries of one (batch, head): four waves of 32
// queries.  Keys stream through LDS in tiles of 64 (K and V, 8 KiB each,
// double-buffered, copied by direct-to-LDS buffer loads issued while the tile
// before is computed).  Per tile a wave forms S^T = K Q^T (keys x
// queries) so each lane holds 32 scores of one query: the row maximum is a
// reduction within the lane plus one exchange between the two lane halves,
// and the probabilities P^T are already in the register layout of the B
// operand of O^T = V^T P^T (the key order inside each 16-key MFMA step is
// permuted the same way on both operands).  V^T fragments come from LDS by
// ds_read_b64_tr_b16.  Online softmax in base 2 (scores scaled by
// scale * log2 e; the running maximum moves only when a tile's exceeds it by
// more than 2^8, so most tiles skip rescaling O), P rounded to bf16 for the
// second product, O accumulated in fp32 and divided by the row sum once at
// the end.  The log-sum-exp per query
// (natural log, [B][H][S] fp32) is what torch's memory-efficient attention
// backward reads, so the step pairs this forward with that backward.
//
// MFMA 32x32x16 operand/result layout (per wave of 64 lanes):
//   A: lane l holds A[i = l%32][k = 8*(l/32) .. +7]
//   B: lane l holds B[k = 8*(l/32) .. +7][j = l%32]
//   D: register r of lane l is D[i = 8*(r/4) + 4*(l/32) + r%4][j = l%32]
#include "vq_internal.h"

namespace vq {

namespace {

typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef short v4i16 __attribute__((ext_vector_type(4)));
typedef short v8i16 __attribute__((ext_vector_type(8)));
typedef __attribute__((address_space(3))) v4i16 lds_v4i16;

constexpr int kHead = 64;                    // head dim
constexpr int kQTile = 128;                  // queries per workgroup
constexpr int kKTile = 64;                   // keys per LDS tile
constexpr int kRowBytes = kHead * 2;         // 128 bytes per key row
constexpr int kMatBytes = kKTile * kRowBytes;  // 8 KiB: one K or V tile
constexpr float kLn2 = 0.693147180559945309f;

// Byte offset of (key row, 16-byte chunk) in a tile: chunks are XOR-swizzled
// by swz(row) = 4 ((row / 2) % 2) + (row / 4) % 4, so the 16 rows of one
// 16-byte fragment read pass (same chunk) and the 4 rows x 4 chunks of one
// transposed 8-byte read pass each cover 256 distinct bytes of the 64 banks
// (a row is 128 bytes: rows of one parity share banks, and swz takes 8
// distinct values over the 8 rows of each parity in 16 consecutive rows).
__device__ __forceinline__ int swz(int row) { return (((row >> 1) & 1) << 2) | ((row >> 2) & 3); }
__device__ __forceinline__ int tile_off(int row, int chunk) { return row * kRowBytes + ((chunk ^ swz(row)) << 4); }

typedef __attribute__((address_space(3))) void lds_void_t;
constexpr uint32_t kRange = 0x7ffffff0u;  // buffer descriptor size in bytes
constexpr uint32_t kOOB = 0x80000000u;    // an offset past kRange: the load returns zeros
constexpr float kSlack = 8.0f;            // log2 units the running maximum may lag the true one

__device__ __forceinline__ __amdgpu_buffer_rsrc_t tile_rsrc(const bf16_t* base) {
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<bf16_t*>(base), (short)0, (int)kRange, 0x00020000);
}

// The register's values in lanes l % 32 and 32 + l % 32, one in each output,
// in every lane l (v_permlane32_swap_b32 of the register with itself: a VALU
// exchange of the two 32-lane halves, no LDS round trip).  lo + hi and
// max(lo, hi) are then the same in both halves.
__device__ __forceinline__ void halves(float x, float& lo, float& hi) {
    const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
    lo = __uint_as_float(r[0]);
    hi = __uint_as_float(r[1]);
}

__device__ __forceinline__ float max3f(float a, float b, float c) {
    return __builtin_elementwise_maximum(__builtin_elementwise_maximum(a, b), c);
}

// IEEE maximum (NaN-propagating: v_maximum3_f32, which needs no
// canonicalisation of the MFMA results as fmaxf would) of 32 values as a
// tree of three-input maxima: 16 instructions instead of 24 pairwise ones
__device__ __forceinline__ float max_of_32(const f32x16& a, const f32x16& b) {
    float m[11];
#pragma unroll
    for (int i = 0; i < 5; ++i) {
        m[2 * i] = max3f(a[3 * i], a[3 * i + 1], a[3 * i + 2]);
        m[2 * i + 1] = max3f(b[3 * i], b[3 * i + 1], b[3 * i + 2]);
    }
    m[10] = __builtin_elementwise_maximum(a[15], b[15]);
    const float n0 = max3f(m[0], m[1], m[2]), n1 = max3f(m[3], m[4], m[5]), n2 = max3f(m[6], m[7], m[8]);
    return max3f(n0, n1, max3f(n2, m[9], m[10]));
}

__global__ __launch_bounds__(256) void attn_fwd_kernel(const bf16_t* __restrict__ q, const bf16_t* __restrict__ k,
                                                       const bf16_t* __restrict__ v, bf16_t* __restrict__ o,
                                                       float* __restrict__ lse, int S, int H, int Hk, int BH, int nqt,
                                                       int64_t qsb, int64_t qss, int64_t qsh, int64_t ksb, int64_t kss,
                                                       int64_t ksh, int64_t vsb, int64_t vss, int64_t vsh, int64_t osb,
                                                       int64_t oss, int64_t osh, float c2) {
    __shared__ __attribute__((aligned(16))) uint8_t smem[2][2 * kMatBytes];
    // heaviest query tiles first; a (batch, head)'s tiles share bid % 8, so
    // when BH % 8 == 0 they run on one XCD and share its L2 for K and V
    const int bid = blockIdx.x;
    const int qt = nqt - 1 - bid / BH;
    const int bh = bid - (bid / BH) * BH;
    const int b = bh / H, h = bh - (bh / H) * H;
    const int hk = h / (H / Hk);
    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int g = lane >> 5, col = lane & 31;
    const int q0 = qt * kQTile;
    const int qw0 = q0 + 32 * wave;
    const int qrow = qw0 + col;

    // Q^T as the B operand: lane holds Q[qrow][16 c + 8 g .. +7]; rows past S
    // read row S - 1 (their results are not stored)
    bf16x8_t qf[4];
    {
        const bf16_t* qp = q + (int64_t)b * qsb + (int64_t)min(qrow, S - 1) * qss + (int64_t)h * qsh + 8 * g;
#pragma unroll
        for (int c = 0; c < 4; ++c) qf[c] = *reinterpret_cast<const bf16x8_t*>(qp + 16 * c);
    }

    // K and V tiles go global -> LDS by direct-to-LDS buffer loads: lane l of
    // wave w's instruction i writes LDS slot s = 64 (4 i + w) + l of the stage
    // (16 bytes each; slots 0-511 K, 512-1023 V), which is tile_off(row, c) for
    // row = (s % 512) / 8 and chunk c = (s % 8) ^ swz(row), so the lane loads
    // that chunk.  Keys past S read zeros.
    const bf16_t* kb0 = k + (int64_t)b * ksb + (int64_t)hk * ksh;
    const bf16_t* vb0 = v + (int64_t)b * vsb + (int64_t)hk * vsh;
    uint32_t voff[4];
    int vrow[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const int w = ((4 * i + wave) * 64 + lane) & 511;
        const int row = w >> 3, c = (w & 7) ^ swz(row);
        vrow[i] = row;
        voff[i] = (uint32_t)(row * (i < 2 ? kss : vss) * 2 + 16 * c);
    }
    auto issue = [&](int j, uint8_t* dst) __attribute__((always_inline)) {
        const __amdgpu_buffer_rsrc_t rk = tile_rsrc(kb0 + (int64_t)j * kKTile * kss);
        const __amdgpu_buffer_rsrc_t rv = tile_rsrc(vb0 + (int64_t)j * kKTile * vss);
        const int lim = S - j * kKTile;
#pragma unroll
        for (int i = 0; i < 4; ++i)
            __builtin_amdgcn_raw_ptr_buffer_load_lds(i < 2 ? rk : rv, (lds_void_t*)(dst + (4 * i + wave) * 1024),
                                                     16, vrow[i] < lim ? voff[i] : kOOB, 0, 0, 0);
    };

    const int S_tiles = (S + kKTile - 1) / kKTile;
    const int nt = min(S_tiles, (q0 + kQTile + kKTile - 1) / kKTile);
    f32x16 oacc[2];
#pragma unroll
    for (int db = 0; db < 2; ++db)
#pragma unroll
        for (int r = 0; r < 16; ++r) oacc[db][r] = 0.0f;
    float m_run = -INFINITY, l_run = 0.0f;

    issue(0, smem[0]);
    asm volatile("s_waitcnt vmcnt(0)\n\ts_barrier" ::: "memory");
    // tile j: read this tile's K and V fragments, then copy tile j + 1 into
    // the other stage (whose last readers passed the last barrier), then the
    // softmax and the value product, then the barrier.  The copies come after
    // the tile's last LDS read because the compiler cannot tell the stages
    // apart and would make every later read wait for them.
    for (int j = 0; j < nt; ++j) {
        const uint8_t* ks = smem[j & 1];
        const uint8_t* vs = ks + kMatBytes;
        const int k0 = j * kKTile;
        const bool active = k0 <= qw0 + 31;  // some key of the tile is visible to some query of the wave
        f32x16 s[2];
        bf16x8_t vf[4][2];
        if (active) {
#pragma unroll
            for (int kb = 0; kb < 2; ++kb) {
#pragma unroll
                for (int r = 0; r < 16; ++r) s[kb][r] = 0.0f;
                const int row = 32 * kb + col;
#pragma unroll
                for (int c = 0; c < 4; ++c) {
                    const bf16x8_t a = *reinterpret_cast<const bf16x8_t*>(ks + tile_off(row, 2 * c + g));
                    s[kb] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, qf[c], s[kb], 0, 0, 0);
                }
            }
            // V^T fragments of the value product: step t takes keys
            // 16 t + 4 g + {0..3} and 16 t + 8 + 4 g + {0..3} in lane half g.
            // ds_read_b64_tr_b16: output lane l element e = element l%4 of the
            // 8 bytes addressed by lane 16 (l/16) + 4 e + (l%16)/4, so lane l
            // receives V[key0 + e][d0 + l%16] when the lane at index u of its
            // 16-lane group G addresses V[key0 + u/4][d0 + 4 (u%4)]
            const int G = lane >> 4, u = lane & 15;
#pragma unroll
            for (int t = 0; t < 4; ++t) {
                const int key = 16 * t + 4 * (G >> 1) + (u >> 2);
#pragma unroll
                for (int db = 0; db < 2; ++db) {
                    const int d = 32 * db + 16 * (G & 1) + 4 * (u & 3);
                    const uint8_t* lo = vs + tile_off(key, d >> 3) + ((d & 7) << 1);
                    const uint8_t* hi = vs + tile_off(key + 8, d >> 3) + ((d & 7) << 1);
                    const v4i16 vlo = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_v4i16*)(lo));
                    const v4i16 vhi = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_v4i16*)(hi));
                    vf[t][db] = __builtin_bit_cast(bf16x8_t, __builtin_shufflevector(vlo, vhi, 0, 1, 2, 3, 4, 5, 6, 7));
                }
            }
        }
        if (j + 1 < nt) issue(j + 1, smem[(j + 1) & 1]);
        if (active) {
            if (k0 + kKTile - 1 > qw0) {  // the causal edge crosses the wave's queries
#pragma unroll
                for (int kb = 0; kb < 2; ++kb)
#pragma unroll
                    for (int r = 0; r < 16; ++r) {
                        const int key = k0 + 32 * kb + 8 * (r >> 2) + 4 * g + (r & 3);
                        if (key > qrow) s[kb][r] = -INFINITY;
                    }
            }
            float mx = max_of_32(s[0], s[1]);
            float mlo, mhi;
            halves(mx, mlo, mhi);
            mx = __builtin_elementwise_maximum(mlo, mhi) * c2;
            // the running maximum moves only when the tile's exceeds it by more
            // than kSlack, so most tiles skip the rescale (exponents stay <= 2^8)
            if (__builtin_amdgcn_ballot_w64(mx > m_run + kSlack)) {
                const float m_new = fmaxf(m_run, mx);
                const float alpha = __builtin_amdgcn_exp2f(m_run - m_new);
                m_run = m_new;
                l_run *= alpha;
#pragma unroll
                for (int db = 0; db < 2; ++db)
#pragma unroll
                    for (int r = 0; r < 16; ++r) oacc[db][r] *= alpha;
            }
            float sum = 0.0f;
#pragma unroll
            for (int kb = 0; kb < 2; ++kb)
#pragma unroll
                for (int r = 0; r < 16; ++r) {
                    const float p = __builtin_amdgcn_exp2f(fmaf(s[kb][r], c2, -m_run));
                    s[kb][r] = p;
                    sum += p;
                }
            l_run += sum;
            // O^T += V^T P^T over the tile's 64 keys, 16 per MFMA
#pragma unroll
            for (int t = 0; t < 4; ++t) {
                const f32x16& sp = s[t >> 1];
                const int r0 = 8 * (t & 1);
                typedef uint32_t u32x4v __attribute__((ext_vector_type(4)));
                const u32x4v pw = {pk_bf16(sp[r0], sp[r0 + 1]), pk_bf16(sp[r0 + 2], sp[r0 + 3]),
                                   pk_bf16(sp[r0 + 4], sp[r0 + 5]), pk_bf16(sp[r0 + 6], sp[r0 + 7])};
                const bf16x8_t pf = __builtin_bit_cast(bf16x8_t, pw);
#pragma unroll
                for (int db = 0; db < 2; ++db)
                    oacc[db] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(vf[t][db], pf, oacc[db], 0, 0, 0);
            }
        }
        // this wave's copies of tile j + 1 have landed and every wave is past
        // its reads of tile j
        asm volatile("s_waitcnt vmcnt(0) lgkmcnt(0)\n\ts_barrier" ::: "memory");
    }

    float llo, lhi;
    halves(l_run, llo, lhi);
    const float lt = llo + lhi;
    if (qrow < S) {
        const float inv = 1.0f / lt;
        bf16_t* op = o + (int64_t)b * osb + (int64_t)qrow * oss + (int64_t)h * osh;
#pragma unroll
        for (int db = 0; db < 2; ++db)
#pragma unroll
            for (int a = 0; a < 4; ++a) {
                const int d = 32 * db + 8 * a + 4 * g;
                uint2 w;
                w.x = pk_bf16(oacc[db][4 * a] * inv, oacc[db][4 * a + 1] * inv);
                w.y = pk_bf16(oacc[db][4 * a + 2] * inv, oacc[db][4 * a + 3] * inv);
                *reinterpret_cast<uint2*>(op + d) = w;
            }
        if (lse && g == 0) lse[(int64_t)bh * S + qrow] = (m_run + __log2f(lt)) * kLn2;
    }
}

// ---------------------------------------------------------------- backward
// Two kernels, no atomics, deterministic (the sums run in a fixed order):
//   attn_bwd_dq_kernel: per 128-query tile (4 waves x 32 queries), over the
//     key tiles up to the diagonal: S^T = K Q^T, dP^T = V dO^T, P = exp(S
//     scale - lse), dS = P (dP - D), dQ^T += K^T dS^T; D = rowsum(dO o O) is
//     formed from the wave's own rows first; lse log2 e and -D per query go
//     to the workspace the second kernel reads.  dP accumulates onto -D, so
//     the MFMAs give dP - D with no subtraction.
//   attn_bwd_dkdv_kernel: per 128-key block (4 waves x 32 keys), over the
//     query tiles from the diagonal on: S = Q K^T, dP = dO V^T, P, dS,
//     dV^T += dO^T P, dK^T += Q^T dS.
// P and dS are rounded to bf16 for the products (as the forward's P); the
// softmax scale is applied to dQ and dK once at the end.  Grouped-query K/V:
// query head h reads K/V head h / (H / Hk) in both kernels, and dK, dV are
// written per query head (the gradients of the repeated heads; a caller sums
// each group), so no workgroup walks several query heads.

struct AttnStrides {
    int64_t q[3], k[3], v[3], o[3], d[3], dq[3], dk[3], dv[3];  // {batch, position, head}, elements
};

// A-operand fragment (16 bytes, rows k-contiguous) of a 64 x 64 tile
__device__ __forceinline__ bf16x8_t tile_frag(const uint8_t* t, int row, int chunk) {
    return *reinterpret_cast<const bf16x8_t*>(t + tile_off(row, chunk));
}

// Transposed fragment of a 64 x 64 tile T[row][d] for MFMA step `ts`, d-block
// db: lane l receives T[16 ts + 4 (l/32) + {0..3}, 16 ts + 8 + 4 (l/32) +
// {0..3}][32 db + l%32] (ds_read_b64_tr_b16: output lane l element e = element
// l%4 of the 8 bytes addressed by lane 16 (l/16) + 4 e + (l%16)/4)
__device__ __forceinline__ bf16x8_t tile_frag_tr(const uint8_t* t, int ts, int db, int lane) {
    const int G = lane >> 4, u = lane & 15;
    const int row = 16 * ts + 4 * (G >> 1) + (u >> 2);
    const int d = 32 * db + 16 * (G & 1) + 4 * (u & 3);
    const v4i16 lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_v4i16*)(t + tile_off(row, d >> 3) + ((d & 7) << 1)));
    const v4i16 hi =
        __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_v4i16*)(t + tile_off(row + 8, d >> 3) + ((d & 7) << 1)));
    return __builtin_bit_cast(bf16x8_t, __builtin_shufflevector(lo, hi, 0, 1, 2, 3, 4, 5, 6, 7));
}

// Registers r0 .. r0 + 7 of an accumulator as a bf16 B (or A) fragment
__device__ __forceinline__ bf16x8_t pack8(const f32x16& a, int r0) {
    typedef uint32_t u32x4v __attribute__((ext_vector_type(4)));
    const u32x4v w = {pk_bf16(a[r0], a[r0 + 1]), pk_bf16(a[r0 + 2], a[r0 + 3]), pk_bf16(a[r0 + 4], a[r0 + 5]),
                      pk_bf16(a[r0 + 6], a[r0 + 7])};
    return __builtin_bit_cast(bf16x8_t, w);
}

__device__ __forceinline__ void zero16(f32x16& a) {
#pragma unroll
    for (int r = 0; r < 16; ++r) a[r] = 0.0f;
}

// Row `row` of a [.., 64] bf16 tensor as 4 B fragments (lane holds elements
// 16 c + 8 (l/32) .. +7)
__device__ __forceinline__ void row_frags(const bf16_t* p, int g, bf16x8_t (&f)[4]) {
#pragma unroll
    for (int c = 0; c < 4; ++c) f[c] = *reinterpret_cast<const bf16x8_t*>(p + 16 * c + 8 * g);
}

// Stores a transposed accumulator pair (registers of lane l: T[8 (r/4) + 4 (l/32)
// + r%4 (+32 for the second)][l%32]) times `mul` as the bf16 row of lane l.
__device__ __forceinline__ void store_row(bf16_t* p, const f32x16 (&acc)[2], float mul, int g) {
#pragma unroll
    for (int db = 0; db < 2; ++db)
#pragma unroll
        for (int a = 0; a < 4; ++a) {
            uint2 w;
            w.x = pk_bf16(acc[db][4 * a] * mul, acc[db][4 * a + 1] * mul);
            w.y = pk_bf16(acc[db][4 * a + 2] * mul, acc[db][4 * a + 3] * mul);
            *reinterpret_cast<uint2*>(p + 32 * db + 8 * a + 4 * g) = w;
        }
}

constexpr float kLog2e = 1.44269504088896340736f;

__global__ __launch_bounds__(256) void attn_bwd_dq_kernel(const bf16_t* __restrict__ q, const bf16_t* __restrict__ k,
                                                          const bf16_t* __restrict__ v, const bf16_t* __restrict__ o,
                                                          const bf16_t* __restrict__ dout,
                                                          const float* __restrict__ lse, float* __restrict__ stats,
                                                          bf16_t* __restrict__ dq, int S, int S_pad, int H, int Hk,
                                                          int BH, int nqt, AttnStrides st, float c2, float scale) {
    __shared__ __attribute__((aligned(16))) uint8_t smem[2][2 * kMatBytes];  // K tile, V tile
    const int bid = blockIdx.x;
    const int qt = nqt - 1 - bid / BH;  // heaviest query tiles first
    const int bh = bid - (bid / BH) * BH;
    const int b = bh / H, h = bh - (bh / H) * H;
    const int hk = h / (H / Hk);  // the K/V head the query head reads
    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int g = lane >> 5, col = lane & 31;
    const int q0 = qt * kQTile;
    const int qw0 = q0 + 32 * wave;
    const int qrow = qw0 + col;
    const int qc = min(qrow, S - 1);

    // Q^T and dO^T as B operands (lane: row qc, elements 16 c + 8 g ..), and
    // D = rowsum(dO o O) in fp32
    bf16x8_t qf[4], df[4], of[4];
    row_frags(q + (int64_t)b * st.q[0] + (int64_t)qc * st.q[1] + (int64_t)h * st.q[2], g, qf);
    row_frags(dout + (int64_t)b * st.d[0] + (int64_t)qc * st.d[1] + (int64_t)h * st.d[2], g, df);
    row_frags(o + (int64_t)b * st.o[0] + (int64_t)qc * st.o[1] + (int64_t)h * st.o[2], g, of);
    float dsum = 0.0f;
#pragma unroll
    for (int c = 0; c < 4; ++c)
#pragma unroll
        for (int e = 0; e < 8; ++e) dsum = fmaf((float)df[c][e], (float)of[c][e], dsum);
    dsum += __shfl_xor(dsum, 32);
    const float lse2 = lse[(int64_t)bh * S + qc] * kLog2e;
    // per (batch, head): lse log2 e for S_pad queries, then -D, for the
    // key-side kernel; padding queries up to S_pad get zeros
    if (g == 0 && qrow < S_pad) {
        stats[(int64_t)bh * 2 * S_pad + qrow] = qrow < S ? lse2 : 0.0f;
        stats[(int64_t)bh * 2 * S_pad + S_pad + qrow] = qrow < S ? -dsum : 0.0f;
    }
    // dP^T accumulates onto -D, so the MFMAs give dP^T - D directly
    f32x16 negd;
#pragma unroll
    for (int r = 0; r < 16; ++r) negd[r] = -dsum;

    // K and V tiles by direct-to-LDS loads (the forward's slot mapping)
    const bf16_t* kb0 = k + (int64_t)b * st.k[0] + (int64_t)hk * st.k[2];
    const bf16_t* vb0 = v + (int64_t)b * st.v[0] + (int64_t)hk * st.v[2];
    uint32_t voff[4];
    int vrow[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const int w = ((4 * i + wave) * 64 + lane) & 511;
        const int row = w >> 3, c = (w & 7) ^ swz(row);
        vrow[i] = row;
        voff[i] = (uint32_t)(row * (i < 2 ? st.k[1] : st.v[1]) * 2 + 16 * c);
    }
    auto issue = [&](int j, uint8_t* dst) __attribute__((always_inline)) {
        const __amdgpu_buffer_rsrc_t rk = tile_rsrc(kb0 + (int64_t)j * kKTile * st.k[1]);
        const __amdgpu_buffer_rsrc_t rv = tile_rsrc(vb0 + (int64_t)j * kKTile * st.v[1]);
        const int lim = S - j * kKTile;
#pragma unroll
        for (int i = 0; i < 4; ++i)
            __builtin_amdgcn_raw_ptr_buffer_load_lds(i < 2 ? rk : rv, (lds_void_t*)(dst + (4 * i + wave) * 1024),
                                                     16, vrow[i] < lim ? voff[i] : kOOB, 0, 0, 0);
    };

    const int S_tiles = (S + kKTile - 1) / kKTile;
    const int nt = min(S_tiles, (q0 + kQTile + kKTile - 1) / kKTile);
    f32x16 acc[2];
    zero16(acc[0]);
    zero16(acc[1]);
    issue(0, smem[0]);
    asm volatile("s_waitcnt vmcnt(0)\n\ts_barrier" ::: "memory");
    // as the forward: the tile's LDS reads come before the next tile's copies
    for (int j = 0; j < nt; ++j) {
        const uint8_t* ks = smem[j & 1];
        const uint8_t* vs = ks + kMatBytes;
        const int k0 = j * kKTile;
        const bool active = k0 <= qw0 + 31;
        f32x16 s[2], dp[2];
        bf16x8_t kt[4][2];
        if (active) {
#pragma unroll
            for (int kb = 0; kb < 2; ++kb) {
                zero16(s[kb]);
                dp[kb] = negd;
                const int row = 32 * kb + col;
#pragma unroll
                for (int c = 0; c < 4; ++c) {
                    s[kb] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(tile_frag(ks, row, 2 * c + g), qf[c], s[kb], 0, 0, 0);
                    dp[kb] =
                        __builtin_amdgcn_mfma_f32_32x32x16_bf16(tile_frag(vs, row, 2 * c + g), df[c], dp[kb], 0, 0, 0);
                }
            }
#pragma unroll
            for (int t = 0; t < 4; ++t)
#pragma unroll
                for (int db = 0; db < 2; ++db) kt[t][db] = tile_frag_tr(ks, t, db, lane);
        }
        if (j + 1 < nt) issue(j + 1, smem[(j + 1) & 1]);
        if (active) {
            if (k0 + kKTile - 1 > qw0) {  // the causal edge crosses the wave's queries (a branch of its own)
#pragma unroll
                for (int kb = 0; kb < 2; ++kb)
#pragma unroll
                    for (int r = 0; r < 16; ++r)
                        if (k0 + 32 * kb + 8 * (r >> 2) + 4 * g + (r & 3) > qrow) s[kb][r] = -INFINITY;
            }
#pragma unroll
            for (int kb = 0; kb < 2; ++kb)
#pragma unroll
                for (int r = 0; r < 16; ++r) {
                    const float p = __builtin_amdgcn_exp2f(fmaf(s[kb][r], c2, -lse2));
                    s[kb][r] = p * dp[kb][r];
                }
            // dQ^T += K^T dS^T, 16 keys per MFMA (the forward's key order)
#pragma unroll
            for (int t = 0; t < 4; ++t) {
                const bf16x8_t dsf = pack8(s[t >> 1], 8 * (t & 1));
#pragma unroll
                for (int db = 0; db < 2; ++db)
                    acc[db] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(kt[t][db], dsf, acc[db], 0, 0, 0);
            }
        }
        asm volatile("s_waitcnt vmcnt(0) lgkmcnt(0)\n\ts_barrier" ::: "memory");
    }
    if (qrow < S) store_row(dq + (int64_t)b * st.dq[0] + (int64_t)qrow * st.dq[1] + (int64_t)h * st.dq[2], acc, scale, g);
}

__global__ __launch_bounds__(256) void attn_bwd_dkdv_kernel(const bf16_t* __restrict__ q,
                                                            const bf16_t* __restrict__ k,
                                                            const bf16_t* __restrict__ v,
                                                            const bf16_t* __restrict__ dout,
                                                            const float* __restrict__ stats, bf16_t* __restrict__ dk,
                                                            bf16_t* __restrict__ dv, int S, int S_pad, int H, int Hk,
                                                            int BH, AttnStrides st, float c2, float scale) {
    // a stage: Q tile and dO tile of 128 queries (16 KiB each), then lse log2 e
    // [128] and -D [128] of those queries
    constexpr int kQBytes = 128 * kRowBytes;
    constexpr int kStage = 2 * kQBytes + 1024;
    __shared__ __attribute__((aligned(16))) uint8_t smem[2][kStage];
    const int bid = blockIdx.x;
    const int kt_idx = bid / BH;  // key block 0 sees the most queries: first
    const int bh = bid - kt_idx * BH;
    const int b = bh / H, h = bh - (bh / H) * H;
    const int hk = h / (H / Hk);  // the K/V head the query head reads
    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int g = lane >> 5, col = lane & 31;
    const int kv0 = kt_idx * 128;
    const int kw0 = kv0 + 32 * wave;
    const int key = kw0 + col;
    const int kc = min(key, S - 1);

    // K^T and V^T as B operands (lane: row kc, elements 16 c + 8 g ..)
    bf16x8_t kf[4], vf[4];
    row_frags(k + (int64_t)b * st.k[0] + (int64_t)kc * st.k[1] + (int64_t)hk * st.k[2], g, kf);
    row_frags(v + (int64_t)b * st.v[0] + (int64_t)kc * st.v[1] + (int64_t)hk * st.v[2], g, vf);

    // Q and dO tiles by direct-to-LDS loads: lane l of wave w's instruction i
    // (0-7) writes stage slot s = 64 (4 i + w) + l (slots 0-1023 Q, 1024-2047
    // dO), which is tile_off(row, c) for row = (s % 1024) / 8 and chunk
    // c = (s % 8) ^ swz(row); queries past S read zeros.  Wave 0 also copies
    // the stats: lanes 0-31 four lse log2 e each, lanes 32-63 four -D each.
    const bf16_t* qb0 = q + (int64_t)b * st.q[0] + (int64_t)h * st.q[2];
    const bf16_t* db0 = dout + (int64_t)b * st.d[0] + (int64_t)h * st.d[2];
    const float* sb0 = stats + (int64_t)bh * S_pad * 2;  // lse log2 e [S_pad], then -D [S_pad]
    uint32_t voff[8];
    int vrow[8];
#pragma unroll
    for (int i = 0; i < 8; ++i) {
        const int w = ((4 * i + wave) * 64 + lane) & 1023;
        const int row = w >> 3, c = (w & 7) ^ swz(row);
        vrow[i] = row;
        voff[i] = (uint32_t)(row * (i < 4 ? st.q[1] : st.d[1]) * 2 + 16 * c);
    }
    const uint32_t soff = (uint32_t)(((lane < 32 ? 0 : S_pad - 128) + 4 * lane) * 4);
    auto issue = [&](int i, uint8_t* dst) __attribute__((always_inline)) {
        const __amdgpu_buffer_rsrc_t rq = tile_rsrc(qb0 + (int64_t)i * 128 * st.q[1]);
        const __amdgpu_buffer_rsrc_t rd = tile_rsrc(db0 + (int64_t)i * 128 * st.d[1]);
        const int lim = S - i * 128;
#pragma unroll
        for (int ii = 0; ii < 8; ++ii)
            __builtin_amdgcn_raw_ptr_buffer_load_lds(ii < 4 ? rq : rd, (lds_void_t*)(dst + (4 * ii + wave) * 1024),
                                                     16, vrow[ii] < lim ? voff[ii] : kOOB, 0, 0, 0);
        if (wave == 0)
            __builtin_amdgcn_raw_ptr_buffer_load_lds(
                __builtin_amdgcn_make_buffer_rsrc(const_cast<float*>(sb0 + i * 128), (short)0, (int)kRange, 0x00020000),
                (lds_void_t*)(dst + 2 * kQBytes), 16, soff, 0, 0, 0);
    };

    f32x16 dka[2], dva[2];
    zero16(dka[0]);
    zero16(dka[1]);
    zero16(dva[0]);
    zero16(dva[1]);
    // query tile i: copy tile i + 1 into the other stage (whose last readers
    // passed the last barrier), compute on this one, then the barrier.
    // Unrolled by two so each step names its two stages as fixed buffers: the
    // compiler then tells the copies into one from the reads of the other.
    auto step = [&](int i, const uint8_t* __restrict__ cur, uint8_t* __restrict__ nxt, int ni)
                    __attribute__((always_inline)) {
        if (i + 1 < ni) issue(i + 1, nxt);
        const uint8_t* qs = cur;
        const uint8_t* ds_ = cur + kQBytes;
        const float* sts = reinterpret_cast<const float*>(cur + 2 * kQBytes);
#pragma unroll
        for (int qb = 0; qb < 4; ++qb) {
            const int qs0 = i * 128 + 32 * qb;  // first query of the sub-block
            if (qs0 + 31 < kw0) continue;       // every query precedes every key of the wave
            f32x16 sc, dp;
            // dP accumulates onto -D of each register's query (4 consecutive
            // queries per 16-byte read), so the MFMAs give dP - D directly
            zero16(sc);
            float l2[16];
#pragma unroll
            for (int a = 0; a < 4; ++a) {
                const float4 x = *reinterpret_cast<const float4*>(sts + 32 * qb + 8 * a + 4 * g);
                const float4 y = *reinterpret_cast<const float4*>(sts + 128 + 32 * qb + 8 * a + 4 * g);
                l2[4 * a] = x.x, l2[4 * a + 1] = x.y, l2[4 * a + 2] = x.z, l2[4 * a + 3] = x.w;
                dp[4 * a] = y.x, dp[4 * a + 1] = y.y, dp[4 * a + 2] = y.z, dp[4 * a + 3] = y.w;
            }
            const int row = 32 * qb + col;
#pragma unroll
            for (int c = 0; c < 4; ++c) {
                sc = __builtin_amdgcn_mfma_f32_32x32x16_bf16(tile_frag(qs, row, 2 * c + g), kf[c], sc, 0, 0, 0);
                dp = __builtin_amdgcn_mfma_f32_32x32x16_bf16(tile_frag(ds_, row, 2 * c + g), vf[c], dp, 0, 0, 0);
            }
            // register r of lane l: query qs0 + 8 (r/4) + 4 g + r%4, key `key`
            if (kw0 + 31 > qs0) {  // the causal edge crosses the sub-block (a branch of its own)
#pragma unroll
                for (int r = 0; r < 16; ++r)
                    if (key > qs0 + 8 * (r >> 2) + 4 * g + (r & 3)) sc[r] = -INFINITY;
            }
#pragma unroll
            for (int r = 0; r < 16; ++r) {
                const float p = __builtin_amdgcn_exp2f(fmaf(sc[r], c2, -l2[r]));
                sc[r] = p;
                dp[r] *= p;
            }
            // dV^T += dO^T P and dK^T += Q^T dS, 16 queries per MFMA
#pragma unroll
            for (int t = 0; t < 2; ++t) {
                const bf16x8_t pf = pack8(sc, 8 * t);
                const bf16x8_t dsf = pack8(dp, 8 * t);
#pragma unroll
                for (int db = 0; db < 2; ++db) {
                    dva[db] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(tile_frag_tr(ds_, 2 * qb + t, db, lane), pf,
                                                                      dva[db], 0, 0, 0);
                    dka[db] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(tile_frag_tr(qs, 2 * qb + t, db, lane), dsf,
                                                                      dka[db], 0, 0, 0);
                }
            }
        }
        // this wave's copies of tile i + 1 have landed and every wave is past
        // its reads of tile i
        asm volatile("s_waitcnt vmcnt(0) lgkmcnt(0)\n\ts_barrier" ::: "memory");
    };
    const int i0 = kv0 / 128;  // queries before the key block see none of its keys
    const int ni = S_pad / 128;
    issue(i0, smem[0]);
    // a wait the compiler sees (the K/V fragments and the first copies are in),
    // so it does not wait again for the fragments inside the loop
    __builtin_amdgcn_s_waitcnt(0);
    asm volatile("s_barrier" ::: "memory");
    for (int i = i0; i < ni; i += 2) {
        step(i, smem[0], smem[1], ni);
        if (i + 1 < ni) step(i + 1, smem[1], smem[0], ni);
    }
    if (key < S) {
        store_row(dk + (int64_t)b * st.dk[0] + (int64_t)key * st.dk[1] + (int64_t)h * st.dk[2], dka, scale, g);
        store_row(dv + (int64_t)b * st.dv[0] + (int64_t)key * st.dv[1] + (int64_t)h * st.dv[2], dva, 1.0f, g);
    }
}

}  // namespace

hipError_t launch_attention_fwd(const bf16_t* q, const bf16_t* k, const bf16_t* v, bf16_t* o, float* lse, int B,
                                int S, int H, int Hk, const int64_t* qs, const int64_t* ks, const int64_t* vs,
                                const int64_t* os, float scale, hipStream_t s) {
    const int BH = B * H;
    const int nqt = (S + kQTile - 1) / kQTile;
    const int64_t blocks = (int64_t)BH * nqt;
    if (blocks == 0) return hipSuccess;
    const float c2 = scale * 1.44269504088896340736f;  // scores in base 2
    attn_fwd_kernel<<<dim3((unsigned)blocks), 256, 0, s>>>(q, k, v, o, lse, S, H, Hk, BH, nqt, qs[0], qs[1], qs[2],
                                                          ks[0], ks[1], ks[2], vs[0], vs[1], vs[2], os[0], os[1],
                                                          os[2], c2);
    return hipGetLastError();
}

int64_t attention_bwd_workspace(int B, int S, int H) {
    const int64_t S_pad = (int64_t)(S + 127) / 128 * 128;
    return (int64_t)B * H * S_pad * 2 * (int64_t)sizeof(float);
}

hipError_t launch_attention_bwd(const bf16_t* q, const bf16_t* k, const bf16_t* v, const bf16_t* o,
                                const bf16_t* dout, const float* lse, bf16_t* dq, bf16_t* dk, bf16_t* dv, int B,
                                int S, int H, int Hk, const int64_t* strides, float scale, float* stats, hipStream_t s) {
    const int BH = B * H;
    if (BH == 0 || S == 0) return hipSuccess;
    AttnStrides st;
    for (int i = 0; i < 3; ++i) {
        st.q[i] = strides[i];
        st.k[i] = strides[3 + i];
        st.v[i] = strides[6 + i];
        st.o[i] = strides[9 + i];
        st.d[i] = strides[12 + i];
        st.dq[i] = strides[15 + i];
        st.dk[i] = strides[18 + i];
        st.dv[i] = strides[21 + i];
    }
    const int S_pad = (S + 127) / 128 * 128;  // the key-side kernel's query tiles
    const int nqt = (S + kQTile - 1) / kQTile;
    const float c2 = scale * kLog2e;
    attn_bwd_dq_kernel<<<dim3((unsigned)(BH * nqt)), 256, 0, s>>>(q, k, v, o, dout, lse, stats, dq, S, S_pad, H, Hk,
                                                                 BH, nqt, st, c2, scale);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return e;
    const int nkt = (S + 127) / 128;
    attn_bwd_dkdv_kernel<<<dim3((unsigned)(BH * nkt)), 256, 0, s>>>(q, k, v, dout, stats, dk, dv, S, S_pad, H, Hk,
                                                                   BH, st, c2, scale);
    return hipGetLastError();
}

}  // namespace vq
