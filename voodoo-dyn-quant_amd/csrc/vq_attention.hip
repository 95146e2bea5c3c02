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
            // IEEE maximum (NaN-propagating: v_maximum3_f32), which needs no
            // canonicalisation of the MFMA results as fmaxf would
            float mx = __builtin_elementwise_maximum(s[0][0], s[1][0]);
#pragma unroll
            for (int r = 1; r < 16; ++r)
                mx = __builtin_elementwise_maximum(mx, __builtin_elementwise_maximum(s[0][r], s[1][r]));
            mx = __builtin_elementwise_maximum(mx, __shfl_xor(mx, 32)) * c2;
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

    const float lt = l_run + __shfl_xor(l_run, 32);
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

}  // namespace vq
