// Fused decode + mix GEMMs for few tokens: Y = X W_eff^T and dX = dY W_eff
// with W_eff = sum_k p_k W_k built tile by tile in LDS from the K packed
// candidates, so W_eff never exists in HBM.  At a few dozen tokens the
// products are bound by reading the weights: these kernels read only the
// packed candidates (3.9 B per weight for the six K-quant formats) where the
// materialised path reads them, writes a bf16 W_eff and reads it again
// (7.9 B per weight).  Every tile is decoded once per 32-token block, so the
// cost grows with the token count; the caller picks this path below a
// measured crossover.
//
// A workgroup (8 waves) walks a fixed sequence of steps.  Each step fills one
// slot of a 4-slot LDS ring with exactly kFzLoads direct-to-LDS loads per
// lane (lanes with nothing to load read zeros), so the wait for a step is a
// compile-time vmcnt with the next two steps still in flight:
//   * a candidate step stages candidate k's bytes of 32 weight rows for one
//     256-weight group (each row span rounded out to 16-byte chunks, as the
//     gate epilogue stages them), and every thread adds its 16 weights of one
//     row, p_k * (dl * u + c), into fp32 registers:
//         acc = fma(p_k dl, u, acc),   cacc += p_k c
//     (two operations per weight and candidate instead of the four of the
//     separately rounded reference mixture: the tile is within a bf16 ulp of
//     the materialised W_eff, not bit-identical to it);
//   * the operand step stages the activation tile (X for the forward, dY for
//     dX); the thread rounds acc + cacc to bf16 into the W tile, and the
//     waves multiply.
// Products are split across workgroups along the reduction (the forward along
// D, dX along N) when the output alone gives too few workgroups; the parts
// are summed in a fixed order by fused_reduce_kernel, so results are
// deterministic.
#include "vq_gemm_impl.h"

namespace vq {

constexpr int kFzThreads = 512;                        // 8 waves
constexpr int kFzWaves = kFzThreads / 64;
constexpr int kFzRows = 32;                            // weight rows per decode step
constexpr int kFzBM = 32;                              // tokens per workgroup
constexpr int kFzSlotChunks = 1024;                    // 16-byte chunks per ring slot (16 KiB)
constexpr int kFzLoads = kFzSlotChunks / kFzThreads;   // loads per lane per step
constexpr int kFzRing = 4;                             // ring slots
// Every format's row span is staged at the pitch of the largest (Q8_0: 19
// chunks, an odd count, so rows fall on distinct 16-byte bank groups); a
// lane's (row, chunk) pair is then the same at every step, and the loads of a
// smaller format skip the chunks past its span.
constexpr int kFzPitch = gate_span_chunks(272);
static_assert(kFzRows * kFzPitch <= kFzSlotChunks, "a step of 32 row spans fits one slot");
static_assert(kFzBM * 32 <= kFzSlotChunks, "an X tile (32 tokens x 256 k) fits one slot");
constexpr size_t kFzLds = (size_t)(kFzRing * kFzSlotChunks + kFzRows * 32) * 16;  // ring + W tile: 80 KiB

struct FusedParams {
    const bf16_t* act;  // X [M][D] (forward) or dY [M][N] (dX)
    CandSet cs;
    const float* probs;
    int M, N, D;        // tokens, weight rows, weight columns used (D <= 256 * row_groups)
    bf16_t* out;        // Y [M][N] or dX [M][D] (no split)
    float* ws;          // [splits][M][N or D] fp32 parts (split > 1)
    int splits;
    int per_split;      // groups (forward) or 32-row blocks (dX) per split
};

// XOR swizzle of a [rows][32 chunks] tile: chunk c of row r sits in slot
// c ^ sw8(r), so the 8 rows one ds_read_b128 pass serves hit distinct 16-byte
// bank groups (rows are 512 bytes apart, so they alias without it).
__device__ __forceinline__ int sw8(int r) { return (r ^ (r >> 3)) & 7; }
// [32][4 chunks] tile (64-byte rows, two per 128 bytes)
__device__ __forceinline__ int sw4(int r) { return ((r >> 1) ^ (r >> 3)) & 3; }

// The staging chunks one lane copies: load i of the lane fills slot chunk
// (i * kFzWaves + wave) * 64 + lane = row * kFzPitch + c.
struct FzLane {
    int row[kFzLoads], c[kFzLoads];
    __device__ __forceinline__ FzLane() {
        const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
#pragma unroll
        for (int i = 0; i < kFzLoads; ++i) {
            const int id = (i * kFzWaves + wave) * 64 + lane;
            row[i] = id / kFzPitch;
            c[i] = id % kFzPitch;
        }
    }
};

// Where candidate bytes of rows [r0, r0 + 32) sit: `origin` is the 16-byte
// boundary at or below row r0's first byte, rows are `stride` bytes apart
// and `head` = (row r0's first byte) mod 16.  Row r0 + r's span of group g
// starts `head + r * stride + g * gb` bytes past origin.
struct FzRows {
    int64_t origin;
    int stride, head, gb;
    __device__ __forceinline__ FzRows(int qt, int64_t rg, int r0) {
        gb = group_bytes(qt);
        stride = (int)(rg * gb);
        const int64_t first = (int64_t)r0 * stride;
        origin = first & ~int64_t(15);
        head = (int)(first & 15);
    }
};

// Candidate k's spans of rows [r0, r0 + 32) (rows past N read row r0) for
// group g, into slot: chunk `row * kFzPitch + c` holds bytes [16 c, 16 c + 16)
// of the row's span rounded down to 16 bytes.  Always kFzLoads loads per lane.
__device__ __forceinline__ void fz_stage_cand(u32x4* slot, const FzLane& ln, const uint8_t* __restrict__ q, int qt,
                                              int64_t rg, int r0, int g, int N) {
    const FzRows rw(qt, rg, r0);
    const int nch = gate_span_chunks(rw.gb);
    const int64_t bytes = (int64_t)N * rw.stride - rw.origin;
    const __amdgpu_buffer_rsrc_t rs = __builtin_amdgcn_make_buffer_rsrc(
        const_cast<uint8_t*>(q + rw.origin), (short)0, (int)(bytes < (int64_t)kRange ? bytes : (int64_t)kRange),
        0x00020000);
    const int wave = __builtin_amdgcn_readfirstlane((int)threadIdx.x >> 6);
    const int gofs = rw.head + g * rw.gb;
#pragma unroll
    for (int i = 0; i < kFzLoads; ++i) {
        const int r = r0 + ln.row[i] < N ? ln.row[i] : 0;
        const uint32_t off = (uint32_t)(((r * rw.stride + gofs) & ~15) + 16 * ln.c[i]);
        const bool ok = ln.row[i] < kFzRows && ln.c[i] < nch;
        __builtin_amdgcn_raw_ptr_buffer_load_lds(rs, (lds_void_t*)(slot + (i * kFzWaves + wave) * 64), 16,
                                                 ok ? off : kOOB, 0, 0, 0);
    }
}

// Loads that fill nothing (past the last step): the same count, all zeros.
__device__ __forceinline__ void fz_stage_none(u32x4* slot, const void* any) {
    const __amdgpu_buffer_rsrc_t rs = make_rsrc(any);
    const int wave = __builtin_amdgcn_readfirstlane((int)threadIdx.x >> 6);
#pragma unroll
    for (int i = 0; i < kFzLoads; ++i)
        __builtin_amdgcn_raw_ptr_buffer_load_lds(rs, (lds_void_t*)(slot + (i * kFzWaves + wave) * 64), 16, kOOB, 0,
                                                 0, 0);
}

// The forward's X tile: tokens [m0, m0 + 32) x k [256 g, 256 g + 256), slot
// chunk 32 r + (c ^ sw8(r)) = X[m0 + r][256 g + 8 c .. + 8] (zeros past M or D).
__device__ __forceinline__ void fz_stage_x(u32x4* slot, const bf16_t* __restrict__ x, int m0, int g, int M, int D) {
    const __amdgpu_buffer_rsrc_t rs = make_rsrc(x + (int64_t)m0 * D);
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane((int)threadIdx.x >> 6);
#pragma unroll
    for (int i = 0; i < kFzLoads; ++i) {
        const int base = (i * kFzWaves + wave) * 64;
        const int id = base + lane;
        const int r = id >> 5, c = (id & 31) ^ sw8(id >> 5);
        const int k = 256 * g + 8 * c;
        const bool ok = m0 + r < M && k < D;
        __builtin_amdgcn_raw_ptr_buffer_load_lds(rs, (lds_void_t*)(slot + base), 16,
                                                 ok ? (uint32_t)(((int64_t)r * D + k) * 2) : kOOB, 0, 0, 0);
    }
}

// dX's dY tile: tokens [m0, m0 + 32) x rows [r0, r0 + 32), slot chunk
// 4 i + (c ^ sw4(i)) = dY[m0 + i][r0 + 8 c .. + 8] (zeros past M or N).
__device__ __forceinline__ void fz_stage_dy(u32x4* slot, const bf16_t* __restrict__ dy, int m0, int r0, int M, int N) {
    const __amdgpu_buffer_rsrc_t rs = make_rsrc(dy + (int64_t)m0 * N);
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane((int)threadIdx.x >> 6);
#pragma unroll
    for (int i = 0; i < kFzLoads; ++i) {
        const int base = (i * kFzWaves + wave) * 64;
        const int id = base + lane;
        const int r = id >> 2, c = (id & 3) ^ sw4(id >> 2);
        const bool ok = id < kFzBM * 4 && m0 + r < M && r0 + 8 * c < N;
        __builtin_amdgcn_raw_ptr_buffer_load_lds(rs, (lds_void_t*)(slot + base), 16,
                                                 ok ? (uint32_t)(((int64_t)r * N + r0 + 8 * c) * 2) : kOOB, 0, 0, 0);
    }
}

// acc[r] += p * (dl * u_r + c) for this thread's 16 weights (row t / 16,
// weights 16 (t % 16) .. + 15 of the group) of the staged candidate.  Only
// the decode is specialised per format; the accumulation is shared, so the
// accumulators stay in the same registers whichever format a step holds.
template <bool IQ>
__device__ __forceinline__ void fz_decode_rt(int qt, const u32x4* slot, int64_t rg, int r0, int g, int N, float pk,
                                             float (&acc)[16], float& cacc) {
    const FzRows rw(qt, rg, r0);
    const int t = threadIdx.x;
    const int row = t >> 4, p = 16 * (t & 15);
    const int r = r0 + row < N ? row : 0;
    const int head = (r * rw.stride + rw.head + g * rw.gb) & 15;
    const uint8_t* gp = reinterpret_cast<const uint8_t*>(slot) + row * 16 * kFzPitch + head;
    uint32_t uw[4];
    float dl, c;
    switch (qt) {
    case Q8_0: decode_affine<Q8_0, 16>(gp, p, uw, dl, c); break;
    case Q2_K: decode_affine<Q2_K, 16>(gp, p, uw, dl, c); break;
    case Q3_K: decode_affine<Q3_K, 16>(gp, p, uw, dl, c); break;
    case Q4_K: decode_affine<Q4_K, 16>(gp, p, uw, dl, c); break;
    case Q5_K: decode_affine<Q5_K, 16>(gp, p, uw, dl, c); break;
    case Q6_K: decode_affine<Q6_K, 16>(gp, p, uw, dl, c); break;
    default:
        if constexpr (IQ)
            decode_affine_iq<16>(qt, gp, p, uw, dl, c);
        else
            decode_affine<Q6_K, 16>(gp, p, uw, dl, c);
        break;
    }
    const float pdl = pk * dl;
    cacc = fmaf(pk, c, cacc);
#pragma unroll
    for (int r2 = 0; r2 < 16; ++r2) acc[r2] = fmaf(pdl, (float)((uw[r2 >> 2] >> (8 * (r2 & 3))) & 0xffu), acc[r2]);
}

// Round this thread's 16 weights to bf16 into the W tile: two chunks of row
// t / 16 at chunk positions 2 (t % 16), + 1, placed by `slot_of(row, chunk)`.
template <class SlotOf>
__device__ __forceinline__ void fz_put_w(u32x4* wt, float (&acc)[16], float cacc, SlotOf slot_of) {
    const int t = threadIdx.x;
    const int row = t >> 4, c0 = 2 * (t & 15);
#pragma unroll
    for (int h = 0; h < 2; ++h) {
        u32x4 v;
#pragma unroll
        for (int e = 0; e < 4; ++e) v[e] = f2bf2(acc[8 * h + 2 * e] + cacc, acc[8 * h + 2 * e + 1] + cacc);
        wt[slot_of(row, c0 + h)] = v;
    }
#pragma unroll
    for (int r = 0; r < 16; ++r) acc[r] = 0.0f;
}

// The step loop shared by both kernels: units [0, nunits), each K candidate
// steps then the operand step, through a ring of kFzRing slots.
// unit_of(u, r0, g) names unit u's rows and group; stage_op(slot, r0, g)
// stages its operand tile; consume(slot, W tile, u) runs after the operand
// step's wait with the W tile complete.  The issue position (unit, step) is
// carried along with the consume position, so no step needs a division.
template <bool IQ, class UnitOf, class StageOp, class Consume, class PutW>
__device__ __forceinline__ void fz_steps(const FusedParams& p, u32x4* smem, int nunits, UnitOf unit_of,
                                         StageOp stage_op, PutW put_w, Consume consume) {
    const CandSet& cs = p.cs;
    const int K = cs.ncand;
    u32x4* wt = smem + kFzRing * kFzSlotChunks;
    const FzLane ln;
    int iu = 0, ij = 0, islot = 0;  // the next step to issue: unit, step within it, ring slot
    auto issue = [&]() {
        u32x4* slot = smem + islot * kFzSlotChunks;
        if (iu >= nunits) {
            fz_stage_none(slot, p.act);
        } else {
            int r0, g;
            unit_of(iu, r0, g);
            if (ij < K)
                fz_stage_cand(slot, ln, cs.qbytes[ij], cs.qtype[ij], cs.row_groups, r0, g, p.N);
            else
                stage_op(slot, r0, g);
        }
        islot = (islot + 1) & (kFzRing - 1);
        if (++ij > K) {
            ij = 0;
            ++iu;
        }
    };
    static_assert((kFzRing & (kFzRing - 1)) == 0, "ring slots: a power of two");
    // the probabilities in SGPRs before the loop: a global load inside it
    // would make its wait cover every staging load issued before it
    float pr[kMaxCand];
#pragma unroll
    for (int q = 0; q < kMaxCand; ++q)
        pr[q] = __int_as_float(__builtin_amdgcn_readfirstlane(q < K ? __float_as_int(p.probs[q]) : 0));
    float acc[16];
#pragma unroll
    for (int r = 0; r < 16; ++r) acc[r] = 0.0f;
    float cacc = 0.0f;
#pragma unroll
    for (int q = 0; q < kFzRing - 1; ++q) issue();
    int slot_i = 0;
    for (int u = 0; u < nunits; ++u) {
        int r0, g;
        unit_of(u, r0, g);
        for (int j = 0; j <= K; ++j) {
            // this step has landed (the two after it may still be in flight),
            // and every wave is done with the previous step, whose slot the
            // next issue refills
            wait_vmcnt_barrier<(kFzRing - 2) * kFzLoads>();
            issue();
            const u32x4* slot = smem + slot_i * kFzSlotChunks;
            slot_i = (slot_i + 1) & (kFzRing - 1);
            if (j < K) {
                float pk = pr[0];
#pragma unroll
                for (int q = 1; q < kMaxCand; ++q)
                    if (j == q) pk = pr[q];
                fz_decode_rt<IQ>(cs.qtype[j], slot, cs.row_groups, r0, g, p.N, pk, acc, cacc);
            } else {
                put_w(wt, acc, cacc);
                cacc = 0.0f;
                // the W tile is complete (LDS writes and a barrier only: the
                // staging loads in flight stay in flight)
                asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
                consume(slot, wt, u);
            }
        }
    }
    wait_vmcnt_barrier<0>();  // the zero loads past the end have landed before LDS is reused
}

// Forward: work item (32-row block blockIdx.x, group split blockIdx.y, token
// block blockIdx.z).  Wave w multiplies k slice [32 w, 32 w + 32) of every
// group; the eight partial tiles are summed in wave order at the end.
// IQ: the candidate set may hold IQ formats.  Their table-lookup decode needs
// more registers; held to 4 waves per SIMD (two workgroups per CU) it spills
// a few bytes, which the K-quant-only instantiation does not.
template <bool IQ>
__global__ __launch_bounds__(kFzThreads) __attribute__((amdgpu_waves_per_eu(4))) void fused_fwd_kernel(FusedParams p) {
    extern __shared__ u32x4 smem[];
    const int r0 = blockIdx.x * kFzRows;
    const int G = (p.D + 255) / 256;  // groups past D only hold zero-padding columns
    const int g0 = blockIdx.y * p.per_split;
    const int ng = min(p.per_split, G - g0);
    const int m0 = blockIdx.z * kFzBM;
    if (ng <= 0) return;
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    f32x16 yacc;
#pragma unroll
    for (int r = 0; r < 16; ++r) yacc[r] = 0.0f;
    auto unit_of = [&](int u, int& rr0, int& g) {
        rr0 = r0;
        g = g0 + u;
    };
    auto stage_op = [&](u32x4* slot, int, int g) { fz_stage_x(slot, p.act, m0, g, p.M, p.D); };
    auto put_w = [&](u32x4* wt, float(&acc)[16], float cacc) {
        fz_put_w(wt, acc, cacc, [](int row, int c) { return row * 32 + (c ^ sw8(row)); });
    };
    auto consume = [&](const u32x4* xs, const u32x4* wt, int) {
        // A = X[token][k], B = W[row][k]: lane l reads row l % 32, chunk
        // 4 w + 2 ks + l / 32 of both tiles
#pragma unroll
        for (int ks = 0; ks < 2; ++ks) {
            const int c = 4 * wave + 2 * ks + (lane >> 5), r = lane & 31;
            const bf16x8_t a = __builtin_bit_cast(bf16x8_t, xs[r * 32 + (c ^ sw8(r))]);
            const bf16x8_t b = __builtin_bit_cast(bf16x8_t, wt[r * 32 + (c ^ sw8(r))]);
            yacc = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b, yacc, 0, 0, 0);
        }
    };
    fz_steps<IQ>(p, smem, ng, unit_of, stage_op, put_w, consume);
    // sum the waves' partial tiles in wave order: [wave][register][lane]
    float* red = reinterpret_cast<float*>(smem);
#pragma unroll
    for (int r = 0; r < 16; ++r) red[(wave * 16 + r) * 64 + lane] = yacc[r];
    __syncthreads();
    for (int e = threadIdx.x; e < 16 * 64; e += kFzThreads) {
        float s = 0.0f;
        for (int w = 0; w < kFzWaves; ++w) s += red[w * 1024 + e];
        const int r = e >> 6, l = e & 63;
        const int m = m0 + 8 * (r >> 2) + 4 * (l >> 5) + (r & 3);
        const int n = r0 + (l & 31);
        if (m < p.M && n < p.N) {
            if (p.splits == 1)
                p.out[(int64_t)m * p.N + n] = f2bf(s);
            else
                p.ws[((int64_t)blockIdx.y * p.M + m) * p.N + n] = s;
        }
    }
}

// dX: work item (column group g, 32-row-block split sp) for token block
// blockIdx.z.  Items are ordered split-major and dealt to the XCDs in
// contiguous ranges (workgroup b runs on XCD b % 8), so the workgroups that
// read neighbouring groups of the same rows -- and so the same cache lines --
// share one XCD's L2.  The W tile is [32 rows (the reduction)][256 columns]
// in the [K][rows] layout the transposed fragment reads want; wave w owns
// output columns [32 w, 32 w + 32) of the group.
template <bool IQ>
__global__ __launch_bounds__(kFzThreads) __attribute__((amdgpu_waves_per_eu(4))) void fused_dx_kernel(FusedParams p) {
    extern __shared__ u32x4 smem[];
    using WL = DmaNS<256, 32, kFzThreads>;  // W tile as [32 k-rows][256 columns]
    const int G = (p.D + 255) / 256;
    const int items = G * p.splits;
    const int per_xcd = (items + 7) / 8;
    const int item = (int)(blockIdx.x % 8) * per_xcd + (int)(blockIdx.x / 8);
    if (item >= items) return;
    const int g = item % G, sp = item / G;
    const int nb = (p.N + kFzRows - 1) / kFzRows;
    const int b0 = sp * p.per_split;
    const int nblk = min(p.per_split, nb - b0);
    const int m0 = blockIdx.z * kFzBM;
    if (nblk <= 0) return;
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    f32x16 acc;
#pragma unroll
    for (int r = 0; r < 16; ++r) acc[r] = 0.0f;
    auto unit_of = [&](int u, int& r0, int& gg) {
        r0 = (b0 + u) * kFzRows;
        gg = g;
    };
    auto stage_op = [&](u32x4* slot, int r0, int) { fz_stage_dy(slot, p.act, m0, r0, p.M, p.N); };
    auto put_w = [&](u32x4* wt, float(&a)[16], float cacc) {
        fz_put_w(wt, a, cacc, [](int row, int c) { return row * 32 + (c ^ (4 * (row & 3))); });
    };
    auto consume = [&](const u32x4* dys, const u32x4* wt, int) {
        // A = dY[token][row]: lane l reads token l % 32, chunk 2 ks + l / 32
#pragma unroll
        for (int ks = 0; ks < 2; ++ks) {
            const int i = lane & 31, c = 2 * ks + (lane >> 5);
            const bf16x8_t a = __builtin_bit_cast(bf16x8_t, dys[i * 4 + (c ^ sw4(i))]);
            const bf16x8_t b = WL::read_frag(wt, 32 * wave, ks, lane);
            acc = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b, acc, 0, 0, 0);
        }
    };
    fz_steps<IQ>(p, smem, nblk, unit_of, stage_op, put_w, consume);
    const int d = 256 * g + 32 * wave + (lane & 31);
#pragma unroll
    for (int r = 0; r < 16; ++r) {
        const int m = m0 + 8 * (r >> 2) + 4 * (lane >> 5) + (r & 3);
        if (m < p.M && d < p.D) {
            if (p.splits == 1)
                p.out[(int64_t)m * p.D + d] = f2bf(acc[r]);
            else
                p.ws[((int64_t)sp * p.M + m) * p.D + d] = acc[r];
        }
    }
}

// out[i] = bf16(sum_s ws[s][i]) over i < count, parts in order.
__global__ __launch_bounds__(256) void fused_reduce_kernel(const float* __restrict__ ws, int splits, int64_t count,
                                                           bf16_t* __restrict__ out) {
    const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
    if (i >= count) return;
    float s = 0.0f;
    for (int k = 0; k < splits; ++k) s += ws[(int64_t)k * count + i];
    out[i] = f2bf(s);
}

// Parts of the reduction: `units` steps-groups (groups of the forward, row
// blocks of dX) shared out over `items` output tiles.  Two workgroups are
// resident per CU; the pick minimises the modelled time, rounds of resident
// workgroups x (units per part + the ring's fill, about four units' time).
static int fused_splits(int64_t items, int units, int cus) {
    const int64_t slots = 2 * (int64_t)cus;
    int best = 1;
    double best_t = 1e300;
    for (int s = 1; s <= units && s <= 64; ++s) {
        const int per = (units + s - 1) / s;
        const int parts = (units + per - 1) / per;
        if (parts != s) continue;
        const int64_t wgs = items * parts;
        const double t = (double)((wgs + slots - 1) / slots) * (per + 4.0);
        if (t < best_t * 0.98) {
            best_t = t;
            best = s;
        }
    }
    return best;
}

FusedPlan fused_plan(bool dx, int M, int N, int D) {
    FusedPlan pl{};
    const int mb = (M + kFzBM - 1) / kFzBM;
    if (!dx) {
        const int nb = (N + kFzRows - 1) / kFzRows;
        const int G = (D + 255) / 256;
        int s = fused_splits((int64_t)nb * mb, G, device_cus());
        pl.per_split = (G + s - 1) / s;
        pl.splits = (G + pl.per_split - 1) / pl.per_split;
        pl.grid_x = nb;
        pl.ws_bytes = pl.splits > 1 ? (int64_t)pl.splits * M * N * 4 : 0;
    } else {
        const int nb = (N + kFzRows - 1) / kFzRows;
        const int G = (D + 255) / 256;
        int s = fused_splits((int64_t)G * mb, nb, device_cus());
        pl.per_split = (nb + s - 1) / s;
        pl.splits = (nb + pl.per_split - 1) / pl.per_split;
        pl.grid_x = 8 * ((G * pl.splits + 7) / 8);  // items dealt to the XCDs (see fused_dx_kernel)
        pl.ws_bytes = pl.splits > 1 ? (int64_t)pl.splits * M * D * 4 : 0;
    }
    pl.grid_z = mb;
    return pl;
}

hipError_t launch_fused(bool dx, const bf16_t* act, const CandSet& cs, const float* probs, int M, int N, int D,
                        bf16_t* out, float* ws, hipStream_t s) {
    if (M <= 0) return hipSuccess;
    const FusedPlan pl = fused_plan(dx, M, N, D);
    FusedParams p{};
    p.act = act;
    p.cs = cs;
    p.probs = probs;
    p.M = M;
    p.N = N;
    p.D = D;
    p.out = out;
    p.ws = ws;
    p.splits = pl.splits;
    p.per_split = pl.per_split;
    static bool attr_done[2][2] = {};  // [dx][iq]
    const bool iq = any_iq(cs);
    const void* kern = dx ? (iq ? (const void*)fused_dx_kernel<true> : (const void*)fused_dx_kernel<false>)
                          : (iq ? (const void*)fused_fwd_kernel<true> : (const void*)fused_fwd_kernel<false>);
    bool& done = attr_done[dx][iq];
    if (!done) {
        hipError_t e = hipFuncSetAttribute(kern, hipFuncAttributeMaxDynamicSharedMemorySize, (int)kFzLds);
        if (e != hipSuccess) {
            (void)hipGetLastError();
            return e;
        }
        done = true;
    }
    const dim3 grid(pl.grid_x, dx ? 1 : pl.splits, pl.grid_z);
    if (dx && iq)
        fused_dx_kernel<true><<<grid, dim3(kFzThreads), kFzLds, s>>>(p);
    else if (dx)
        fused_dx_kernel<false><<<grid, dim3(kFzThreads), kFzLds, s>>>(p);
    else if (iq)
        fused_fwd_kernel<true><<<grid, dim3(kFzThreads), kFzLds, s>>>(p);
    else
        fused_fwd_kernel<false><<<grid, dim3(kFzThreads), kFzLds, s>>>(p);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess || pl.splits == 1) return e;
    const int64_t count = (int64_t)M * (dx ? D : N);
    fused_reduce_kernel<<<dim3((unsigned)((count + 255) / 256)), dim3(256), 0, s>>>(ws, pl.splits, count, out);
    return hipGetLastError();
}

}  // namespace vq
