// bf16 MFMA GEMM machinery of the gated Linear on gfx950
// (v_mfma_f32_32x32x16_bf16).  Included by vq_gemm.hip, which instantiates
// the tile configurations.
//
// One kernel template computes C[i][j] = sum_k A[i][k] * B[j][k] with both
// operands staged in LDS as [rows][BK] tiles whose reduction index k is
// contiguous, which is the operand layout the MFMA reads (each lane holds 8
// consecutive k of one row).  Loaders fill those tiles from global memory:
//   LoaderK  - the source already has k contiguous (row-major [rows][K]);
//   LoaderT  - the source is [K][rows] (rows contiguous): a thread loads an
//              8x8 bf16 block with eight 16-byte loads and transposes it in
//              registers before its 16-byte LDS writes.
// The three products of the path:
//   forward  Y[m][n]  = sum_d X[m][d] W[n][d]        A=X (K), B=W (K)
//   dX       dX[m][d] = sum_n dY[m][n] W[n][d]       A=dY (K), B=W (T)
//   gate     dW[d][n] = sum_m X[m][d] dY[m][n]       A=X (T), B=dY (T)
// The gate product never reaches global memory: its epilogue stages the fp32
// tile through LDS (reusing the main-loop buffers) and dots every candidate's
// exactly decoded weights against it, writing one partial per candidate per
// work item.  <dW, W_k> is linear in dW, so the M reduction may also be split
// across work items with no dW reduction at all.  A second kernel sums the
// partials in a fixed order: gate gradients are deterministic.
//
// MFMA 32x32x16 operand/result layout (per wave of 64 lanes):
//   A: lane l holds A[i = l%32][k = 8*(l/32) .. +7]
//   B: lane l holds B[k = 8*(l/32) .. +7][j = l%32]
//   D: register r of lane l is D[i = 8*(r/4) + 4*(l/32) + r%4][j = l%32]
#pragma once

#include "vq_internal.h"

namespace vq {

typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef float f32x16 __attribute__((ext_vector_type(16)));

// ---------------------------------------------------------------- LDS layout
// Tile [rows][BK] bf16 in 16-byte chunks; chunk index XOR-swizzled with bits
// of the row so that both the MFMA fragment reads (32 consecutive rows, one
// chunk) and the transposed loader's writes (rows 8 apart) spread over banks.
template <int BK>
__device__ __forceinline__ int lds_chunk(int row, int chunk) {
    constexpr int CPR = BK / 8;
    const int sw = (row ^ (row >> 3)) & (CPR - 1);
    return row * CPR + (chunk ^ sw);
}

// ---------------------------------------------------------------- loaders
// Global reads go through raw buffer loads: an element outside the matrix is
// given an offset past the descriptor's range, and the hardware returns zeros
// for it, so edge tiles need no branches.  Descriptors are rebased per tile so
// every offset stays far below 2^31.
constexpr uint32_t kRange = 0x7ffffff0u;  // descriptor size in bytes (in-range offsets stay below 2^30)
constexpr uint32_t kOOB = 0x80000000u;    // offset past kRange: the load returns zeros

__device__ __forceinline__ __amdgpu_buffer_rsrc_t make_rsrc(const void* base) {
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), (short)0, (int)kRange, 0x00020000);
}

__device__ __forceinline__ u32x4 buf_load16(__amdgpu_buffer_rsrc_t r, uint32_t off) {
    return __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(r, (int)off, 0, 0));
}

template <int ROWS, int BK, int THREADS>
struct LoaderK {
    static constexpr int CPR = BK / 8;
    static constexpr int NL = ROWS * CPR / THREADS;
    static_assert(NL * THREADS == ROWS * CPR, "tile must split evenly over threads");
    u32x4 reg[NL];

    // rows [r0, r0 + ROWS) x k [k0, k0 + BK) of src[row * ld + k], zero past kend
    __device__ __forceinline__ void load(const bf16_t* __restrict__ src, int64_t ld, int r0, int rows, int k0,
                                         int kend) {
        const __amdgpu_buffer_rsrc_t rs = make_rsrc(src + (int64_t)r0 * ld + k0);
#pragma unroll
        for (int i = 0; i < NL; ++i) {
            const int id = i * THREADS + (int)threadIdx.x;
            const int row = id / CPR, c = id % CPR;
            const bool ok = r0 + row < rows && k0 + 8 * c < kend;
            reg[i] = buf_load16(rs, ok ? (uint32_t)((row * ld + 8 * c) * 2) : kOOB);
        }
    }
    __device__ __forceinline__ void store(u32x4* __restrict__ lds) const {
#pragma unroll
        for (int i = 0; i < NL; ++i) {
            const int id = i * THREADS + (int)threadIdx.x;
            lds[lds_chunk<BK>(id / CPR, id % CPR)] = reg[i];
        }
    }
};

// A thread moves one KB x 8 block (KB k-rows of 8 consecutive tile rows): KB
// 16-byte global loads, a register transpose, then 8 LDS writes of KB bf16.
// KB = 4 when the tile has enough blocks for every thread (fewer staging
// registers), else 8.
template <int ROWS, int BK, int THREADS>
struct LoaderT {
    static constexpr int RB = ROWS / 8;  // 8-row blocks along the tile rows
    static constexpr int KB = (RB * (BK / 4) >= THREADS) ? 4 : 8;
    static constexpr int NB = RB * (BK / KB);  // blocks per tile
    static constexpr int NBT = (NB + THREADS - 1) / THREADS;
    u32x4 reg[NBT][KB];

    // rows [r0, r0 + ROWS) x k [k0, k0 + BK) of src[k * ld + row], zero past kend
    __device__ __forceinline__ void load(const bf16_t* __restrict__ src, int64_t ld, int r0, int rows, int k0,
                                         int kend) {
        const __amdgpu_buffer_rsrc_t rs = make_rsrc(src + (int64_t)k0 * ld + r0);
#pragma unroll
        for (int i = 0; i < NBT; ++i) {
            const int b = i * THREADS + (int)threadIdx.x;
            const int rb = b % RB, kb = b / RB;
            const bool rok = (NB % THREADS == 0 || b < NB) && r0 + 8 * rb < rows;
#pragma unroll
            for (int kk = 0; kk < KB; ++kk) {
                const int kr = KB * kb + kk;
                const bool ok = rok && k0 + kr < kend;
                reg[i][kk] = buf_load16(rs, ok ? (uint32_t)((kr * ld + 8 * rb) * 2) : kOOB);
            }
        }
    }
    // Element rr of k-rows a and b, packed as two consecutive k.
    static __device__ __forceinline__ uint32_t pair(uint32_t a, uint32_t b, int odd) {
        return odd ? ((a >> 16) | (b & 0xffff0000u)) : ((a & 0xffffu) | (b << 16));
    }
    __device__ __forceinline__ void store(u32x4* __restrict__ lds) const {
#pragma unroll
        for (int i = 0; i < NBT; ++i) {
            const int b = i * THREADS + (int)threadIdx.x;
            if (NB % THREADS != 0 && b >= NB) continue;
            const int rb = b % RB, kb = b / RB;
#pragma unroll
            for (int rr = 0; rr < 8; ++rr) {
                const int w = rr >> 1, odd = rr & 1;
                if constexpr (KB == 8) {
                    u32x4 o;
                    o.x = pair(reg[i][0][w], reg[i][1][w], odd);
                    o.y = pair(reg[i][2][w], reg[i][3][w], odd);
                    o.z = pair(reg[i][4][w], reg[i][5][w], odd);
                    o.w = pair(reg[i][6][w], reg[i][7][w], odd);
                    lds[lds_chunk<BK>(8 * rb + rr, kb)] = o;
                } else {
                    uint2 o;
                    o.x = pair(reg[i][0][w], reg[i][1][w], odd);
                    o.y = pair(reg[i][2][w], reg[i][3][w], odd);
                    uint2* dst = reinterpret_cast<uint2*>(lds + lds_chunk<BK>(8 * rb + rr, kb >> 1)) + (kb & 1);
                    *dst = o;
                }
            }
        }
    }
};

// ---------------------------------------------------------------- work order
// Workgroups are dispatched round-robin over the 8 XCDs (workgroup w runs on
// XCD w % 8).  Remap so that each XCD works through a contiguous run of the
// grouped tile order: tiles sharing A rows and B rows then meet in the same L2.
struct WorkItem {
    int tm, tn, split, logical;
};

__device__ __forceinline__ WorkItem map_work(int tiles_m, int tiles_n, int splits, int group_m) {
    const int total = tiles_m * tiles_n * splits;
    const int w = blockIdx.x;
    const int per = total / 8, rem = total % 8;
    const int xcd = w % 8, local = w / 8;
    const int logical = xcd * per + min(xcd, rem) + local;
    const int tile = logical / splits;
    const int group_size = group_m * tiles_n;
    const int group = tile / group_size;
    const int first_m = group * group_m;
    const int gm = min(tiles_m - first_m, group_m);
    const int in_group = tile % group_size;
    WorkItem wi;
    wi.tm = first_m + in_group % gm;
    wi.tn = in_group / gm;
    wi.split = logical % splits;
    wi.logical = logical;
    return wi;
}

enum Epi : int { EPI_STORE = 0, EPI_GATE = 1 };

struct GemmParams {
    const bf16_t* A;
    int64_t lda;
    const bf16_t* B;
    int64_t ldb;
    int I, J, K;  // C is I x J, reduction length K
    int splits;   // reduction splits (gate epilogue only)
    bf16_t* C;
    int64_t ldc;
    // gate epilogue: i indexes d (< dlimit), j indexes n; candidates are rows n
    CandSet cs;
    int dlimit;
    float* partials;  // [work items][ncand]
};

template <int BI, int BJ, int BK, int WI, int WJ>
struct GemmShape {
    static constexpr int THREADS = WI * WJ * 64;
    static constexpr int WTI = BI / WI, WTJ = BJ / WJ;  // wave tile
    static constexpr int MI = WTI / 32, NJ = WTJ / 32;
    static constexpr int A_CH = BI * BK / 8, B_CH = BJ * BK / 8;  // 16-byte chunks per tile
    static constexpr size_t MAIN_LDS = (size_t)2 * (A_CH + B_CH) * 16;
};

// Double-buffered main loop over k in [kbeg, kend): global loads of stage
// s+1 are issued before the MFMAs of stage s and written to the other LDS
// buffer after them; one barrier per stage.
template <class LA, class LB, int BI, int BJ, int BK, int WI, int WJ>
__device__ __forceinline__ void gemm_mainloop(const GemmParams& p, int i0, int j0, int kbeg, int kend,
                                              u32x4* __restrict__ smem,
                                              f32x16 (&acc)[GemmShape<BI, BJ, BK, WI, WJ>::MI]
                                                           [GemmShape<BI, BJ, BK, WI, WJ>::NJ]) {
    using S = GemmShape<BI, BJ, BK, WI, WJ>;
    u32x4* const sA0 = smem;
    u32x4* const sA1 = smem + S::A_CH;
    u32x4* const sB0 = smem + 2 * S::A_CH;
    u32x4* const sB1 = smem + 2 * S::A_CH + S::B_CH;
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int wi = wave / WJ, wj = wave % WJ;

#pragma unroll
    for (int a = 0; a < S::MI; ++a)
#pragma unroll
        for (int b = 0; b < S::NJ; ++b)
#pragma unroll
            for (int r = 0; r < 16; ++r) acc[a][b][r] = 0.0f;

    LA la;
    LB lb;
    la.load(p.A, p.lda, i0, p.I, kbeg, kend);
    lb.load(p.B, p.ldb, j0, p.J, kbeg, kend);
    la.store(sA0);
    lb.store(sB0);
    __syncthreads();

    const int nk = (kend - kbeg + BK - 1) / BK;
    for (int kt = 0; kt < nk; ++kt) {
        const bool more = kt + 1 < nk;
        if (more) {
            la.load(p.A, p.lda, i0, p.I, kbeg + (kt + 1) * BK, kend);
            lb.load(p.B, p.ldb, j0, p.J, kbeg + (kt + 1) * BK, kend);
        }
        const u32x4* sa = (kt & 1) ? sA1 : sA0;
        const u32x4* sb = (kt & 1) ? sB1 : sB0;
#pragma unroll
        for (int ks = 0; ks < BK / 16; ++ks) {
            bf16x8_t fa[S::MI], fb[S::NJ];
            const int ch = 2 * ks + (lane >> 5);
#pragma unroll
            for (int a = 0; a < S::MI; ++a)
                fa[a] = __builtin_bit_cast(bf16x8_t, sa[lds_chunk<BK>(wi * S::WTI + 32 * a + (lane & 31), ch)]);
#pragma unroll
            for (int b = 0; b < S::NJ; ++b)
                fb[b] = __builtin_bit_cast(bf16x8_t, sb[lds_chunk<BK>(wj * S::WTJ + 32 * b + (lane & 31), ch)]);
#pragma unroll
            for (int a = 0; a < S::MI; ++a)
#pragma unroll
                for (int b = 0; b < S::NJ; ++b)
                    acc[a][b] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(fa[a], fb[b], acc[a][b], 0, 0, 0);
        }
        if (more) {
            la.store((kt & 1) ? sA0 : sA1);
            lb.store((kt & 1) ? sB0 : sB1);
        }
        __syncthreads();
    }
}

// ---------------------------------------------------------------- gate epilogue
// Each wave stages its own fp32 sub-tile through a private LDS region, half
// the d rows at a time (rows a = 2h, 2h+1 of its 32-row MFMA blocks), as
// T[n][d] with PITCH floats per n row; its lanes then dot runs of 8
// consecutive d of one n against every candidate.  Only the half being
// processed and the other half's accumulators are live at once.
template <int WTI, int WTJ>
struct GateStage {
    static constexpr int HALF = WTI / 2;       // d rows per half
    static constexpr int PITCH = HALF + 4;     // floats per n row (+16 B against bank conflicts)
    static constexpr int RUNS_PER_ROW = HALF / 8;
    static constexpr int RUNS = WTJ * RUNS_PER_ROW / 64;  // per lane
    static constexpr size_t WAVE_LDS = (size_t)WTJ * PITCH * 4;
};

template <int QT, int RUNS, int RUNS_PER_ROW>
__device__ __forceinline__ float gate_runs(const float (&v)[RUNS][8], const uint8_t* __restrict__ qbytes,
                                           int64_t row_groups, int nbase, int dbase, int lane, int J, int dlimit) {
    constexpr int GB = group_bytes(QT);
    float s = 0.0f;
#pragma unroll
    for (int i = 0; i < RUNS; ++i) {
        // branch-free: out-of-range runs read row 0 / group 0 and are masked,
        // so the loads of every run can be issued together
        const int run = i * 64 + lane;
        const int n = nbase + run / RUNS_PER_ROW;
        const int d = dbase + 8 * (run % RUNS_PER_ROW);
        const bool ok = n < J && d < dlimit;
        const uint8_t* g = qbytes + ((int64_t)(ok ? n : 0) * row_groups + (ok ? (d >> 8) : 0)) * GB;
        const float t = dot_run<QT, 8>(g, d & 255, v[i]);
        s += ok ? t : 0.0f;
    }
    return s;
}

template <int BI, int BJ, int BK, int WI, int WJ>
__device__ __forceinline__ void gate_epilogue(const GemmParams& p, const WorkItem& w, int i0, int j0,
                                              u32x4* __restrict__ smem,
                                              const f32x16 (&acc)[GemmShape<BI, BJ, BK, WI, WJ>::MI]
                                                                 [GemmShape<BI, BJ, BK, WI, WJ>::NJ]) {
    using S = GemmShape<BI, BJ, BK, WI, WJ>;
    using G = GateStage<S::WTI, S::WTJ>;
    constexpr int NW = WI * WJ;
    static_assert(S::MI % 2 == 0 && G::RUNS * 64 == S::WTJ * G::RUNS_PER_ROW, "gate staging shape");
    __shared__ float red[NW][kMaxCand];
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int wi = wave / WJ, wj = wave % WJ;
    float* T = reinterpret_cast<float*>(smem) + wave * (G::WAVE_LDS / 4);
    __syncthreads();  // every wave is past its last main-loop LDS read
#pragma unroll
    for (int h = 0; h < 2; ++h) {
#pragma unroll
        for (int a2 = 0; a2 < S::MI / 2; ++a2) {
            const int a = h * (S::MI / 2) + a2;
#pragma unroll
            for (int b = 0; b < S::NJ; ++b)
#pragma unroll
                for (int g = 0; g < 4; ++g) {
                    const int dl = 32 * a2 + 8 * g + 4 * (lane >> 5);
                    const int nl = 32 * b + (lane & 31);
                    *reinterpret_cast<float4*>(T + nl * G::PITCH + dl) = make_float4(
                        acc[a][b][4 * g], acc[a][b][4 * g + 1], acc[a][b][4 * g + 2], acc[a][b][4 * g + 3]);
                }
        }
        float v[G::RUNS][8];
#pragma unroll
        for (int i = 0; i < G::RUNS; ++i) {
            const int run = i * 64 + lane;
            const float* src = T + (run / G::RUNS_PER_ROW) * G::PITCH + 8 * (run % G::RUNS_PER_ROW);
            const float4 lo = *reinterpret_cast<const float4*>(src);
            const float4 hi = *reinterpret_cast<const float4*>(src + 4);
            v[i][0] = lo.x; v[i][1] = lo.y; v[i][2] = lo.z; v[i][3] = lo.w;
            v[i][4] = hi.x; v[i][5] = hi.y; v[i][6] = hi.z; v[i][7] = hi.w;
        }
        const int dbase = i0 + wi * S::WTI + h * G::HALF;
        const int nbase = j0 + wj * S::WTJ;
        for (int k = 0; k < p.cs.ncand; ++k) {
            const uint8_t* q = p.cs.qbytes[k];
            const int64_t rg = p.cs.row_groups;
            float s;
            switch (p.cs.qtype[k]) {
            case Q8_0: s = gate_runs<Q8_0, G::RUNS, G::RUNS_PER_ROW>(v, q, rg, nbase, dbase, lane, p.J, p.dlimit); break;
            case Q2_K: s = gate_runs<Q2_K, G::RUNS, G::RUNS_PER_ROW>(v, q, rg, nbase, dbase, lane, p.J, p.dlimit); break;
            case Q3_K: s = gate_runs<Q3_K, G::RUNS, G::RUNS_PER_ROW>(v, q, rg, nbase, dbase, lane, p.J, p.dlimit); break;
            case Q4_K: s = gate_runs<Q4_K, G::RUNS, G::RUNS_PER_ROW>(v, q, rg, nbase, dbase, lane, p.J, p.dlimit); break;
            case Q5_K: s = gate_runs<Q5_K, G::RUNS, G::RUNS_PER_ROW>(v, q, rg, nbase, dbase, lane, p.J, p.dlimit); break;
            default: s = gate_runs<Q6_K, G::RUNS, G::RUNS_PER_ROW>(v, q, rg, nbase, dbase, lane, p.J, p.dlimit); break;
            }
#pragma unroll
            for (int off = 32; off >= 1; off >>= 1) s += __shfl_xor(s, off);
            if (lane == 0) red[wave][k] = h == 0 ? s : red[wave][k] + s;
        }
    }
    __syncthreads();
    if ((int)threadIdx.x < p.cs.ncand) {
        float s = 0.0f;
        for (int wv = 0; wv < NW; ++wv) s += red[wv][threadIdx.x];
        p.partials[(int64_t)w.logical * p.cs.ncand + threadIdx.x] = s;
    }
}

// ---------------------------------------------------------------- kernel
template <class LA, class LB, int BI, int BJ, int BK, int WI, int WJ, int EPI>
__global__ __launch_bounds__(WI* WJ * 64) void gemm_kernel(GemmParams p) {
    using S = GemmShape<BI, BJ, BK, WI, WJ>;
    extern __shared__ u32x4 smem[];
    const int tiles_i = (p.I + BI - 1) / BI, tiles_j = (p.J + BJ - 1) / BJ;
    const WorkItem w = map_work(tiles_i, tiles_j, EPI == EPI_GATE ? p.splits : 1, 8);
    const int i0 = w.tm * BI, j0 = w.tn * BJ;
    int kbeg = 0, kend = p.K;
    if (EPI == EPI_GATE && p.splits > 1) {
        const int chunk = ((p.K + p.splits - 1) / p.splits + BK - 1) / BK * BK;
        kbeg = min(p.K, w.split * chunk);
        kend = min(p.K, kbeg + chunk);
    }
    f32x16 acc[S::MI][S::NJ];
    gemm_mainloop<LA, LB, BI, BJ, BK, WI, WJ>(p, i0, j0, kbeg, kend, smem, acc);

    if constexpr (EPI == EPI_STORE) {
        const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
        const int wi = wave / WJ, wj = wave % WJ;
#pragma unroll
        for (int a = 0; a < S::MI; ++a)
#pragma unroll
            for (int b = 0; b < S::NJ; ++b) {
                const int gj = j0 + wj * S::WTJ + 32 * b + (lane & 31);
#pragma unroll
                for (int r = 0; r < 16; ++r) {
                    const int gi = i0 + wi * S::WTI + 32 * a + 8 * (r >> 2) + 4 * (lane >> 5) + (r & 3);
                    if (gi < p.I && gj < p.J) p.C[(int64_t)gi * p.ldc + gj] = f2bf(acc[a][b][r]);
                }
            }
    } else {
        gate_epilogue<BI, BJ, BK, WI, WJ>(p, w, i0, j0, smem, acc);
    }
}

template <class LA, class LB, int BI, int BJ, int BK, int WI, int WJ, int EPI>
constexpr size_t gemm_lds_bytes() {
    using S = GemmShape<BI, BJ, BK, WI, WJ>;
    constexpr size_t gate = (size_t)WI * WJ * GateStage<S::WTI, S::WTJ>::WAVE_LDS;
    return EPI == EPI_GATE && gate > S::MAIN_LDS ? gate : S::MAIN_LDS;
}

template <class LA, class LB, int BI, int BJ, int BK, int WI, int WJ, int EPI>
static hipError_t launch_gemm(const GemmParams& p, hipStream_t s) {
    if (p.I <= 0 || p.J <= 0) return hipSuccess;
    auto kern = gemm_kernel<LA, LB, BI, BJ, BK, WI, WJ, EPI>;
    constexpr size_t lds = gemm_lds_bytes<LA, LB, BI, BJ, BK, WI, WJ, EPI>();
    static bool attr_set = false;  // per instantiation
    if (!attr_set) {
        hipError_t e = hipFuncSetAttribute((const void*)kern, hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds);
        if (e != hipSuccess) return e;
        attr_set = true;
    }
    const int splits = EPI == EPI_GATE ? p.splits : 1;
    const int items = ((p.I + BI - 1) / BI) * ((p.J + BJ - 1) / BJ) * splits;
    kern<<<dim3(items), dim3(WI * WJ * 64), lds, s>>>(p);
    return hipGetLastError();
}

}  // namespace vq
