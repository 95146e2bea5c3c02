// bf16 MFMA GEMMs of the gated Linear on gfx950 (v_mfma_f32_32x32x16_bf16).
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
// The gate product never leaves registers: its epilogue decodes every
// candidate's weights at the lane's accumulator positions (exact fp32, the same
// decoder as dequant) and accumulates <dW, W_k> per tile; a second kernel sums
// the tile partials in a fixed order, so gate gradients are deterministic.
//
// MFMA 32x32x16 operand/result layout (per wave of 64 lanes):
//   A: lane l holds A[i = l%32][k = 8*(l/32) .. +7]
//   B: lane l holds B[k = 8*(l/32) .. +7][j = l%32]
//   D: register r of lane l is D[i = 8*(r/4) + 4*(l/32) + r%4][j = l%32]
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

    // rows [r0, r0 + ROWS) x k [k0, k0 + BK) of src[row * ld + k]
    __device__ __forceinline__ void load(const bf16_t* __restrict__ src, int64_t ld, int r0, int rows, int k0,
                                         int K) {
        const __amdgpu_buffer_rsrc_t rs = make_rsrc(src + (int64_t)r0 * ld + k0);
#pragma unroll
        for (int i = 0; i < NL; ++i) {
            const int id = i * THREADS + (int)threadIdx.x;
            const int row = id / CPR, c = id % CPR;
            const bool ok = r0 + row < rows && k0 + 8 * c < K;
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

template <int ROWS, int BK, int THREADS>
struct LoaderT {
    static constexpr int RB = ROWS / 8;         // 8-row blocks along the tile rows
    static constexpr int NB = RB * (BK / 8);    // 8x8 blocks per tile
    static constexpr int NBT = (NB + THREADS - 1) / THREADS;
    u32x4 reg[NBT][8];

    // rows [r0, r0 + ROWS) x k [k0, k0 + BK) of src[k * ld + row]
    __device__ __forceinline__ void load(const bf16_t* __restrict__ src, int64_t ld, int r0, int rows, int k0,
                                         int K) {
        const __amdgpu_buffer_rsrc_t rs = make_rsrc(src + (int64_t)k0 * ld + r0);
#pragma unroll
        for (int i = 0; i < NBT; ++i) {
            const int b = i * THREADS + (int)threadIdx.x;
            const int rb = b % RB, kb = b / RB;
            const bool rok = (NB % THREADS == 0 || b < NB) && r0 + 8 * rb < rows;
#pragma unroll
            for (int kk = 0; kk < 8; ++kk) {
                const int kr = 8 * kb + kk;
                const bool ok = rok && k0 + kr < K;
                reg[i][kk] = buf_load16(rs, ok ? (uint32_t)((kr * ld + 8 * rb) * 2) : kOOB);
            }
        }
    }
    // Half `rr` of the 8 loaded k-rows -> 8 consecutive k of tile row rr.
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
                u32x4 o;
                o.x = pair(reg[i][0][w], reg[i][1][w], odd);
                o.y = pair(reg[i][2][w], reg[i][3][w], odd);
                o.z = pair(reg[i][4][w], reg[i][5][w], odd);
                o.w = pair(reg[i][6][w], reg[i][7][w], odd);
                lds[lds_chunk<BK>(8 * rb + rr, kb)] = o;
            }
        }
    }
};

// ---------------------------------------------------------------- tile order
// Workgroups are dispatched round-robin over the 8 XCDs (workgroup w runs on
// XCD w % 8).  Remap so that each XCD works through a contiguous run of the
// grouped tile order: tiles sharing A rows and B rows then meet in the same L2.
struct TileCoord {
    int tm, tn, logical;
};

__device__ __forceinline__ TileCoord map_tile(int tiles_m, int tiles_n, int group_m) {
    const int T = tiles_m * tiles_n;
    const int w = blockIdx.x;
    const int per = T / 8, rem = T % 8;
    const int xcd = w % 8, local = w / 8;
    const int logical = xcd * per + min(xcd, rem) + local;
    const int group_size = group_m * tiles_n;
    const int group = logical / group_size;
    const int first_m = group * group_m;
    const int gm = min(tiles_m - first_m, group_m);
    const int in_group = logical % group_size;
    TileCoord tc;
    tc.tm = first_m + in_group % gm;
    tc.tn = in_group / gm;
    tc.logical = logical;
    return tc;
}

// ---------------------------------------------------------------- kernel
enum Epi : int { EPI_STORE = 0, EPI_GATE = 1 };

struct GemmParams {
    const bf16_t* A;
    int64_t lda;
    const bf16_t* B;
    int64_t ldb;
    int I, J, K;  // C is I x J, reduction length K
    bf16_t* C;
    int64_t ldc;
    // gate epilogue: i indexes d (< dlimit), j indexes n; candidates are rows n
    CandSet cs;
    int dlimit;
    float* partials;  // [tiles][ncand]
};

// <dW_tile, W_k> over the lane's accumulators: register r of block (a, b) is
// dW[d = dbase + 32a + 8(r/4) + r%4][n = nbase + 32b] (d, n relative to the
// wave's tile origin), decoded 4 consecutive d at a time.
template <int QT, int MI, int NJ>
__device__ __forceinline__ float gate_dot(const f32x16 (&acc)[MI][NJ], const uint8_t* __restrict__ qbytes,
                                          int64_t row_groups, int nbase, int dbase, int J, int dlimit) {
    constexpr int GB = group_bytes(QT);
    float s = 0.0f;
#pragma unroll
    for (int b = 0; b < NJ; ++b) {
        const int n = nbase + 32 * b;
        const bool nok = n < J;
        const uint8_t* row = qbytes + (int64_t)(nok ? n : 0) * row_groups * GB;
#pragma unroll
        for (int a = 0; a < MI; ++a)
#pragma unroll
            for (int g = 0; g < 4; ++g) {
                const int d = dbase + 32 * a + 8 * g;
                if (nok && d < dlimit) {
                    float w[4];
                    decode_run<QT, 4>(row + (int64_t)(d >> 8) * GB, d & 255, w);
#pragma unroll
                    for (int t = 0; t < 4; ++t) s = fmaf(acc[a][b][4 * g + t], w[t], s);
                }
                // keep the scheduler from hoisting every run's byte loads at once
                __builtin_amdgcn_sched_barrier(0);
            }
    }
    return s;
}

template <class LA, class LB, int BI, int BJ, int BK, int WI, int WJ, int EPI>
__global__ __launch_bounds__(WI* WJ * 64) void gemm_kernel(GemmParams p) {
    constexpr int WTI = BI / WI, WTJ = BJ / WJ;  // wave tile
    constexpr int MI = WTI / 32, NJ = WTJ / 32;
    constexpr int A_CH = BI * BK / 8, B_CH = BJ * BK / 8;
    extern __shared__ u32x4 smem[];
    u32x4* const sA0 = smem;
    u32x4* const sA1 = smem + A_CH;
    u32x4* const sB0 = smem + 2 * A_CH;
    u32x4* const sB1 = smem + 2 * A_CH + B_CH;

    const int tiles_i = (p.I + BI - 1) / BI, tiles_j = (p.J + BJ - 1) / BJ;
    const TileCoord tc = map_tile(tiles_i, tiles_j, 8);
    const int i0 = tc.tm * BI, j0 = tc.tn * BJ;

    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int wi = wave / WJ, wj = wave % WJ;

    f32x16 acc[MI][NJ];
#pragma unroll
    for (int a = 0; a < MI; ++a)
#pragma unroll
        for (int b = 0; b < NJ; ++b)
#pragma unroll
            for (int r = 0; r < 16; ++r) acc[a][b][r] = 0.0f;

    LA la;
    LB lb;
    la.load(p.A, p.lda, i0, p.I, 0, p.K);
    lb.load(p.B, p.ldb, j0, p.J, 0, p.K);
    la.store(sA0);
    lb.store(sB0);
    __syncthreads();

    const int nk = (p.K + BK - 1) / BK;
    for (int kt = 0; kt < nk; ++kt) {
        const bool more = kt + 1 < nk;
        if (more) {
            la.load(p.A, p.lda, i0, p.I, (kt + 1) * BK, p.K);
            lb.load(p.B, p.ldb, j0, p.J, (kt + 1) * BK, p.K);
        }
        const u32x4* sa = (kt & 1) ? sA1 : sA0;
        const u32x4* sb = (kt & 1) ? sB1 : sB0;
#pragma unroll
        for (int ks = 0; ks < BK / 16; ++ks) {
            bf16x8_t fa[MI], fb[NJ];
            const int ch = 2 * ks + (lane >> 5);
#pragma unroll
            for (int a = 0; a < MI; ++a)
                fa[a] = __builtin_bit_cast(bf16x8_t, sa[lds_chunk<BK>(wi * WTI + 32 * a + (lane & 31), ch)]);
#pragma unroll
            for (int b = 0; b < NJ; ++b)
                fb[b] = __builtin_bit_cast(bf16x8_t, sb[lds_chunk<BK>(wj * WTJ + 32 * b + (lane & 31), ch)]);
#pragma unroll
            for (int a = 0; a < MI; ++a)
#pragma unroll
                for (int b = 0; b < NJ; ++b)
                    acc[a][b] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(fa[a], fb[b], acc[a][b], 0, 0, 0);
        }
        if (more) {
            la.store((kt & 1) ? sA0 : sA1);
            lb.store((kt & 1) ? sB0 : sB1);
        }
        __syncthreads();
    }

    if constexpr (EPI == EPI_STORE) {
#pragma unroll
        for (int a = 0; a < MI; ++a)
#pragma unroll
            for (int b = 0; b < NJ; ++b) {
                const int gj = j0 + wj * WTJ + 32 * b + (lane & 31);
#pragma unroll
                for (int r = 0; r < 16; ++r) {
                    const int gi = i0 + wi * WTI + 32 * a + 8 * (r >> 2) + 4 * (lane >> 5) + (r & 3);
                    if (gi < p.I && gj < p.J) p.C[(int64_t)gi * p.ldc + gj] = f2bf(acc[a][b][r]);
                }
            }
    } else {
        // Gate epilogue: rows i are d, columns j are n.  Each lane owns runs of
        // 4 consecutive d of one row n: decode them exactly and dot.
        __shared__ float red[WI * WJ][kMaxCand];
        const int dbase = i0 + wi * WTI + 4 * (lane >> 5);
        const int nbase = j0 + wj * WTJ + (lane & 31);
        for (int k = 0; k < p.cs.ncand; ++k) {
            const uint8_t* q = p.cs.qbytes[k];
            float s;
            switch (p.cs.qtype[k]) {
            case Q8_0: s = gate_dot<Q8_0, MI, NJ>(acc, q, p.cs.row_groups, nbase, dbase, p.J, p.dlimit); break;
            case Q2_K: s = gate_dot<Q2_K, MI, NJ>(acc, q, p.cs.row_groups, nbase, dbase, p.J, p.dlimit); break;
            case Q3_K: s = gate_dot<Q3_K, MI, NJ>(acc, q, p.cs.row_groups, nbase, dbase, p.J, p.dlimit); break;
            case Q4_K: s = gate_dot<Q4_K, MI, NJ>(acc, q, p.cs.row_groups, nbase, dbase, p.J, p.dlimit); break;
            case Q5_K: s = gate_dot<Q5_K, MI, NJ>(acc, q, p.cs.row_groups, nbase, dbase, p.J, p.dlimit); break;
            default: s = gate_dot<Q6_K, MI, NJ>(acc, q, p.cs.row_groups, nbase, dbase, p.J, p.dlimit); break;
            }
#pragma unroll
            for (int off = 32; off >= 1; off >>= 1) s += __shfl_xor(s, off);
            if (lane == 0) red[wave][k] = s;
        }
        __syncthreads();
        if ((int)threadIdx.x < p.cs.ncand) {
            float s = 0.0f;
            for (int w = 0; w < WI * WJ; ++w) s += red[w][threadIdx.x];
            p.partials[(int64_t)tc.logical * p.cs.ncand + threadIdx.x] = s;
        }
    }
}

template <class LA, class LB, int BI, int BJ, int BK, int WI, int WJ, int EPI>
static hipError_t launch_gemm(const GemmParams& p, hipStream_t s) {
    if (p.I <= 0 || p.J <= 0) return hipSuccess;
    auto kern = gemm_kernel<LA, LB, BI, BJ, BK, WI, WJ, EPI>;
    const size_t lds = (size_t)2 * (BI + BJ) * BK * sizeof(bf16_t);
    static bool attr_set = false;  // per instantiation
    if (!attr_set) {
        hipError_t e = hipFuncSetAttribute((const void*)kern, hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds);
        if (e != hipSuccess) return e;
        attr_set = true;
    }
    const int tiles = ((p.I + BI - 1) / BI) * ((p.J + BJ - 1) / BJ);
    kern<<<dim3(tiles), dim3(WI * WJ * 64), lds, s>>>(p);
    return hipGetLastError();
}

// Tile configurations: 256x256 output tiles, BK = 64.  The forward and dX
// products run 8 waves (each 128x64, two waves per SIMD); the gate product keeps
// 4 waves (each 128x128) because its epilogue holds the whole tile while it
// decodes candidates.
template <int WI, int WJ>
struct Cfg {
    static constexpr int BI = 256, BJ = 256, BK = 64, THREADS = WI * WJ * 64;
};
using CfgFwd = Cfg<2, 4>;
using CfgDx = Cfg<2, 4>;
using CfgGate = Cfg<2, 2>;

hipError_t launch_gemm_fwd(const bf16_t* X, const bf16_t* W, int64_t ldw, bf16_t* Y, int M, int N, int D,
                           hipStream_t s) {
    using C = CfgFwd;
    GemmParams p{};
    p.A = X; p.lda = D; p.B = W; p.ldb = ldw; p.I = M; p.J = N; p.K = D; p.C = Y; p.ldc = N;
    return launch_gemm<LoaderK<C::BI, C::BK, C::THREADS>, LoaderK<C::BJ, C::BK, C::THREADS>, C::BI, C::BJ, C::BK,
                       2, 4, EPI_STORE>(p, s);
}

hipError_t launch_gemm_dx(const bf16_t* dY, const bf16_t* W, int64_t ldw, bf16_t* dX, int M, int N, int D,
                          hipStream_t s) {
    using C = CfgDx;
    GemmParams p{};
    p.A = dY; p.lda = N; p.B = W; p.ldb = ldw; p.I = M; p.J = D; p.K = N; p.C = dX; p.ldc = D;
    return launch_gemm<LoaderK<C::BI, C::BK, C::THREADS>, LoaderT<C::BJ, C::BK, C::THREADS>, C::BI, C::BJ, C::BK,
                       2, 4, EPI_STORE>(p, s);
}

int64_t gate_partial_count(int N, int D) {
    using C = CfgGate;
    return (int64_t)((D + C::BI - 1) / C::BI) * ((N + C::BJ - 1) / C::BJ);
}

hipError_t launch_gemm_gate(const bf16_t* dY, const bf16_t* X, const CandSet& cs, float* partials, int M, int N,
                            int D, hipStream_t s) {
    using C = CfgGate;
    GemmParams p{};
    p.A = X; p.lda = D; p.B = dY; p.ldb = N; p.I = D; p.J = N; p.K = M;
    p.cs = cs; p.dlimit = D; p.partials = partials;
    return launch_gemm<LoaderT<C::BI, C::BK, C::THREADS>, LoaderT<C::BJ, C::BK, C::THREADS>, C::BI, C::BJ, C::BK,
                       2, 2, EPI_GATE>(p, s);
}

// Fixed-order fp64 sum of the tile partials: dprobs[k] = sum_t partials[t][k].
__global__ __launch_bounds__(256) void gate_reduce_kernel(const float* __restrict__ partials, int64_t ntiles,
                                                          int ncand, float* __restrict__ dprobs) {
    __shared__ double sh[256];
    const int k = blockIdx.x;
    double s = 0.0;
    for (int64_t t = threadIdx.x; t < ntiles; t += 256) s += (double)partials[t * ncand + k];
    sh[threadIdx.x] = s;
    __syncthreads();
    for (int w = 128; w >= 1; w >>= 1) {
        if ((int)threadIdx.x < w) sh[threadIdx.x] += sh[threadIdx.x + w];
        __syncthreads();
    }
    if (threadIdx.x == 0) dprobs[k] = (float)sh[0];
}

hipError_t launch_gate_reduce(const float* partials, int64_t ntiles, int ncand, float* dprobs, hipStream_t s) {
    gate_reduce_kernel<<<dim3(ncand), dim3(256), 0, s>>>(partials, ntiles, ncand, dprobs);
    return hipGetLastError();
}

}  // namespace vq
