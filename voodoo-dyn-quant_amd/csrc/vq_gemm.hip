// Tile configurations and launchers of the gated-Linear GEMMs (the kernel
// templates live in vq_gemm_impl.h).
#include "vq_gemm_impl.h"

namespace vq {

// 256x256 output tiles, 4 waves of 128x128 (256 fp32 accumulators per lane,
// held in AGPRs), operands copied global -> LDS by direct-to-LDS loads into two
// padded LDS stages with the stage switch inside the MFMA stream.  BK = 64 for
// the forward and dX products, 32 for the gate product (its epilogue, not the
// main loop, sets the LDS size; measured on MI355X at 8192 x 5120 x 17408).
// Operands stored [K][rows] (dX's W, both gate operands) keep that orientation
// in LDS and are read with ds_read_b64_tr_b16.
using FwdLA = DmaK<256, 64, 256>;
using FwdLB = DmaK<256, 64, 256>;
using DxLA = DmaK<256, 64, 256>;
using DxLB = DmaN<256, 64, 256>;
using GateL = DmaN<256, 32, 256>;
constexpr int kGateBI = 256, kGateBJ = 256;

static int device_cus() {
    static int cus = 0;
    if (cus == 0) {
        int dev = 0;
        hipDeviceProp_t prop;
        if (hipGetDevice(&dev) == hipSuccess && hipGetDeviceProperties(&prop, dev) == hipSuccess)
            cus = prop.multiProcessorCount;
        else
            cus = 256;
    }
    return cus;
}

// Reduction splits of the gate product: more work items shorten the last
// round of tiles, each split repeats the epilogue (measured: about as long
// as 1200 rows of the reduction).
int gate_splits(int M, int N, int D) {
    const int tiles = ((D + kGateBI - 1) / kGateBI) * ((N + kGateBJ - 1) / kGateBJ);
    const int cus = device_cus();
    int best = 1;
    double best_t = 1e30;
    for (int s = 1; s <= 4; ++s) {
        if (s > 1 && M / s < 1024) break;
        const int64_t rounds = ((int64_t)tiles * s + cus - 1) / cus;
        const double t = (double)rounds * (1.0 / s + 1200.0 / (M > 0 ? M : 1));
        if (t < best_t - 1e-9) {
            best_t = t;
            best = s;
        }
    }
    return best;
}

int64_t gate_partial_count(int M, int N, int D) {
    return (int64_t)((D + kGateBI - 1) / kGateBI) * ((N + kGateBJ - 1) / kGateBJ) * gate_splits(M, N, D);
}

hipError_t launch_gemm_fwd(const bf16_t* X, const bf16_t* W, int64_t ldw, bf16_t* Y, int M, int N, int D,
                           hipStream_t s) {
    GemmParams p{};
    p.A = X; p.lda = D; p.B = W; p.ldb = ldw; p.I = M; p.J = N; p.K = D; p.splits = 1; p.C = Y; p.ldc = N;
    return launch_gemm<FwdLA, FwdLB, 256, 256, 64, 2, 2, EPI_STORE, 2>(p, s);
}

hipError_t launch_gemm_dx(const bf16_t* dY, const bf16_t* W, int64_t ldw, bf16_t* dX, int M, int N, int D,
                          hipStream_t s) {
    GemmParams p{};
    p.A = dY; p.lda = N; p.B = W; p.ldb = ldw; p.I = M; p.J = D; p.K = N; p.splits = 1; p.C = dX; p.ldc = D;
    return launch_gemm<DxLA, DxLB, 256, 256, 64, 2, 2, EPI_STORE, 2>(p, s);
}

hipError_t launch_gemm_gate(const bf16_t* dY, const bf16_t* X, const CandSet& cs, float* partials, int M, int N,
                            int D, hipStream_t s) {
    GemmParams p{};
    p.A = X; p.lda = D; p.B = dY; p.ldb = N; p.I = D; p.J = N; p.K = M;
    p.splits = gate_splits(M, N, D);
    p.cs = cs; p.dlimit = D; p.partials = partials;
    return launch_gemm<GateL, GateL, kGateBI, kGateBJ, 32, 2, 2, EPI_GATE, 2>(p, s);
}

// Fixed-order fp64 sum of the work-item partials: dprobs[k] = sum_t partials[t][k].
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
