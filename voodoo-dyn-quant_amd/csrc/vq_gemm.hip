// Tile configurations and launchers of the gated-Linear GEMMs (the kernel
// templates live in vq_gemm_impl.h).
#include "vq_gemm_impl.h"

namespace vq {

// 256x256 output tiles, 8 waves in a 4 x 2 layout (64x128 each, 128 fp32
// accumulators per lane) and two waves per SIMD, so one wave's fragment reads
// and copies hide under the other's MFMAs; operands copied global -> LDS by
// direct-to-LDS loads into two padded LDS stages with the stage switch inside
// the MFMA stream, BK = 64; the stage-switch order is chosen per product.
// Measured on MI355X at 8192 tokens against the same tiles with 4 waves of
// 128x128 and one wave per SIMD: forward 5120 -> 17408 1238 vs 1336 us,
// 17408 -> 5120 1226 vs 1392 us, 4096 -> 28672 1594 vs 1702 us; dX + gate
// 2659 vs 2690 us.
// Operands stored [K][rows] (dX's W, both gate operands) keep that orientation
// in LDS and are read with ds_read_b64_tr_b16.
constexpr int kWaves = 8;
using FwdLA = DmaKS<256, 64, 64 * kWaves>;
using FwdLB = DmaKS<256, 64, 64 * kWaves>;
using DxLA = DmaKS<256, 64, 64 * kWaves>;
using DxLB = DmaNS<256, 64, 64 * kWaves>;
using GateL = DmaNS<256, 64, 64 * kWaves>;
using GateLA = DmaNS<256, 64, 64 * kWaves, 1>;  // weight rows permuted for the gate epilogue
constexpr int kGateBI = 256, kGateBJ = 256;

hipError_t stream_fence(hipStream_t from, hipStream_t to) {
    if (from == to) return hipSuccess;
    constexpr int kDevices = 64, kRing = 8;
    static thread_local hipEvent_t ring[kDevices][kRing];  // held until the thread ends
    static thread_local int next[kDevices];
    int dev = 0;
    hipError_t e = from ? hipStreamGetDevice(from, &dev) : hipGetDevice(&dev);
    if (e != hipSuccess) return e;
    if (dev < 0 || dev >= kDevices) return hipErrorInvalidDevice;
    hipEvent_t& ev = ring[dev][next[dev]];
    next[dev] = (next[dev] + 1) % kRing;
    if (!ev) {  // created on the stream's device
        int cur = 0;
        if ((e = hipGetDevice(&cur)) != hipSuccess) return e;
        if (cur != dev && (e = hipSetDevice(dev)) != hipSuccess) return e;
        e = hipEventCreateWithFlags(&ev, hipEventDisableTiming);
        if (cur != dev) (void)hipSetDevice(cur);
        if (e != hipSuccess) {
            ev = nullptr;
            return e;
        }
    }
    if ((e = hipEventRecord(ev, from)) != hipSuccess) return e;
    return hipStreamWaitEvent(to, ev, 0);
}

int device_cus() {
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

// Every 8-wave product issues each refill in two halves (COPY_SPLIT) and
// pins its schedule only at each stage's first k-step (SWITCH_LOOSE).  The
// forward: split refills 0.3-4% faster at every swept shape, then SWITCH_LOOSE
// 0.1-1.0% faster than SWITCH_READ_FIRST at 8192 tokens and 5120 -> 17408,
// 4096 -> 28672, 14336 -> 4096, 1024 -> 6144, 1024 -> 1536.  The backward:
// 3.0-3.1% faster than dX SWITCH_FREE + gate SWITCH_LOOSE with single-burst
// refills at 5120 -> 17408, 17408 -> 5120, 4096 -> 28672 (0.6-1.3% at
// 1024-wide).
using FwdCfg = GemmCfg<FwdLA, FwdLB, 256, 256, 64, 4, 2, EPI_STORE, 2, SWITCH_LOOSE, 2, COPY_SPLIT>;
// Products with fewer 256x256 tiles than three quarters of the CUs (the 0.8B
// decoder's 1024-wide projections at 8192 tokens) fill the chip better with
// 128x128 tiles, four waves of 64x64 and two workgroups per CU (measured on
// MI355X at 8192 tokens: 1024 -> 1024 25 vs 33 us, 3072 -> 1024 55 vs 67 us);
// from 192 tiles on the 8-wave 256x256 tiles win (1024 -> 1536 33 vs 39 us,
// 1024 -> 3072 65 vs 68 us).  Reads first with split refills: 3-12% faster
// than a fenced stage switch with one burst per refill (8192 tokens at
// 1024 -> 1024, 2048 -> 1024, 3072 -> 1024; 4096 tokens at 1024 -> 1024).
using FwdSmallCfg =
    GemmCfg<DmaKS<128, 64, 256>, DmaKS<128, 64, 256>, 128, 128, 64, 2, 2, EPI_STORE, 2, SWITCH_READ_FIRST, 2, COPY_SPLIT>;

static bool small_product(int M, int N) {
    const int64_t tiles = (int64_t)((M + 255) / 256) * ((N + 255) / 256);
    return 4 * tiles < 3 * (int64_t)device_cus();
}
using DxCfg = GemmCfg<DxLA, DxLB, 256, 256, 64, 4, 2, EPI_STORE, 2, SWITCH_LOOSE, 2, COPY_SPLIT>;
using GateCfg = GemmCfg<GateLA, GateL, kGateBI, kGateBJ, 64, 4, 2, EPI_GATE, 2, SWITCH_LOOSE, 2, COPY_SPLIT>;
using GatePartsCfg = GemmCfg<GateLA, GateL, kGateBI, kGateBJ, 64, 4, 2, EPI_PARTS, 2, SWITCH_LOOSE, 2, COPY_SPLIT>;

static GemmParams fwd_params(const bf16_t* X, const bf16_t* W, int64_t ldw, bf16_t* Y, int M, int N, int D) {
    GemmParams p{};
    p.A = X; p.lda = D; p.B = W; p.ldb = ldw; p.I = M; p.J = N; p.K = D; p.C = Y; p.ldc = N;
    return p;
}

static GemmParams dx_params(const bf16_t* dY, const bf16_t* W, int64_t ldw, bf16_t* dX, int M, int N, int D) {
    GemmParams p{};
    p.A = dY; p.lda = N; p.B = W; p.ldb = ldw; p.I = M; p.J = D; p.K = N; p.C = dX; p.ldc = D;
    return p;
}

static GemmParams gate_params(const bf16_t* dY, const bf16_t* X, const CandGroup& cg, float* partials, int M, int N,
                              int D) {
    GemmParams p{};
    p.A = X; p.lda = D; p.B = dY; p.ldb = N; p.I = D; p.J = N; p.K = M;
    p.cg = cg; p.dlimit = D; p.partials = partials;
    return p;
}

// One partial per gate grid block (split tail parts and idle padding blocks
// included; the latter write zeros).
int64_t gate_partial_count(int M, int N, int D) {
    GemmParams p = gate_params(nullptr, nullptr, CandGroup{}, nullptr, M, N, D);
    return GateCfg::plan(p, device_cus(), true);
}

// Gate products whose 256x256 dW tiles are few enough that the fused plan
// splits them along M run every candidate's decode and dot once per part, and
// the epilogue (VALU-bound, K decodes of 65536 weights) then outlasts the
// part's main loop.  Where the fused plan splits tiles 4 ways or more, those
// products write fp32 parts instead (EPI_PARTS) and one pass over the summed
// parts takes the dots (launch_gate_dot).  Measured on MI355X at 8192 tokens,
// K = 6, backward launches together: 1024 -> 1536 93 -> 76 us, 3072 -> 1024
// 140 -> 126 us, 1024 -> 1024 65 -> 63 us; at 1024 -> 6144 (tiles split 2
// ways) the parts lost, 217 -> 238 us: the parts' round trip through memory
// (the dot pass reads them at about 4 TB/s) outweighs a twice-run epilogue.
// Parts per tile: what the CUs left over by dX's work items hold, at least 2,
// at most kMaxGateParts, each part at least 4 K steps; the buffer is capped at
// kMaxPartsBytes.
constexpr int64_t kMaxPartsBytes = (int64_t)64 << 20;

int gate_parts(int M, int N, int D) {
    if (M <= 0 || N <= 0 || D <= 0) return 0;
    const int cus = device_cus();
    GemmParams g = gate_params(nullptr, nullptr, CandGroup{}, nullptr, M, N, D);
    GateCfg::plan(g, cus, true);
    if (g.s_max < 4) return 0;  // each tile's epilogue runs at most 3 times
    const int64_t tiles = (int64_t)GateCfg::tiles_i(g) * GateCfg::tiles_j(g);
    GemmParams x = dx_params(nullptr, nullptr, 0, nullptr, M, N, D);
    const int dx_items = DxCfg::plan(x, cus, true);
    int64_t s = (cus - dx_items) / tiles;
    s = s < 2 ? 2 : s > kMaxGateParts ? kMaxGateParts : s;
    if (s > GateCfg::ksteps(g) / 4) s = GateCfg::ksteps(g) / 4;
    if (s < 2 || tiles * s * kGateBI * kGateBJ * 4 > kMaxPartsBytes) return 0;
    return (int)s;
}

static int64_t parts_floats(int parts, int N, int D) {
    return (int64_t)((D + kGateBI - 1) / kGateBI) * ((N + kGateBJ - 1) / kGateBJ) * parts * kGateBI * kGateBJ;
}

int64_t gate_parts_bytes(int M, int N, int D) {
    const int s = gate_parts(M, N, D);
    return s == 0 ? 0 : parts_floats(s, N, D) * 4;
}

// fp32 workspace for the K parts of dX's split tail tiles.
int64_t dx_tail_bytes(int M, int N, int D) {
    GemmParams p = dx_params(nullptr, nullptr, 0, nullptr, M, N, D);
    DxCfg::plan(p, device_cus(), true);
    return DxCfg::tail_bytes(p);
}

// fp32 workspace for the K parts of the forward's split tail tiles.
int64_t fwd_tail_bytes(int M, int N, int D) {
    GemmParams p = fwd_params(nullptr, nullptr, 0, nullptr, M, N, D);
    if (small_product(M, N)) {
        FwdSmallCfg::plan(p, device_cus(), true);
        return FwdSmallCfg::tail_bytes(p);
    }
    FwdCfg::plan(p, device_cus(), true);
    return FwdCfg::tail_bytes(p);
}

hipError_t launch_gemm_fwd(const bf16_t* X, const bf16_t* W, int64_t ldw, bf16_t* Y, int M, int N, int D,
                           float* tail_ws, hipStream_t s) {
    if (small_product(M, N))
        return launch_gemm_cfg<FwdSmallCfg>(fwd_params(X, W, ldw, Y, M, N, D), device_cus(), tail_ws, s);
    return launch_gemm_cfg<FwdCfg>(fwd_params(X, W, ldw, Y, M, N, D), device_cus(), tail_ws, s);
}

hipError_t launch_gemm_dx(const bf16_t* dY, const bf16_t* W, int64_t ldw, bf16_t* dX, int M, int N, int D,
                          float* tail_ws, hipStream_t s) {
    return launch_gemm_cfg<DxCfg>(dx_params(dY, W, ldw, dX, M, N, D), device_cus(), tail_ws, s);
}

static GemmParams parts_params(const bf16_t* dY, const bf16_t* X, float* dwp, int parts, int M, int N, int D) {
    GemmParams p = gate_params(dY, X, CandGroup{}, nullptr, M, N, D);
    p.dwp = dwp;
    p.parts = parts;
    return p;
}

hipError_t launch_gemm_gate(const bf16_t* dY, const bf16_t* X, const CandGroup& cg, float* partials, int M, int N,
                            int D, float* dwp, hipStream_t s, hipStream_t ds) {
    if (dwp) {
        const int np = gate_parts(M, N, D);
        if (np == 0) return hipErrorInvalidValue;
        hipError_t e = launch_gemm_cfg<GatePartsCfg>(parts_params(dY, X, dwp, np, M, N, D), device_cus(), nullptr, s);
        if (e == hipSuccess) e = stream_fence(s, ds);
        if (e != hipSuccess) return e;
        return launch_gate_dot(cg, N, D, dwp, np, partials, ds);
    }
    if (any_iq(cg))
        return launch_gemm_cfg<GateCfg, true>(gate_params(dY, X, cg, partials, M, N, D), device_cus(), nullptr, s);
    return launch_gemm_cfg<GateCfg>(gate_params(dY, X, cg, partials, M, N, D), device_cus(), nullptr, s);
}

// dX and gate products of one backward in a single launch (dX work items,
// the longer ones, first).
hipError_t launch_gemm_dx_gate(const bf16_t* dY, const bf16_t* W, int64_t ldw, bf16_t* dX, const bf16_t* X,
                               const CandGroup& cg, float* partials, int M, int N, int D, float* tail_ws,
                               float* dwp, hipStream_t s, hipStream_t ds) {
    if (dwp) {
        const int np = gate_parts(M, N, D);
        if (np == 0) return hipErrorInvalidValue;
        hipError_t e = launch_gemm_dual<DxCfg, GatePartsCfg>(dx_params(dY, W, ldw, dX, M, N, D),
                                                             parts_params(dY, X, dwp, np, M, N, D), device_cus(),
                                                             tail_ws, s);
        if (e == hipSuccess) e = stream_fence(s, ds);
        if (e != hipSuccess) return e;
        return launch_gate_dot(cg, N, D, dwp, np, partials, ds);
    }
    if (any_iq(cg))
        return launch_gemm_dual<DxCfg, GateCfg, true>(dx_params(dY, W, ldw, dX, M, N, D),
                                                        gate_params(dY, X, cg, partials, M, N, D), device_cus(),
                                                        tail_ws, s);
    return launch_gemm_dual<DxCfg, GateCfg>(dx_params(dY, W, ldw, dX, M, N, D),
                                            gate_params(dY, X, cg, partials, M, N, D), device_cus(), tail_ws, s);
}

// PTQR forward: token rows grouped by candidate, each group multiplied by its
// candidate's bf16 decode (the mainloop and store of the forward product, with
// A rows gathered and Y rows scattered through perm).
// SWITCH_LOOSE: 1.1-2.2% faster than SWITCH_READ_FIRST at 8192 tokens over six
// candidates (5120 -> 17408, 4096 -> 28672, 1024 -> 6144)
using RoutedCfg = GemmCfg<DmaKSG<256, 64, 64 * kWaves>, FwdLB, 256, 256, 64, 4, 2, EPI_STORE, 2, SWITCH_LOOSE, 2, COPY_SPLIT>;

hipError_t launch_routed_fwd(const bf16_t* X, int M, int D, const bf16_t* const* cand_bf16, int64_t ldw, int N,
                             int ncand, const int* perm, const int* group_off, bf16_t* Y, hipStream_t s) {
    GemmParams p = fwd_params(X, nullptr, ldw, Y, M, N, D);
    p.rowmap = perm;
    p.group_off = group_off;
    p.ngroups = ncand;
    p.map_rows = M;
    for (int k = 0; k < ncand; ++k) p.bk[k] = cand_bf16[k];
    return launch_routed_gemm<RoutedCfg>(p, M, device_cus(), s);
}

// Fixed-order fp64 sum of the work-item partials: dprobs[k] = sum_t partials[t * stride + k].
__global__ __launch_bounds__(256) void gate_reduce_kernel(const float* __restrict__ partials, int64_t ntiles,
                                                          int stride, float* __restrict__ dprobs) {
    __shared__ double sh[256];
    const int k = blockIdx.x;
    double s = 0.0;
    for (int64_t t = threadIdx.x; t < ntiles; t += 256) s += (double)partials[t * stride + k];
    sh[threadIdx.x] = s;
    __syncthreads();
    for (int w = 128; w >= 1; w >>= 1) {
        if ((int)threadIdx.x < w) sh[threadIdx.x] += sh[threadIdx.x + w];
        __syncthreads();
    }
    if (threadIdx.x == 0) dprobs[k] = (float)sh[0];
}

// Every member of a stacked product in one launch: block (k, i) reduces
// member i's candidate k (slot i * kstride + k of each partial row).
__global__ __launch_bounds__(256) void gate_reduce_group_kernel(const float* __restrict__ partials, int64_t ntiles,
                                                                int stride, GateReduceOut out) {
    __shared__ double sh[256];
    const int k = blockIdx.x, i = blockIdx.y;
    if (k >= out.ncand[i]) return;
    const int slot = i * out.kstride + k;
    double s = 0.0;
    for (int64_t t = threadIdx.x; t < ntiles; t += 256) s += (double)partials[t * stride + slot];
    sh[threadIdx.x] = s;
    __syncthreads();
    for (int w = 128; w >= 1; w >>= 1) {
        if ((int)threadIdx.x < w) sh[threadIdx.x] += sh[threadIdx.x + w];
        __syncthreads();
    }
    if (threadIdx.x == 0) out.dprobs[i][k] = (float)sh[0];
}

hipError_t launch_gate_reduce_group(const float* partials, int64_t ntiles, int stride, const GateReduceOut& out,
                                    int nmembers, hipStream_t s) {
    gate_reduce_group_kernel<<<dim3(out.kstride, nmembers), dim3(256), 0, s>>>(partials, ntiles, stride, out);
    return hipGetLastError();
}

hipError_t launch_gate_reduce(const float* partials, int64_t ntiles, int ncand, float* dprobs, hipStream_t s) {
    return launch_gate_reduce_strided(partials, ntiles, ncand, ncand, dprobs, s);
}

hipError_t launch_gate_reduce_strided(const float* partials, int64_t ntiles, int stride, int ncand, float* dprobs,
                                      hipStream_t s) {
    gate_reduce_kernel<<<dim3(ncand), dim3(256), 0, s>>>(partials, ntiles, stride, dprobs);
    return hipGetLastError();
}

}  // namespace vq
