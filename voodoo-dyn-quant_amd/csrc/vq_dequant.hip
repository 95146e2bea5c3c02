// HBM-bound streaming kernels: GGUF block dequantisation to fp32 (bit-exact
// to ggml's dequantize_row_*) and the softmax mixture of K candidates to a bf16
// W_eff (bit-exact to the fp32 k-ordered mixture of the reference's
// _MixedWeightFunction.forward, voodoo_quant/layers.py:336-352, followed by
// the source-dtype cast).
//
// Data layout: a candidate is N rows of D_pad/256 groups; every format packs a
// row's groups contiguously and rows back to back, so the flattened group index
// g covers weights [256 g, 256 g + 256) of the row-major [N][D_pad] matrix.
// A workgroup streams consecutive groups (of every candidate, for the mix)
// into LDS with 16-byte direct-to-LDS loads (the byte range of 16 groups is a
// multiple of 16 for every format), then each thread decodes runs of 8
// weights from LDS and writes them with 16-byte stores.
#include <mutex>
#include <unordered_map>

#include "vq_internal.h"

namespace vq {

hipError_t allow_dynamic_lds(const void* kern, size_t lds) {
    if (lds <= 64 * 1024) return hipSuccess;
    static std::mutex mu;
    static std::unordered_map<const void*, size_t> granted;  // largest size set per kernel
    std::lock_guard<std::mutex> lock(mu);
    auto it = granted.find(kern);
    if (it != granted.end() && it->second >= lds) return hipSuccess;
    // exactly the size asked for: the kernel's static LDS counts against the same 160 KiB
    hipError_t e = hipFuncSetAttribute(kern, hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds);
    if (e != hipSuccess) {
        (void)hipGetLastError();
        return e;
    }
    granted[kern] = lds;
    return hipSuccess;
}

// Copy `len` bytes at `src` (16-byte aligned) to LDS `dst` (16-byte aligned)
// with direct-to-LDS loads (buffer_load_dwordx4 ... lds: lane l of a wave's
// instruction lands at M0 + 16 l), so a thread's loads of every candidate are
// in flight together and no register holds them; stage_wait() then waits for
// them before the workgroup synchronises.  Whole 16-byte chunks only: lanes
// past them are masked off, and the last `len % 16` bytes are copied by
// ordinary byte loads.
__device__ __forceinline__ void stage_bytes(uint8_t* __restrict__ dst, const uint8_t* __restrict__ src, int len) {
    typedef __attribute__((address_space(3))) void lds_void;
    const int nvec = len >> 4;
    const __amdgpu_buffer_rsrc_t rs =
        __builtin_amdgcn_make_buffer_rsrc(const_cast<uint8_t*>(src), (short)0, len, 0x00020000);
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane((int)threadIdx.x >> 6);
    const int stride = (int)blockDim.x;  // a multiple of 64
    for (int base = 64 * wave; base < nvec; base += stride) {
        // cache policy 2: streamed once (non-temporal)
        if (base + lane < nvec)
            __builtin_amdgcn_raw_ptr_buffer_load_lds(rs, (lds_void*)(dst + 16 * base), 16, 16 * (base + lane), 0, 0,
                                                     2);
    }
    const int tail = len & 15;
    if ((int)threadIdx.x < tail) dst[(nvec << 4) + threadIdx.x] = src[(nvec << 4) + threadIdx.x];
}

// This thread's stage_bytes copies have landed in LDS (a __syncthreads()
// after it makes everyone's visible).
__device__ __forceinline__ void stage_wait() { asm volatile("s_waitcnt vmcnt(0)" ::: "memory"); }

// Output placement of one run of 8 weights: lanes 2k and 2k + 1 of a wave
// decode run k (weights 8k .. 8k + 7) of two neighbouring groups A and B, and
// swap halves, so that each fp32 store instruction writes one whole group
// (lane l: weights 4l .. 4l + 3, 1 KB contiguous per instruction) straight from
// registers.  Against writing each thread's run as two 16-byte halves 32 bytes
// apart (each instruction covering half of a 2 KB span) this is the 1 KB
// pattern of an LDS round trip without the LDS buffer and its barrier, which
// leaves a workgroup's LDS to its staged bytes (and an IQ format's code book).
template <class OUT>
__device__ __forceinline__ void store_run(OUT* __restrict__ out, int64_t group_a, const float (&y)[8], int lane) {
    if constexpr (sizeof(OUT) == 4) {
        const bool odd = lane & 1;
        float4 send = odd ? make_float4(y[0], y[1], y[2], y[3]) : make_float4(y[4], y[5], y[6], y[7]);
        float4 recv;
        recv.x = __shfl_xor(send.x, 1);
        recv.y = __shfl_xor(send.y, 1);
        recv.z = __shfl_xor(send.z, 1);
        recv.w = __shfl_xor(send.w, 1);
        const float4 mine_lo = make_float4(y[0], y[1], y[2], y[3]), mine_hi = make_float4(y[4], y[5], y[6], y[7]);
        const float4 a = odd ? recv : mine_lo;  // group A, weights 4 lane .. + 3
        const float4 b = odd ? mine_hi : recv;  // group B, weights 4 lane .. + 3
        reinterpret_cast<float4*>(out + group_a * 256)[lane] = a;
        reinterpret_cast<float4*>(out + (group_a + 1) * 256)[lane] = b;
    } else {
        // bf16: a lane's 8 weights are 16 contiguous bytes already
        uint4 v;
        v.x = f2bf2(y[0], y[1]);
        v.y = f2bf2(y[2], y[3]);
        v.z = f2bf2(y[4], y[5]);
        v.w = f2bf2(y[6], y[7]);
        *reinterpret_cast<uint4*>(out + (group_a + (lane & 1)) * 256 + 8 * (lane >> 1)) = v;
    }
}

// Runs of 8 weights per thread, per format: a workgroup of kStreamThreads
// threads stages and decodes 8 * RUNS groups.  The bytes one workgroup keeps
// in flight set the rate (the fp32 output stream is the same 235 MB for every
// format at 4096 x 14336, and a write-only stream of it runs at 6.4-6.5 TB/s
// on MI355X).  Measured there, fraction of 8 TB/s at 16 / 32 / 64 / 128 / 256
// groups per workgroup: Q2_K 0.66 / 0.73 / 0.77 / 0.79 / 0.72, Q3_K 0.67 /
// 0.71 / 0.74 / 0.71-0.76 / 0.64, the code-book IQ formats 0.55-0.61 /
// 0.58-0.67 / 0.69-0.76 / 0.75-0.78 / 0.70-0.76; Q4_K 0.76 / 0.79 / 0.77,
// Q5_K and Q6_K best at 32 (0.76, 0.73), IQ4_XS at 32 (0.80), Q8_0 (272
// bytes per group) at 16 (0.79 against 0.77 at 32).
__host__ __device__ constexpr int dequant_runs(int qt) {
    return qt == Q8_0 ? 2 : (qt == Q4_K || qt == Q5_K || qt == Q6_K || qt == IQ4_XS) ? 4 : 16;
}

// Formats whose code book is copied to LDS by the workgroup (the lookups then
// read LDS instead of gathering 64 scattered words per wave instruction
// through L1): measured faster for IQ3_XXS (1 KB book) and IQ3_S (2 KB) at 16
// and 32 groups per workgroup (0.59 -> 0.67-0.69 at 16), level at 128, and
// slower for the larger books (IQ2_S 8 KB, IQ1_S / IQ1_M 16 KB: the copy and
// the LDS it takes cost more than the lookups save) and for IQ2_XXS / IQ2_XS.
__host__ __device__ constexpr bool dequant_book_in_lds(int qt) { return qt == IQ3_XXS || qt == IQ3_S; }

// OUT = float: ggml's fp32 values bit for bit; OUT = bf16_t: those values
// rounded to bf16 (torch's rounding), the source-dtype candidate the
// reference's lazy path holds.  Wave w decodes groups 2 (w + 4 u) and
// 2 (w + 4 u) + 1, u < RUNS.  A partial last workgroup with an odd group
// count decodes the group past its end from stale LDS (every code-book index
// stays inside its book) and stores nothing of it.
template <int QT, class OUT, int RUNS, class Books>
__device__ __forceinline__ void dequant_groups(const uint8_t* __restrict__ lds, OUT* __restrict__ out, int64_t g0,
                                               int ng, const Books& bk) {
    constexpr int GB = group_bytes(QT);
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
#pragma unroll
    for (int u = 0; u < RUNS; ++u) {
        const int pair = wave + (kStreamThreads / 64) * u;  // groups 2 pair, 2 pair + 1
        const int j = 2 * pair + (lane & 1);
        if (2 * pair < ng) {
            float y[8];
            if constexpr (is_iq(QT))
                decode_run_iq<8>(QT, lds + j * GB, 8 * (lane >> 1), y, bk);
            else
                decode_run<QT, 8>(lds + j * GB, 8 * (lane >> 1), y);
            if (2 * pair + 1 < ng) {
                store_run<OUT>(out, g0 + 2 * pair, y, lane);
            } else {  // the last group of an odd count: group A only
                if constexpr (sizeof(OUT) == 4) {
                    const bool odd = lane & 1;
                    float4 send = odd ? make_float4(y[0], y[1], y[2], y[3]) : make_float4(y[4], y[5], y[6], y[7]);
                    float4 recv;
                    recv.x = __shfl_xor(send.x, 1);
                    recv.y = __shfl_xor(send.y, 1);
                    recv.z = __shfl_xor(send.z, 1);
                    recv.w = __shfl_xor(send.w, 1);
                    const float4 a = odd ? recv : make_float4(y[0], y[1], y[2], y[3]);
                    reinterpret_cast<float4*>(out + (g0 + 2 * pair) * 256)[lane] = a;
                } else if (!(lane & 1)) {
                    uint4 v;
                    v.x = f2bf2(y[0], y[1]);
                    v.y = f2bf2(y[2], y[3]);
                    v.z = f2bf2(y[4], y[5]);
                    v.w = f2bf2(y[6], y[7]);
                    *reinterpret_cast<uint4*>(out + (g0 + 2 * pair) * 256 + 8 * (lane >> 1)) = v;
                }
            }
        }
    }
}

template <int QT, class OUT>
__global__ __launch_bounds__(kStreamThreads) void dequant_kernel(const uint8_t* __restrict__ q,
                                                                 OUT* __restrict__ out, int64_t ngroups) {
    constexpr int GB = group_bytes(QT);
    constexpr int RUNS = dequant_runs(QT);
    constexpr int GPB = kStreamThreads / 32 * RUNS;  // groups per workgroup
    constexpr int BOOK = dequant_book_in_lds(QT) ? iq_book_bytes(QT) : 16;
    static_assert(BOOK % 16 == 0, "a code book of whole 16-byte chunks");
    __shared__ __attribute__((aligned(16))) uint8_t book[BOOK];
    __shared__ __attribute__((aligned(16))) uint8_t lds[GPB * GB + 16];
    const int64_t g0 = (int64_t)blockIdx.x * GPB;
    const int ng = (int)min<int64_t>(GPB, ngroups - g0);
    if constexpr (dequant_book_in_lds(QT)) stage_bytes(book, iq_book_src(QT), BOOK);
    stage_bytes(lds, q + g0 * GB, ng * GB);
    stage_wait();
    __syncthreads();
    if constexpr (dequant_book_in_lds(QT))
        dequant_groups<QT, OUT, RUNS>(lds, out, g0, ng, LdsBook{(const __attribute__((address_space(3))) uint8_t*)book});
    else
        dequant_groups<QT, OUT, RUNS>(lds, out, g0, ng, GlobalBooks());
}

template <int QT, class OUT>
static void launch_dequant_qt(const uint8_t* q, OUT* out, int64_t ngroups, hipStream_t s) {
    constexpr int GPB = kStreamThreads / 32 * dequant_runs(QT);
    const dim3 grid((unsigned)((ngroups + GPB - 1) / GPB));
    dequant_kernel<QT, OUT><<<grid, kStreamThreads, 0, s>>>(q, out, ngroups);
}

template <class OUT>
static hipError_t launch_dequant_t(int qtype, const uint8_t* q, OUT* out, int64_t ngroups, hipStream_t s) {
    if (ngroups <= 0) return hipSuccess;
    switch (qtype) {
    case Q8_0: launch_dequant_qt<Q8_0, OUT>(q, out, ngroups, s); break;
    case Q2_K: launch_dequant_qt<Q2_K, OUT>(q, out, ngroups, s); break;
    case Q3_K: launch_dequant_qt<Q3_K, OUT>(q, out, ngroups, s); break;
    case Q4_K: launch_dequant_qt<Q4_K, OUT>(q, out, ngroups, s); break;
    case Q5_K: launch_dequant_qt<Q5_K, OUT>(q, out, ngroups, s); break;
    case Q6_K: launch_dequant_qt<Q6_K, OUT>(q, out, ngroups, s); break;
    case IQ2_XXS: launch_dequant_qt<IQ2_XXS, OUT>(q, out, ngroups, s); break;
    case IQ2_XS: launch_dequant_qt<IQ2_XS, OUT>(q, out, ngroups, s); break;
    case IQ2_S: launch_dequant_qt<IQ2_S, OUT>(q, out, ngroups, s); break;
    case IQ3_XXS: launch_dequant_qt<IQ3_XXS, OUT>(q, out, ngroups, s); break;
    case IQ3_S: launch_dequant_qt<IQ3_S, OUT>(q, out, ngroups, s); break;
    case IQ1_S: launch_dequant_qt<IQ1_S, OUT>(q, out, ngroups, s); break;
    case IQ1_M: launch_dequant_qt<IQ1_M, OUT>(q, out, ngroups, s); break;
    case IQ4_XS: launch_dequant_qt<IQ4_XS, OUT>(q, out, ngroups, s); break;
    default: return hipErrorInvalidValue;
    }
    return hipGetLastError();
}

hipError_t launch_dequant(int qtype, const uint8_t* q, float* out, int64_t ngroups, hipStream_t s) {
    return launch_dequant_t<float>(qtype, q, out, ngroups, s);
}

hipError_t launch_dequant_bf16(int qtype, const uint8_t* q, bf16_t* out, int64_t ngroups, hipStream_t s) {
    return launch_dequant_t<bf16_t>(qtype, q, out, ngroups, s);
}

// ---------------------------------------------------------------------------
// Mixture: W_eff = bf16( (((0 + p0 W0) + p1 W1) + ...) ) with every product and
// sum rounded separately, exactly as the fp32 torch ops of the reference.
// One launch mixes up to kMaxSets tensors (the members of a stacked
// product); a workgroup covers RUNS * 16 groups of one tensor (launched with
// RUNS = 1).  A thread takes 16 consecutive weights of a group per run (one
// scale decode per candidate and run).
// ---------------------------------------------------------------------------
struct MixPlan {
    int nsets;
    CandSet sets[kMaxSets];
    const float* probs[kMaxSets];
    bf16_t* out[kMaxSets];
    int64_t ngroups[kMaxSets];
    int64_t block0[kMaxSets + 1];  // first workgroup of each set
    // per set and candidate: bytes per group, and where the candidate's
    // staged groups start in LDS (filled on the host)
    int gbytes[kMaxSets][kMaxCand];
    int lds_off[kMaxSets][kMaxCand];
};

constexpr int kMixRun = 16;                                     // weights per thread and run
constexpr int kMixGroupsPerPass = kStreamThreads * kMixRun / 256;  // 16

// IQ: the sets may hold IQ formats (the K-quant-only instantiation keeps its
// lower register count and occupancy).
template <int RUNS, bool IQ>
__global__ __launch_bounds__(kStreamThreads) void mix_kernel(MixPlan mp) {
    extern __shared__ __attribute__((aligned(16))) uint8_t lds[];
    constexpr int GPB = kMixGroupsPerPass * RUNS;  // groups per workgroup
    int si = 0;
#pragma unroll
    for (int q = 1; q < kMaxSets; ++q)
        if (q < mp.nsets && (int64_t)blockIdx.x >= mp.block0[q]) si = q;
    const CandSet& cs = mp.sets[si];
    const int64_t g0 = ((int64_t)blockIdx.x - mp.block0[si]) * GPB;
    const int ng = (int)min<int64_t>(GPB, mp.ngroups[si] - g0);
    for (int k = 0; k < cs.ncand; ++k) {
        const int gb = mp.gbytes[si][k];
        stage_bytes(lds + mp.lds_off[si][k], cs.qbytes[k] + g0 * gb, ng * gb);
    }
    // the probabilities, read once per workgroup (one short LDS read per
    // candidate and run instead of a global load in the loop)
    __shared__ float sp[kMaxCand];
    if ((int)threadIdx.x < cs.ncand) sp[threadIdx.x] = mp.probs[si][threadIdx.x];
    stage_wait();
    __syncthreads();
    const int t = threadIdx.x;
    bf16_t* w_eff = mp.out[si];
    const int p = kMixRun * (t & 15);
#pragma unroll
    for (int u = 0; u < RUNS; ++u) {
        const int j = (t >> 4) + kMixGroupsPerPass * u;
        if (j >= ng) continue;
        float mixed[kMixRun];
#pragma unroll
        for (int r = 0; r < kMixRun; ++r) mixed[r] = 0.0f;
        for (int k = 0; k < cs.ncand; ++k) {
            const int qt = cs.qtype[k];
            float w[kMixRun];
            const uint8_t* g = lds + mp.lds_off[si][k] + j * mp.gbytes[si][k];
            switch (qt) {
            case Q8_0: decode_mix<Q8_0, kMixRun>(g, p, w); break;
            case Q2_K: decode_mix<Q2_K, kMixRun>(g, p, w); break;
            case Q3_K: decode_mix<Q3_K, kMixRun>(g, p, w); break;
            case Q4_K: decode_mix<Q4_K, kMixRun>(g, p, w); break;
            case Q5_K: decode_mix<Q5_K, kMixRun>(g, p, w); break;
            case Q6_K: decode_mix<Q6_K, kMixRun>(g, p, w); break;
            default:
                if constexpr (IQ)
                    decode_mix_iq<kMixRun>(qt, g, p, w);
                else
                    decode_mix<Q6_K, kMixRun>(g, p, w);
                break;
            }
            const float pk = sp[k];
            {
                // product and sum rounded separately, like the two torch ops
#pragma clang fp contract(off)
#pragma unroll
                for (int r = 0; r < kMixRun; ++r) mixed[r] = mixed[r] + pk * w[r];
            }
        }
        uint4 v[2];
#pragma unroll
        for (int h = 0; h < 2; ++h) {
            v[h].x = f2bf2(mixed[8 * h + 0], mixed[8 * h + 1]);
            v[h].y = f2bf2(mixed[8 * h + 2], mixed[8 * h + 3]);
            v[h].z = f2bf2(mixed[8 * h + 4], mixed[8 * h + 5]);
            v[h].w = f2bf2(mixed[8 * h + 6], mixed[8 * h + 7]);
        }
        uint4* o = reinterpret_cast<uint4*>(w_eff + (g0 + j) * 256 + p);
        o[0] = v[0];
        o[1] = v[1];
    }
}

hipError_t launch_mix_sets(int nsets, const CandSet* sets, const float* const* probs, bf16_t* const* out,
                           const int64_t* ngroups, hipStream_t s) {
    MixPlan mp{};
    mp.nsets = nsets;
    // 16 groups per workgroup: with the staging copies all in flight at once,
    // 32- and 64-group workgroups were 13% and 40% slower at 17408 x 5120
    // (K = 6), and slower at 1536 x 1024 and 6144 x 1024 too
    const int gpb = kMixGroupsPerPass;
    size_t lds = 0;
    int64_t blocks = 0;
    for (int i = 0; i < nsets; ++i) {
        mp.sets[i] = sets[i];
        mp.probs[i] = probs[i];
        mp.out[i] = out[i];
        mp.ngroups[i] = ngroups[i];
        mp.block0[i] = blocks;
        blocks += (ngroups[i] + gpb - 1) / gpb;
        size_t l = 0;
        for (int k = 0; k < sets[i].ncand; ++k) {
            mp.gbytes[i][k] = group_bytes(sets[i].qtype[k]);
            mp.lds_off[i][k] = (int)l;
            l += (gpb * mp.gbytes[i][k] + 15) & ~15;
        }
        lds = l > lds ? l : lds;
    }
    mp.block0[nsets] = blocks;
    if (blocks <= 0) return hipSuccess;
    bool iq = false;
    for (int i = 0; i < nsets; ++i) iq = iq || any_iq(sets[i]);
    // 16 Q8_0 candidates stage 68 KiB
    const hipError_t e = allow_dynamic_lds(iq ? (const void*)mix_kernel<1, true> : (const void*)mix_kernel<1, false>, lds);
    if (e != hipSuccess) return e;
    if (iq)
        mix_kernel<1, true><<<dim3((unsigned)blocks), kStreamThreads, lds, s>>>(mp);
    else
        mix_kernel<1, false><<<dim3((unsigned)blocks), kStreamThreads, lds, s>>>(mp);
    return hipGetLastError();
}

hipError_t launch_mix(const CandSet& cs, const float* probs, bf16_t* w_eff, int64_t ngroups, hipStream_t s) {
    return launch_mix_sets(1, &cs, &probs, &w_eff, &ngroups, s);
}

// ---------------------------------------------------------------------------
// Gate dots from dW parts (the EPI_PARTS gate product):
//   partials[block][set * kstride + k] = sum over the block's weights of
//   dW[n][d] * W_k[n][d],
// dW[n][d] the fp32 sum, in part order, of the parts
//   dwp[(tm * tiles_j + tn) * parts + part][n % 256][d % 256],
// tm = d / 256, tn = n / 256, n counted over the stacked members.  A
// workgroup takes 16 consecutive groups (row, 256 weights) of one member and
// stages every candidate's bytes for them in LDS as the mix does; a thread
// takes 16 consecutive weights of one group.  Weights past D have no
// gradient.  The block sums are reduced in a fixed order (launch_gate_reduce*).
// ---------------------------------------------------------------------------
struct GateDotPlan {
    int nsets, kstride, parts, tiles_j, dlimit;
    int64_t row_groups;
    const float* dwp;
    float* partials;
    CandSet sets[kMaxSets];
    int set_j0[kMaxSets + 1];
    int64_t ngroups[kMaxSets];
    int64_t block0[kMaxSets + 1];
    int gbytes[kMaxSets][kMaxCand];
    int lds_off[kMaxSets][kMaxCand];
};

template <bool IQ>
__global__ __launch_bounds__(kStreamThreads) void gate_dot_kernel(GateDotPlan gp) {
    extern __shared__ __attribute__((aligned(16))) uint8_t lds[];
    __shared__ float red[kStreamThreads / 64][kMaxCand];
    int si = 0;
#pragma unroll
    for (int q = 1; q < kMaxSets; ++q)
        if (q < gp.nsets && (int64_t)blockIdx.x >= gp.block0[q]) si = q;
    const CandSet& cs = gp.sets[si];
    const int64_t g0 = ((int64_t)blockIdx.x - gp.block0[si]) * kMixGroupsPerPass;
    const int ng = (int)min<int64_t>(kMixGroupsPerPass, gp.ngroups[si] - g0);
    for (int k = 0; k < cs.ncand; ++k) {
        const int gb = gp.gbytes[si][k];
        stage_bytes(lds + gp.lds_off[si][k], cs.qbytes[k] + g0 * gb, ng * gb);
    }
    // this thread's 16 weights of dW, summed over the parts while the copies fly
    const int t = threadIdx.x, j = t >> 4, p = kMixRun * (t & 15);
    float v[kMixRun];
#pragma unroll
    for (int r = 0; r < kMixRun; ++r) v[r] = 0.0f;
    if (j < ng) {
        const int64_t gi = g0 + j;
        const int grp = (int)(gi % gp.row_groups);
        const int d0 = grp * 256 + p;
        if (d0 < gp.dlimit) {
            const int64_t n = gp.set_j0[si] + gi / gp.row_groups;
            const float4* src = reinterpret_cast<const float4*>(
                gp.dwp + ((int64_t)grp * gp.tiles_j + n / 256) * gp.parts * 65536 + (n % 256) * 256 + p);
            // every part's loads in flight before the first add (one wave per
            // SIMD: a load-add loop would wait out one memory latency per part)
            float4 q[kMaxGateParts][kMixRun / 4];
#pragma unroll
            for (int part = 0; part < kMaxGateParts; ++part)
                if (part < gp.parts)
#pragma unroll
                    for (int h = 0; h < kMixRun / 4; ++h) q[part][h] = src[part * 16384 + h];
#pragma unroll
            for (int part = 0; part < kMaxGateParts; ++part)
                if (part < gp.parts)
#pragma unroll
                    for (int h = 0; h < kMixRun / 4; ++h) {
                        v[4 * h] += q[part][h].x;
                        v[4 * h + 1] += q[part][h].y;
                        v[4 * h + 2] += q[part][h].z;
                        v[4 * h + 3] += q[part][h].w;
                    }
#pragma unroll
            for (int r = 0; r < kMixRun; ++r)
                if (d0 + r >= gp.dlimit) v[r] = 0.0f;
        }
    }
    stage_wait();
    __syncthreads();
    const int lane = t & 63, wave = t >> 6;
    for (int k = 0; k < cs.ncand; ++k) {
        float dot = 0.0f;
        if (j < ng) {
            const int qt = cs.qtype[k];
            const uint8_t* g = lds + gp.lds_off[si][k] + j * gp.gbytes[si][k];
            switch (qt) {
            case Q8_0: dot = dot_run<Q8_0, kMixRun>(g, p, v); break;
            case Q2_K: dot = dot_run<Q2_K, kMixRun>(g, p, v); break;
            case Q3_K: dot = dot_run<Q3_K, kMixRun>(g, p, v); break;
            case Q4_K: dot = dot_run<Q4_K, kMixRun>(g, p, v); break;
            case Q5_K: dot = dot_run<Q5_K, kMixRun>(g, p, v); break;
            case Q6_K: dot = dot_run<Q6_K, kMixRun>(g, p, v); break;
            default:
                if constexpr (IQ)
                    dot = dot_run_iq<kMixRun>(qt, g, p, v);
                else
                    dot = dot_run<Q6_K, kMixRun>(g, p, v);
                break;
            }
        }
#pragma unroll
        for (int off = 32; off >= 1; off >>= 1) dot += __shfl_xor(dot, off);
        if (lane == 0) red[wave][k] = dot;
    }
    __syncthreads();
    // this block's slots of every member: its own sums, zeros for the others
    const int nslot = gp.nsets * gp.kstride;
    if (t < nslot) {
        const int k = t - si * gp.kstride;
        float sum = 0.0f;
        if (k >= 0 && k < cs.ncand)
            for (int w = 0; w < kStreamThreads / 64; ++w) sum += red[w][k];
        gp.partials[(int64_t)blockIdx.x * nslot + t] = sum;
    }
}

int64_t gate_dot_blocks(int nsets, const int64_t* n, int64_t row_groups) {
    int64_t b = 0;
    for (int i = 0; i < nsets; ++i) b += (n[i] * row_groups + kMixGroupsPerPass - 1) / kMixGroupsPerPass;
    return b;
}

hipError_t launch_gate_dot(const CandGroup& cg, int N, int D, const float* dwp, int parts, float* partials,
                           hipStream_t s) {
    if (cg.nsets < 1 || cg.nsets > kMaxSets || cg.nsets * cg.kstride > kStreamThreads || parts < 1 ||
        parts > kMaxGateParts)
        return hipErrorInvalidValue;
    GateDotPlan gp{};
    gp.nsets = cg.nsets;
    gp.kstride = cg.kstride;
    gp.parts = parts;
    gp.tiles_j = (N + 255) / 256;
    gp.dlimit = D;
    gp.row_groups = cg.sets[0].row_groups;
    gp.dwp = dwp;
    gp.partials = partials;
    size_t lds = 0;
    int64_t blocks = 0;
    bool iq = false;
    for (int i = 0; i < cg.nsets; ++i) {
        if (cg.sets[i].row_groups != gp.row_groups || (int64_t)(D + 255) / 256 > gp.row_groups)
            return hipErrorInvalidValue;
        gp.sets[i] = cg.sets[i];
        gp.set_j0[i] = cg.set_j0[i];
        gp.ngroups[i] = (int64_t)(cg.set_j0[i + 1] - cg.set_j0[i]) * gp.row_groups;
        gp.block0[i] = blocks;
        blocks += (gp.ngroups[i] + kMixGroupsPerPass - 1) / kMixGroupsPerPass;
        size_t l = 0;
        for (int k = 0; k < cg.sets[i].ncand; ++k) {
            gp.gbytes[i][k] = group_bytes(cg.sets[i].qtype[k]);
            gp.lds_off[i][k] = (int)l;
            l += (kMixGroupsPerPass * gp.gbytes[i][k] + 15) & ~15;
        }
        lds = l > lds ? l : lds;
        iq = iq || any_iq(cg.sets[i]);
    }
    gp.set_j0[cg.nsets] = cg.set_j0[cg.nsets];
    gp.block0[cg.nsets] = blocks;
    if (blocks <= 0) return hipSuccess;
    const void* kern = iq ? (const void*)gate_dot_kernel<true> : (const void*)gate_dot_kernel<false>;
    const hipError_t e = allow_dynamic_lds(kern, lds);
    if (e != hipSuccess) return e;
    if (iq)
        gate_dot_kernel<true><<<dim3((unsigned)blocks), kStreamThreads, lds, s>>>(gp);
    else
        gate_dot_kernel<false><<<dim3((unsigned)blocks), kStreamThreads, lds, s>>>(gp);
    return hipGetLastError();
}

}  // namespace vq
