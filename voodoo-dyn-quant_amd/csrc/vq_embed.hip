// Embedding rows straight from the packed candidates: the row-select lookup of
// a gated embedding (reference layers.py:670-750, 753-790) and the Q8_0
// teacher's embedding (training/q8_teacher.py:131-173).
//
// Every supported format stores a weight row as row_groups consecutive
// 256-weight groups, so row `id` of candidate k is the byte span
// [id * row_groups * gb_k, (id + 1) * row_groups * gb_k).  A workgroup takes
// one requested row and a segment of at most kGroupsPerBlock groups of it,
// stages that segment of every candidate it needs into LDS with 16-byte loads,
// and decodes it the way the full-matrix kernels do:
//   mixture:  out = ((0 + p0 W0) + p1 W1) + ..., the mix kernel's arithmetic
//             (fp32, products and sums rounded separately), stored as bf16
//             (the same row of W_eff bit for bit) or as fp32;
//   routed:   out = W_k(r), ggml's exact value, as bf16 or fp32;
//   backward: part[b][k] = <G rows of block b, W_k rows> for a bf16 or fp32 G,
//             reduced over blocks in a fixed order in fp64 (dL/dp_k).
// Row ids (and routes) outside their range give a zero row and a zero
// contribution; the kernels never read outside the candidate buffers.
#include "vq_internal.h"

namespace vq {

namespace {

// LDS bytes reserved for one candidate's segment: up to 15 bytes ahead of the
// segment (kept so every field sits at the same address mod 16 as in global
// memory) plus the segment itself.
__host__ __device__ constexpr int span_cap(int gb) { return (kGroupsPerBlock * gb + 15 + 15) & ~15; }

// Copy [src, src + len) to dst + (src mod 16), dst 16-byte aligned in LDS.
// Whole 16-byte chunks move as direct-to-LDS loads (buffer_load_dwordx4 ...
// lds: lane l of a wave's instruction lands at M0 + 16 l) from the 16-byte
// boundary at or below src (never below the 16-byte aligned buffer that holds
// src), so every candidate's copies are in flight together; the last partial
// chunk moves byte by byte, so nothing past src + len is read.  span_wait()
// waits for this thread's copies.  Returns src mod 16.
__device__ __forceinline__ int stage_span(uint8_t* __restrict__ dst, const uint8_t* __restrict__ src, int len) {
    typedef __attribute__((address_space(3))) void lds_void;
    const int head = (int)(reinterpret_cast<uintptr_t>(src) & 15u);
    const uint8_t* base = src - head;
    const int total = head + len;
    const int nvec = total >> 4;
    const __amdgpu_buffer_rsrc_t rs =
        __builtin_amdgcn_make_buffer_rsrc(const_cast<uint8_t*>(base), (short)0, total, 0x00020000);
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane((int)threadIdx.x >> 6);
    for (int b = 64 * wave; b < nvec; b += (int)blockDim.x)
        if (b + lane < nvec)
            __builtin_amdgcn_raw_ptr_buffer_load_lds(rs, (lds_void*)(dst + 16 * b), 16, 16 * (b + lane), 0, 0, 0);
    const int tail = total & 15;
    if ((int)threadIdx.x < tail) dst[(nvec << 4) + threadIdx.x] = base[(nvec << 4) + threadIdx.x];
    return head;
}

__device__ __forceinline__ void span_wait() { asm volatile("s_waitcnt vmcnt(0)" ::: "memory"); }

struct RowSeg {
    int64_t r;   // requested row (output row)
    int s0;      // first group of the segment
    int ng;      // groups in the segment
};

__device__ __forceinline__ RowSeg row_segment(int nseg, int seg, int gused) {
    RowSeg rs;
    const int64_t b = blockIdx.x;
    rs.r = b / nseg;
    rs.s0 = (int)(b - rs.r * nseg) * seg;
    rs.ng = min(seg, gused - rs.s0);
    return rs;
}

__device__ __forceinline__ void decode8_mix_rt(int qt, const uint8_t* g, int p, float (&w)[8]) {
    switch (qt) {
    case Q8_0: decode8_mix<Q8_0>(g, p, w); break;
    case Q2_K: decode8_mix<Q2_K>(g, p, w); break;
    case Q3_K: decode8_mix<Q3_K>(g, p, w); break;
    case Q4_K: decode8_mix<Q4_K>(g, p, w); break;
    case Q5_K: decode8_mix<Q5_K>(g, p, w); break;
    case Q6_K: decode8_mix<Q6_K>(g, p, w); break;
    default: decode_mix_iq<8>(qt, g, p, w); break;
    }
}

__device__ __forceinline__ float dot8_rt(int qt, const uint8_t* g, int p, const float* v) {
    switch (qt) {
    case Q8_0: return dot_run<Q8_0, 8>(g, p, v);
    case Q2_K: return dot_run<Q2_K, 8>(g, p, v);
    case Q3_K: return dot_run<Q3_K, 8>(g, p, v);
    case Q4_K: return dot_run<Q4_K, 8>(g, p, v);
    case Q5_K: return dot_run<Q5_K, 8>(g, p, v);
    case Q6_K: return dot_run<Q6_K, 8>(g, p, v);
    default: return dot_run_iq<8>(qt, g, p, v);
    }
}

__device__ __forceinline__ void store8(bf16_t* o, const float (&v)[8]) {
    uint4 q;
    q.x = f2bf2(v[0], v[1]);
    q.y = f2bf2(v[2], v[3]);
    q.z = f2bf2(v[4], v[5]);
    q.w = f2bf2(v[6], v[7]);
    *reinterpret_cast<uint4*>(o) = q;
}

__device__ __forceinline__ void store8(float* o, const float (&v)[8]) {
    float4* o4 = reinterpret_cast<float4*>(o);
    o4[0] = make_float4(v[0], v[1], v[2], v[3]);
    o4[1] = make_float4(v[4], v[5], v[6], v[7]);
}

__device__ __forceinline__ void load8(const bf16_t* g, float (&v)[8]) {
    const uint4 q = *reinterpret_cast<const uint4*>(g);
    const uint32_t w[4] = {q.x, q.y, q.z, q.w};
#pragma unroll
    for (int r = 0; r < 4; ++r) {
        v[2 * r] = __uint_as_float(w[r] << 16);
        v[2 * r + 1] = __uint_as_float(w[r] & 0xffff0000u);
    }
}

__device__ __forceinline__ void load8(const float* g, float (&v)[8]) {
    const float4 a = reinterpret_cast<const float4*>(g)[0];
    const float4 b = reinterpret_cast<const float4*>(g)[1];
    v[0] = a.x; v[1] = a.y; v[2] = a.z; v[3] = a.w;
    v[4] = b.x; v[5] = b.y; v[6] = b.z; v[7] = b.w;
}

}  // namespace

template <bool ROUTED, class OUT>
__global__ __launch_bounds__(kStreamThreads) void embed_rows_kernel(CandSet cs, const float* __restrict__ probs,
                                                                    const int64_t* __restrict__ routing,
                                                                    const int64_t* __restrict__ ids, int64_t vocab,
                                                                    int nseg, int seg, int gused, int64_t dim,
                                                                    OUT* __restrict__ out) {
    extern __shared__ __attribute__((aligned(16))) uint8_t lds[];
    __shared__ int sbase[kMaxCand];
    __shared__ float sp[kMaxCand];  // the probabilities, read once per workgroup
    const RowSeg rs = row_segment(nseg, seg, gused);
    const int64_t id = ids[rs.r];
    bool valid = id >= 0 && id < vocab;
    int k0 = 0, k1 = cs.ncand;
    if (!ROUTED && (int)threadIdx.x < cs.ncand) sp[threadIdx.x] = probs[threadIdx.x];
    if constexpr (ROUTED) {
        const int64_t kr = routing[rs.r];
        valid = valid && kr >= 0 && kr < cs.ncand;
        k0 = valid ? (int)kr : 0;
        k1 = k0 + 1;
    }
    if (valid) {
        int off = 0;
        for (int k = k0; k < k1; ++k) {
            const int gb = group_bytes(cs.qtype[k]);
            const uint8_t* src = cs.qbytes[k] + (id * cs.row_groups + rs.s0) * gb;
            const int head = stage_span(lds + off, src, rs.ng * gb);
            if (threadIdx.x == 0) sbase[k] = off + head;
            off += span_cap(gb);
        }
    }
    span_wait();
    __syncthreads();
    const int t = threadIdx.x;
    const int p = 8 * (t & 31);
#pragma unroll
    for (int u = 0; u < kRunsPerThread; ++u) {
        const int j = (t >> 5) + 8 * u;
        if (j >= rs.ng) continue;
        const int64_t col = (int64_t)(rs.s0 + j) * 256 + p;
        if (col >= dim) continue;
        float val[8];
#pragma unroll
        for (int r = 0; r < 8; ++r) val[r] = 0.0f;
        if (valid) {
            if constexpr (ROUTED) {
                const int qt = cs.qtype[k0];
                decode_run_rt<8>(qt, lds + sbase[k0] + j * group_bytes(qt), p, val);
            } else {
                for (int k = 0; k < cs.ncand; ++k) {
                    const int qt = cs.qtype[k];
                    float w[8];
                    decode8_mix_rt(qt, lds + sbase[k] + j * group_bytes(qt), p, w);
                    const float pk = sp[k];
                    {
                        // product and sum rounded separately, as in the mix kernel
#pragma clang fp contract(off)
#pragma unroll
                        for (int r = 0; r < 8; ++r) val[r] = val[r] + pk * w[r];
                    }
                }
            }
        }
        store8(out + rs.r * dim + col, val);
    }
}

// part[b][k] = sum over block b's weights of G[r][c] * W_k[id][c].
template <class GT>
__global__ __launch_bounds__(kStreamThreads) void embed_rows_bwd_kernel(CandSet cs, const int64_t* __restrict__ ids,
                                                                        int64_t vocab, int nseg, int seg, int gused,
                                                                        int64_t dim, const GT* __restrict__ grad,
                                                                        float* __restrict__ partials) {
    extern __shared__ __attribute__((aligned(16))) uint8_t lds[];
    __shared__ int sbase[kMaxCand];
    __shared__ float red[kMaxCand][kStreamThreads / 64];
    const RowSeg rs = row_segment(nseg, seg, gused);
    const int64_t id = ids[rs.r];
    const bool valid = id >= 0 && id < vocab;
    if (valid) {
        int off = 0;
        for (int k = 0; k < cs.ncand; ++k) {
            const int gb = group_bytes(cs.qtype[k]);
            const uint8_t* src = cs.qbytes[k] + (id * cs.row_groups + rs.s0) * gb;
            const int head = stage_span(lds + off, src, rs.ng * gb);
            if (threadIdx.x == 0) sbase[k] = off + head;
            off += span_cap(gb);
        }
    }
    // this thread's gradient values, kept across the candidates
    const int t = threadIdx.x;
    const int p = 8 * (t & 31);
    float v[kRunsPerThread][8];
    bool live[kRunsPerThread];
#pragma unroll
    for (int u = 0; u < kRunsPerThread; ++u) {
        const int j = (t >> 5) + 8 * u;
        const int64_t col = (int64_t)(rs.s0 + j) * 256 + p;
        live[u] = valid && j < rs.ng && col < dim;
#pragma unroll
        for (int r = 0; r < 8; ++r) v[u][r] = 0.0f;
        if (live[u]) load8(grad + rs.r * dim + col, v[u]);
    }
    span_wait();
    __syncthreads();
    const int wave = t >> 6;
    for (int k = 0; k < cs.ncand; ++k) {
        const int qt = cs.qtype[k];
        const int gb = group_bytes(qt);
        float a = 0.0f;
#pragma unroll
        for (int u = 0; u < kRunsPerThread; ++u) {
            if (live[u]) a += dot8_rt(qt, lds + sbase[k] + ((t >> 5) + 8 * u) * gb, p, v[u]);
        }
#pragma unroll
        for (int m = 32; m >= 1; m >>= 1) a += __shfl_xor(a, m, 64);
        if ((t & 63) == 0) red[k][wave] = a;
    }
    __syncthreads();
    if (t < cs.ncand) {
        float s = 0.0f;
#pragma unroll
        for (int w = 0; w < kStreamThreads / 64; ++w) s += red[t][w];
        partials[(int64_t)blockIdx.x * cs.ncand + t] = s;
    }
}

EmbedPlan embed_plan(int64_t nids, int64_t dim) {
    EmbedPlan pl;
    pl.gused = (int)((dim + 255) / 256);
    pl.nseg = (pl.gused + kGroupsPerBlock - 1) / kGroupsPerBlock;
    pl.seg = pl.nseg > 0 ? (pl.gused + pl.nseg - 1) / pl.nseg : 0;
    pl.blocks = nids * pl.nseg;
    return pl;
}

static size_t embed_lds(const CandSet& cs, bool routed) {
    size_t lds = 0;
    for (int k = 0; k < cs.ncand; ++k) {
        const size_t c = span_cap(group_bytes(cs.qtype[k]));
        lds = routed ? (c > lds ? c : lds) : lds + c;
    }
    return lds;
}

template <class OUT>
static hipError_t embed_rows_t(const CandSet& cs, const float* probs, const int64_t* routing, const int64_t* ids,
                               int64_t vocab, int64_t dim, const EmbedPlan& pl, OUT* out, hipStream_t s) {
    const dim3 grid((unsigned)pl.blocks);
    const size_t lds = embed_lds(cs, routing != nullptr);
    const hipError_t e = allow_dynamic_lds(
        routing ? (const void*)embed_rows_kernel<true, OUT> : (const void*)embed_rows_kernel<false, OUT>, lds);
    if (e != hipSuccess) return e;
    if (routing)
        embed_rows_kernel<true, OUT><<<grid, kStreamThreads, lds, s>>>(cs, probs, routing, ids, vocab, pl.nseg, pl.seg,
                                                                       pl.gused, dim, out);
    else
        embed_rows_kernel<false, OUT><<<grid, kStreamThreads, lds, s>>>(cs, probs, nullptr, ids, vocab, pl.nseg,
                                                                        pl.seg, pl.gused, dim, out);
    return hipSuccess;
}

hipError_t launch_embed_rows(const CandSet& cs, const float* probs, const int64_t* routing, const int64_t* ids,
                             int64_t nids, int64_t vocab, int64_t dim, void* out, bool out_f32, hipStream_t s) {
    const EmbedPlan pl = embed_plan(nids, dim);
    if (pl.blocks <= 0) return hipSuccess;
    const hipError_t e = out_f32 ? embed_rows_t(cs, probs, routing, ids, vocab, dim, pl, static_cast<float*>(out), s)
                                 : embed_rows_t(cs, probs, routing, ids, vocab, dim, pl, static_cast<bf16_t*>(out), s);
    if (e != hipSuccess) return e;
    return hipGetLastError();
}

hipError_t launch_embed_rows_bwd(const CandSet& cs, const int64_t* ids, int64_t nids, int64_t vocab, int64_t dim,
                                 const void* grad, bool grad_f32, float* partials, float* dprobs, hipStream_t s) {
    const EmbedPlan pl = embed_plan(nids, dim);
    if (pl.blocks <= 0) {
        // no rows: dL/dp is zero (written by a kernel, not a memset, so the call can be captured)
        return launch_gate_reduce(partials, 0, cs.ncand, dprobs, s);
    }
    const dim3 grid((unsigned)pl.blocks);
    const size_t lds = embed_lds(cs, false);
    const hipError_t ea = allow_dynamic_lds(
        grad_f32 ? (const void*)embed_rows_bwd_kernel<float> : (const void*)embed_rows_bwd_kernel<bf16_t>, lds);
    if (ea != hipSuccess) return ea;
    if (grad_f32)
        embed_rows_bwd_kernel<float><<<grid, kStreamThreads, lds, s>>>(cs, ids, vocab, pl.nseg, pl.seg, pl.gused,
                                                                       dim, static_cast<const float*>(grad), partials);
    else
        embed_rows_bwd_kernel<bf16_t><<<grid, kStreamThreads, lds, s>>>(cs, ids, vocab, pl.nseg, pl.seg, pl.gused,
                                                                        dim, static_cast<const bf16_t*>(grad),
                                                                        partials);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return e;
    return launch_gate_reduce(partials, pl.blocks, cs.ncand, dprobs, s);
}

}  // namespace vq
