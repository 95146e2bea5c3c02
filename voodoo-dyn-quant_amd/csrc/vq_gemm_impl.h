// bf16 MFMA GEMM machinery of the gated Linear on gfx950
// (v_mfma_f32_32x32x16_bf16).  Included by vq_gemm.hip, which instantiates
// the tile configurations.
//
// One kernel template computes C[i][j] = sum_k A[i][k] * B[j][k] with both
// operands copied global -> LDS by direct-to-LDS buffer loads into XOR-
// swizzled stages, then read as MFMA fragments (each lane holds 8
// consecutive k of one row):
//   DmaKS - the source has k contiguous (row-major [rows][K]); fragments
//           with ds_read_b128;
//   DmaNS - the source is [K][rows] (rows contiguous), kept in that
//           orientation; fragments with ds_read_b64_tr_b16.
// The three products of the path:
//   forward  Y[m][n]  = sum_d X[m][d] W[n][d]        A=X (KS), B=W (KS)
//   dX       dX[m][d] = sum_n dY[m][n] W[n][d]       A=dY (KS), B=W (NS)
//   gate     dW[d][n] = sum_m X[m][d] dY[m][n]       A=X (NS), B=dY (NS)
// The gate product never reaches global memory: its epilogue keeps the fp32
// tile in the accumulators, stages each candidate's bytes for the tile into
// LDS (reusing the main-loop buffers) and dots the exactly decoded weights
// against it, writing one partial per candidate per work item.  <dW, W_k> is linear in dW, so the M reduction may also be split
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

// ---------------------------------------------------------------- direct-to-LDS loaders
// buffer_load_dwordx4 ... lds: lane l of one wave instruction writes its 16
// bytes at M0 + 16 l, so one instruction fills 64 consecutive LDS chunks and
// no register ever holds the tile.  Lanes on rows or k past the matrix use
// an out-of-range offset and write zeros without touching memory.  A lane's offset depends only on (instruction,
// wave, lane) and the tile origin, so offsets are computed once per work
// item and the k origin moves the descriptor base.
typedef __attribute__((address_space(3))) void lds_void_t;

// K-major tiles: a tile row keeps its CPR = BK/8 data chunks, no padding,
// and chunk c of row r sits in slot c ^ sw(r) of that row.  The copy fills
// LDS slots in order (lane l of an instruction writes slot M0/16 + l), so a
// lane fetches the global chunk its slot holds; a fragment read addresses the
// slot of its chunk.  sw spreads the 8 (16) rows one ds_read_b128 pass serves
// over distinct 16-byte bank groups with 32 (64) banks of 4 bytes: for CPR = 8,
// rows r and r + 8 differ through r >> 3; for CPR = 4 (64-byte rows, two rows
// per 128 bytes), the rows of one parity within 8, and the rows of one residue
// mod 4 within 16, take distinct slots.  Against a layout padded by one chunk
// per row the stage is 1/9 (BK 64) smaller, and no copy lane writes padding.
template <int ROWS, int BK, int THREADS>
struct DmaKS {
    static constexpr bool kDma = true;
    static constexpr int kPerm = 0;
    static constexpr int kFragReads = 1;
    static constexpr int CPR = BK / 8;
    static_assert(CPR == 4 || CPR == 8, "BK 32 or 64");
    static constexpr int NW = THREADS / 64;
    static constexpr int NI = ROWS * CPR / (64 * NW);  // instructions per wave per stage
    static_assert(NI * 64 * NW == ROWS * CPR, "the tile splits evenly over the waves");
    static constexpr int CHUNKS = ROWS * CPR;
    uint32_t voff[NI];
    int kpos[NI];

    static __device__ __forceinline__ int sw(int r) {
        if constexpr (CPR == 4)
            return ((r >> 1) ^ (r >> 3)) & 3;
        else
            return (r ^ (r >> 3)) & 7;
    }
    // tile rows [r0, r0 + ROWS) of src[row * ld + k]
    __device__ __forceinline__ void init(int64_t ld, int r0, int rows, const int* = nullptr, int = 0) {
        const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
#pragma unroll
        for (int i = 0; i < NI; ++i) {
            const int L = (i * NW + wave) * 64 + lane;
            const int row = L / CPR;
            const int c = (L % CPR) ^ sw(row);
            voff[i] = r0 + row < rows ? (uint32_t)((row * ld + 8 * c) * 2) : kOOB;
            kpos[i] = 8 * c + 8;  // k extent this lane's chunk needs
        }
    }
    __device__ __forceinline__ void issue(u32x4* lds, const bf16_t* __restrict__ src, int64_t ld, int r0, int k0,
                                          int kvalid) const {
        const __amdgpu_buffer_rsrc_t rs = make_rsrc(src + (int64_t)r0 * ld + k0);
        const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
#pragma unroll
        for (int i = 0; i < NI; ++i)
            __builtin_amdgcn_raw_ptr_buffer_load_lds(rs, (lds_void_t*)(lds + (i * NW + wave) * 64), 16,
                                                     kpos[i] <= kvalid ? voff[i] : kOOB, 0, 0, 0);
    }
    // MFMA fragment: tile row `row + lane%32`, k = 16 ks + 8 (lane/32) .. +7
    static __device__ __forceinline__ bf16x8_t read_frag(const u32x4* __restrict__ lds, int row, int ks, int lane) {
        const int r = row + (lane & 31);
        return __builtin_bit_cast(bf16x8_t, lds[r * CPR + ((2 * ks + (lane >> 5)) ^ sw(r))]);
    }
};

// [K][rows] tiles: k-row kr keeps its RCH = ROWS/8 chunks, no padding, chunk c in
// slot c ^ 4 (kr % 4).  One ds_read_b64_tr_b16 pass reads 4 consecutive
// k-rows x 32 tile rows (4 chunks, 64 bytes, aligned: fragment rows start at
// multiples of 32); the XOR moves the 4 k-rows' 64-byte blocks onto distinct
// quarters of 256 bytes (as a 64-byte pad per k-row would).  The read at
// k + 4 keeps the same XOR.
// PERM = 1 reorders each 32-row fragment by 4-row granules: MFMA row 4 q + t
// reads tile row 4 rot(q) + t, rot(q) = 4 (q % 2) + q / 2.  Accumulator
// element 4 u + t of lane l (MFMA row 8 u + 4 (l / 32) + t) then holds tile
// row 16 (l / 32) + 4 u + t: each lane's 16 values of a 32x32 block are 16
// consecutive tile rows.  Each 32-lane half still reads whole 64-byte blocks
// of the same 4 k-rows, so the reads stay conflict-free.
template <int ROWS, int BK, int THREADS, int PERM = 0>
struct DmaNS {
    static constexpr bool kDma = true;
    static constexpr int kPerm = PERM;
    static constexpr int kFragReads = 2;
    static constexpr int RCH = ROWS / 8;  // chunks per k-row
    static_assert(RCH % 16 == 0, "the XOR of up to 12 stays inside the k-row");
    static constexpr int NW = THREADS / 64;
    static constexpr int NI = BK * RCH / (64 * NW);
    static_assert(NI * 64 * NW == BK * RCH, "the tile splits evenly over the waves");
    static constexpr int CHUNKS = BK * RCH;
    uint32_t voff[NI];
    int kpos[NI];

    // tile rows [r0, r0 + ROWS) of src[k * ld + row]
    __device__ __forceinline__ void init(int64_t ld, int r0, int rows, const int* = nullptr, int = 0) {
        const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
#pragma unroll
        for (int i = 0; i < NI; ++i) {
            const int L = (i * NW + wave) * 64 + lane;
            const int kr = L / RCH;
            const int c = (L % RCH) ^ (4 * (kr & 3));
            voff[i] = r0 + 8 * c < rows ? (uint32_t)((kr * ld + 8 * c) * 2) : kOOB;
            kpos[i] = kr + 1;
        }
    }
    __device__ __forceinline__ void issue(u32x4* lds, const bf16_t* __restrict__ src, int64_t ld, int r0, int k0,
                                          int kvalid) const {
        const __amdgpu_buffer_rsrc_t rs = make_rsrc(src + (int64_t)k0 * ld + r0);
        const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
#pragma unroll
        for (int i = 0; i < NI; ++i)
            __builtin_amdgcn_raw_ptr_buffer_load_lds(rs, (lds_void_t*)(lds + (i * NW + wave) * 64), 16,
                                                     kpos[i] <= kvalid ? voff[i] : kOOB, 0, 0, 0);
    }
    // ds_read_b64_tr_b16, per 16-lane group, gives output lane l element j =
    // element l%4 of the 8 bytes addressed by lane 16 (l/16) + 4 j + (l%16)/4
    // (measured on gfx950), so when lane s addresses
    //     k = kk + 8 (s/32) + (s%16)/4,   row = r + 16 ((s/16)%2) + 4 (s%4)
    // lane l receives rows r + l%32 at k = kk + 8 (l/32) + 0..3: the MFMA layout
    // (PERM = 1 moves each addressed 4-row granule as described above)
    static __device__ __forceinline__ bf16x8_t read_frag(const u32x4* __restrict__ lds, int row, int ks, int lane) {
        typedef short v4i16 __attribute__((ext_vector_type(4)));
        typedef __attribute__((address_space(3))) v4i16 lds_v4i16;
        const int k = 16 * ks + 8 * (lane >> 5) + ((lane & 15) >> 2);
        const int q = 4 * ((lane >> 4) & 1) + (lane & 3);  // 4-row granule of the MFMA rows
        const int r = row + 4 * (PERM ? (((q & 1) << 2) | (q >> 1)) : q);
        const bf16_t* base =
            reinterpret_cast<const bf16_t*>(lds) + 8 * (k * RCH + ((r >> 3) ^ (4 * (k & 3)))) + (r & 7);
        const v4i16 lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_v4i16*)(base));
        const v4i16 hi = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_v4i16*)(base + 8 * 4 * RCH));
        typedef short v8i16 __attribute__((ext_vector_type(8)));
        const v8i16 v = __builtin_shufflevector(lo, hi, 0, 1, 2, 3, 4, 5, 6, 7);
        return __builtin_bit_cast(bf16x8_t, v);
    }
};

// DmaKS with gathered rows: tile row r is source row map[r0 + r] (rows
// r0 + r >= rows are zeros).  The per-lane offsets carry the whole row offset,
// so the descriptor base moves with k only; the host bounds m * ld * 2 < 2^31.
template <int ROWS, int BK, int THREADS>
struct DmaKSG : DmaKS<ROWS, BK, THREADS> {
    using Base = DmaKS<ROWS, BK, THREADS>;
    using Base::CPR;
    using Base::NI;
    using Base::NW;
    // map_rows: valid source rows; an entry outside [0, map_rows) reads zeros
    __device__ __forceinline__ void init(int64_t ld, int r0, int rows, const int* map, int map_rows) {
        const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
#pragma unroll
        for (int i = 0; i < NI; ++i) {
            const int L = (i * NW + wave) * 64 + lane;
            const int row = L / CPR;
            const int c = (L % CPR) ^ Base::sw(row);
            const int src = r0 + row < rows ? map[r0 + row] : -1;
            const bool ok = (unsigned)src < (unsigned)map_rows;
            this->voff[i] = ok ? (uint32_t)(((int64_t)src * ld + 8 * c) * 2) : kOOB;
            this->kpos[i] = 8 * c + 8;
        }
    }
    __device__ __forceinline__ void issue(u32x4* lds, const bf16_t* __restrict__ src, int64_t, int, int k0,
                                          int kvalid) const {
        const __amdgpu_buffer_rsrc_t rs = make_rsrc(src + k0);
        const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
#pragma unroll
        for (int i = 0; i < NI; ++i)
            __builtin_amdgcn_raw_ptr_buffer_load_lds(rs, (lds_void_t*)(lds + (i * NW + wave) * 64), 16,
                                                     this->kpos[i] <= kvalid ? this->voff[i] : kOOB, 0, 0, 0);
    }
};

// ---------------------------------------------------------------- work order
// tile-rows per group of the grouped tile order. Against 4 and 16 at 8192
// tokens (forward, dX and gate over four Linear shapes), 8 was best or within
// 1% of best in 11 of 12 cases; 4 was 2.6% faster for the forward at
// 4096 -> 28672, and 16 was never best.
constexpr int kGroupM = 8;

// Workgroups are dispatched round-robin over the 8 XCDs (workgroup w runs on
// XCD w % 8, its local index w / 8).  The tiles, in grouped order (group_m
// tile-rows at a time, so tiles sharing A rows and B rows meet in one L2), are
// dealt to the XCDs in contiguous ranges.  An XCD with C CUs runs R = tiles/C
// whole rounds of whole tiles; its last `tail` tiles are each split along K
// into s parts (s = C / tail, each part keeping at least 4 k-steps), so the
// final round takes a fraction of a tile's time instead of leaving CUs idle.
struct XcdPlan {
    int t0, tiles;  // the XCD's tile range
    int full;       // tiles run whole
    int tail, s;    // tiles split along K, and parts per tile
    __host__ __device__ int items() const { return full + tail * s; }
};

// min_saved: split only when a part is at least this many K steps shorter
// than the whole tile (a split store tile pays a fixup launch).
__host__ __device__ inline XcdPlan xcd_plan(int x, int total_tiles, int cus_per_xcd, int ksteps, bool split_ok,
                                            int min_saved = 0, int max_split = 8) {
    const int base = total_tiles / 8, rem = total_tiles % 8;
    XcdPlan pl;
    pl.tiles = base + (x < rem ? 1 : 0);
    pl.t0 = x * base + (x < rem ? x : rem);
    const int c = cus_per_xcd > 0 ? cus_per_xcd : 1;
    const int t = pl.tiles % c;
    int sp = t > 0 ? c / t : 1;
    if (sp > max_split) sp = max_split;
    if (sp > ksteps / 4) sp = ksteps / 4;
    if (sp >= 2 && ksteps - (ksteps + sp - 1) / sp < min_saved) sp = 1;
    if (!split_ok || t == 0 || sp < 2) {
        pl.full = pl.tiles;
        pl.tail = 0;
        pl.s = 1;
    } else {
        pl.full = pl.tiles - t;
        pl.tail = t;
        pl.s = sp;
    }
    return pl;
}

struct WorkItem {
    int tm, tn;      // tile coordinates
    int split, ns;   // K part and parts of this tile (ns = 1: whole)
    int tail_slot;   // split tiles: x * tail_max + tail index, else -1
    bool idle;       // padding block of a shorter XCD
};

__device__ __forceinline__ void tile_coords(int tile, int tiles_m, int tiles_n, int group_m, int& tm, int& tn) {
    const int group_size = group_m * tiles_n;
    const int group = tile / group_size;
    const int first_m = group * group_m;
    const int gm = min(tiles_m - first_m, group_m);
    const int in_group = tile % group_size;
    tm = first_m + in_group % gm;
    tn = in_group / gm;
}

__device__ __forceinline__ WorkItem map_work(int w, int tiles_m, int tiles_n, int ksteps, int cus_per_xcd,
                                             bool split_ok, int tail_max, int group_m, int min_saved = 0,
                                             int max_split = 8) {
    const int x = w % 8, local = w / 8;
    const XcdPlan pl = xcd_plan(x, tiles_m * tiles_n, cus_per_xcd, ksteps, split_ok, min_saved, max_split);
    WorkItem wi;
    wi.idle = local >= pl.items();
    wi.split = 0;
    wi.ns = 1;
    wi.tail_slot = -1;
    int tile = pl.t0 + local;
    if (!wi.idle && local >= pl.full) {
        const int q = local - pl.full, tt = q / pl.s;
        tile = pl.t0 + pl.full + tt;
        wi.split = q % pl.s;
        wi.ns = pl.s;
        wi.tail_slot = x * tail_max + tt;
    }
    if (wi.idle) tile = 0;
    tile_coords(tile, tiles_m, tiles_n, group_m, wi.tm, wi.tn);
    return wi;
}

// EPI_STORE: C rounded to bf16.  EPI_GATE: the tile's dots with every
// candidate (partials per block).  EPI_PARTS: a gate product whose tiles are
// split along K into p.parts parts writes each part's fp32 tile to p.dwp and
// leaves the candidate dots to one pass over the summed parts.
enum Epi : int { EPI_STORE = 0, EPI_GATE = 1, EPI_PARTS = 2 };

struct GemmParams {
    const bf16_t* A;
    int64_t lda;
    const bf16_t* B;
    int64_t ldb;
    int I, J, K;  // C is I x J, reduction length K
    bf16_t* C;
    int64_t ldc;
    // work decomposition (set by the launcher): CUs per XCD, whether tail
    // tiles may be split along K, and the largest per-XCD tail and split
    int cus_per_xcd;
    int split_ok;
    int split_min_saved;  // see xcd_plan
    int split_max;        // most K parts of one tile
    int tail_max, s_max;
    // gate epilogue: i indexes d (< dlimit), j indexes n; candidates are rows n
    CandGroup cg;
    int dlimit;
    // gate epilogue: [grid blocks][nsets * kstride] partial sums; store epilogue with
    // split tails: [8 * tail_max][s_max][BI * BJ] fp32 partial tiles
    float* partials;
    // parts epilogue: [tile (tm * tiles_j + tn)][part][BJ][BI] fp32, n-major
    float* dwp;
    int parts;
    // routed product: A rows gathered and C rows scattered through rowmap;
    // group g owns rowmap[group_off[g] .. group_off[g + 1]) and multiplies
    // by bk[g]
    const int* rowmap;
    const int* group_off;
    int ngroups;
    int map_rows;  // rows of A and C (entries of rowmap outside [0, map_rows) are skipped)
    const bf16_t* bk[kMaxCand];
};

template <int BI, int BJ, int BK, int WI, int WJ>
struct GemmShape {
    static constexpr int THREADS = WI * WJ * 64;
    static constexpr int WTI = BI / WI, WTJ = BJ / WJ;  // wave tile
    static constexpr int MI = WTI / 32, NJ = WTJ / 32;
};

template <class LA, class LB, int DEPTH = 1>
struct StageLds {
    static constexpr int A_CH = LA::CHUNKS, B_CH = LB::CHUNKS;  // 16-byte chunks per stage
    static constexpr size_t BYTES = (size_t)DEPTH * (A_CH + B_CH) * 16;  // DEPTH stages
};

// Main loop with direct-to-LDS loaders and NS LDS stages: the loads of stage
// kt + NS - 1 are issued right after the barrier that retires stage kt - 1,
// so NS - 1 stages are in flight while stage kt is multiplied.  One barrier
// per stage; each wave waits (vmcnt) only for its own copies of stage kt.
// Wait until at most N of this wave's vector-memory operations are pending,
// then for its LDS operations, then for the other waves.  A plain
// __syncthreads() would also drain vmcnt (its release fence), retiring the
// stages still in flight.
template <int N>
__device__ __forceinline__ void wait_vmcnt_barrier() {
    static_assert(N >= 0 && N < 64, "vmcnt field is 6 bits");
    asm volatile("s_waitcnt vmcnt(%0) lgkmcnt(0)\n\ts_barrier" ::"n"(N) : "memory");
}

// Main loop over direct-to-LDS stages: NS LDS stages, NS - 1 of them in
// flight while one is multiplied.  The stage switch sits inside the MFMA
// stream: the wait for stage kt + 1 and the barrier come after the last
// k-step's fragments of stage kt are in registers, so the next stage's first
// fragment reads and the copies of stage kt + NS (into the buffer stage kt just
// vacated) are issued among the last k-step's MFMAs instead of in front of an
// idle matrix pipe.  Each wave waits (vmcnt) only for its own copies; the
// barrier then covers everyone's.
// Order of the stage switch, measured per product on MI355X (operand layout
// and tile count change which one keeps the matrix pipe busiest):
//   SWITCH_COPY_FIRST   copies of stage kt + NS, then reads of stage kt + 1
//   SWITCH_READ_FIRST   reads first, so the copies can interleave the MFMAs
//   SWITCH_FENCED       reads first, and the barrier fenced with
//                       sched_barrier so no MFMA or read crosses it
//   SWITCH_LOOSE        reads first; inside a stage only "the first k-step's
//                       reads, then its MFMAs" is pinned, the rest is left to
//                       the scheduler
//   SWITCH_LOOSE2       SWITCH_LOOSE with the stage switch unpinned too
//   SWITCH_FREE         no scheduling hints at all (order of issue only)
enum StageSwitch : int {
    SWITCH_COPY_FIRST = 0,
    SWITCH_READ_FIRST = 1,
    SWITCH_FENCED = 2,
    SWITCH_LOOSE = 3,
    SWITCH_LOOSE2 = 4,
    SWITCH_FREE = 5
};

// COPY_SPLIT: the refill of the buffer a stage switch frees is issued in two
// halves, the A tile at the switch and the B tile after the next stage's first
// k-step, so the two bursts of LDS writes land apart (two stages only: every
// switch then waits for all copies).
enum CopyIssue : int { COPY_BURST = 0, COPY_SPLIT = 1 };

template <class LA, class LB, int BI, int BJ, int BK, int WI, int WJ, int NS, int SWITCH, int COPY = COPY_BURST>
__device__ __forceinline__ void gemm_mainloop_pp(const GemmParams& p, int i0, int j0, int kbeg, int kend,
                                                 u32x4* __restrict__ smem,
                                                 f32x16 (&acc)[GemmShape<BI, BJ, BK, WI, WJ>::MI]
                                                              [GemmShape<BI, BJ, BK, WI, WJ>::NJ]) {
    static_assert(NS >= 2 && NS <= 4, "2 to 4 LDS stages");
    static_assert(COPY == COPY_BURST || NS == 2, "split refills need the wait-for-all of two stages");
    using S = GemmShape<BI, BJ, BK, WI, WJ>;
    constexpr int STAGE = LA::CHUNKS + LB::CHUNKS;
    constexpr int KS = BK / 16;
    static_assert(KS % 2 == 0, "fragment buffers alternate per k-step");
    constexpr int FR = LA::kFragReads * S::MI + LB::kFragReads * S::NJ;  // LDS reads per k-step
    constexpr int MF = S::MI * S::NJ;                                     // MFMAs per k-step
    constexpr int NI = LA::NI + LB::NI;                                   // copies per stage
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int wi = wave / WJ, wj = wave % WJ;
    LA la;
    LB lb;
    la.init(p.lda, i0, p.I, p.rowmap, p.map_rows);
    lb.init(p.ldb, j0, p.J);
#pragma unroll
    for (int a = 0; a < S::MI; ++a)
#pragma unroll
        for (int b = 0; b < S::NJ; ++b)
#pragma unroll
            for (int r = 0; r < 16; ++r) acc[a][b][r] = 0.0f;

    const int nk = (kend - kbeg + BK - 1) / BK;
    // stage kt past the end copies nothing (zeros into a free buffer)
    auto issue = [&](int kt) {
        u32x4* st = smem + (kt % NS) * STAGE;
        const int k0 = min(kbeg + kt * BK, kend);
        const int kvalid = min(BK, kend - k0);
        la.issue(st, p.A, p.lda, i0, k0, kvalid);
        lb.issue(st + LA::CHUNKS, p.B, p.ldb, j0, k0, kvalid);
    };
    auto issue_a = [&](int kt) {
        u32x4* st = smem + (kt % NS) * STAGE;
        const int k0 = min(kbeg + kt * BK, kend);
        la.issue(st, p.A, p.lda, i0, k0, min(BK, kend - k0));
    };
    auto issue_b = [&](int kt) {
        u32x4* st = smem + (kt % NS) * STAGE;
        const int k0 = min(kbeg + kt * BK, kend);
        lb.issue(st + LA::CHUNKS, p.B, p.ldb, j0, k0, min(BK, kend - k0));
    };
    bf16x8_t fa[2][S::MI], fb[2][S::NJ];
    auto read = [&](const u32x4* st, int ks, int buf) {
#pragma unroll
        for (int a = 0; a < S::MI; ++a) fa[buf][a] = LA::read_frag(st, wi * S::WTI + 32 * a, ks, lane);
#pragma unroll
        for (int b = 0; b < S::NJ; ++b) fb[buf][b] = LB::read_frag(st + LA::CHUNKS, wj * S::WTJ + 32 * b, ks, lane);
    };
    auto mfma = [&](int buf) {
#pragma unroll
        for (int a = 0; a < S::MI; ++a)
#pragma unroll
            for (int b = 0; b < S::NJ; ++b)
                acc[a][b] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(fa[buf][a], fb[buf][b], acc[a][b], 0, 0, 0);
    };

    if (nk <= 0) return;
#pragma unroll
    for (int s = 0; s < NS; ++s) issue(s);
    wait_vmcnt_barrier<(NS - 1) * NI>();
    read(smem, 0, 0);
    for (int kt = 0; kt < nk; ++kt) {
        const u32x4* st = smem + (kt % NS) * STAGE;
#pragma unroll
        for (int ks = 0; ks + 1 < KS; ++ks) {
            read(st, ks + 1, (ks + 1) & 1);
            mfma(ks & 1);
            // the B half of the refill issued at the last switch
            if constexpr (COPY == COPY_SPLIT)
                if (ks == 0 && kt >= 1) issue_b(kt - 1 + NS);
        }
        if constexpr (SWITCH != SWITCH_FREE) __builtin_amdgcn_sched_group_barrier(0x100, FR, 0);  // reads of k-step 1 first
        if constexpr (SWITCH != SWITCH_LOOSE && SWITCH != SWITCH_FREE && SWITCH != SWITCH_LOOSE2) {
#pragma unroll
            for (int ks = 1; ks + 1 < KS; ++ks) {
#pragma unroll
                for (int r = 0; r < FR; ++r) {
                    __builtin_amdgcn_sched_group_barrier(0x008, (MF + FR - 1) / FR, 0);
                    __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);
                }
            }
        }
        if constexpr (SWITCH != SWITCH_FREE) __builtin_amdgcn_sched_group_barrier(0x008, MF, 0);
        // all of stage kt is in registers: wait for stage kt + 1 (stages
        // kt + 2 .. kt + NS - 1 may still be in flight), then stage kt's
        // buffer is free for stage kt + NS (past the end: harmless zeros and
        // reads, so the body has no branch and one set of accumulators)
        // SWITCH_FENCED: the barrier becomes a hard scheduling boundary (the
        // scheduler otherwise moves register-only MFMAs from above past it and
        // fragment reads from below ahead of it)
        if constexpr (SWITCH == SWITCH_FENCED) __builtin_amdgcn_sched_barrier(0);
        wait_vmcnt_barrier<(NS - 2) * NI>();
        if constexpr (SWITCH == SWITCH_FENCED) __builtin_amdgcn_sched_barrier(0);
        // reads first: the compiler cannot tell stage buffers apart, so copies
        // issued first stay ahead of every later read (and MFMA)
        if constexpr (COPY == COPY_SPLIT) {
            read(smem + ((kt + 1) % NS) * STAGE, 0, 0);
            issue_a(kt + NS);
        } else if constexpr (SWITCH == SWITCH_COPY_FIRST) {
            issue(kt + NS);
            read(smem + ((kt + 1) % NS) * STAGE, 0, 0);
        } else {
            read(smem + ((kt + 1) % NS) * STAGE, 0, 0);
            issue(kt + NS);
        }
        mfma((KS - 1) & 1);
        if constexpr (SWITCH != SWITCH_FREE && SWITCH != SWITCH_LOOSE2) {
            __builtin_amdgcn_sched_group_barrier(0x100, FR, 1);
#pragma unroll
            for (int r = 0; r < MF; ++r) {
                __builtin_amdgcn_sched_group_barrier(0x008, 1, 1);
                __builtin_amdgcn_sched_group_barrier(0x020, (NI + MF - 1) / MF, 1);
            }
        }
    }
    wait_vmcnt_barrier<0>();  // the zero copies have landed before anyone reuses LDS
}

// ---------------------------------------------------------------- gate epilogue
// The work item's dW tile stays in the accumulators.  Its d range is exactly
// one 256-weight group of every candidate row (BI = 256, i0 a multiple of
// 256), so for each candidate the tile needs 256 spans of GB bytes, one per
// row n.  Those spans are copied into LDS by direct-to-LDS buffer loads
// (buffer_load_dwordx4 ... lds: lane l of an instruction lands at M0 + 16 l),
// each span rounded out to whole 16-byte chunks so the LDS copy keeps the
// global alignment of every field.  Candidate k+1 streams in while candidate k
// is decoded in the accumulator layout.  The descriptor starts at the 16-byte
// boundary at or below the tile's first row and ends with the candidate's
// bytes, so the rounded-out tail of the last span reads zeros and every offset
// stays within the tile's 256 row spans (below 2^30 for any row length the
// C ABI accepts), however large the candidate; rows past J load the tile's
// first row (their dW is zero).
// A staged span takes an odd number of 16-byte chunks: the 32 rows one wave
// reads at the same offset then fall on 16 distinct 16-byte bank groups
// instead of 4 or 8 (even pitches repeat after 4 or 8 rows).
__host__ __device__ constexpr int gate_span_chunks(int gb) { return ((gb + 15 + 15) / 16) | 1; }
constexpr int kGateMaxChunks = gate_span_chunks(272);  // worst type (Q8_0)

__device__ __forceinline__ int gate_row_chunks(int qt) { return gate_span_chunks(group_bytes(qt)); }

template <int BJ, int THREADS>
__device__ __forceinline__ void gate_stage_lds(u32x4* __restrict__ buf, const uint8_t* __restrict__ qbytes, int qt,
                                               int64_t row_groups, int j0, int group, int J) {
    typedef __attribute__((address_space(3))) void lds_void;
    const int gb = group_bytes(qt), nch = gate_row_chunks(qt);
    const int64_t origin = ((int64_t)j0 * row_groups * gb) & ~int64_t(15);
    const int64_t bytes = (int64_t)J * row_groups * gb - origin;
    const __amdgpu_buffer_rsrc_t rs = __builtin_amdgcn_make_buffer_rsrc(
        const_cast<uint8_t*>(qbytes + origin), (short)0, (int)(bytes < (int64_t)kRange ? bytes : (int64_t)kRange),
        0x00020000);
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    constexpr int NW = THREADS / 64;
    const int total = BJ * nch;
    for (int base = wave * 64; base < total; base += NW * 64) {
        const int id = base + lane;
        const int row = id / nch, c = id % nch;
        const int n = (j0 + row < J && id < total) ? j0 + row : j0;
        const int64_t span = ((int64_t)n * row_groups + group) * gb;
        // one instruction per wave: lanes land at buf + 16 (base + lane)
        __builtin_amdgcn_raw_ptr_buffer_load_lds(rs, (lds_void*)(buf + base), 16,
                                                 (uint32_t)((span & ~int64_t(15)) - origin + 16 * c), 0, 0, 0);
    }
}

// <acc, W_k> over the lane's accumulators: with the A operand's rows
// permuted (DmaNS PERM = 1), block (a, b) holds, for row n = 32 b + lane%32,
// the 16 consecutive weights 32 a + 16 (lane/32) + r, r = 0..15 (relative to
// the wave's tile origin).
template <int QT, int MI, int NJ, int WTI, int WTJ>
__device__ __forceinline__ float gate_dot_lds(const f32x16 (&acc)[MI][NJ], const float (&sv)[MI][NJ],
                                              const uint8_t* __restrict__ buf, int64_t row_groups, int j0, int group,
                                              int wi, int wj, int lane, int J) {
    constexpr int GB = group_bytes(QT);
    constexpr int PITCH = 16 * gate_span_chunks(GB);  // bytes per staged row span
    float s = 0.0f;
#pragma unroll
    for (int b = 0; b < NJ; ++b) {
        const int nl = wj * WTJ + 32 * b + (lane & 31);
        // rows past J were staged from the tile's first row: locate their bytes the same way
        const int n = j0 + nl < J ? j0 + nl : j0;
        const int64_t span = ((int64_t)n * row_groups + group) * GB;
        const uint8_t* g = buf + nl * PITCH + (int)(span & 15);
#pragma unroll
        for (int a = 0; a < MI; ++a) {
            float v[16];
#pragma unroll
            for (int r = 0; r < 16; ++r) v[r] = acc[a][b][r];
            s += dot_sub16<QT>(g, wi * WTI + 32 * a + 16 * (lane >> 5), v, sv[a][b]);
        }
    }
    return s;
}

// gate_dot_lds for the IQ formats (type known at run time, uniform)
template <int MI, int NJ, int WTI, int WTJ>
__device__ __forceinline__ float gate_dot_lds_iq(int qt, const f32x16 (&acc)[MI][NJ], const float (&sv)[MI][NJ],
                                                 const uint8_t* __restrict__ buf, int64_t row_groups, int j0,
                                                 int group, int wi, int wj, int lane, int J) {
    const int gb = group_bytes(qt);
    const int pitch = 16 * gate_span_chunks(gb);
    float s = 0.0f;
#pragma unroll
    for (int b = 0; b < NJ; ++b) {
        const int nl = wj * WTJ + 32 * b + (lane & 31);
        const int n = j0 + nl < J ? j0 + nl : j0;
        const int64_t span = ((int64_t)n * row_groups + group) * gb;
        const uint8_t* g = buf + nl * pitch + (int)(span & 15);
#pragma unroll
        for (int a = 0; a < MI; ++a) {
            float v[16];
#pragma unroll
            for (int r = 0; r < 16; ++r) v[r] = acc[a][b][r];
            s += dot_sub16_iq(qt, g, wi * WTI + 32 * a + 16 * (lane >> 5), v, sv[a][b]);
        }
    }
    return s;
}

// IQ: the candidate set may hold IQ formats (their table-lookup decode needs
// registers the K-quant-only instantiation keeps for itself).
template <int BI, int BJ, int BK, int WI, int WJ, bool IQ>
__device__ __forceinline__ void gate_epilogue(const GemmParams& p, int block, int i0, int j0,
                                              u32x4* __restrict__ smem,
                                              const f32x16 (&acc)[GemmShape<BI, BJ, BK, WI, WJ>::MI]
                                                                 [GemmShape<BI, BJ, BK, WI, WJ>::NJ]) {
    using S = GemmShape<BI, BJ, BK, WI, WJ>;
    static_assert(BI == 256, "the gate tile covers exactly one 256-weight group per row");
    constexpr int NW = WI * WJ;
    constexpr int BUF_CH = BJ * kGateMaxChunks;  // 16-byte chunks per candidate buffer
    // per-wave candidate sums, after the two candidate buffers (inside the
    // dynamic allocation: a static array would push an 8-wave workgroup whose
    // main loop takes all 160 KiB past the limit)
    float(*red)[kMaxCand] = reinterpret_cast<float(*)[kMaxCand]>(smem + 2 * BUF_CH);
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);  // uniform: scale fields index by it
    const int wi = wave / WJ, wj = wave % WJ;
    const int group = i0 / 256;
    // the gated tensor this tile's rows belong to (uniform per block)
    int g = 0;
#pragma unroll
    for (int q = 1; q < kMaxSets; ++q)
        if (q < p.cg.nsets && j0 >= p.cg.set_j0[q]) g = q;
    const CandSet& cs = p.cg.sets[g];
    const int jl0 = j0 - p.cg.set_j0[g];                 // first row within the tensor
    const int jn = p.cg.set_j0[g + 1] - p.cg.set_j0[g];  // the tensor's rows
    const int64_t rg = cs.row_groups;
    // candidate-independent sums of each accumulator block
    float sv[S::MI][S::NJ];
#pragma unroll
    for (int a = 0; a < S::MI; ++a)
#pragma unroll
        for (int b = 0; b < S::NJ; ++b) {
            float t = 0.0f;
#pragma unroll
            for (int r = 0; r < 16; ++r) t += acc[a][b][r];
            sv[a][b] = t;
        }
    __syncthreads();  // every wave is past its last main-loop LDS read
    gate_stage_lds<BJ, S::THREADS>(smem, cs.qbytes[0], cs.qtype[0], rg, jl0, group, jn);
    for (int k = 0; k < cs.ncand; ++k) {
        // this wave's direct-to-LDS copies of candidate k have landed, then
        // everyone's have; buffer (k+1) % 2 is no longer read
        asm volatile("s_waitcnt vmcnt(0) lgkmcnt(0)" ::: "memory");
        __syncthreads();
        if (k + 1 < cs.ncand)
            gate_stage_lds<BJ, S::THREADS>(smem + ((k + 1) & 1) * BUF_CH, cs.qbytes[k + 1], cs.qtype[k + 1], rg, jl0,
                                           group, jn);
        const uint8_t* buf = reinterpret_cast<const uint8_t*>(smem + (k & 1) * BUF_CH);
        float sum;
        switch (cs.qtype[k]) {
        case Q8_0: sum = gate_dot_lds<Q8_0, S::MI, S::NJ, S::WTI, S::WTJ>(acc, sv, buf, rg, jl0, group, wi, wj, lane, jn); break;
        case Q2_K: sum = gate_dot_lds<Q2_K, S::MI, S::NJ, S::WTI, S::WTJ>(acc, sv, buf, rg, jl0, group, wi, wj, lane, jn); break;
        case Q3_K: sum = gate_dot_lds<Q3_K, S::MI, S::NJ, S::WTI, S::WTJ>(acc, sv, buf, rg, jl0, group, wi, wj, lane, jn); break;
        case Q4_K: sum = gate_dot_lds<Q4_K, S::MI, S::NJ, S::WTI, S::WTJ>(acc, sv, buf, rg, jl0, group, wi, wj, lane, jn); break;
        case Q5_K: sum = gate_dot_lds<Q5_K, S::MI, S::NJ, S::WTI, S::WTJ>(acc, sv, buf, rg, jl0, group, wi, wj, lane, jn); break;
        default:
            if constexpr (IQ) {
                if (is_iq(cs.qtype[k])) {
                    sum = gate_dot_lds_iq<S::MI, S::NJ, S::WTI, S::WTJ>(cs.qtype[k], acc, sv, buf, rg, jl0, group, wi,
                                                                        wj, lane, jn);
                    break;
                }
            }
            sum = gate_dot_lds<Q6_K, S::MI, S::NJ, S::WTI, S::WTJ>(acc, sv, buf, rg, jl0, group, wi, wj, lane, jn);
            break;
        }
#pragma unroll
        for (int off = 32; off >= 1; off >>= 1) sum += __shfl_xor(sum, off);
        if (lane == 0) red[wave][k] = sum;
    }
    __syncthreads();
    // this block's slots of every tensor: its own sums, zeros for the others
    const int nslot = p.cg.nsets * p.cg.kstride;
    if ((int)threadIdx.x < nslot) {
        const int k = (int)threadIdx.x - g * p.cg.kstride;
        float s = 0.0f;
        if (k >= 0 && k < cs.ncand)
            for (int wv = 0; wv < NW; ++wv) s += red[wv][k];
        p.partials[(int64_t)block * nslot + threadIdx.x] = s;
    }
}

// ---------------------------------------------------------------- kernels
// One GEMM configuration: loaders, tile, wave layout, epilogue, pipeline depth.
// K steps a split part of a store tile must save (see GemmCfg::plan).  14
// against 10: the dual backward at 8192 tokens, 1024 -> 1536 (24 K steps of
// dX, no longer split in two) 94 -> 82 us; within 0.5% at 5120 -> 17408,
// 4096 -> 28672 and the other 1024-wide products.
constexpr int kMinSavedSplitSteps = 14;

template <class LA_, class LB_, int BI_, int BJ_, int BK_, int WI_, int WJ_, int EPI_, int DEPTH_,
          int SWITCH_ = SWITCH_FENCED, int OCC_ = 1, int COPY_ = COPY_BURST>
struct GemmCfg {
    using LA = LA_;
    using LB = LB_;
    static constexpr int BI = BI_, BJ = BJ_, BK = BK_, WI = WI_, WJ = WJ_, EPI = EPI_, DEPTH = DEPTH_;
    static constexpr int SWITCH = SWITCH_;
    static constexpr int OCC = OCC_;  // waves per SIMD the registers are budgeted for
    static constexpr int COPY = COPY_;
    static constexpr int THREADS = WI * WJ * 64;
    static constexpr size_t main_lds() { return StageLds<LA, LB, DEPTH>::BYTES; }
    static constexpr size_t lds() {
        constexpr size_t gate = (size_t)2 * BJ * kGateMaxChunks * 16 + (size_t)WI * WJ * kMaxCand * 4;  // two candidate buffers, wave sums
        constexpr size_t store = (size_t)BI * (BJ + 8) * 2 + BI * 4;   // bf16 staging of the tile, row map
        constexpr size_t epi = EPI == EPI_GATE ? gate : EPI == EPI_PARTS ? 0 : store;
        return epi > main_lds() ? epi : main_lds();
    }
    static int tiles_i(const GemmParams& p) { return (p.I + BI - 1) / BI; }
    static int tiles_j(const GemmParams& p) { return (p.J + BJ - 1) / BJ; }
    static __host__ __device__ int ksteps(const GemmParams& p) { return (p.K + BK - 1) / BK; }
    // Fill in the work decomposition; returns the grid size (8 * blocks per XCD).
    static int plan(GemmParams& p, int cus, bool split_ok) {
        if (p.I <= 0 || p.J <= 0) return 0;
        if constexpr (EPI == EPI_PARTS) {
            // every tile in p.parts parts, the XCDs' tile ranges as for whole tiles
            p.cus_per_xcd = cus / 8 > 0 ? cus / 8 : 1;
            p.split_ok = 0;
            p.tail_max = 0;
            p.s_max = 1;
            const int tiles = tiles_i(p) * tiles_j(p);
            int items = 0;
            for (int x = 0; x < 8; ++x) {
                const XcdPlan pl = xcd_plan(x, tiles, p.cus_per_xcd, ksteps(p), false);
                items = pl.tiles * p.parts > items ? pl.tiles * p.parts : items;
            }
            return 8 * items;
        }
        // a split store tile pays for its partial writes and a fixup launch:
        // split only when a part saves at least kMinSavedSplitSteps K steps
        p.split_min_saved = EPI == EPI_STORE ? kMinSavedSplitSteps : 0;
        // more than 8 parts (tried for the gate at 1024 x 1024) loses: the
        // parts of a dual launch then overflow one round of the CUs
        p.split_max = 8;
        p.cus_per_xcd = cus / 8 > 0 ? cus / 8 : 1;
        p.split_ok = split_ok ? 1 : 0;
        const int tiles = tiles_i(p) * tiles_j(p);
        int items = 0;
        p.tail_max = 0;
        p.s_max = 1;
        for (int x = 0; x < 8; ++x) {
            const XcdPlan pl = xcd_plan(x, tiles, p.cus_per_xcd, ksteps(p), split_ok, p.split_min_saved, p.split_max);
            items = pl.items() > items ? pl.items() : items;
            p.tail_max = pl.tail > p.tail_max ? pl.tail : p.tail_max;
            p.s_max = pl.s > p.s_max ? pl.s : p.s_max;
        }
        return 8 * items;
    }
    // fp32 workspace the split tails of a store epilogue need
    static int64_t tail_bytes(const GemmParams& p) {
        return p.tail_max > 0 ? (int64_t)8 * p.tail_max * p.s_max * BI * BJ * 4 : 0;
    }
};

// Store epilogue: the tile goes through LDS as bf16 ([BI][BJ + 8], the pad
// puts the two row halves of an MFMA write on different banks), then out with
// 16-byte stores, 32 consecutive threads per 512-byte row segment, so C is
// written in whole cache lines.  C's row length J is a multiple of 8.  The
// stores are non-temporal: every CU writes its tile at about the same moment,
// and streaming the burst past L2 measured 4-6% faster on the forward at
// 8192 x 5120 -> 17408 and 8192 x 1024 -> 1536 / 6144 (within 1% elsewhere).
template <int BI, int BJ, int BK, int WI, int WJ>
__device__ __forceinline__ void store_tile_lds(const GemmParams& p, int i0, int j0, u32x4* __restrict__ smem,
                                               const f32x16 (&acc)[GemmShape<BI, BJ, BK, WI, WJ>::MI]
                                                                  [GemmShape<BI, BJ, BK, WI, WJ>::NJ]) {
    using S = GemmShape<BI, BJ, BK, WI, WJ>;
    constexpr int PITCH = BJ + 8;  // bf16 per LDS row
    static_assert((size_t)BI * PITCH * 2 + BI * 4 <= 160 * 1024, "tile and row map fit in LDS");
    static_assert(S::THREADS >= BI, "one thread per tile row loads the row map");
    bf16_t* t = reinterpret_cast<bf16_t*>(smem);
    int* rows_at = reinterpret_cast<int*>(t + BI * PITCH);  // routed: the tile's destination rows
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int wi = wave / WJ, wj = wave % WJ;
    // one map load per tile row, in flight while the accumulators go to LDS
    // (the store loop below would otherwise wait on a global load per chunk)
    int dest = -1;
    if (p.rowmap && (int)threadIdx.x < BI && i0 + (int)threadIdx.x < p.I) dest = p.rowmap[i0 + threadIdx.x];
    __syncthreads();  // every wave is past its last main-loop LDS read
    if (p.rowmap && (int)threadIdx.x < BI) rows_at[threadIdx.x] = dest;
    // rows il and il + 1 of a lane's column convert as one pair
    // (v_cvt_pk_bf16_f32: one instruction for two values, where the software
    // rounding takes six per value; a NaN stays a quiet NaN)
#pragma unroll
    for (int a = 0; a < S::MI; ++a)
#pragma unroll
        for (int b = 0; b < S::NJ; ++b) {
            const int jl = wj * S::WTJ + 32 * b + (lane & 31);
#pragma unroll
            for (int r = 0; r < 16; r += 2) {
                const int il = wi * S::WTI + 32 * a + 8 * (r >> 2) + 4 * (lane >> 5) + (r & 3);
                const uint32_t h = pk_bf16(acc[a][b][r], acc[a][b][r + 1]);
                t[il * PITCH + jl] = (bf16_t)h;
                t[(il + 1) * PITCH + jl] = (bf16_t)(h >> 16);
            }
        }
    __syncthreads();
    constexpr int CPR = BJ / 8;  // 16-byte chunks per tile row
    const int rows = min(BI, p.I - i0), cols = min(BJ, p.J - j0);
#pragma unroll 4
    for (int c = threadIdx.x; c < BI * CPR; c += S::THREADS) {
        const int il = c / CPR, jc = c % CPR;
        if (il < rows && 8 * jc < cols) {
            const u32x4 v = *reinterpret_cast<const u32x4*>(t + il * PITCH + 8 * jc);
            const int64_t gi = p.rowmap ? rows_at[il] : i0 + il;  // routed: scatter rows
            if (!p.rowmap || (uint64_t)gi < (uint64_t)p.map_rows)
                __builtin_nontemporal_store(v, reinterpret_cast<u32x4*>(p.C + gi * p.ldc + j0 + 8 * jc));
        }
    }
}

// Work item `block` of problem p.  IQ: a gate product whose candidate sets
// may hold IQ formats (their table-lookup decode needs registers the
// K-quant-only instantiation keeps for itself).
template <class C, bool IQ = false>
__device__ __forceinline__ void gemm_body(const GemmParams& p, int block, u32x4* __restrict__ smem) {
    using LA = typename C::LA;
    using LB = typename C::LB;
    constexpr int BI = C::BI, BJ = C::BJ, BK = C::BK, WI = C::WI, WJ = C::WJ, EPI = C::EPI, DEPTH = C::DEPTH;
    using S = GemmShape<BI, BJ, BK, WI, WJ>;
    const int tiles_i = (p.I + BI - 1) / BI, tiles_j = (p.J + BJ - 1) / BJ;
    const int ksteps = (p.K + BK - 1) / BK;
    if constexpr (EPI == EPI_PARTS) {
        // item (tile, part): XCD x = block % 8 takes its tile range part by part
        static_assert(LA::kPerm == 1, "each lane holds 16 consecutive rows i of an accumulator block");
        const int x = block % 8, local = block / 8;
        const XcdPlan pl = xcd_plan(x, tiles_i * tiles_j, p.cus_per_xcd, ksteps, false);
        if (local >= pl.tiles * p.parts) return;
        int tm, tn;
        tile_coords(pl.t0 + local / p.parts, tiles_i, tiles_j, kGroupM, tm, tn);
        const int part = local % p.parts;
        const int chunk = (ksteps + p.parts - 1) / p.parts * BK;
        const int kbeg = min(p.K, part * chunk), kend = min(p.K, kbeg + chunk);
        f32x16 acc[S::MI][S::NJ];
        gemm_mainloop_pp<LA, LB, BI, BJ, BK, WI, WJ, DEPTH, C::SWITCH, C::COPY>(p, tm * BI, tn * BJ, kbeg, kend, smem,
                                                                                acc);
        // acc[a][b][r] is element (i, j) = (wi WTI + 32 a + 16 (lane >> 5) + r, wj WTJ + 32 b + lane % 32):
        // four 16-byte stores per lane and block, two lanes per 128-byte row segment
        const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
        const int wi = wave / WJ, wj = wave % WJ;
        float* slot = p.dwp + ((int64_t)(tm * tiles_j + tn) * p.parts + part) * (BI * BJ);
#pragma unroll
        for (int a = 0; a < S::MI; ++a)
#pragma unroll
            for (int b = 0; b < S::NJ; ++b) {
                const int jl = wj * S::WTJ + 32 * b + (lane & 31);
                const int il = wi * S::WTI + 32 * a + 16 * (lane >> 5);
                float4* o = reinterpret_cast<float4*>(slot + jl * BI + il);
#pragma unroll
                for (int q = 0; q < 4; ++q)
                    o[q] = make_float4(acc[a][b][4 * q], acc[a][b][4 * q + 1], acc[a][b][4 * q + 2], acc[a][b][4 * q + 3]);
            }
        return;
    }
    const WorkItem w = map_work(block, tiles_i, tiles_j, ksteps, p.cus_per_xcd, p.split_ok != 0, p.tail_max, kGroupM,
                                p.split_min_saved, p.split_max);
    if (w.idle) {
        if constexpr (EPI == EPI_GATE) {
            const int nslot = p.cg.nsets * p.cg.kstride;
            if ((int)threadIdx.x < nslot) p.partials[(int64_t)block * nslot + threadIdx.x] = 0.0f;
        }
        return;
    }
    const int i0 = w.tm * BI, j0 = w.tn * BJ;
    int kbeg = 0, kend = p.K;
    if (w.ns > 1) {
        const int chunk = (ksteps + w.ns - 1) / w.ns * BK;
        kbeg = min(p.K, w.split * chunk);
        kend = min(p.K, kbeg + chunk);
    }
    f32x16 acc[S::MI][S::NJ];
    static_assert(LA::kDma && LB::kDma, "direct-to-LDS loaders");
    gemm_mainloop_pp<LA, LB, BI, BJ, BK, WI, WJ, DEPTH, C::SWITCH, C::COPY>(p, i0, j0, kbeg, kend, smem, acc);

    if constexpr (EPI == EPI_STORE) {
        if (w.ns > 1) {
            // K part of a split tail tile: fp32 partial, [element][thread]
            float* slot = p.partials + ((int64_t)w.tail_slot * p.s_max + w.split) * (BI * BJ);
#pragma unroll
            for (int a = 0; a < S::MI; ++a)
#pragma unroll
                for (int b = 0; b < S::NJ; ++b)
#pragma unroll
                    for (int r = 0; r < 16; ++r)
                        slot[((a * S::NJ + b) * 16 + r) * S::THREADS + threadIdx.x] = acc[a][b][r];
            return;
        }
        store_tile_lds<BI, BJ, BK, WI, WJ>(p, i0, j0, smem, acc);
    } else if constexpr (EPI == EPI_GATE) {
        static_assert(LA::kPerm == 1, "the gate epilogue reads 16 consecutive weights per accumulator block");
        gate_epilogue<BI, BJ, BK, WI, WJ, IQ>(p, block, i0, j0, smem, acc);
    }
}

// Sum of the K parts of each split tail tile of a store epilogue, in part
// order, rounded to bf16 into C.  One block per (XCD tail slot, accumulator
// block (a, b)): every thread loads its 16 values of each part at once.
template <class C>
__global__ __launch_bounds__(C::THREADS) void gemm_tail_fixup_kernel(GemmParams p) {
    using S = GemmShape<C::BI, C::BJ, C::BK, C::WI, C::WJ>;
    constexpr int BLOCKS = S::MI * S::NJ;
    constexpr int TILE = C::BI * C::BJ;
    const int slot = blockIdx.x / BLOCKS, ab = blockIdx.x % BLOCKS;
    const int a = ab / S::NJ, b = ab % S::NJ;
    const int x = slot / p.tail_max, tt = slot % p.tail_max;
    const int tiles_i = (p.I + C::BI - 1) / C::BI, tiles_j = (p.J + C::BJ - 1) / C::BJ;
    const XcdPlan pl = xcd_plan(x, tiles_i * tiles_j, p.cus_per_xcd, C::ksteps(p), p.split_ok != 0, p.split_min_saved,
                                p.split_max);
    if (tt >= pl.tail) return;
    int tm, tn;
    tile_coords(pl.t0 + pl.full + tt, tiles_i, tiles_j, kGroupM, tm, tn);
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int wi = wave / C::WJ, wj = wave % C::WJ;
    const float* base = p.partials + (int64_t)slot * p.s_max * TILE + (ab * 16) * S::THREADS + threadIdx.x;
    float v[16];
#pragma unroll
    for (int r = 0; r < 16; ++r) v[r] = base[r * S::THREADS];
#pragma unroll
    for (int sp = 1; sp < 8; ++sp) {
        if (sp < pl.s) {
            float t[16];
#pragma unroll
            for (int r = 0; r < 16; ++r) t[r] = base[(int64_t)sp * TILE + r * S::THREADS];
#pragma unroll
            for (int r = 0; r < 16; ++r) v[r] += t[r];
        }
    }
    const int gj = tn * C::BJ + wj * S::WTJ + 32 * b + (lane & 31);
#pragma unroll
    for (int r = 0; r < 16; ++r) {
        const int gi = tm * C::BI + wi * S::WTI + 32 * a + 8 * (r >> 2) + 4 * (lane >> 5) + (r & 3);
        if (gi < p.I && gj < p.J) p.C[(int64_t)gi * p.ldc + gj] = f2bf(v[r]);
    }
}

// The register budget is set by the waves per SIMD the configuration runs at
// (OCC: one for four-wave 256x256 tiles with 256 accumulators per lane, two
// for eight-wave ones or two 128x128 workgroups per CU): telling the compiler
// so lets it keep fragments in flight instead of minimising registers for an
// occupancy the LDS use rules out anyway.
template <class C, bool IQ = false>
__global__ __launch_bounds__(C::THREADS) __attribute__((amdgpu_waves_per_eu(C::OCC, C::OCC)))
void gemm_kernel(GemmParams p) {
#if defined(__HIP_DEVICE_COMPILE__)  // the host pass needs only the launch stub (see gemm_dual_kernel)
    extern __shared__ u32x4 smem[];
    gemm_body<C, IQ>(p, blockIdx.x, smem);
#endif
}

// Two independent products in one launch: blocks [0, n1) run problem 1,
// blocks [n1, ...) problem 2 (n1 is a multiple of 8, so both keep the XCD
// mapping of map_work; blocks past problem 1's items exit).  One grid lets
// the second product's work items fill the last, partial round of the first
// instead of each launch idling CUs in its own tail.
template <class C1, class C2, bool IQ1 = false, bool IQ2 = false>
__global__ __launch_bounds__(C1::THREADS) __attribute__((amdgpu_waves_per_eu(C1::OCC, C1::OCC)))
void gemm_dual_kernel(GemmParams p1, int items1, int n1, GemmParams p2) {
    static_assert(C1::THREADS == C2::THREADS && C1::OCC == C2::OCC, "both problems use the same workgroup shape");
    // Kernel bodies are compiled for the device only: the host pass needs just
    // the launch stub, and with a configuration instantiated for both IQ
    // values it rejects the second instantiation of gemm_mainloop_pp
    // (a substitution failure on the accumulator array parameter that the
    // device pass does not report).
#if defined(__HIP_DEVICE_COMPILE__)
    extern __shared__ u32x4 smem[];
    const int b = blockIdx.x;
    if (b < n1) {
        if (b < items1) gemm_body<C1, IQ1>(p1, b, smem);
    } else {
        gemm_body<C2, IQ2>(p2, b - n1, smem);
    }
#endif
}

template <class C>
static hipError_t set_lds_attr(const void* kern, size_t lds, bool& done) {
    if (done) return hipSuccess;
    hipError_t e = hipFuncSetAttribute(kern, hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds);
    if (e == hipSuccess)
        done = true;
    else
        (void)hipGetLastError();  // report it once, here, not again at the caller's next launch
    return e;
}

// Launch of one product.  `cus` is the device's CU count; a store epilogue
// splits tail tiles only when `tail_ws` (tail_bytes of the plan) is given.
template <class C, bool IQ = false>
static hipError_t launch_gemm_cfg(GemmParams p, int cus, float* tail_ws, hipStream_t s) {
    const bool split_ok = C::EPI == EPI_GATE || tail_ws != nullptr;
    const int grid = C::plan(p, cus, split_ok);
    if (grid == 0) return hipSuccess;
    if (C::EPI == EPI_STORE) p.partials = tail_ws;
    constexpr size_t lds = C::lds();
    static_assert(lds <= 160 * 1024, "exceeds the 160 KiB of LDS per workgroup");
    static bool attr_set = false;  // per instantiation
    auto kern = gemm_kernel<C, IQ>;
    hipError_t e = set_lds_attr<C>((const void*)kern, lds, attr_set);
    if (e != hipSuccess) return e;
    kern<<<dim3(grid), dim3(C::THREADS), lds, s>>>(p);
    e = hipGetLastError();
    if (e != hipSuccess || C::EPI != EPI_STORE || p.tail_max == 0) return e;
    constexpr int FIX_BLOCKS = GemmShape<C::BI, C::BJ, C::BK, C::WI, C::WJ>::MI * GemmShape<C::BI, C::BJ, C::BK, C::WI, C::WJ>::NJ;
    gemm_tail_fixup_kernel<C><<<dim3(8 * p.tail_max * FIX_BLOCKS), dim3(C::THREADS), 0, s>>>(p);
    return hipGetLastError();
}

// Two products in one launch (see gemm_dual_kernel): problem 1, a store
// product with split tails (tail_ws1), and problem 2, a gate product.  The
// gate product's work items come first and the store product's fill the
// tail (its split parts are fixed up after the launch): 0.8-1.5% faster than
// the other order at 8192 tokens and 5120 -> 17408, 0.9-1.2% at
// 4096 -> 28672, neutral at 17408 -> 5120 and the 1024-wide products.
template <class C1, class C2, bool IQ2 = false>
static hipError_t launch_gemm_dual(GemmParams p1, GemmParams p2, int cus, float* tail_ws1, hipStream_t s) {
    static_assert(C1::EPI == EPI_STORE && (C2::EPI == EPI_GATE || C2::EPI == EPI_PARTS),
                  "a store product and a gate product");
    const int grid1 = C1::plan(p1, cus, tail_ws1 != nullptr);
    const int grid2 = C2::plan(p2, cus, true);
    p1.partials = tail_ws1;
    if (grid1 == 0) return launch_gemm_cfg<C2, IQ2>(p2, cus, nullptr, s);
    if (grid2 == 0) return launch_gemm_cfg<C1>(p1, cus, tail_ws1, s);
    constexpr size_t lds = C1::lds() > C2::lds() ? C1::lds() : C2::lds();
    static_assert(lds <= 160 * 1024, "exceeds the 160 KiB of LDS per workgroup");
    static bool attr_set = false;
    auto kern = gemm_dual_kernel<C2, C1, IQ2, false>;
    hipError_t e = set_lds_attr<C2>((const void*)kern, lds, attr_set);
    if (e != hipSuccess) return e;
    kern<<<dim3(grid2 + grid1), dim3(C2::THREADS), lds, s>>>(p2, grid2, grid2, p1);
    e = hipGetLastError();
    if (e != hipSuccess || C1::EPI != EPI_STORE || p1.tail_max == 0) return e;
    constexpr int FIX_BLOCKS = GemmShape<C1::BI, C1::BJ, C1::BK, C1::WI, C1::WJ>::MI * GemmShape<C1::BI, C1::BJ, C1::BK, C1::WI, C1::WJ>::NJ;
    gemm_tail_fixup_kernel<C1><<<dim3(8 * p1.tail_max * FIX_BLOCKS), dim3(C1::THREADS), 0, s>>>(p1);
    return hipGetLastError();
}

// ---------------------------------------------------------------- routed product
// Grouped GEMM: C[rowmap[r]] = A[rowmap[r]] . bk[g]^T for the rows r of each
// group g (group_off on the device, so the host never waits for the counts).
// The grid covers ceil(m / BI) + ngroups - 1 tile-rows, the most the groups can
// need; every block counts the tile-rows the groups do need, takes its tile of
// those (the XCDs get even contiguous ranges, the spare blocks spread over all
// of them) and finds the tile's group by walking the group sizes.  Measured on
// MI355X at 8192 tokens, 5120 -> 17408, six candidates: group-ordered tiles and
// the row map staged once per tile took six Gumbel-sized groups from 1.380 to
// 1.338 ms and six 256-aligned groups from 1.236-1.260 to 1.214 ms (one group
// 1.145 ms, the dense forward 1.147 ms).
template <class C>
__global__ __launch_bounds__(C::THREADS) __attribute__((amdgpu_waves_per_eu(C::OCC, C::OCC)))
void routed_gemm_kernel(GemmParams p, int tile_rows) {
    using LA = typename C::LA;
    using LB = typename C::LB;
    constexpr int BI = C::BI, BJ = C::BJ, BK = C::BK, WI = C::WI, WJ = C::WJ;
    using S = GemmShape<BI, BJ, BK, WI, WJ>;
    extern __shared__ u32x4 smem[];
    const int tiles_j = (p.J + BJ - 1) / BJ;
    // group bounds clamped to [0, map_rows] and made monotonic, so bad
    // offsets cannot index rowmap out of range; the work is spread over the
    // tile-rows the groups actually have (the grid covers the most they can)
    int used_rows = 0;
    for (int g = 0, h = 0; g < p.ngroups; ++g) {
        const int l = min(max(p.group_off[g], h), p.map_rows);
        h = min(max(p.group_off[g + 1], l), p.map_rows);
        used_rows += (h - l + BI - 1) / BI;
    }
    used_rows = min(used_rows, tile_rows);
    // the XCDs take contiguous ranges of the tiles (as in map_work); the tiles
    // run group by group, each group's tile-rows in blocks of kGroupM with the
    // tile-rows fastest, so the tiles an XCD runs at once read one candidate's
    // B panels and share them in its L2
    const int x = blockIdx.x % 8, local = blockIdx.x / 8;
    const XcdPlan pl = xcd_plan(x, used_rows * tiles_j, p.cus_per_xcd, 0, false);
    if (local >= pl.items()) return;
    int tile = pl.t0 + local, tm = 0, tn = 0, g = 0, lo = 0, hi = 0;
    for (; g < p.ngroups; ++g) {
        lo = min(max(p.group_off[g], hi), p.map_rows);
        hi = min(max(p.group_off[g + 1], lo), p.map_rows);
        const int nt = (hi - lo + BI - 1) / BI;
        if (tile < nt * tiles_j) {
            tile_coords(tile, nt, tiles_j, kGroupM, tm, tn);
            break;
        }
        tile -= nt * tiles_j;
    }
    if (g >= p.ngroups) return;
    GemmParams q = p;
    q.B = p.bk[g];
    q.I = hi;  // end of the group's rows in rowmap
    const int i0 = lo + tm * BI, j0 = tn * BJ;
    f32x16 acc[S::MI][S::NJ];
    gemm_mainloop_pp<LA, LB, BI, BJ, BK, WI, WJ, C::DEPTH, C::SWITCH, C::COPY>(q, i0, j0, 0, q.K, smem, acc);
    store_tile_lds<BI, BJ, BK, WI, WJ>(q, i0, j0, smem, acc);
}

template <class C>
static hipError_t launch_routed_gemm(GemmParams p, int m, int cus, hipStream_t s) {
    if (m <= 0 || p.J <= 0 || p.ngroups <= 0) return hipSuccess;
    const int tile_rows = (m + C::BI - 1) / C::BI + p.ngroups - 1;
    const int tiles = tile_rows * ((p.J + C::BJ - 1) / C::BJ);
    p.cus_per_xcd = cus / 8 > 0 ? cus / 8 : 1;
    p.split_ok = 0;
    int items = 0;
    for (int x = 0; x < 8; ++x) {
        const XcdPlan pl = xcd_plan(x, tiles, p.cus_per_xcd, C::ksteps(p), false);
        items = pl.items() > items ? pl.items() : items;
    }
    constexpr size_t lds = C::lds();
    static bool attr_set = false;
    auto kern = routed_gemm_kernel<C>;
    hipError_t e = set_lds_attr<C>((const void*)kern, lds, attr_set);
    if (e != hipSuccess) return e;
    kern<<<dim3(8 * items), dim3(C::THREADS), lds, s>>>(p, tile_rows);
    return hipGetLastError();
}

}  // namespace vq
