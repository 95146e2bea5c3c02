// C ABI of libvoodoo_hip.so (declared in include/voodoo_hip.h): argument
// validation, error strings and kernel sequencing.  No entry point allocates.
#include <cstdarg>
#include <cstdio>
#include <mutex>
#include <string>

#include "../../include/voodoo_hip.h"
#include "vq_internal.h"

namespace {

thread_local std::string g_last_error;

int fail(int code, const char* fmt, ...) {
    char buf[512];
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(buf, sizeof(buf), fmt, ap);
    va_end(ap);
    g_last_error = buf;
    return code;
}

int ok() {
    g_last_error.clear();
    return VQ_OK;
}

int hip_check(hipError_t e, const char* what) {
    if (e != hipSuccess) return fail(VQ_ERR_HIP, "%s: %s", what, hipGetErrorString(e));
    return VQ_OK;
}

bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

const char* qtype_name(int qt) {
    switch (qt) {
    case vq::Q8_0: return "Q8_0";
    case vq::Q2_K: return "Q2_K";
    case vq::Q3_K: return "Q3_K";
    case vq::Q4_K: return "Q4_K";
    case vq::Q5_K: return "Q5_K";
    case vq::Q6_K: return "Q6_K";
    case vq::IQ2_XXS: return "IQ2_XXS";
    case vq::IQ2_XS: return "IQ2_XS";
    case vq::IQ3_XXS: return "IQ3_XXS";
    case vq::IQ1_S: return "IQ1_S";
    case vq::IQ3_S: return "IQ3_S";
    case vq::IQ2_S: return "IQ2_S";
    case vq::IQ4_XS: return "IQ4_XS";
    case vq::IQ1_M: return "IQ1_M";
    default: return "?";
    }
}

int block_size(int qt) { return qt == vq::Q8_0 ? 32 : 256; }

int check_types(int ncand, const int* qtypes, const void* const* qbytes, bool need_ptrs) {
    if (ncand < 1 || ncand > vq::kMaxCand)
        return fail(VQ_ERR_SHAPE, "ncand=%d outside [1, %d]", ncand, vq::kMaxCand);
    if (!qtypes) return fail(VQ_ERR_NULL, "qtypes is NULL");
    if (need_ptrs && !qbytes) return fail(VQ_ERR_NULL, "qbytes is NULL");
    for (int k = 0; k < ncand; ++k) {
        if (!vq::qtype_supported(qtypes[k]))
            return fail(VQ_ERR_QTYPE, "candidate %d: unsupported ggml type %d (supported: Q8_0, Q2_K..Q6_K)", k,
                        qtypes[k]);
        if (need_ptrs) {
            if (!qbytes[k]) return fail(VQ_ERR_NULL, "candidate %d (%s): qbytes is NULL", k, qtype_name(qtypes[k]));
            if (!aligned16(qbytes[k]))
                return fail(VQ_ERR_ALIGN, "candidate %d (%s): qbytes not 16-byte aligned", k, qtype_name(qtypes[k]));
        }
    }
    return VQ_OK;
}

int check_candidates(int ncand, const int* qtypes, const void* const* qbytes, int64_t n, int64_t d, int64_t d_pad,
                     bool need_ptrs) {
    const int rc = check_types(ncand, qtypes, qbytes, need_ptrs);
    if (rc != VQ_OK) return rc;
    if (n <= 0 || d <= 0 || d_pad <= 0) return fail(VQ_ERR_SHAPE, "n=%lld d=%lld d_pad=%lld must be positive",
                                                   (long long)n, (long long)d, (long long)d_pad);
    if (d_pad % 256 != 0) return fail(VQ_ERR_ALIGN, "d_pad=%lld is not a multiple of 256", (long long)d_pad);
    if (d > d_pad) return fail(VQ_ERR_SHAPE, "d=%lld exceeds d_pad=%lld", (long long)d, (long long)d_pad);
    if (n % 8 != 0 || d % 8 != 0)
        return fail(VQ_ERR_ALIGN, "n=%lld and d=%lld must be multiples of 8", (long long)n, (long long)d);
    // GEMM tiles address at most 256 rows of a row-major operand from a rebased
    // buffer descriptor: keep 256 * 2 * (row length) below 2^30.
    if (n > (1 << 21) || d_pad > (1 << 21))
        return fail(VQ_ERR_SHAPE, "n=%lld / d_pad=%lld exceed the 2^21 limit of one dimension", (long long)n,
                    (long long)d_pad);
    return VQ_OK;
}

vq::CandSet make_set(int ncand, const int* qtypes, const void* const* qbytes, int64_t d_pad) {
    vq::CandSet cs{};
    cs.ncand = ncand;
    cs.row_groups = d_pad / 256;
    for (int k = 0; k < ncand; ++k) {
        cs.qtype[k] = qtypes[k];
        cs.qbytes[k] = static_cast<const uint8_t*>(qbytes[k]);
    }
    return cs;
}

int64_t align256(int64_t x) { return (x + 255) & ~int64_t(255); }

// One gated tensor as a group of one.
vq::CandGroup group_of(const vq::CandSet& cs, int64_t n) {
    vq::CandGroup g{};
    g.nsets = 1;
    g.kstride = cs.ncand;
    g.set_j0[0] = 0;
    g.set_j0[1] = (int)n;
    g.sets[0] = cs;
    return g;
}

// Checks of a stacked group of gated tensors sharing one input; fills cg and
// the total row count.
int check_group(int nmembers, const int64_t* n, const int* ncand, const int* qtypes, const void* const* qbytes,
                int64_t d, int64_t d_pad, vq::CandGroup& cg, int64_t& n_total) {
    if (nmembers < 1 || nmembers > vq::kMaxSets)
        return fail(VQ_ERR_SHAPE, "nmembers=%d outside [1, %d]", nmembers, vq::kMaxSets);
    if (!n || !ncand || !qtypes || !qbytes) return fail(VQ_ERR_NULL, "n/ncand/qtypes/qbytes is NULL");
    cg = vq::CandGroup{};
    cg.nsets = nmembers;
    n_total = 0;
    int off = 0;
    for (int i = 0; i < nmembers; ++i) {
        int rc = check_candidates(ncand[i], qtypes + off, qbytes + off, n[i], d, d_pad, true);
        if (rc != VQ_OK) return rc;
        if (nmembers > 1 && n[i] % 256 != 0)
            return fail(VQ_ERR_ALIGN, "member %d: n=%lld must be a multiple of 256 in a group", i, (long long)n[i]);
        cg.sets[i] = make_set(ncand[i], qtypes + off, qbytes + off, d_pad);
        cg.set_j0[i] = (int)n_total;
        cg.kstride = ncand[i] > cg.kstride ? ncand[i] : cg.kstride;
        n_total += n[i];
        off += ncand[i];
    }
    if (n_total > (1 << 21)) return fail(VQ_ERR_SHAPE, "stacked n=%lld exceeds 2^21", (long long)n_total);
    cg.set_j0[nmembers] = (int)n_total;
    return VQ_OK;
}

// Shared checks of the embedding-row entry points.
int check_embed(int ncand, const int* qtypes, const void* const* qbytes, const int64_t* ids, int64_t nids,
                int64_t vocab, int64_t dim, int64_t d_pad) {
    int rc = check_types(ncand, qtypes, qbytes, true);
    if (rc != VQ_OK) return rc;
    if (vocab <= 0 || dim <= 0 || d_pad <= 0 || nids < 0)
        return fail(VQ_ERR_SHAPE, "num_embeddings=%lld dim=%lld d_pad=%lld nids=%lld", (long long)vocab,
                    (long long)dim, (long long)d_pad, (long long)nids);
    if (d_pad % 256 != 0) return fail(VQ_ERR_ALIGN, "d_pad=%lld is not a multiple of 256", (long long)d_pad);
    if (dim > d_pad) return fail(VQ_ERR_SHAPE, "embedding_dim=%lld exceeds d_pad=%lld", (long long)dim, (long long)d_pad);
    if (dim % 8 != 0) return fail(VQ_ERR_ALIGN, "embedding_dim=%lld must be a multiple of 8", (long long)dim);
    if (d_pad > (1 << 21)) return fail(VQ_ERR_SHAPE, "d_pad=%lld exceeds 2^21", (long long)d_pad);
    if (vq::embed_plan(nids, dim).blocks >= ((int64_t)1 << 31))
        return fail(VQ_ERR_SHAPE, "nids=%lld: too many rows for one launch", (long long)nids);
    if (nids > 0 && !ids) return fail(VQ_ERR_NULL, "ids is NULL");
    return VQ_OK;
}


// Checks shared by the two gated-Linear backward entry points.
int check_bwd(const uint16_t* dy, const uint16_t* x, int64_t m, int64_t n, int64_t d, int64_t d_pad, int ncand,
              const int* qtypes, const void* const* qbytes, const uint16_t* w_eff, const uint16_t* dx) {
    int rc = check_candidates(ncand, qtypes, qbytes, n, d, d_pad, true);
    if (rc != VQ_OK) return rc;
    if (m < 0 || m > INT32_MAX) return fail(VQ_ERR_SHAPE, "m=%lld out of range", (long long)m);
    if (!dy || !x) return fail(VQ_ERR_NULL, "dy/x is NULL");
    if (!aligned16(dy) || !aligned16(x)) return fail(VQ_ERR_ALIGN, "dy/x not 16-byte aligned");
    if (dx && !aligned16(dx)) return fail(VQ_ERR_ALIGN, "dx not 16-byte aligned");
    if (w_eff && !aligned16(w_eff)) return fail(VQ_ERR_ALIGN, "w_eff not 16-byte aligned");
    return VQ_OK;
}

// The gate product's share of a backward workspace: its partials (one per
// gate block, or one per dot block where the product writes fp32 dW parts)
// and those parts.  With allow_parts the partial area holds either count, so
// the workspace sizes (which see d but not d_pad) bound every call; the parts
// run when the shape asks for them and d_pad is d rounded up to 256.  Without
// allow_parts: the fused epilogue and its partials only.
struct GateWs {
    bool parts;
    int64_t part_bytes;  // 256-aligned partial area
    int64_t dwp_bytes;   // 256-aligned parts area (0 without allow_parts or parts)
};

GateWs gate_ws(int64_t m, int64_t d, int64_t d_pad, int nsets, const int64_t* n, int64_t n_total, int nslot,
               bool allow_parts) {
    GateWs g{};
    const int64_t fused = vq::gate_partial_count((int)m, (int)n_total, (int)d);
    const bool possible = allow_parts && vq::gate_parts((int)m, (int)n_total, (int)d) > 0;
    const int64_t dot = possible ? vq::gate_dot_blocks(nsets, n, (d + 255) / 256) : 0;
    g.parts = possible && d_pad == (d + 255) / 256 * 256;
    g.part_bytes = align256((fused > dot ? fused : dot) * nslot * (int64_t)sizeof(float));
    g.dwp_bytes = possible ? align256(vq::gate_parts_bytes((int)m, (int)n_total, (int)d)) : 0;
    return g;
}

// The backward's launches: an optional re-mix of W_eff into remix_buf, the
// dX and gate products (one launch when both run), the fixed-order reduce.
// partials: gw.part_bytes of gate partials; tail_ws: dX's split-tail partial
// tiles, or NULL to run dX's tiles whole; dwp: the gate's dW parts when
// gw.parts.  gs: the stream the gate gradient is finished on (the parts
// path's dot pass and the reduce), fenced after the products on s.
int run_bwd(const uint16_t* dy, const uint16_t* x, int64_t m, int64_t n, int64_t d, int64_t d_pad,
            const vq::CandSet& cs, const float* probs, const uint16_t* w_eff, uint16_t* remix_buf, uint16_t* dx,
            float* dprobs, const GateWs& gw, float* partials, float* tail_ws, float* dwp, hipStream_t s,
            hipStream_t gs) {
    int rc = VQ_OK;
    const int ncand = cs.ncand;
    // the parts path when the shape takes it and its buffer is there
    float* parts = gw.parts ? dwp : nullptr;
    if (dx) {
        const uint16_t* w = w_eff;
        if (remix_buf) {
            rc = hip_check(vq::launch_mix(cs, probs, remix_buf, n * d_pad / 256, s), "mix launch");
            if (rc != VQ_OK) return rc;
            w = remix_buf;
        }
        if (m > 0 && dprobs) {
            // both products in one launch: each fills the other's last round
            rc = hip_check(vq::launch_gemm_dx_gate(dy, w, d_pad, dx, x, group_of(cs, n), partials, (int)m, (int)n,
                                                   (int)d, tail_ws, parts, s, gs),
                           "dX + gate GEMM launch");
            if (rc != VQ_OK) return rc;
        } else if (m > 0) {
            rc = hip_check(vq::launch_gemm_dx(dy, w, d_pad, dx, (int)m, (int)n, (int)d, tail_ws, s),
                           "dX GEMM launch");
            if (rc != VQ_OK) return rc;
        }
    }
    if (dprobs) {
        if (m == 0) {
            // no tokens: dL/dp = 0 (written by the reduce over zero partials)
            rc = hip_check(vq::stream_fence(s, gs), "stream fence");
            if (rc == VQ_OK) rc = hip_check(vq::launch_gate_reduce(partials, 0, ncand, dprobs, gs), "gate reduce launch");
            return rc == VQ_OK ? ok() : rc;
        }
        if (!dx) {
            rc = hip_check(
                vq::launch_gemm_gate(dy, x, group_of(cs, n), partials, (int)m, (int)n, (int)d, parts, s, gs),
                "gate GEMM launch");
            if (rc != VQ_OK) return rc;
        }
        // partials: one per dot block on the parts path, one per gate block otherwise
        const int64_t nparts = parts ? vq::gate_dot_blocks(1, &n, d_pad / 256)
                                     : vq::gate_partial_count((int)m, (int)n, (int)d);
        rc = hip_check(vq::stream_fence(s, gs), "stream fence");
        if (rc != VQ_OK) return rc;
        rc = hip_check(vq::launch_gate_reduce(partials, nparts, ncand, dprobs, gs), "gate reduce launch");
        if (rc != VQ_OK) return rc;
    }
    return ok();
}

// Scratch memory of vq_gated_linear_bwd_static, for callers that cannot
// allocate: gate partials, then dX's split-tail tiles when they fit.  One copy
// per device (the code object's own global), held until the process ends;
// its device address is looked up once per device with that device current.
constexpr int64_t kStaticScratchBytes = VQ_STATIC_SCRATCH_BYTES;
static __device__ __align__(256) uint8_t scratch[kStaticScratchBytes];
constexpr int kMaxDevices = 64;
char* g_scratch_ptr[kMaxDevices];
std::mutex g_scratch_mu;

// The device address of `scratch` on the device `s` runs on (the current
// device for the NULL stream).
int static_scratch(hipStream_t s, char** out) {
    int cur = 0;
    int rc = hip_check(hipGetDevice(&cur), "hipGetDevice");
    if (rc != VQ_OK) return rc;
    int dev = cur;
    if (s) {
        rc = hip_check(hipStreamGetDevice(s, &dev), "hipStreamGetDevice");
        if (rc != VQ_OK) return rc;
    }
    if (dev < 0 || dev >= kMaxDevices) return fail(VQ_ERR_HIP, "device %d: beyond the %d devices tracked", dev, kMaxDevices);
    std::lock_guard<std::mutex> lock(g_scratch_mu);
    if (!g_scratch_ptr[dev]) {
        if (dev != cur && (rc = hip_check(hipSetDevice(dev), "hipSetDevice")) != VQ_OK) return rc;
        void* p = nullptr;
        const hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
        if (dev != cur) (void)hipSetDevice(cur);
        rc = hip_check(e, "hipGetSymbolAddress(scratch)");
        if (rc != VQ_OK) return rc;
        g_scratch_ptr[dev] = static_cast<char*>(p);
    }
    *out = g_scratch_ptr[dev];
    return VQ_OK;
}

}  // namespace

extern "C" {

int vq_version(void) { return 100; }

const char* vq_last_error_string(void) { return g_last_error.c_str(); }

int64_t vq_group_bytes(int qtype) { return vq::group_bytes(qtype); }

int64_t vq_qbytes_size(int qtype, int64_t nrows, int64_t ncols) {
    if (!vq::qtype_supported(qtype)) return fail(VQ_ERR_QTYPE, "unsupported ggml type %d", qtype), -1;
    if (nrows < 0 || ncols < 0 || ncols % block_size(qtype) != 0) {
        fail(VQ_ERR_ALIGN, "%s requires in_features %% %d == 0, got %lld", qtype_name(qtype), block_size(qtype),
             (long long)ncols);
        return -1;
    }
    const int64_t bytes_per_block = qtype == vq::Q8_0 ? 34 : vq::group_bytes(qtype);
    return nrows * (ncols / block_size(qtype)) * bytes_per_block;
}

int vq_validate_candidates(int ncand, const int* qtypes, int64_t n, int64_t d, int64_t d_pad) {
    const int rc = check_candidates(ncand, qtypes, nullptr, n, d, d_pad, false);
    return rc == VQ_OK ? ok() : rc;
}

int vq_dequant(int qtype, const void* qbytes, float* out, int64_t nrows, int64_t ncols, void* stream) {
    if (!vq::qtype_supported(qtype)) return fail(VQ_ERR_QTYPE, "unsupported ggml type %d", qtype);
    if (!qbytes || !out) return fail(VQ_ERR_NULL, "qbytes/out is NULL");
    if (nrows < 0 || ncols < 0) return fail(VQ_ERR_SHAPE, "negative size");
    if (ncols % block_size(qtype) != 0)
        return fail(VQ_ERR_ALIGN, "%s requires in_features %% %d == 0, got %lld", qtype_name(qtype),
                    block_size(qtype), (long long)ncols);
    const int64_t total = nrows * ncols;
    if (total % 256 != 0)
        return fail(VQ_ERR_ALIGN, "%s: weight count %lld is not a multiple of 256", qtype_name(qtype),
                    (long long)total);
    if (!aligned16(qbytes) || !aligned16(out)) return fail(VQ_ERR_ALIGN, "qbytes/out not 16-byte aligned");
    int rc = hip_check(vq::launch_dequant(qtype, static_cast<const uint8_t*>(qbytes), out, total / 256,
                                          static_cast<hipStream_t>(stream)),
                       "dequant launch");
    return rc == VQ_OK ? ok() : rc;
}

int vq_dequant_bf16(int qtype, const void* qbytes, uint16_t* out, int64_t nrows, int64_t ncols, void* stream) {
    if (vq::group_bytes(qtype) == 0) return fail(VQ_ERR_QTYPE, "unsupported ggml type %d", qtype);
    if (!qbytes || !out) return fail(VQ_ERR_NULL, "qbytes/out is NULL");
    if (nrows < 0 || ncols < 0) return fail(VQ_ERR_SHAPE, "negative size");
    if (ncols % 256 != 0) return fail(VQ_ERR_ALIGN, "ncols=%lld is not a multiple of 256", (long long)ncols);
    if (!aligned16(qbytes) || !aligned16(out)) return fail(VQ_ERR_ALIGN, "qbytes/out not 16-byte aligned");
    const int64_t total = nrows * ncols;
    int rc = hip_check(vq::launch_dequant_bf16(qtype, static_cast<const uint8_t*>(qbytes), out, total / 256,
                                               static_cast<hipStream_t>(stream)),
                       "dequant launch");
    return rc == VQ_OK ? ok() : rc;
}

int vq_routed_linear_fwd(const uint16_t* x, int64_t m, int64_t n, int64_t d, int64_t d_pad, int ncand,
                         const uint16_t* const* cand_bf16, const int32_t* perm, const int32_t* group_off,
                         uint16_t* y, void* stream) {
    if (ncand < 1 || ncand > vq::kMaxCand) return fail(VQ_ERR_SHAPE, "ncand=%d out of [1, %d]", ncand, vq::kMaxCand);
    if (n <= 0 || d <= 0 || d > d_pad || n > (1 << 21) || d_pad > (1 << 21))
        return fail(VQ_ERR_SHAPE, "sizes n=%lld d=%lld d_pad=%lld", (long long)n, (long long)d, (long long)d_pad);
    if (n % 8 || d % 8 || d_pad % 256) return fail(VQ_ERR_ALIGN, "n, d need multiples of 8 and d_pad of 256");
    if (m < 0 || m * d_pad * 2 >= ((int64_t)1 << 31))
        return fail(VQ_ERR_SHAPE, "m=%lld: m * d_pad * 2 must stay below 2^31", (long long)m);
    if (!x || !y || !perm || !group_off || !cand_bf16) return fail(VQ_ERR_NULL, "x/y/perm/group_off/cand is NULL");
    if (!aligned16(x) || !aligned16(y)) return fail(VQ_ERR_ALIGN, "x/y not 16-byte aligned");
    for (int k = 0; k < ncand; ++k) {
        if (!cand_bf16[k]) return fail(VQ_ERR_NULL, "cand_bf16[%d] is NULL", k);
        if (!aligned16(cand_bf16[k])) return fail(VQ_ERR_ALIGN, "cand_bf16[%d] not 16-byte aligned", k);
    }
    if (m == 0) return ok();
    int rc = hip_check(vq::launch_routed_fwd(x, (int)m, (int)d, cand_bf16, d_pad, (int)n, ncand, perm, group_off, y,
                                             static_cast<hipStream_t>(stream)),
                       "routed GEMM launch");
    return rc == VQ_OK ? ok() : rc;
}

int vq_embedding_rows_fwd(int ncand, const int* qtypes, const void* const* qbytes, const float* probs,
                          const int64_t* routing, const int64_t* ids, int64_t nids, int64_t num_embeddings,
                          int64_t dim, int64_t d_pad, void* out, int out_f32, void* stream) {
    int rc = check_embed(ncand, qtypes, qbytes, ids, nids, num_embeddings, dim, d_pad);
    if (rc != VQ_OK) return rc;
    if (nids == 0) return ok();
    if (!out) return fail(VQ_ERR_NULL, "out is NULL");
    if (!routing && !probs) return fail(VQ_ERR_NULL, "probs is NULL (needed without routing)");
    if (!aligned16(out)) return fail(VQ_ERR_ALIGN, "out not 16-byte aligned");
    const vq::CandSet cs = make_set(ncand, qtypes, qbytes, d_pad);
    rc = hip_check(vq::launch_embed_rows(cs, probs, routing, ids, nids, num_embeddings, dim, out, out_f32 != 0,
                                         static_cast<hipStream_t>(stream)),
                   "embedding rows launch");
    return rc == VQ_OK ? ok() : rc;
}

int64_t vq_embedding_rows_bwd_workspace(int64_t nids, int64_t dim, int ncand) {
    if (nids < 0 || dim <= 0 || ncand < 1 || ncand > vq::kMaxCand) return -1;
    return align256(vq::embed_plan(nids, dim).blocks * ncand * (int64_t)sizeof(float));
}

int vq_embedding_rows_bwd(int ncand, const int* qtypes, const void* const* qbytes, const int64_t* ids,
                          int64_t nids, int64_t num_embeddings, int64_t dim, int64_t d_pad, const void* grad,
                          int grad_f32, float* dprobs, void* workspace, int64_t ws_bytes, void* stream) {
    int rc = check_embed(ncand, qtypes, qbytes, ids, nids, num_embeddings, dim, d_pad);
    if (rc != VQ_OK) return rc;
    if (!dprobs) return fail(VQ_ERR_NULL, "dprobs is NULL");
    if (nids > 0 && !grad) return fail(VQ_ERR_NULL, "grad is NULL");
    if (nids > 0 && !aligned16(grad)) return fail(VQ_ERR_ALIGN, "grad not 16-byte aligned");
    const int64_t need = vq::embed_plan(nids, dim).blocks * ncand * (int64_t)sizeof(float);
    if (need > 0 && (!workspace || ws_bytes < need))
        return fail(VQ_ERR_WORKSPACE, "workspace of %lld bytes needed, %lld given", (long long)need,
                    (long long)ws_bytes);
    const vq::CandSet cs = make_set(ncand, qtypes, qbytes, d_pad);
    rc = hip_check(vq::launch_embed_rows_bwd(cs, ids, nids, num_embeddings, dim, grad, grad_f32 != 0,
                                             static_cast<float*>(workspace), dprobs,
                                             static_cast<hipStream_t>(stream)),
                   "embedding rows backward launch");
    return rc == VQ_OK ? ok() : rc;
}

int vq_mix_weight(int ncand, const int* qtypes, const void* const* qbytes, const float* probs, int64_t n,
                  int64_t d_pad, uint16_t* w_eff, void* stream) {
    // the mix streams whole 256-weight groups: any row count (a vocabulary, say) works
    int rc = check_types(ncand, qtypes, qbytes, true);
    if (rc != VQ_OK) return rc;
    if (n <= 0 || d_pad <= 0) return fail(VQ_ERR_SHAPE, "n=%lld d_pad=%lld must be positive", (long long)n,
                                         (long long)d_pad);
    if (d_pad % 256 != 0) return fail(VQ_ERR_ALIGN, "d_pad=%lld is not a multiple of 256", (long long)d_pad);
    if (!probs || !w_eff) return fail(VQ_ERR_NULL, "probs/w_eff is NULL");
    if (!aligned16(w_eff)) return fail(VQ_ERR_ALIGN, "w_eff not 16-byte aligned");
    const vq::CandSet cs = make_set(ncand, qtypes, qbytes, d_pad);
    rc = hip_check(vq::launch_mix(cs, probs, w_eff, n * d_pad / 256, static_cast<hipStream_t>(stream)),
                   "mix launch");
    return rc == VQ_OK ? ok() : rc;
}

int vq_linear_fwd(const uint16_t* x, int64_t m, int64_t n, int64_t d, const uint16_t* w, int64_t ldw, uint16_t* y,
                  void* workspace, int64_t ws_bytes, void* stream) {
    if (n <= 0 || d <= 0 || m < 0 || n > (1 << 21) || d > (1 << 21) || ldw < d || ldw > (1 << 21))
        return fail(VQ_ERR_SHAPE, "sizes m=%lld n=%lld d=%lld ldw=%lld", (long long)m, (long long)n, (long long)d,
                    (long long)ldw);
    if (n % 8 || d % 8 || ldw % 8) return fail(VQ_ERR_ALIGN, "n, d and ldw must be multiples of 8");
    if (m > INT32_MAX) return fail(VQ_ERR_SHAPE, "m=%lld exceeds 2^31 - 1", (long long)m);
    if (!x || !w || !y) return fail(VQ_ERR_NULL, "x/w/y is NULL");
    if (!aligned16(x) || !aligned16(w) || !aligned16(y)) return fail(VQ_ERR_ALIGN, "x/w/y not 16-byte aligned");
    if (m == 0) return ok();
    const int64_t need = vq::fwd_tail_bytes((int)m, (int)n, (int)d);
    float* tail = (workspace && ws_bytes >= need && need > 0) ? static_cast<float*>(workspace) : nullptr;
    int rc = hip_check(vq::launch_gemm_fwd(reinterpret_cast<const vq::bf16_t*>(x),
                                           reinterpret_cast<const vq::bf16_t*>(w), ldw, reinterpret_cast<vq::bf16_t*>(y),
                                           (int)m, (int)n, (int)d, tail, static_cast<hipStream_t>(stream)),
                       "GEMM launch");
    return rc == VQ_OK ? ok() : rc;
}

namespace {
int check_rope(int64_t B, int64_t S, int Hq, int Hkv, int D, const void* cosb, const void* sinb) {
    if (B < 0 || S <= 0 || Hq <= 0 || Hkv <= 0 || D <= 0 || B * S > INT32_MAX)
        return fail(VQ_ERR_SHAPE, "B=%lld S=%lld Hq=%d Hkv=%d D=%d", (long long)B, (long long)S, Hq, Hkv, D);
    if (Hq % Hkv) return fail(VQ_ERR_SHAPE, "Hq=%d is not a multiple of Hkv=%d", Hq, Hkv);
    if (D % 16) return fail(VQ_ERR_ALIGN, "head dim %d must be a multiple of 16", D);
    if (!cosb || !sinb) return fail(VQ_ERR_NULL, "cos/sin is NULL");
    if (!aligned16(cosb) || !aligned16(sinb)) return fail(VQ_ERR_ALIGN, "cos/sin not 16-byte aligned");
    return VQ_OK;
}
}  // namespace

int vq_rope_qkv_fwd(const uint16_t* qkv, int64_t B, int64_t S, int Hq, int Hkv, int kv_heads_out, int D,
                    const float* cosb, const float* sinb, uint16_t* q, uint16_t* k, uint16_t* v, void* stream) {
    int rc = check_rope(B, S, Hq, Hkv, D, cosb, sinb);
    if (rc != VQ_OK) return rc;
    if (kv_heads_out != Hq && kv_heads_out != Hkv)
        return fail(VQ_ERR_SHAPE, "kv_heads_out=%d: Hq (%d, heads repeated) or Hkv (%d)", kv_heads_out, Hq, Hkv);
    if (B == 0) return ok();
    if (!qkv || !q || !k || !v) return fail(VQ_ERR_NULL, "qkv/q/k/v is NULL");
    if (!aligned16(qkv) || !aligned16(q) || !aligned16(k) || !aligned16(v))
        return fail(VQ_ERR_ALIGN, "qkv/q/k/v not 16-byte aligned");
    rc = hip_check(vq::launch_rope_qkv_fwd(reinterpret_cast<const vq::bf16_t*>(qkv), B * S, (int)S, Hq, Hkv,
                                           kv_heads_out, D, cosb, sinb, reinterpret_cast<vq::bf16_t*>(q), reinterpret_cast<vq::bf16_t*>(k),
                                           reinterpret_cast<vq::bf16_t*>(v), static_cast<hipStream_t>(stream)),
                   "rope launch");
    return rc == VQ_OK ? ok() : rc;
}

int vq_rope_qkv_bwd(const uint16_t* dq, const uint16_t* dk, const uint16_t* dv, int64_t stride_b, int64_t stride_h,
                    int64_t stride_s, int64_t B, int64_t S, int Hq, int Hkv, int D, const float* cosb,
                    const float* sinb, uint16_t* dqkv, void* stream) {
    int rc = check_rope(B, S, Hq, Hkv, D, cosb, sinb);
    if (rc != VQ_OK) return rc;
    if (B == 0) return ok();
    if (!dq || !dk || !dv || !dqkv) return fail(VQ_ERR_NULL, "dq/dk/dv/dqkv is NULL");
    if (!aligned16(dq) || !aligned16(dk) || !aligned16(dv) || !aligned16(dqkv) || stride_b % 8 || stride_h % 8 ||
        stride_s % 8)
        return fail(VQ_ERR_ALIGN, "gradients not 16-byte aligned (pointers and strides)");
    rc = hip_check(vq::launch_rope_qkv_bwd(reinterpret_cast<const vq::bf16_t*>(dq),
                                           reinterpret_cast<const vq::bf16_t*>(dk),
                                           reinterpret_cast<const vq::bf16_t*>(dv), stride_b, stride_h, stride_s,
                                           B * S, (int)S, Hq, Hkv, D, cosb, sinb, reinterpret_cast<vq::bf16_t*>(dqkv),
                                           static_cast<hipStream_t>(stream)),
                   "rope backward launch");
    return rc == VQ_OK ? ok() : rc;
}

int vq_swiglu_fwd(const uint16_t* gu, int64_t tokens, int64_t F, uint16_t* out, void* stream) {
    if (tokens < 0 || F <= 0 || F > INT32_MAX) return fail(VQ_ERR_SHAPE, "tokens=%lld F=%lld", (long long)tokens, (long long)F);
    if (F % 8) return fail(VQ_ERR_ALIGN, "F=%lld must be a multiple of 8", (long long)F);
    if (tokens == 0) return ok();
    if (!gu || !out) return fail(VQ_ERR_NULL, "gu/out is NULL");
    if (!aligned16(gu) || !aligned16(out)) return fail(VQ_ERR_ALIGN, "gu/out not 16-byte aligned");
    int rc = hip_check(vq::launch_swiglu_fwd(reinterpret_cast<const vq::bf16_t*>(gu), tokens, (int)F,
                                             reinterpret_cast<vq::bf16_t*>(out), static_cast<hipStream_t>(stream)),
                       "swiglu launch");
    return rc == VQ_OK ? ok() : rc;
}

int vq_swiglu_bwd(const uint16_t* gu, const uint16_t* dy, int64_t tokens, int64_t F, uint16_t* dgu, void* stream) {
    if (tokens < 0 || F <= 0 || F > INT32_MAX) return fail(VQ_ERR_SHAPE, "tokens=%lld F=%lld", (long long)tokens, (long long)F);
    if (F % 8) return fail(VQ_ERR_ALIGN, "F=%lld must be a multiple of 8", (long long)F);
    if (tokens == 0) return ok();
    if (!gu || !dy || !dgu) return fail(VQ_ERR_NULL, "gu/dy/dgu is NULL");
    if (!aligned16(gu) || !aligned16(dy) || !aligned16(dgu)) return fail(VQ_ERR_ALIGN, "gu/dy/dgu not 16-byte aligned");
    int rc = hip_check(vq::launch_swiglu_bwd(reinterpret_cast<const vq::bf16_t*>(gu),
                                             reinterpret_cast<const vq::bf16_t*>(dy), tokens, (int)F,
                                             reinterpret_cast<vq::bf16_t*>(dgu), static_cast<hipStream_t>(stream)),
                       "swiglu backward launch");
    return rc == VQ_OK ? ok() : rc;
}

static int check_norm(int64_t rows, int64_t dim) {
    if (rows < 0 || dim <= 0 || dim > INT32_MAX)
        return fail(VQ_ERR_SHAPE, "rows=%lld dim=%lld", (long long)rows, (long long)dim);
    if (dim % 8) return fail(VQ_ERR_ALIGN, "dim=%lld must be a multiple of 8", (long long)dim);
    return VQ_OK;
}

int vq_add_rmsnorm_fwd(const uint16_t* h, const uint16_t* a, const uint16_t* w, int64_t rows, int64_t dim, float eps,
                       uint16_t* s_out, uint16_t* n_out, float* rstd_out, void* stream) {
    int rc = check_norm(rows, dim);
    if (rc != VQ_OK) return rc;
    if (!(eps >= 0.0f)) return fail(VQ_ERR_SHAPE, "eps must be >= 0");
    if (rows == 0) return ok();
    if (!h || !w || !n_out) return fail(VQ_ERR_NULL, "h/w/n_out is NULL");
    if (!aligned16(h) || !aligned16(w) || !aligned16(n_out) || (a && !aligned16(a)) || (s_out && !aligned16(s_out)))
        return fail(VQ_ERR_ALIGN, "h/a/w/s_out/n_out not 16-byte aligned");
    rc = hip_check(vq::launch_add_rmsnorm_fwd(reinterpret_cast<const vq::bf16_t*>(h),
                                              reinterpret_cast<const vq::bf16_t*>(a),
                                              reinterpret_cast<const vq::bf16_t*>(w), rows, (int)dim, eps,
                                              reinterpret_cast<vq::bf16_t*>(s_out), reinterpret_cast<vq::bf16_t*>(n_out),
                                              rstd_out, static_cast<hipStream_t>(stream)),
                   "add_rmsnorm launch");
    return rc == VQ_OK ? ok() : rc;
}

int vq_rmsnorm_bwd(const uint16_t* dn, const uint16_t* ds, const uint16_t* s, const uint16_t* w, const float* rstd,
                   int64_t rows, int64_t dim, uint16_t* dh, void* stream) {
    int rc = check_norm(rows, dim);
    if (rc != VQ_OK) return rc;
    if (rows == 0) return ok();
    if (!dn || !s || !w || !rstd || !dh) return fail(VQ_ERR_NULL, "dn/s/w/rstd/dh is NULL");
    if (!aligned16(dn) || !aligned16(s) || !aligned16(w) || !aligned16(dh) || (ds && !aligned16(ds)))
        return fail(VQ_ERR_ALIGN, "dn/ds/s/w/dh not 16-byte aligned");
    rc = hip_check(vq::launch_rmsnorm_bwd(reinterpret_cast<const vq::bf16_t*>(dn),
                                          reinterpret_cast<const vq::bf16_t*>(ds),
                                          reinterpret_cast<const vq::bf16_t*>(s),
                                          reinterpret_cast<const vq::bf16_t*>(w), rstd, rows, (int)dim,
                                          reinterpret_cast<vq::bf16_t*>(dh), static_cast<hipStream_t>(stream)),
                   "rmsnorm backward launch");
    return rc == VQ_OK ? ok() : rc;
}

int vq_attention_fwd(const uint16_t* q, const uint16_t* k, const uint16_t* v, uint16_t* o, float* lse, int64_t B,
                     int64_t S, int Hq, int Hk, int D, const int64_t* q_strides, const int64_t* k_strides,
                     const int64_t* v_strides, const int64_t* o_strides, float scale, void* stream) {
    if (B < 0 || S < 0 || S > INT32_MAX / 2 || Hq <= 0 || Hk <= 0 || Hq % Hk)
        return fail(VQ_ERR_SHAPE, "B=%lld S=%lld Hq=%d Hk=%d", (long long)B, (long long)S, Hq, Hk);
    if (D != 64) return fail(VQ_ERR_SHAPE, "head dim %d: only 64 is supported", D);
    if (B * Hq * ((S + 127) / 128) > INT32_MAX)
        return fail(VQ_ERR_SHAPE, "B=%lld Hq=%d S=%lld: too many query tiles", (long long)B, Hq, (long long)S);
    if (!(scale > 0.0f) || scale > 1e30f) return fail(VQ_ERR_SHAPE, "scale must be positive and finite");
    if (B == 0 || S == 0) return ok();
    if (!q || !k || !v || !o) return fail(VQ_ERR_NULL, "q/k/v/o is NULL");
    if (!q_strides || !k_strides || !v_strides || !o_strides) return fail(VQ_ERR_NULL, "a stride array is NULL");
    if (!aligned16(q) || !aligned16(k) || !aligned16(v) || !aligned16(o) || (lse && (reinterpret_cast<uintptr_t>(lse) & 3)))
        return fail(VQ_ERR_ALIGN, "q/k/v/o not 16-byte aligned (or lse not 4-byte aligned)");
    for (const int64_t* st : {q_strides, k_strides, v_strides, o_strides})
        for (int i = 0; i < 3; ++i)
            if (st[i] < 0 || st[i] % 8) return fail(VQ_ERR_ALIGN, "strides must be non-negative multiples of 8");
    // a 64-key tile is addressed by 32-bit byte offsets from its first row
    if (k_strides[1] > (1 << 22) || v_strides[1] > (1 << 22))
        return fail(VQ_ERR_SHAPE, "k/v position strides above 2^22 elements");
    int rc = hip_check(vq::launch_attention_fwd(reinterpret_cast<const vq::bf16_t*>(q),
                                                reinterpret_cast<const vq::bf16_t*>(k),
                                                reinterpret_cast<const vq::bf16_t*>(v), reinterpret_cast<vq::bf16_t*>(o),
                                                lse, (int)B, (int)S, Hq, Hk, q_strides, k_strides, v_strides, o_strides,
                                                scale, static_cast<hipStream_t>(stream)),
                       "attention launch");
    return rc == VQ_OK ? ok() : rc;
}

int64_t vq_attention_bwd_workspace(int64_t B, int64_t S, int Hq) {
    if (B < 0 || S < 0 || S > INT32_MAX / 2 || Hq <= 0 || B * Hq > INT32_MAX) return -1;
    return align256(vq::attention_bwd_workspace((int)B, (int)S, Hq));
}

int vq_attention_bwd(const uint16_t* q, const uint16_t* k, const uint16_t* v, const uint16_t* o, const uint16_t* dout,
                     const float* lse, uint16_t* dq, uint16_t* dk, uint16_t* dv, int64_t B, int64_t S, int Hq, int Hk,
                     int D, const int64_t* strides, float scale, void* workspace, int64_t ws_bytes, void* stream) {
    if (B < 0 || S < 0 || S > INT32_MAX / 2 || Hq <= 0 || Hk <= 0 || Hq % Hk)
        return fail(VQ_ERR_SHAPE, "B=%lld S=%lld Hq=%d Hk=%d", (long long)B, (long long)S, Hq, Hk);
    if (D != 64) return fail(VQ_ERR_SHAPE, "head dim %d: only 64 is supported", D);
    if (B * Hq * ((S + 127) / 128) > INT32_MAX)
        return fail(VQ_ERR_SHAPE, "B=%lld Hq=%d S=%lld: too many tiles", (long long)B, Hq, (long long)S);
    if (!(scale > 0.0f) || scale > 1e30f) return fail(VQ_ERR_SHAPE, "scale must be positive and finite");
    if (B == 0 || S == 0) return ok();
    if (!q || !k || !v || !o || !dout || !lse || !dq || !dk || !dv) return fail(VQ_ERR_NULL, "a tensor pointer is NULL");
    if (!strides) return fail(VQ_ERR_NULL, "strides is NULL");
    for (const void* p : {(const void*)q, (const void*)k, (const void*)v, (const void*)o, (const void*)dout,
                          (const void*)dq, (const void*)dk, (const void*)dv})
        if (!aligned16(p)) return fail(VQ_ERR_ALIGN, "tensors must be 16-byte aligned");
    if (reinterpret_cast<uintptr_t>(lse) & 3) return fail(VQ_ERR_ALIGN, "lse not 4-byte aligned");
    for (int i = 0; i < 24; ++i)
        if (strides[i] < 0 || strides[i] % 8) return fail(VQ_ERR_ALIGN, "strides must be non-negative multiples of 8");
    // 64-key and 128-query tiles are addressed by 32-bit byte offsets from their first row
    if (strides[1] > (1 << 22) || strides[4] > (1 << 22) || strides[7] > (1 << 22) || strides[13] > (1 << 22))
        return fail(VQ_ERR_SHAPE, "q/k/v/dout position strides above 2^22 elements");
    const int64_t need = vq_attention_bwd_workspace(B, S, Hq);
    if (!workspace || ws_bytes < need || !aligned16(workspace))
        return fail(VQ_ERR_WORKSPACE, "workspace %lld bytes at %p, need %lld (16-byte aligned)", (long long)ws_bytes,
                    workspace, (long long)need);
    int rc = hip_check(vq::launch_attention_bwd(reinterpret_cast<const vq::bf16_t*>(q),
                                                reinterpret_cast<const vq::bf16_t*>(k),
                                                reinterpret_cast<const vq::bf16_t*>(v),
                                                reinterpret_cast<const vq::bf16_t*>(o),
                                                reinterpret_cast<const vq::bf16_t*>(dout), lse,
                                                reinterpret_cast<vq::bf16_t*>(dq), reinterpret_cast<vq::bf16_t*>(dk),
                                                reinterpret_cast<vq::bf16_t*>(dv), (int)B, (int)S, Hq, Hk, strides, scale,
                                                static_cast<float*>(workspace), static_cast<hipStream_t>(stream)),
                       "attention backward launch");
    return rc == VQ_OK ? ok() : rc;
}

int64_t vq_distill_loss_workspace(int64_t rows) {
    if (rows < 0) return -1;
    return align256((5 * rows + 2) * (int64_t)sizeof(float));
}

namespace {
int check_distill(const uint16_t* logits, const uint16_t* teacher_logits, const int64_t* labels, int64_t rows,
                  int64_t vocab, float temperature, const void* ws, int64_t ws_bytes) {
    if (rows <= 0 || vocab <= 0 || rows > INT32_MAX)
        return fail(VQ_ERR_SHAPE, "rows=%lld vocab=%lld", (long long)rows, (long long)vocab);
    if (vocab % 8) return fail(VQ_ERR_ALIGN, "vocab=%lld must be a multiple of 8", (long long)vocab);
    if (!(temperature > 0.0f)) return fail(VQ_ERR_SHAPE, "temperature must be positive");
    if (!logits || !teacher_logits || !labels) return fail(VQ_ERR_NULL, "logits/teacher_logits/labels is NULL");
    if (!aligned16(logits) || !aligned16(teacher_logits)) return fail(VQ_ERR_ALIGN, "logits not 16-byte aligned");
    if (!ws || ws_bytes < (5 * rows + 2) * (int64_t)sizeof(float))
        return fail(VQ_ERR_WORKSPACE, "workspace of %lld bytes needed", (long long)((5 * rows + 2) * 4));
    return VQ_OK;
}
}  // namespace

int vq_distill_loss_fwd(const uint16_t* logits, const uint16_t* teacher_logits, const int64_t* labels, int64_t rows,
                        int64_t vocab, float temperature, float* out, void* workspace, int64_t ws_bytes,
                        void* stream) {
    int rc = check_distill(logits, teacher_logits, labels, rows, vocab, temperature, workspace, ws_bytes);
    if (rc != VQ_OK) return rc;
    if (!out) return fail(VQ_ERR_NULL, "out is NULL");
    rc = hip_check(vq::launch_distill_fwd(reinterpret_cast<const vq::bf16_t*>(logits),
                                          reinterpret_cast<const vq::bf16_t*>(teacher_logits), labels, rows, vocab,
                                          temperature, out, static_cast<float*>(workspace),
                                          static_cast<hipStream_t>(stream)),
                   "distillation loss launch");
    return rc == VQ_OK ? ok() : rc;
}

int vq_distill_loss_bwd(const uint16_t* logits, const uint16_t* teacher_logits, const int64_t* labels, int64_t rows,
                        int64_t vocab, float temperature, const float* grad_out, uint16_t* grad_logits,
                        const void* workspace, int64_t ws_bytes, void* stream) {
    int rc = check_distill(logits, teacher_logits, labels, rows, vocab, temperature, workspace, ws_bytes);
    if (rc != VQ_OK) return rc;
    if (!grad_out || !grad_logits) return fail(VQ_ERR_NULL, "grad_out/grad_logits is NULL");
    if (!aligned16(grad_logits)) return fail(VQ_ERR_ALIGN, "grad_logits not 16-byte aligned");
    rc = hip_check(vq::launch_distill_bwd(reinterpret_cast<const vq::bf16_t*>(logits),
                                          reinterpret_cast<const vq::bf16_t*>(teacher_logits), labels, rows, vocab,
                                          temperature, grad_out, reinterpret_cast<vq::bf16_t*>(grad_logits),
                                          static_cast<const float*>(workspace), static_cast<hipStream_t>(stream)),
                   "distillation loss backward launch");
    return rc == VQ_OK ? ok() : rc;
}

int64_t vq_gated_linear_fwd_workspace(int64_t m, int64_t n, int64_t d) {
    if (m < 0 || n <= 0 || d <= 0 || m > INT32_MAX || n > INT32_MAX || d > INT32_MAX) return -1;
    return align256(vq::fwd_tail_bytes((int)m, (int)n, (int)d));
}

int vq_gated_linear_fwd(const uint16_t* x, int64_t m, int64_t n, int64_t d, int64_t d_pad, int ncand,
                        const int* qtypes, const void* const* qbytes, const float* probs, uint16_t* w_eff,
                        uint16_t* y, void* workspace, int64_t ws_bytes, void* stream) {
    int rc = check_candidates(ncand, qtypes, qbytes, n, d, d_pad, true);
    if (rc != VQ_OK) return rc;
    if (m < 0 || m > INT32_MAX) return fail(VQ_ERR_SHAPE, "m=%lld out of range", (long long)m);
    if (!probs || !w_eff) return fail(VQ_ERR_NULL, "probs/w_eff is NULL");
    if (m > 0 && (!x || !y)) return fail(VQ_ERR_NULL, "x/y is NULL");  // m == 0: the mix alone
    if (!aligned16(x) || !aligned16(w_eff) || !aligned16(y))
        return fail(VQ_ERR_ALIGN, "x/w_eff/y not 16-byte aligned");
    hipStream_t s = static_cast<hipStream_t>(stream);
    const vq::CandSet cs = make_set(ncand, qtypes, qbytes, d_pad);
    rc = hip_check(vq::launch_mix(cs, probs, w_eff, n * d_pad / 256, s), "mix launch");
    if (rc != VQ_OK) return rc;
    if (m == 0) return ok();
    if (workspace && !aligned16(workspace)) return fail(VQ_ERR_ALIGN, "workspace not 16-byte aligned");
    const int64_t tail_bytes = vq::fwd_tail_bytes((int)m, (int)n, (int)d);
    float* tail_ws = workspace && tail_bytes > 0 && ws_bytes >= tail_bytes ? static_cast<float*>(workspace) : nullptr;
    rc = hip_check(vq::launch_gemm_fwd(x, w_eff, d_pad, y, (int)m, (int)n, (int)d, tail_ws, s),
                   "forward GEMM launch");
    return rc == VQ_OK ? ok() : rc;
}

int64_t vq_gated_linear_bwd_workspace(int64_t m, int64_t n, int64_t d, int64_t d_pad, int ncand, int need_w_eff) {
    if (m < 0 || n <= 0 || d <= 0 || ncand < 1 || m > INT32_MAX || n > INT32_MAX || d > INT32_MAX) return -1;
    // [gate partials][dX split-tail partial tiles][gate dW parts][re-mixed W_eff]
    const GateWs gw = gate_ws(m, d, d_pad, 1, &n, n, ncand, true);
    int64_t bytes = gw.part_bytes + align256(vq::dx_tail_bytes((int)m, (int)n, (int)d)) + gw.dwp_bytes;
    if (need_w_eff) bytes += align256(n * d_pad * 2);
    return bytes;
}

int vq_gated_linear_bwd(const uint16_t* dy, const uint16_t* x, int64_t m, int64_t n, int64_t d, int64_t d_pad,
                        int ncand, const int* qtypes, const void* const* qbytes, const float* probs,
                        const uint16_t* w_eff, uint16_t* dx, float* dprobs, void* workspace, int64_t ws_bytes,
                        void* stream) {
    return vq_gated_linear_bwd_gate_stream(dy, x, m, n, d, d_pad, ncand, qtypes, qbytes, probs, w_eff, dx, dprobs,
                                           workspace, ws_bytes, stream, stream);
}

int vq_gated_linear_bwd_gate_stream(const uint16_t* dy, const uint16_t* x, int64_t m, int64_t n, int64_t d,
                                    int64_t d_pad, int ncand, const int* qtypes, const void* const* qbytes,
                                    const float* probs, const uint16_t* w_eff, uint16_t* dx, float* dprobs,
                                    void* workspace, int64_t ws_bytes, void* stream, void* gate_stream) {
    int rc = check_bwd(dy, x, m, n, d, d_pad, ncand, qtypes, qbytes, w_eff, dx);
    if (rc != VQ_OK) return rc;
    const bool remix = dx != nullptr && w_eff == nullptr;
    const int64_t need = vq_gated_linear_bwd_workspace(m, n, d, d_pad, ncand, remix ? 1 : 0);
    const GateWs gw = gate_ws(m, d, d_pad, 1, &n, n, ncand, true);
    const int64_t part_bytes = gw.part_bytes;
    if ((dprobs || remix) && (!workspace || ws_bytes < need))
        return fail(VQ_ERR_WORKSPACE, "workspace of %lld bytes required, got %lld", (long long)need,
                    (long long)(workspace ? ws_bytes : 0));
    if (workspace && !aligned16(workspace)) return fail(VQ_ERR_ALIGN, "workspace not 16-byte aligned");
    float* partials = static_cast<float*>(workspace);
    const int64_t tail_bytes = align256(vq::dx_tail_bytes((int)m, (int)n, (int)d));
    // dX splits its tail tiles along K only with room for their partials
    float* tail_ws = nullptr;
    if (workspace && tail_bytes > 0 && ws_bytes >= part_bytes + tail_bytes)
        tail_ws = reinterpret_cast<float*>(static_cast<char*>(workspace) + part_bytes);
    float* dwp = gw.parts && workspace && ws_bytes >= need
                     ? reinterpret_cast<float*>(static_cast<char*>(workspace) + part_bytes + tail_bytes)
                     : nullptr;
    uint16_t* remix_buf = nullptr;
    if (remix) {
        if (!probs) return fail(VQ_ERR_NULL, "probs is NULL");
        remix_buf = reinterpret_cast<uint16_t*>(static_cast<char*>(workspace) + part_bytes + tail_bytes + gw.dwp_bytes);
    }
    return run_bwd(dy, x, m, n, d, d_pad, make_set(ncand, qtypes, qbytes, d_pad), probs, w_eff, remix_buf, dx, dprobs,
                   gw, partials, tail_ws, dwp, static_cast<hipStream_t>(stream), static_cast<hipStream_t>(gate_stream));
}

int vq_gated_linear_bwd_static(const uint16_t* dy, const uint16_t* x, int64_t m, int64_t n, int64_t d, int64_t d_pad,
                               int ncand, const int* qtypes, const void* const* qbytes, const uint16_t* w_eff,
                               uint16_t* dx, float* dprobs, void* stream) {
    int rc = check_bwd(dy, x, m, n, d, d_pad, ncand, qtypes, qbytes, w_eff, dx);
    if (rc != VQ_OK) return rc;
    if (dx && !w_eff) return fail(VQ_ERR_NULL, "dx needs the forward's w_eff (this entry point does not re-mix)");
    // the fused gate epilogue only: dW parts would not fit the scratch
    const GateWs gw = gate_ws(m, d, d_pad, 1, &n, n, ncand, false);
    const int64_t part_bytes = gw.part_bytes;
    if (dprobs && part_bytes > kStaticScratchBytes)
        return fail(VQ_ERR_WORKSPACE, "m=%lld n=%lld d=%lld ncand=%d needs %lld bytes of gate partials; the static "
                    "scratch holds %lld (use vq_gated_linear_bwd with a workspace)", (long long)m, (long long)n,
                    (long long)d, ncand, (long long)part_bytes, (long long)kStaticScratchBytes);
    hipStream_t s = static_cast<hipStream_t>(stream);
    char* scratch_ptr = nullptr;
    rc = static_scratch(s, &scratch_ptr);
    if (rc != VQ_OK) return rc;
    // dX runs whole tiles: a split tail keeps 8 XCDs x (tiles x parts, at least
    // 8 for any split the plan makes with 32 CUs per XCD) x 256 KiB of fp32
    // partials, 16 MiB or more, which the scratch never holds
    return run_bwd(dy, x, m, n, d, d_pad, make_set(ncand, qtypes, qbytes, d_pad), nullptr, w_eff, nullptr, dx, dprobs,
                   gw, reinterpret_cast<float*>(scratch_ptr), nullptr, nullptr, s, s);
}

int64_t vq_gated_linear_fused_workspace(int64_t m, int64_t n, int64_t d, int dx) {
    if (m < 0 || n <= 0 || d <= 0 || m > INT32_MAX || n > (1 << 21) || d > (1 << 21)) return -1;
    if (m == 0) return 0;
    return align256(vq::fused_plan(dx != 0, (int)m, (int)n, (int)d).ws_bytes);
}

namespace {
int run_fused(bool dx, const uint16_t* act, int64_t m, int64_t n, int64_t d, int64_t d_pad, int ncand,
              const int* qtypes, const void* const* qbytes, const float* probs, uint16_t* out, void* workspace,
              int64_t ws_bytes, void* stream) {
    int rc = check_candidates(ncand, qtypes, qbytes, n, d, d_pad, true);
    if (rc != VQ_OK) return rc;
    if (m < 0 || m > INT32_MAX) return fail(VQ_ERR_SHAPE, "m=%lld out of range", (long long)m);
    if (!act || !probs || !out) return fail(VQ_ERR_NULL, "%s/probs/%s is NULL", dx ? "dy" : "x", dx ? "dx" : "y");
    if (!aligned16(act) || !aligned16(out)) return fail(VQ_ERR_ALIGN, "activations/output not 16-byte aligned");
    if (m == 0) return ok();
    const int64_t need = vq::fused_plan(dx, (int)m, (int)n, (int)d).ws_bytes;
    if (need > 0 && (!workspace || ws_bytes < need))
        return fail(VQ_ERR_WORKSPACE, "workspace of %lld bytes required, got %lld", (long long)need,
                    (long long)(workspace ? ws_bytes : 0));
    if (workspace && !aligned16(workspace)) return fail(VQ_ERR_ALIGN, "workspace not 16-byte aligned");
    rc = hip_check(vq::launch_fused(dx, act, make_set(ncand, qtypes, qbytes, d_pad), probs, (int)m, (int)n, (int)d,
                                    out, need > 0 ? static_cast<float*>(workspace) : nullptr,
                                    static_cast<hipStream_t>(stream)),
                   dx ? "fused dX launch" : "fused forward launch");
    return rc == VQ_OK ? ok() : rc;
}
}  // namespace

int vq_gated_linear_fwd_fused(const uint16_t* x, int64_t m, int64_t n, int64_t d, int64_t d_pad, int ncand,
                              const int* qtypes, const void* const* qbytes, const float* probs, uint16_t* y,
                              void* workspace, int64_t ws_bytes, void* stream) {
    return run_fused(false, x, m, n, d, d_pad, ncand, qtypes, qbytes, probs, y, workspace, ws_bytes, stream);
}

int vq_gated_linear_dx_fused(const uint16_t* dy, int64_t m, int64_t n, int64_t d, int64_t d_pad, int ncand,
                             const int* qtypes, const void* const* qbytes, const float* probs, uint16_t* dx,
                             void* workspace, int64_t ws_bytes, void* stream) {
    return run_fused(true, dy, m, n, d, d_pad, ncand, qtypes, qbytes, probs, dx, workspace, ws_bytes, stream);
}

int vq_gated_linear_group_fwd(const uint16_t* x, int64_t m, int64_t d, int64_t d_pad, int nmembers, const int64_t* n,
                              const int* ncand, const int* qtypes, const void* const* qbytes,
                              const float* const* probs, uint16_t* w_eff, uint16_t* y, void* workspace,
                              int64_t ws_bytes, void* stream) {
    vq::CandGroup cg;
    int64_t n_total = 0;
    int rc = check_group(nmembers, n, ncand, qtypes, qbytes, d, d_pad, cg, n_total);
    if (rc != VQ_OK) return rc;
    if (m < 0 || m > INT32_MAX) return fail(VQ_ERR_SHAPE, "m=%lld out of range", (long long)m);
    if (!probs || !w_eff) return fail(VQ_ERR_NULL, "probs/w_eff is NULL");
    if (m > 0 && (!x || !y)) return fail(VQ_ERR_NULL, "x/y is NULL");  // m == 0: the mixes alone
    if (!aligned16(x) || !aligned16(w_eff) || !aligned16(y))
        return fail(VQ_ERR_ALIGN, "x/w_eff/y not 16-byte aligned");
    hipStream_t s = static_cast<hipStream_t>(stream);
    vq::bf16_t* outs[vq::kMaxSets];
    int64_t ngroups[vq::kMaxSets];
    for (int i = 0; i < nmembers; ++i) {
        if (!probs[i]) return fail(VQ_ERR_NULL, "probs[%d] is NULL", i);
        outs[i] = w_eff + (int64_t)cg.set_j0[i] * d_pad;
        ngroups[i] = n[i] * d_pad / 256;
    }
    rc = hip_check(vq::launch_mix_sets(nmembers, cg.sets, probs, outs, ngroups, s), "mix launch");
    if (rc != VQ_OK) return rc;
    if (m == 0) return ok();
    if (workspace && !aligned16(workspace)) return fail(VQ_ERR_ALIGN, "workspace not 16-byte aligned");
    const int64_t tail_bytes = vq::fwd_tail_bytes((int)m, (int)n_total, (int)d);
    float* tail_ws = workspace && tail_bytes > 0 && ws_bytes >= tail_bytes ? static_cast<float*>(workspace) : nullptr;
    rc = hip_check(vq::launch_gemm_fwd(x, w_eff, d_pad, y, (int)m, (int)n_total, (int)d, tail_ws, s),
                   "forward GEMM launch");
    return rc == VQ_OK ? ok() : rc;
}

int64_t vq_gated_linear_group_bwd_workspace(int64_t m, int64_t d, int nmembers, const int64_t* n, const int* ncand) {
    if (m < 0 || d <= 0 || m > INT32_MAX || d > INT32_MAX || nmembers < 1 || nmembers > vq::kMaxSets || !n || !ncand)
        return -1;
    int64_t n_total = 0;
    int kstride = 0;
    for (int i = 0; i < nmembers; ++i) {
        if (n[i] <= 0 || ncand[i] < 1 || ncand[i] > vq::kMaxCand) return -1;
        n_total += n[i];
        kstride = ncand[i] > kstride ? ncand[i] : kstride;
    }
    if (n_total > INT32_MAX) return -1;
    // [gate partials][dX split-tail partial tiles][gate dW parts]; d_pad = the
    // 256-multiple the candidates are padded to
    const GateWs gw = gate_ws(m, d, (d + 255) / 256 * 256, nmembers, n, n_total, nmembers * kstride, true);
    return gw.part_bytes + align256(vq::dx_tail_bytes((int)m, (int)n_total, (int)d)) + gw.dwp_bytes;
}

int vq_gated_linear_group_bwd(const uint16_t* dy, const uint16_t* x, int64_t m, int64_t d, int64_t d_pad, int nmembers,
                              const int64_t* n, const int* ncand, const int* qtypes, const void* const* qbytes,
                              const uint16_t* w_eff, uint16_t* dx, float* const* dprobs, void* workspace,
                              int64_t ws_bytes, void* stream) {
    return vq_gated_linear_group_bwd_gate_stream(dy, x, m, d, d_pad, nmembers, n, ncand, qtypes, qbytes, w_eff, dx,
                                                 dprobs, workspace, ws_bytes, stream, stream);
}

int vq_gated_linear_group_bwd_gate_stream(const uint16_t* dy, const uint16_t* x, int64_t m, int64_t d, int64_t d_pad,
                                          int nmembers, const int64_t* n, const int* ncand, const int* qtypes,
                                          const void* const* qbytes, const uint16_t* w_eff, uint16_t* dx,
                                          float* const* dprobs, void* workspace, int64_t ws_bytes, void* stream,
                                          void* gate_stream) {
    vq::CandGroup cg;
    int64_t n_total = 0;
    int rc = check_group(nmembers, n, ncand, qtypes, qbytes, d, d_pad, cg, n_total);
    if (rc != VQ_OK) return rc;
    if (m < 0 || m > INT32_MAX) return fail(VQ_ERR_SHAPE, "m=%lld out of range", (long long)m);
    if (!dy || !x) return fail(VQ_ERR_NULL, "dy/x is NULL");
    if (!aligned16(dy) || !aligned16(x)) return fail(VQ_ERR_ALIGN, "dy/x not 16-byte aligned");
    if (dx && (!w_eff || !aligned16(dx) || !aligned16(w_eff)))
        return fail(w_eff ? VQ_ERR_ALIGN : VQ_ERR_NULL, "dx needs the forward's 16-byte aligned w_eff");
    if (dprobs)
        for (int i = 0; i < nmembers; ++i)
            if (!dprobs[i]) return fail(VQ_ERR_NULL, "dprobs[%d] is NULL", i);
    hipStream_t s = static_cast<hipStream_t>(stream), gs = static_cast<hipStream_t>(gate_stream);
    const int64_t need = vq_gated_linear_group_bwd_workspace(m, d, nmembers, n, ncand);
    const int nslot = nmembers * cg.kstride;
    const GateWs gw = gate_ws(m, d, d_pad, nmembers, n, n_total, nslot, true);
    const int64_t part_bytes = gw.part_bytes;
    if (dprobs && (!workspace || ws_bytes < need))
        return fail(VQ_ERR_WORKSPACE, "workspace of %lld bytes required, got %lld", (long long)need,
                    (long long)(workspace ? ws_bytes : 0));
    if (workspace && !aligned16(workspace)) return fail(VQ_ERR_ALIGN, "workspace not 16-byte aligned");
    float* partials = static_cast<float*>(workspace);
    const int64_t tail_bytes = align256(vq::dx_tail_bytes((int)m, (int)n_total, (int)d));
    float* tail_ws = nullptr;
    if (workspace && tail_bytes > 0 && ws_bytes >= part_bytes + tail_bytes)
        tail_ws = reinterpret_cast<float*>(static_cast<char*>(workspace) + part_bytes);
    float* dwp = gw.parts && workspace && ws_bytes >= need
                     ? reinterpret_cast<float*>(static_cast<char*>(workspace) + part_bytes + tail_bytes)
                     : nullptr;
    // every member in one reduce; no tokens: a reduce over zero partials
    // writes dL/dp = 0; the parts path when the shape takes it and its buffer is there
    vq::GateReduceOut out{};
    out.kstride = cg.kstride;
    if (dprobs)
        for (int i = 0; i < nmembers; ++i) {
            out.dprobs[i] = dprobs[i];
            out.ncand[i] = ncand[i];
        }
    if (dx && m > 0) {
        if (dprobs)
            rc = hip_check(vq::launch_gemm_dx_gate(dy, w_eff, d_pad, dx, x, cg, partials, (int)m, (int)n_total, (int)d,
                                                   tail_ws, dwp, s, gs),
                           "dX + gate GEMM launch");
        else
            rc = hip_check(vq::launch_gemm_dx(dy, w_eff, d_pad, dx, (int)m, (int)n_total, (int)d, tail_ws, s),
                           "dX GEMM launch");
        if (rc != VQ_OK) return rc;
    }
    if (dprobs) {
        if (!dx && m > 0) {
            rc = hip_check(vq::launch_gemm_gate(dy, x, cg, partials, (int)m, (int)n_total, (int)d, dwp, s, gs),
                           "gate GEMM launch");
            if (rc != VQ_OK) return rc;
        }
        // partials: one per dot block on the parts path, one per gate block otherwise
        const int64_t nparts = m == 0 ? 0
                               : dwp  ? vq::gate_dot_blocks(nmembers, n, d_pad / 256)
                                      : vq::gate_partial_count((int)m, (int)n_total, (int)d);
        rc = hip_check(vq::stream_fence(s, gs), "stream fence");
        if (rc != VQ_OK) return rc;
        rc = hip_check(vq::launch_gate_reduce_group(partials, nparts, nslot, out, nmembers, gs), "gate reduce launch");
        if (rc != VQ_OK) return rc;
    }
    return ok();
}

}  // extern "C"
