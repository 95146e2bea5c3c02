// Measurement probes for bench.py (libvq_probe.so, not part of the product's
// C ABI): the sustained bf16 MFMA rate of the chip and its HBM read and copy
// bandwidth, so the roofline can be stated against what the card delivers
// under load as well as against the published peaks.
#include <hip/hip_runtime.h>
#include <stdint.h>

namespace {

typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

constexpr int kChains = 8;  // independent accumulators per wave: enough to issue back to back

// Every wave issues `iters` rounds of kChains independent
// v_mfma_f32_32x32x16_bf16 (32 * 32 * 16 * 2 FLOP each) on register
// operands: no memory traffic, only the matrix pipe (and the clock it holds).
__global__ __launch_bounds__(256) void mfma_peak_kernel(int64_t iters, float* __restrict__ sink) {
    const int lane = threadIdx.x & 63;
    bf16x8_t a, b;
#pragma unroll
    for (int i = 0; i < 8; ++i) {
        a[i] = (__bf16)(1.0f + 0.001f * (float)(lane + i));
        b[i] = (__bf16)(0.5f - 0.001f * (float)(lane - i));
    }
    f32x16 acc[kChains];
#pragma unroll
    for (int c = 0; c < kChains; ++c)
#pragma unroll
        for (int r = 0; r < 16; ++r) acc[c][r] = 0.0f;
    for (int64_t it = 0; it < iters; ++it) {
#pragma unroll
        for (int c = 0; c < kChains; ++c) acc[c] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b, acc[c], 0, 0, 0);
    }
    float s = 0.0f;
#pragma unroll
    for (int c = 0; c < kChains; ++c)
#pragma unroll
        for (int r = 0; r < 16; ++r) s += acc[c][r];
    sink[blockIdx.x * blockDim.x + threadIdx.x] = s;
}

// Streams `n16` 16-byte words: each thread reads a strided set and keeps an
// XOR, written once per thread (so the loads are not removed).
__global__ __launch_bounds__(256) void hbm_read_kernel(const u32x4* __restrict__ src, int64_t n16,
                                                       uint32_t* __restrict__ sink) {
    const int64_t stride = (int64_t)gridDim.x * blockDim.x;
    u32x4 x = {0, 0, 0, 0};
    for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n16; i += stride) {
        const u32x4 v = __builtin_nontemporal_load(src + i);
        x ^= v;
    }
    sink[(int64_t)blockIdx.x * blockDim.x + threadIdx.x] = x[0] ^ x[1] ^ x[2] ^ x[3];
}

__global__ __launch_bounds__(256) void hbm_copy_kernel(const u32x4* __restrict__ src, u32x4* __restrict__ dst,
                                                       int64_t n16) {
    const int64_t stride = (int64_t)gridDim.x * blockDim.x;
    for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n16; i += stride)
        __builtin_nontemporal_store(__builtin_nontemporal_load(src + i), dst + i);
}

int cus() {
    int dev = 0;
    hipDeviceProp_t prop;
    if (hipGetDevice(&dev) != hipSuccess || hipGetDeviceProperties(&prop, dev) != hipSuccess) return 256;
    return prop.multiProcessorCount;
}

}  // namespace

extern "C" {

// Workgroups (256 threads each) the MFMA probe launches: two per CU, so each
// SIMD holds two waves.
int vq_probe_mfma_blocks(void) { return 2 * cus(); }

// Launch the MFMA probe on `stream`: vq_probe_mfma_blocks() workgroups, each
// wave `iters` rounds of 8 MFMAs; sink holds blocks * 256 floats.  Returns a
// hipError_t.  FLOP = blocks * 4 waves * iters * 8 * 32768.
int vq_probe_mfma(int64_t iters, float* sink, void* stream) {
    mfma_peak_kernel<<<dim3(vq_probe_mfma_blocks()), dim3(256), 0, static_cast<hipStream_t>(stream)>>>(iters, sink);
    return (int)hipGetLastError();
}

// Workgroups of the HBM probes (a few per CU, grid-stride loops).
int vq_probe_hbm_blocks(void) { return 8 * cus(); }

// Read `bytes` (a multiple of 16) at src; sink holds vq_probe_hbm_blocks() * 256 words.
int vq_probe_hbm_read(const void* src, int64_t bytes, uint32_t* sink, void* stream) {
    hbm_read_kernel<<<dim3(vq_probe_hbm_blocks()), dim3(256), 0, static_cast<hipStream_t>(stream)>>>(
        static_cast<const u32x4*>(src), bytes / 16, sink);
    return (int)hipGetLastError();
}

// Copy `bytes` (a multiple of 16) from src to dst.
int vq_probe_hbm_copy(const void* src, void* dst, int64_t bytes, void* stream) {
    hbm_copy_kernel<<<dim3(vq_probe_hbm_blocks()), dim3(256), 0, static_cast<hipStream_t>(stream)>>>(
        static_cast<const u32x4*>(src), static_cast<u32x4*>(dst), bytes / 16);
    return (int)hipGetLastError();
}

}  // extern "C"
