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

// The same stream on data that changes from one MFMA to the next: four
// fragment pairs of random bf16 values (uniform in [-2, 2), as fresh GEMM
// operands would be), chain c multiplying pair (c % 4, (c + 1) % 4), so no two
// consecutive instructions see the same operands.  The matrix pipe's power
// depends on how many operand bits toggle; constant operands draw the least
// and let the clock run highest.  Block 0's first lane records the shader
// clock (s_memtime) and the constant-rate real-time clock (s_memrealtime)
// before and after its loop, so the host can state the clock the chip held.
__device__ __forceinline__ uint32_t hash32(uint32_t x) {
    x ^= x >> 16;
    x *= 0x7feb352dU;
    x ^= x >> 15;
    x *= 0x846ca68bU;
    x ^= x >> 16;
    return x;
}

template <bool kRandom>
__global__ __launch_bounds__(256) void mfma_clock_kernel(int64_t iters, uint32_t seed, float* __restrict__ sink,
                                                         uint64_t* __restrict__ clocks) {
    const int lane = threadIdx.x & 63;
    constexpr int kSets = kRandom ? 4 : 1;
    bf16x8_t a[kSets], b[kSets];
#pragma unroll
    for (int s = 0; s < kSets; ++s)
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            if constexpr (kRandom) {
                const uint32_t h = hash32(seed ^ hash32((uint32_t)(blockIdx.x * 256 + threadIdx.x) * 64u + s * 16u + i));
                a[s][i] = (__bf16)((float)(int32_t)h * (2.0f / 2147483648.0f));
                b[s][i] = (__bf16)((float)(int32_t)hash32(h + 0x9e3779b9U) * (2.0f / 2147483648.0f));
            } else {
                a[s][i] = (__bf16)(1.0f + 0.001f * (float)(lane + i));
                b[s][i] = (__bf16)(0.5f - 0.001f * (float)(lane - i));
            }
        }
    f32x16 acc[kChains];
#pragma unroll
    for (int c = 0; c < kChains; ++c)
#pragma unroll
        for (int r = 0; r < 16; ++r) acc[c][r] = 0.0f;
    const bool timer = blockIdx.x == 0 && threadIdx.x == 0;
    const uint64_t t0 = __builtin_amdgcn_s_memtime(), r0 = __builtin_amdgcn_s_memrealtime();
    for (int64_t it = 0; it < iters; ++it) {
#pragma unroll
        for (int c = 0; c < kChains; ++c)
            acc[c] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a[c % kSets], b[(c + 1) % kSets], acc[c], 0, 0, 0);
    }
    const uint64_t t1 = __builtin_amdgcn_s_memtime(), r1 = __builtin_amdgcn_s_memrealtime();
    float s = 0.0f;
#pragma unroll
    for (int c = 0; c < kChains; ++c)
#pragma unroll
        for (int r = 0; r < 16; ++r) s += acc[c][r];
    sink[blockIdx.x * blockDim.x + threadIdx.x] = s;
    if (timer) {
        clocks[0] = t1 - t0;
        clocks[1] = r1 - r0;
    }
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

// Copy with 8 16-byte loads in flight per thread (a workgroup moves 32 KB
// per iteration, consecutive threads on consecutive words): the memory-level
// parallelism of the dequant kernels, which a one-word-per-iteration copy
// (about 4.9 TB/s) does not reach.  n16 is a multiple of 8 * 256 here.
constexpr int kCopyUnroll = 8;

__global__ __launch_bounds__(256) void hbm_copy_kernel(const u32x4* __restrict__ src, u32x4* __restrict__ dst,
                                                       int64_t n16) {
    const int64_t per_block = 256 * kCopyUnroll;
    for (int64_t base = (int64_t)blockIdx.x * per_block; base < n16; base += (int64_t)gridDim.x * per_block) {
        u32x4 v[kCopyUnroll];
#pragma unroll
        for (int k = 0; k < kCopyUnroll; ++k) v[k] = src[base + k * 256 + threadIdx.x];
#pragma unroll
        for (int k = 0; k < kCopyUnroll; ++k) dst[base + k * 256 + threadIdx.x] = v[k];
    }
}

// Write-only stream of n16 16-byte words (the output side of dequant alone).
__global__ __launch_bounds__(256) void hbm_write_kernel(u32x4* __restrict__ dst, int64_t n16) {
    const int64_t per_block = 256 * kCopyUnroll;
    const u32x4 v = {1u, 2u, 3u, (uint32_t)threadIdx.x};
    for (int64_t base = (int64_t)blockIdx.x * per_block; base < n16; base += (int64_t)gridDim.x * per_block) {
#pragma unroll
        for (int k = 0; k < kCopyUnroll; ++k) dst[base + k * 256 + threadIdx.x] = v;
    }
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

// The MFMA probe with a clock reading: `random` selects the random-operand
// stream (else the constant operands of vq_probe_mfma).  Same grid, FLOP and
// sink as vq_probe_mfma; clocks[0] = shader-clock ticks and clocks[1] =
// real-time-clock ticks over block 0's loop (2 words on the device).
int vq_probe_mfma_clock(int random, int64_t iters, uint32_t seed, float* sink, uint64_t* clocks, void* stream) {
    const hipStream_t s = static_cast<hipStream_t>(stream);
    if (random)
        mfma_clock_kernel<true><<<dim3(vq_probe_mfma_blocks()), dim3(256), 0, s>>>(iters, seed, sink, clocks);
    else
        mfma_clock_kernel<false><<<dim3(vq_probe_mfma_blocks()), dim3(256), 0, s>>>(iters, seed, sink, clocks);
    return (int)hipGetLastError();
}

// Rate of the clock s_memrealtime reads, in kHz (0 when the runtime does not say).
int vq_probe_wall_clock_khz(void) {
    int dev = 0, khz = 0;
    if (hipGetDevice(&dev) != hipSuccess ||
        hipDeviceGetAttribute(&khz, hipDeviceAttributeWallClockRate, dev) != hipSuccess)
        return 0;
    return khz;
}

// Workgroups of the HBM probes (a few per CU, grid-stride loops).
int vq_probe_hbm_blocks(void) { return 8 * cus(); }

// Read `bytes` (a multiple of 16) at src; sink holds vq_probe_hbm_blocks() * 256 words.
int vq_probe_hbm_read(const void* src, int64_t bytes, uint32_t* sink, void* stream) {
    hbm_read_kernel<<<dim3(vq_probe_hbm_blocks()), dim3(256), 0, static_cast<hipStream_t>(stream)>>>(
        static_cast<const u32x4*>(src), bytes / 16, sink);
    return (int)hipGetLastError();
}

// Copy `bytes` (a multiple of 32 KiB) from src to dst.
int vq_probe_hbm_copy(const void* src, void* dst, int64_t bytes, void* stream) {
    if (bytes % (16 * 256 * kCopyUnroll)) return (int)hipErrorInvalidValue;
    hbm_copy_kernel<<<dim3(vq_probe_hbm_blocks()), dim3(256), 0, static_cast<hipStream_t>(stream)>>>(
        static_cast<const u32x4*>(src), static_cast<u32x4*>(dst), bytes / 16);
    return (int)hipGetLastError();
}

// Write `bytes` (a multiple of 32 KiB) at dst.
int vq_probe_hbm_write(void* dst, int64_t bytes, void* stream) {
    if (bytes % (16 * 256 * kCopyUnroll)) return (int)hipErrorInvalidValue;
    hbm_write_kernel<<<dim3(vq_probe_hbm_blocks()), dim3(256), 0, static_cast<hipStream_t>(stream)>>>(
        static_cast<u32x4*>(dst), bytes / 16);
    return (int)hipGetLastError();
}

}  // extern "C"
