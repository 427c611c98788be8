// Achieved-peak microbenchmarks (include/pe_peaks.h): the bf16 MFMA rate, a streaming HBM read,
// an HBM copy and the direct global-to-LDS read the attention kernels stage with, each written
// with the same instructions those kernels use, so the roofline's spec peaks can be shown beside
// what one MI355X sustains. Measurement only; no attention entry point calls these.
#include "../../include/pe_peaks.h"

#include <hip/hip_runtime.h>

#include "pe_attn_stage.h"

namespace {

using pe::bf16x8;
using pe::f32x16;

constexpr int kThreads = 256;

// Four independent MFMA chains per wave (the matrix core overlaps independent products; a
// chain's dependent MFMAs issue back to back through the accumulator forwarding path).
__global__ __launch_bounds__(kThreads) void mfma_peak_kernel(const bf16x8 *ops, float *sink, int iters) {
    const int t = (int)((blockIdx.x * kThreads + threadIdx.x) & 2047);
    const bf16x8 a = ops[t], b = ops[t + 2048];
    f32x16 c0 = {}, c1 = {}, c2 = {}, c3 = {};
#pragma unroll 4
    for (int i = 0; i < iters; ++i) {
        c0 = pe::mfma32(a, b, c0);
        c1 = pe::mfma32(b, a, c1);
        c2 = pe::mfma32(a, a, c2);
        c3 = pe::mfma32(b, b, c3);
    }
    float s = 0.0f;
#pragma unroll
    for (int j = 0; j < 16; ++j) s += c0[j] + c1[j] + c2[j] + c3[j];
    sink[blockIdx.x * kThreads + threadIdx.x] = s;
}

// Four coalesced 16-byte loads in flight per lane per iteration, grid-strided.
__global__ __launch_bounds__(kThreads) void read_peak_kernel(const int4 *src, int64_t n16, int32_t *sink) {
    const int64_t g = (int64_t)gridDim.x * kThreads;
    int4 acc = make_int4(0, 0, 0, 0);
    for (int64_t i = blockIdx.x * kThreads + threadIdx.x; i < n16; i += 4 * g) {
        int4 v[4];
#pragma unroll
        for (int j = 0; j < 4; ++j) v[j] = i + j * g < n16 ? src[i + j * g] : make_int4(0, 0, 0, 0);
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            acc.x ^= v[j].x;
            acc.y ^= v[j].y;
            acc.z ^= v[j].z;
            acc.w ^= v[j].w;
        }
    }
    sink[blockIdx.x * kThreads + threadIdx.x] = acc.x ^ acc.y ^ acc.z ^ acc.w;
}

__global__ __launch_bounds__(kThreads) void copy_peak_kernel(const int4 *src, int4 *dst, int64_t n16) {
    const int64_t g = (int64_t)gridDim.x * kThreads;
    for (int64_t i = blockIdx.x * kThreads + threadIdx.x; i < n16; i += 4 * g) {
        int4 v[4];
#pragma unroll
        for (int j = 0; j < 4; ++j)
            if (i + j * g < n16) v[j] = src[i + j * g];
#pragma unroll
        for (int j = 0; j < 4; ++j)
            if (i + j * g < n16) dst[i + j * g] = v[j];
    }
}

// 16 KiB chunks, grid-strided, each streamed by the workgroup's four waves (four 1 KiB wave-loads
// each) into one of two LDS stages; a chunk's loads are waited for only after the next chunk's
// are issued, so two chunks are in flight per workgroup. Nothing reads the stages until the end
// (one int per lane read back, so the loads have an observer).
constexpr int kChunk = 16384;

__global__ __launch_bounds__(kThreads) void read_lds_peak_kernel(const char *src, int64_t chunks, int32_t *sink) {
    __shared__ __attribute__((aligned(16))) char stage[2][kChunk];
    const int wave = pe::uniform((int)(threadIdx.x >> 6)), lane = (int)(threadIdx.x & 63);
    const uint32_t base = pe::uniform((int)pe::lds_addr(&stage[0][0]));
    int n = 0;
    for (int64_t c = blockIdx.x; c < chunks; c += gridDim.x, ++n) {
        const __amdgpu_buffer_rsrc_t rs = pe::make_rsrc(src + c * kChunk, kChunk);
        const uint32_t lds0 = base + (n & 1) * kChunk + wave * 4096;
        const uint32_t lds[4] = {lds0, lds0 + 1024, lds0 + 2048, lds0 + 3072};
        const int off[4] = {wave * 4096 + lane * 16, wave * 4096 + 1024 + lane * 16, wave * 4096 + 2048 + lane * 16,
                            wave * 4096 + 3072 + lane * 16};
        pe::dma16x4(lds, off, rs, rs);
        pe::wait_vmcnt<4>();
    }
    pe::wait_vmcnt<0>();
    __syncthreads();
    sink[blockIdx.x * kThreads + threadIdx.x] = reinterpret_cast<const int32_t *>(&stage[0][0])[threadIdx.x];
}

int launched() { return hipGetLastError() == hipSuccess ? 0 : -4; }

}  // namespace

extern "C" {

int pe_peak_mfma_bf16(const void *operands, float *sink, int32_t blocks, int32_t iters, hipStream_t stream) {
    if (!operands || !sink || blocks < 1 || iters < 1) return -1;
    hipLaunchKernelGGL(mfma_peak_kernel, dim3(blocks), dim3(kThreads), 0, stream,
                       static_cast<const bf16x8 *>(operands), sink, iters);
    return launched();
}

int pe_peak_read(const void *src, size_t bytes, int32_t *sink, int32_t blocks, hipStream_t stream) {
    if (!src || !sink || blocks < 1 || bytes % 64 || reinterpret_cast<uintptr_t>(src) % 16) return -1;
    hipLaunchKernelGGL(read_peak_kernel, dim3(blocks), dim3(kThreads), 0, stream, static_cast<const int4 *>(src),
                       (int64_t)(bytes / 16), sink);
    return launched();
}

int pe_peak_copy(const void *src, void *dst, size_t bytes, int32_t blocks, hipStream_t stream) {
    if (!src || !dst || blocks < 1 || bytes % 64 || reinterpret_cast<uintptr_t>(src) % 16 ||
        reinterpret_cast<uintptr_t>(dst) % 16)
        return -1;
    hipLaunchKernelGGL(copy_peak_kernel, dim3(blocks), dim3(kThreads), 0, stream, static_cast<const int4 *>(src),
                       static_cast<int4 *>(dst), (int64_t)(bytes / 16));
    return launched();
}

int pe_peak_read_lds(const void *src, size_t bytes, int32_t *sink, int32_t blocks, hipStream_t stream) {
    if (!src || !sink || blocks < 1 || bytes % kChunk || reinterpret_cast<uintptr_t>(src) % 16) return -1;
    hipLaunchKernelGGL(read_lds_peak_kernel, dim3(blocks), dim3(kThreads), 0, stream, static_cast<const char *>(src),
                       (int64_t)(bytes / kChunk), sink);
    return launched();
}

}  // extern "C"
