// A plain read of a device buffer: the streaming floor that the Q4 GEMV
// kernels are compared with at the same byte counts (a read of 12-25 MB is
// bound by launch ramp and latency as much as by HBM bandwidth).  Each thread
// requests four 16-byte words at once (non-temporal, like the weight loads of
// the GEMV kernels), and each block stores the xor of its 16 KB, so the read
// cannot be optimised away and its result is checkable.
#include "kr_internal.hpp"

namespace kr {

namespace {
constexpr uint32_t kStreamThreads = 256;
constexpr uint32_t kStreamWords = 4;  // 16-byte words per thread
constexpr size_t kStreamBlockBytes = (size_t)kStreamThreads * kStreamWords * 16;
}  // namespace

__global__ __launch_bounds__(256) void stream_read_kernel(const u32x4 *__restrict__ p, size_t n16,
                                                          uint32_t *__restrict__ sink) {
    __shared__ uint32_t wx[kStreamThreads / kWave];
    const size_t base = (size_t)blockIdx.x * kStreamThreads * kStreamWords + threadIdx.x;
    u32x4 v[kStreamWords];
#pragma unroll
    for (uint32_t i = 0; i < kStreamWords; ++i) {
        const size_t j = base + (size_t)i * kStreamThreads;
        v[i] = __builtin_nontemporal_load(p + (j < n16 ? j : n16 - 1));  // clamped: unconditional
    }
    uint32_t x = 0;
#pragma unroll
    for (uint32_t i = 0; i < kStreamWords; ++i)
        if (base + (size_t)i * kStreamThreads < n16) x ^= v[i].x ^ v[i].y ^ v[i].z ^ v[i].w;
#pragma unroll
    for (int m = 32; m >= 1; m >>= 1) x ^= (uint32_t)__shfl_xor((int)x, m);
    if ((threadIdx.x & (kWave - 1)) == 0) wx[threadIdx.x / kWave] = x;
    __syncthreads();
    if (threadIdx.x == 0) sink[blockIdx.x] = (wx[0] ^ wx[1]) ^ (wx[2] ^ wx[3]);
}

size_t stream_read_sink_words(size_t bytes) { return (bytes + kStreamBlockBytes - 1) / kStreamBlockBytes; }

hipError_t launch_stream_read(const void *buf, size_t bytes, uint32_t *sink, hipStream_t s) {
    const size_t blocks = stream_read_sink_words(bytes);
    hipLaunchKernelGGL(stream_read_kernel, dim3((uint32_t)blocks), dim3(kStreamThreads), 0, s,
                       reinterpret_cast<const u32x4 *>(buf), bytes / 16, sink);
    return hipGetLastError();
}

}  // namespace kr
