// A plain read of a device buffer: the streaming floor that the Q4 GEMV
// kernels are compared with at the same byte counts (a read of 12-25 MB is
// bound by launch ramp and latency as much as by HBM bandwidth).  One
// non-temporal 16-byte load per thread over a grid that covers the buffer
// once (measured faster at these sizes than fewer threads with several loads
// each).  A lane stores only when the xor of its 16 bytes equals `match`, so
// the read cannot be optimised away, is checkable, and adds no write traffic
// or cross-lane work when nothing matches (a store per wave measured 30 %
// slower).
#include "kr_internal.hpp"

namespace kr {

namespace {
constexpr uint32_t kStreamThreads = 256;
constexpr size_t kStreamPieceBytes = (size_t)kWave * 16;
}  // namespace

__global__ __launch_bounds__(256) void stream_read_kernel(const u32x4 *__restrict__ p, size_t n16, uint32_t match,
                                                          uint32_t *__restrict__ hits) {
    const size_t j = (size_t)blockIdx.x * kStreamThreads + threadIdx.x;
    const u32x4 v = __builtin_nontemporal_load(p + (j < n16 ? j : n16 - 1));  // clamped: unconditional
    if (j < n16 && ((v.x ^ v.y) ^ (v.z ^ v.w)) == match) hits[j / kWave] = 1u;
}

size_t stream_read_pieces(size_t bytes) { return (bytes + kStreamPieceBytes - 1) / kStreamPieceBytes; }

hipError_t launch_stream_read(const void *buf, size_t bytes, uint32_t match, uint32_t *hits, hipStream_t s) {
    const size_t n16 = bytes / 16;
    const size_t blocks = (n16 + kStreamThreads - 1) / kStreamThreads;
    hipLaunchKernelGGL(stream_read_kernel, dim3((uint32_t)blocks), dim3(kStreamThreads), 0, s,
                       reinterpret_cast<const u32x4 *>(buf), n16, match, hits);
    return hipGetLastError();
}

}  // namespace kr
