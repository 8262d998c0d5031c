// q4_format.hip — format-boundary kernels: bit-exact dequantisation, 36-byte
// block <-> planar conversion, and f16 -> bf16 scale/bias conversion.
//
//   dequantize_q4_group64_to_f32   crates/kriya-core/src/quantizer.rs:112-126
//   BlockQ4Group64 layout          crates/kriya-core/src/tensor.rs:104-115
//   MLX triplet repack             crates/kriya-core/src/safetensors_loader.rs:221-273
//   split planes (ScaledAlignedQ4Block + BlockQ4ScaleBias)
//                                  crates/kriya-core/src/tensor.rs:117-211
//   parse_half_endian              crates/kriya-core/src/safetensors_loader.rs:310-318
//
// All three are HBM-bound byte movers; each thread moves one 16- or 36-byte
// unit with vector loads and stores.
#include "kr_internal.hpp"

namespace kr {

// One thread per u32 word (8 outputs): out = fma(q, s, b), the reference's
// mul_add, which v_fma_f32 computes correctly rounded.
__global__ __launch_bounds__(256) void dequant_kernel(Q4Mat w, float *__restrict__ out, size_t total_words) {
    const size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= total_words) return;
    const uint32_t wpr = w.k >> 3;
    const size_t row = i / wpr;
    const uint32_t word_in_row = (uint32_t)(i - row * wpr);
    const size_t g = row * (w.k >> 6) + (word_in_row >> 3);
    const float s = bf16_to_f32(w.sc[g]);
    const float b = bf16_to_f32(w.bi[g]);
    const uint32_t q = w.qw[i];
    f32x4 lo, hi;
    lo.x = fmaf((float)(q & 15u), s, b);
    lo.y = fmaf((float)((q >> 4) & 15u), s, b);
    lo.z = fmaf((float)((q >> 8) & 15u), s, b);
    lo.w = fmaf((float)((q >> 12) & 15u), s, b);
    hi.x = fmaf((float)((q >> 16) & 15u), s, b);
    hi.y = fmaf((float)((q >> 20) & 15u), s, b);
    hi.z = fmaf((float)((q >> 24) & 15u), s, b);
    hi.w = fmaf((float)(q >> 28), s, b);
    f32x4 *o = reinterpret_cast<f32x4 *>(out + i * 8);
    o[0] = lo;
    o[1] = hi;
}

// One thread per block.  A 36-byte block is nine little-endian u32 words:
// word 0 = scale | bias << 16, words 1..8 = the 32 nibble bytes, which are
// the 8 planar words of group g of row r.
__global__ __launch_bounds__(256) void from_blocks36_kernel(const uint32_t *__restrict__ blocks, size_t nblocks,
                                                            uint32_t *__restrict__ qw, uint16_t *__restrict__ sc,
                                                            uint16_t *__restrict__ bi) {
    const size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= nblocks) return;
    const uint32_t *blk = blocks + i * 9;
    const uint32_t sb = blk[0];
    sc[i] = (uint16_t)(sb & 0xFFFFu);
    bi[i] = (uint16_t)(sb >> 16);
    u32x4 a, b;
    a.x = blk[1]; a.y = blk[2]; a.z = blk[3]; a.w = blk[4];
    b.x = blk[5]; b.y = blk[6]; b.z = blk[7]; b.w = blk[8];
    u32x4 *o = reinterpret_cast<u32x4 *>(qw + i * 8);
    o[0] = a;
    o[1] = b;
}

__global__ __launch_bounds__(256) void to_blocks36_kernel(Q4Mat w, uint32_t *__restrict__ blocks, size_t nblocks) {
    const size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= nblocks) return;
    const u32x4 *q = reinterpret_cast<const u32x4 *>(w.qw + i * 8);
    const u32x4 a = q[0], b = q[1];
    uint32_t *blk = blocks + i * 9;
    blk[0] = (uint32_t)w.sc[i] | ((uint32_t)w.bi[i] << 16);
    blk[1] = a.x; blk[2] = a.y; blk[3] = a.z; blk[4] = a.w;
    blk[5] = b.x; blk[6] = b.y; blk[7] = b.z; blk[8] = b.w;
}

// Split planes (tensor.rs:117-211): block i's 32 nibble bytes are 16-byte
// aligned at qs + 32 i -- the same bytes, in the same order, as the 8 planar
// words of group g of row r (i = r * G + g) -- and its {scale, bias} bf16 pair
// is the u32 sb[i] = scale | bias << 16.  One thread per block.  With qw == qs
// the nibbles are left in place and only the pairs are split.
__global__ __launch_bounds__(256) void from_split_kernel(const u32x4 *qs, const uint32_t *__restrict__ sb,
                                                         size_t nblocks, u32x4 *qw, uint16_t *__restrict__ sc,
                                                         uint16_t *__restrict__ bi) {
    const size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= nblocks) return;
    const uint32_t p = sb[i];
    sc[i] = (uint16_t)(p & 0xFFFFu);
    bi[i] = (uint16_t)(p >> 16);
    if (qw != qs) {
        const u32x4 a = qs[2 * i], b = qs[2 * i + 1];
        qw[2 * i] = a;
        qw[2 * i + 1] = b;
    }
}

__global__ __launch_bounds__(256) void to_split_kernel(Q4Mat w, u32x4 *qs, uint32_t *__restrict__ sb, size_t nblocks) {
    const size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= nblocks) return;
    sb[i] = (uint32_t)w.sc[i] | ((uint32_t)w.bi[i] << 16);
    const u32x4 *q = reinterpret_cast<const u32x4 *>(w.qw);
    if (qs != q) {
        const u32x4 a = q[2 * i], b = q[2 * i + 1];
        qs[2 * i] = a;
        qs[2 * i + 1] = b;
    }
}

// quantizer.rs:31-57 restated on bits (subnormal renormalisation by shifting,
// inf/NaN payload kept), then the RNE of quantizer.rs:19-24.
__device__ __forceinline__ uint32_t f16_bits_to_f32_bits(uint32_t h) {
    const uint32_t sign = (h >> 15) & 1u, e = (h >> 10) & 0x1Fu, mant = h & 0x3FFu;
    if (e == 0) {
        if (mant == 0) return sign << 31;
        const int lz = __clz(mant) - 21;  // shifts until bit 10 is set
        const uint32_t m = (mant << lz) & 0x3FFu;
        const uint32_t ex = (uint32_t)(127 - 14 - lz);
        return (sign << 31) | (ex << 23) | (m << 13);
    }
    if (e == 31) return (sign << 31) | 0x7F800000u | (mant << 13);
    return (sign << 31) | ((e + 112u) << 23) | (mant << 13);
}

__global__ __launch_bounds__(256) void f16_to_bf16_kernel(const uint16_t *in, uint16_t *out, size_t count) {
    const size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= count) return;
    const uint32_t f = f16_bits_to_f32_bits(in[i]);
    out[i] = (uint16_t)((f + 0x7FFFu + ((f >> 16) & 1u)) >> 16);
}

static inline dim3 grid_for(size_t count) { return dim3((unsigned)((count + 255) / 256)); }

hipError_t launch_format_dequant(const Q4Mat &w, float *out, hipStream_t s) {
    const size_t words = (size_t)w.n * (w.k >> 3);
    if (words == 0) return hipSuccess;
    hipLaunchKernelGGL(dequant_kernel, grid_for(words), dim3(256), 0, s, w, out, words);
    return hipGetLastError();
}

hipError_t launch_from_blocks36(const void *blocks, uint32_t n, uint32_t k, uint32_t *qw, uint16_t *sc,
                                uint16_t *bi, hipStream_t s) {
    const size_t nb = (size_t)n * (k >> 6);
    if (nb == 0) return hipSuccess;
    hipLaunchKernelGGL(from_blocks36_kernel, grid_for(nb), dim3(256), 0, s,
                       reinterpret_cast<const uint32_t *>(blocks), nb, qw, sc, bi);
    return hipGetLastError();
}

hipError_t launch_to_blocks36(const Q4Mat &w, void *blocks, hipStream_t s) {
    const size_t nb = (size_t)w.n * (w.k >> 6);
    if (nb == 0) return hipSuccess;
    hipLaunchKernelGGL(to_blocks36_kernel, grid_for(nb), dim3(256), 0, s, w, reinterpret_cast<uint32_t *>(blocks),
                       nb);
    return hipGetLastError();
}

hipError_t launch_from_split(const void *qs, const void *sb, uint32_t n, uint32_t k, uint32_t *qw, uint16_t *sc,
                             uint16_t *bi, hipStream_t s) {
    const size_t nb = (size_t)n * (k >> 6);
    if (nb == 0) return hipSuccess;
    hipLaunchKernelGGL(from_split_kernel, grid_for(nb), dim3(256), 0, s, reinterpret_cast<const u32x4 *>(qs),
                       reinterpret_cast<const uint32_t *>(sb), nb, reinterpret_cast<u32x4 *>(qw), sc, bi);
    return hipGetLastError();
}

hipError_t launch_to_split(const Q4Mat &w, void *qs, void *sb, hipStream_t s) {
    const size_t nb = (size_t)w.n * (w.k >> 6);
    if (nb == 0) return hipSuccess;
    hipLaunchKernelGGL(to_split_kernel, grid_for(nb), dim3(256), 0, s, w, reinterpret_cast<u32x4 *>(qs),
                       reinterpret_cast<uint32_t *>(sb), nb);
    return hipGetLastError();
}

hipError_t launch_f16_to_bf16(const uint16_t *in, uint16_t *out, size_t count, hipStream_t s) {
    if (count == 0) return hipSuccess;
    hipLaunchKernelGGL(f16_to_bf16_kernel, grid_for(count), dim3(256), 0, s, in, out, count);
    return hipGetLastError();
}

}  // namespace kr
