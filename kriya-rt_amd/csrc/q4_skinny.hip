// q4_skinny.hip — Q4_G64 matmul for a few tokens (2 <= m <= 16) on the matrix
// cores: batched decode (config 1 B = 4, 16) and MoE experts with few routed
// tokens.  Replaces the reference's small-M path q4_g64_prefill_gemm /
// _gate_up_gemm (kernels/metal/q4_gemm_and_moe.metal:2173-2486), which re-reads
// each weight tile once per 16-token tile and uses scalar FMAs.
//
// Bound: HBM (the weights are read once; m <= 16 gives AI <= 57 FLOP/B).
//
// Mapping.  v_mfma_f32_16x16x32_f16 with A = X (16 token rows, zero-padded)
// and B = W^T (16 weight rows).  A wave owns a K range of 4 * L columns: lane
// group g = lane / 16 covers [k0 + g L, k0 + (g+1) L) and lane l % 16 its
// token row (A) or weight row (B).  The wave loads its X fragments once and
// keeps them in registers for every N tile it visits; per N tile each lane
// loads L/8 consecutive u32 words (L/2 bytes) of one weight row straight from
// HBM into registers, so a wave instruction reads 16 rows x 64 contiguous
// bytes and no LDS staging or barrier sits between HBM and the MFMA.
// Dequantisation in registers: nibble pairs (j, j+4) under the fp16 pattern
// 0x6400 -> exact (1024+q) halves, v_pk_add_f16 -1024, v_pk_fma_f16 (s, b);
// the resulting order e0 e4 e1 e5 e2 e6 e3 e7 is applied to the X fragments
// too, so it cancels in the dot product.
// A block (4 waves) covers 4 consecutive K ranges; its wave partials are added
// through LDS in wave order.  When K needs more ranges than one block has, K
// is also split over blocks and the f32 partials are reduced in split order by
// q4_mfma_splitk_reduce_kernel.  Blocks loop over N tiles (persistent grid),
// prefetching the next tile's words while the current tile is multiplied.
#include "kr_internal.hpp"

namespace kr {

namespace {

__device__ __forceinline__ uint32_t opq_s(uint32_t v) {
    uint32_t r;
    asm volatile("s_mov_b32 %0, %1" : "=s"(r) : "i"(v));
    return r;
}
__device__ __forceinline__ uint32_t opq_v(uint32_t v) {
    uint32_t r;
    asm volatile("v_mov_b32 %0, %1" : "=v"(r) : "i"(v));
    return r;
}

// 8 bf16 x values (4 u32 words, element order) -> 8 fp16 in the order e0 e4 e1 e5 e2 e6 e3 e7.
__device__ __forceinline__ f16x8_t x_frag(const u32x4 &v) {
    const uint32_t X[4] = {v.x, v.y, v.z, v.w};
    _Float16 e[8];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        e[2 * i] = (_Float16)__uint_as_float(X[i] << 16);
        e[2 * i + 1] = (_Float16)__uint_as_float(X[i] & 0xFFFF0000u);
    }
    f16x8_t r = {e[0], e[4], e[1], e[5], e[2], e[6], e[3], e[7]};
    return r;
}

// one word of 8 nibbles -> B fragment (w0 w4 w1 w5 w2 w6 w3 w7) as fp16
__device__ __forceinline__ f16x8_t w_frag(uint32_t w, f16x2_t s2, f16x2_t b2, uint32_t mask, uint32_t magic) {
    const f16x2_t k1024 = {(_Float16)-1024.0f, (_Float16)-1024.0f};
    f16x2_t pr[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        const f16x2_t q = __builtin_bit_cast(f16x2_t, ((w >> (4 * j)) & mask) | magic) + k1024;
        pr[j] = __builtin_elementwise_fma(q, s2, b2);
    }
    f16x8_t r = {pr[0].x, pr[0].y, pr[1].x, pr[1].y, pr[2].x, pr[2].y, pr[3].x, pr[3].y};
    return r;
}

__device__ __forceinline__ f16x2_t half2_of_bf16(uint32_t bf) {
    const _Float16 h = (_Float16)__uint_as_float(bf << 16);
    f16x2_t r = {h, h};
    return r;
}

}  // namespace

// L: columns per lane group per wave (64 or 128); NW: 1 plain, 2 gate/up.
template <int L, int NW>
__global__ __launch_bounds__(256) void q4_skinny_kernel(SkinnyArgs a) {
    constexpr int kSlices = L / 8;   // MFMA k-slices per wave per N tile (8 columns per lane)
    constexpr int kWords = L / 8;    // u32 words per lane per matrix per N tile
    constexpr int kVec = kWords / 4; // dwordx4 loads per lane per matrix
    constexpr int kGroups = L / 64;  // quantisation groups per lane
    __shared__ f32x4 red[NW][4][64];
    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int g = lane >> 4, r16 = lane & 15;
    const uint32_t K = a.k;
    const uint32_t groups_total = K >> 6;
    const uint32_t range = (blockIdx.x % a.ksplit) * 4 + wave;  // this wave's K range
    const uint32_t k_lane = range * (4 * L) + g * L;            // first column of this lane group
    const bool k_live = k_lane < K;                              // K % 64 == 0 and L % 64 == 0: all or nothing
    const uint32_t kMask = opq_s(0x000F000Fu);
    const uint32_t kMagic = opq_v(0x64006400u);

    // ---- X fragments of this lane (token row r16, columns k_lane .. k_lane + L), kept for all N tiles
    f16x8_t xf[kSlices];
    {
        const bool row_live = (uint32_t)r16 < a.m && k_live;
        const uint16_t *xrow = a.x + (size_t)r16 * a.ldx + k_lane;
#pragma unroll
        for (int s = 0; s < kSlices; ++s) {
            u32x4 v = {0, 0, 0, 0};
            if (row_live) v = *reinterpret_cast<const u32x4 *>(xrow + 8 * s);
            xf[s] = x_frag(v);
        }
    }

    const uint32_t ntiles = (a.w.n + 15) / 16;
    const uint32_t nblk_n = gridDim.x / a.ksplit;
    uint32_t nt = blockIdx.x / a.ksplit;

    u32x4 wv[NW][kVec];
    uint32_t sv[NW][kGroups], bv[NW][kGroups];
    auto fetch = [&](uint32_t t) {
        uint32_t row = t * 16 + r16;
        row = row < a.w.n ? row : a.w.n - 1;  // tail rows re-read a valid row and are never stored
#pragma unroll
        for (int mi = 0; mi < NW; ++mi) {
            const Q4Mat &w = mi == 0 ? a.w : a.w2;
            if (k_live) {
                const u32x4 *src = reinterpret_cast<const u32x4 *>(w.qw + (size_t)row * (K >> 3) + (k_lane >> 3));
#pragma unroll
                for (int i = 0; i < kVec; ++i) wv[mi][i] = ld_stream(src + i);
#pragma unroll
                for (int q = 0; q < kGroups; ++q) {
                    sv[mi][q] = w.sc[(size_t)row * groups_total + (k_lane >> 6) + q];
                    bv[mi][q] = w.bi[(size_t)row * groups_total + (k_lane >> 6) + q];
                }
            }
        }
    };
    if (nt >= ntiles) return;
    fetch(nt);
    for (;;) {
        f32x4 acc[NW];
#pragma unroll
        for (int mi = 0; mi < NW; ++mi) acc[mi] = f32x4{0, 0, 0, 0};
        if (k_live) {
#pragma unroll
            for (int mi = 0; mi < NW; ++mi) {
#pragma unroll
                for (int q = 0; q < kGroups; ++q) {
                    const f16x2_t s2 = half2_of_bf16(sv[mi][q]), b2 = half2_of_bf16(bv[mi][q]);
#pragma unroll
                    for (int s = 0; s < 8; ++s) {  // 8 slices of 8 columns = one group
                        const int widx = q * 8 + s;
                        const uint32_t word = widx % 4 == 0   ? wv[mi][widx / 4].x
                                              : widx % 4 == 1 ? wv[mi][widx / 4].y
                                              : widx % 4 == 2 ? wv[mi][widx / 4].z
                                                              : wv[mi][widx / 4].w;
                        acc[mi] = __builtin_amdgcn_mfma_f32_16x16x32_f16(xf[widx], w_frag(word, s2, b2, kMask, kMagic),
                                                                         acc[mi], 0, 0, 0);
                    }
                }
            }
        }
        const uint32_t tn = nt + nblk_n;
        if (tn < ntiles) fetch(tn);
        // ---- block reduction over the 4 K ranges, in wave order
#pragma unroll
        for (int mi = 0; mi < NW; ++mi) red[mi][wave][lane] = acc[mi];
        __syncthreads();
        if (wave == 0) {
            f32x4 tot[NW];
#pragma unroll
            for (int mi = 0; mi < NW; ++mi) {
                tot[mi] = red[mi][0][lane];
#pragma unroll
                for (int wv_ = 1; wv_ < 4; ++wv_) tot[mi] += red[mi][wv_][lane];
            }
            const uint32_t n = nt * 16 + r16;
            if (n < a.w.n) {
#pragma unroll
                for (int v = 0; v < 4; ++v) {
                    const uint32_t m = 4 * g + v;
                    if (m >= a.m) continue;
                    if (a.partial) {
                        float *dst = a.partial + ((size_t)(blockIdx.x % a.ksplit) * a.m + m) * (size_t)(NW * a.w.n) + n;
                        dst[0] = tot[0][v];
                        if (NW == 2) dst[a.w.n] = tot[NW - 1][v];
                        continue;
                    }
                    float val = tot[0][v];
                    if (NW == 2) val = activation(val, a.act) * tot[NW - 1][v];
                    if (a.bias) val += bf16_to_f32(a.bias[n]);
                    const size_t o = (size_t)m * a.ldo + n;
                    if (a.out_f32) {
                        float *out = reinterpret_cast<float *>(a.out);
                        out[o] = a.accumulate ? out[o] + val : val;
                    } else {
                        uint16_t *out = reinterpret_cast<uint16_t *>(a.out);
                        out[o] = (uint16_t)f32_to_bf16(a.accumulate ? val + bf16_to_f32(out[o]) : val);
                    }
                }
            }
        }
        if (tn >= ntiles) break;
        __syncthreads();  // red is rewritten by the next tile
        nt = tn;
    }
}

template <int L, int NW>
static hipError_t launch_skinny_t(SkinnyArgs &a, uint32_t max_blocks, hipStream_t s) {
    const uint32_t ranges = (a.k + 4 * L - 1) / (4 * L);
    a.ksplit = (ranges + 3) / 4;
    const uint32_t ntiles = (a.w.n + 15) / 16;
    uint32_t nblk_n = ntiles;
    const uint32_t cap = max_blocks / a.ksplit;
    if (cap > 0 && nblk_n > cap) nblk_n = cap;
    const dim3 grid(nblk_n * a.ksplit);
    hipLaunchKernelGGL((q4_skinny_kernel<L, NW>), grid, dim3(256), 0, s, a);
    return hipGetLastError();
}

// Columns per lane group: 128 when a block covers K (k <= 2048, k % 512 == 0 so
// that no lane range straddles the end of a row), 64 otherwise.
static uint32_t skinny_lane_cols(uint32_t k) { return (k <= 2048 && k % 512 == 0) ? 128 : 64; }

hipError_t launch_skinny(SkinnyArgs &a, hipStream_t s) {
    const bool gate_up = a.w2.qw != nullptr;
    const uint32_t max_blocks = (uint32_t)tuning().skinny_max_blocks;
    if (skinny_lane_cols(a.k) == 128)
        return gate_up ? launch_skinny_t<128, 2>(a, max_blocks, s) : launch_skinny_t<128, 1>(a, max_blocks, s);
    return gate_up ? launch_skinny_t<64, 2>(a, max_blocks, s) : launch_skinny_t<64, 1>(a, max_blocks, s);
}

uint32_t skinny_ksplit(uint32_t k) {
    const uint32_t L = skinny_lane_cols(k);
    const uint32_t ranges = (k + 4 * L - 1) / (4 * L);
    return (ranges + 3) / 4;
}

}  // namespace kr
