// q4_mfma.hip — batched (m > 1) Q4_G64 matmul on the gfx950 matrix cores.
//
// Replaces the reference's batched kernels (kernels/metal/q4_gemm_and_moe.metal):
//   q4_g64_prefill_gemm / _qkv_gemm / _gate_up_gemm      :2173-2486  (1 < M < 64)
//   q4_g64_batched_simdgroup_gemm_m64                     :2708-2851  (M >= 64)
//   q4_g64_batched_simdgroup_qkv_gemm_m64                 :2853-3022
//   q4_g64_batched_simdgroup_gate_up_swiglu_gemm_m64      :3024-3215
//
// Y[M, N] = X[M, K] . W[N, K]^T with X bf16 and W planar Q4_G64.
// Bound: MFMA for prefill-sized M (config 2: AI ~ 800 FLOP/B), HBM for the
// batched-decode M <= 16 (config 1 B = 4, 16).
//
// Operands are fp16 with f32 accumulation (v_mfma_f32_16x16x32_f16):
//   * weights: w = fma(q, s, b) rounded once to fp16.  For scales and biases
//     in fp16's normal range this is exact whenever the value has <= 11
//     significant bits, which holds for w = s*(q-8) with bf16 s (8 bits) -- the
//     benchmark distributions; bf16 (8 bits) would round such weights.  The
//     reference's own M >= 64 kernels use half operands as well
//     (q4_gemm_and_moe.metal:2722-2724, 2761-2764).
//   * activations: bf16 -> fp16 is exact for |x| in [2^-14, 65504].  A token row
//     whose largest |x| over the block's K range lies outside [2^-8, 2^16) is
//     staged times 2^e (its largest |x| then in [2^15, 2^16)) and its results
//     multiplied by 2^-e, both exact; the row maxima come from a scan of the
//     block's rows before the first step (this kernel serves the shapes the
//     few-token and prefill kernels do not take).
// Dequantisation per 8 nibbles (one u32 word): for j in 0..3 the pair of
// nibbles (j, j+4) is placed under the fp16 pattern 0x6400 (1024.0, ulp 1),
// v_pk_add_f16 removes the 1024 exactly and v_pk_fma_f16 applies (s, b).
//
// Tiling: a block of 256 threads (4 waves, 2 x 2) computes a BM x BN tile of
// one problem over a K range, in 64-wide K steps (one quantisation group):
// each step stages X (BM x 64) and the dequantised W (BN x 64, twice for the
// gate/up epilogue) in LDS, double-buffered, while the next step's global
// loads are in flight.  Up to three problems (q, k, v) share one launch and X.
// Split-K (grid.y) writes f32 partials to a workspace that a second kernel
// reduces in split order before the epilogue, so results do not depend on
// scheduling.  Block ids are remapped so that the M tiles of one N tile run on
// the same XCD (blocks are dealt round-robin to the 8 XCDs) and share its L2.
#include "kr_internal.hpp"

namespace kr {

namespace {

constexpr int kPitch = 72;  // fp16 per LDS row: 64 + 8 padding (144 B) to spread LDS banks

__device__ __forceinline__ uint32_t opaque_s(uint32_t v) {
    uint32_t r;
    asm volatile("s_mov_b32 %0, %1" : "=s"(r) : "i"(v));
    return r;
}
__device__ __forceinline__ uint32_t opaque_v(uint32_t v) {
    uint32_t r;
    asm volatile("v_mov_b32 %0, %1" : "=v"(r) : "i"(v));
    return r;
}

// bf16 bits times 2^e (sc) -> fp16 bits.  A bf16 value has 8 significant bits, so in fp16's
// normal range the conversion is exact and the rounding mode does not matter:
// one v_cvt_pkrtz_f16_f32 per pair.
__device__ __forceinline__ uint32_t bf16x2_to_f16x2(uint32_t v, float sc) {
    return __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_pkrtz(__uint_as_float(v << 16) * sc,
                                                                   __uint_as_float(v & 0xFFFF0000u) * sc));
}

// 8 nibbles of one word -> 8 fp16 weights in element order (e0..e7) as 4 u32.
__device__ __forceinline__ void dequant_word_f16(uint32_t w, f16x2_t s2, f16x2_t b2, uint32_t mask, uint32_t magic,
                                                 uint32_t (&out)[4]) {
    const f16x2_t k1024 = {(_Float16)-1024.0f, (_Float16)-1024.0f};
    f16x2_t pr[4];  // pr[j] = (w_j, w_{j+4})
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        const uint32_t hbits = ((w >> (4 * j)) & mask) | magic;
        const f16x2_t q = __builtin_bit_cast(f16x2_t, hbits) + k1024;  // exact (q_j, q_{j+4})
        pr[j] = __builtin_elementwise_fma(q, s2, b2);
    }
    // element order: (e0 e1) (e2 e3) (e4 e5) (e6 e7)
    f16x2_t o0 = {pr[0].x, pr[1].x}, o1 = {pr[2].x, pr[3].x}, o2 = {pr[0].y, pr[1].y}, o3 = {pr[2].y, pr[3].y};
    out[0] = __builtin_bit_cast(uint32_t, o0);
    out[1] = __builtin_bit_cast(uint32_t, o1);
    out[2] = __builtin_bit_cast(uint32_t, o2);
    out[3] = __builtin_bit_cast(uint32_t, o3);
}

__device__ __forceinline__ f16x2_t bf16_pair_to_f16x2(uint32_t bf) {
    const _Float16 h = (_Float16)bf16_to_f32(bf);
    f16x2_t r = {h, h};
    return r;
}

}  // namespace

template <int BM, int BN, int NW>
struct MfmaTile {
    static constexpr int kWaveM = BM / 2, kWaveN = BN / 2;       // 2 x 2 waves
    static constexpr int kFragM = kWaveM / 16, kFragN = kWaveN / 16;
    static constexpr int kLdsRows = BM + NW * BN;
    static constexpr int kLdsBytes = 2 * kLdsRows * kPitch * 2;  // double-buffered
    // per-thread staging loads per K step
    static constexpr int kXLoads = (BM * 8 + 255) / 256;         // u32x4 (8 bf16) units
    static constexpr int kWLoads = (BN * 2 + 255) / 256;         // u32x4 (32 nibbles) units per matrix
    static_assert(kWaveM % 16 == 0 && kWaveN % 16 == 0, "wave tile must be a multiple of 16");
};

template <int BM, int BN, int NW, int EPI>
__global__ __launch_bounds__(256) void q4_mfma_gemm_kernel(MfmaArgs args) {
    using T = MfmaTile<BM, BN, NW>;
    extern __shared__ __align__(16) uint16_t lds_raw[];
    __shared__ int s_rowexp[BM];  // staging exponent e of each token row of the block
    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int wm = wave >> 1, wn = wave & 1;

    // ---- block -> (problem, n tile, m tile), XCD-aware: consecutive tiles share an XCD
    const uint32_t nblk = gridDim.x;
    uint32_t bid = blockIdx.x;
    if (nblk >= 8 && (nblk & 7) == 0) bid = (bid & 7) * (nblk >> 3) + (bid >> 3);
    int pi = 0;
#pragma unroll
    for (int i = 1; i < kMaxMfmaProblems; ++i)
        if (i < args.np && bid >= args.p[i].tile_begin) pi = i;
    const MfmaProblem &P = args.p[pi];
    const uint32_t local = bid - P.tile_begin;
    const uint32_t tiles_m = (args.m + BM - 1) / BM;
    const uint32_t mt = local % tiles_m, nt = local / tiles_m;
    const uint32_t m0 = mt * BM, n0 = nt * BN;
    const uint32_t N = P.w.n;
    const uint32_t K = args.k;
    const uint32_t groups = K >> 6;
    const uint32_t ks = blockIdx.y;
    const uint32_t g_begin = ks * args.groups_per_split;
    const uint32_t g_end = min(groups, g_begin + args.groups_per_split);

    const uint32_t kMask = opaque_s(0x000F000Fu);
    const uint32_t kMagic = opaque_v(0x64006400u);

    // ---- staging assignments
    // X: unit u -> row u / 8, 8-element column block u % 8
    // W: unit u -> row u / 2, half-group u % 2 (words 4h..4h+3 = elements 32h..32h+31)
    u32x4 xr[T::kXLoads];
    u32x4 wr[NW][T::kWLoads];
    uint32_t sr[NW][T::kWLoads], br[NW][T::kWLoads];
    auto load_step = [&](uint32_t g) {
#pragma unroll
        for (int i = 0; i < T::kXLoads; ++i) {
            const uint32_t u = tid + 256 * i;
            const uint32_t row = u >> 3, cb = u & 7;
            const uint32_t gm = m0 + row;
            xr[i] = u32x4{0, 0, 0, 0};
            if (u < (uint32_t)BM * 8 && gm < args.m)
                xr[i] = *reinterpret_cast<const u32x4 *>(args.x + (size_t)gm * args.ldx + g * 64 + cb * 8);
        }
#pragma unroll
        for (int mi = 0; mi < NW; ++mi) {
            const Q4Mat &w = mi == 0 ? P.w : P.w2;
#pragma unroll
            for (int i = 0; i < T::kWLoads; ++i) {
                const uint32_t u = tid + 256 * i;
                uint32_t row = n0 + (u >> 1);
                row = row < N ? row : N - 1;  // tail rows re-read a valid row; never stored
                if (u < (uint32_t)BN * 2) {
                    wr[mi][i] = ld_stream(reinterpret_cast<const u32x4 *>(w.qw + (size_t)row * (K >> 3) + g * 8) +
                                          (u & 1));
                    sr[mi][i] = w.sc[(size_t)row * groups + g];
                    br[mi][i] = w.bi[(size_t)row * groups + g];
                }
            }
        }
    };
    auto store_step = [&](int buf) {
        uint16_t *base = lds_raw + buf * T::kLdsRows * kPitch;
#pragma unroll
        for (int i = 0; i < T::kXLoads; ++i) {
            const uint32_t u = tid + 256 * i;
            if (u < (uint32_t)BM * 8) {
                const uint32_t row = u >> 3, cb = u & 7;
                const float sc = exp2_int(s_rowexp[row]);
                u32x4 h;
                h.x = bf16x2_to_f16x2(xr[i].x, sc);
                h.y = bf16x2_to_f16x2(xr[i].y, sc);
                h.z = bf16x2_to_f16x2(xr[i].z, sc);
                h.w = bf16x2_to_f16x2(xr[i].w, sc);
                *reinterpret_cast<u32x4 *>(base + row * kPitch + cb * 8) = h;
            }
        }
#pragma unroll
        for (int mi = 0; mi < NW; ++mi) {
#pragma unroll
            for (int i = 0; i < T::kWLoads; ++i) {
                const uint32_t u = tid + 256 * i;
                if (u < (uint32_t)BN * 2) {
                    const uint32_t row = u >> 1, half = u & 1;
                    const f16x2_t s2 = bf16_pair_to_f16x2(sr[mi][i]);
                    const f16x2_t b2 = bf16_pair_to_f16x2(br[mi][i]);
                    uint16_t *dst = base + (BM + mi * BN + row) * kPitch + half * 32;
                    const uint32_t wd[4] = {wr[mi][i].x, wr[mi][i].y, wr[mi][i].z, wr[mi][i].w};
#pragma unroll
                    for (int q = 0; q < 4; ++q) {
                        uint32_t o[4];
                        dequant_word_f16(wd[q], s2, b2, kMask, kMagic, o);
                        *reinterpret_cast<u32x4 *>(dst + q * 8) = u32x4{o[0], o[1], o[2], o[3]};
                    }
                }
            }
        }
    };

    f32x4 acc[NW][T::kFragM][T::kFragN];
#pragma unroll
    for (int mi = 0; mi < NW; ++mi)
#pragma unroll
        for (int a = 0; a < T::kFragM; ++a)
#pragma unroll
            for (int b = 0; b < T::kFragN; ++b) acc[mi][a][b] = f32x4{0, 0, 0, 0};

    // ---- staging exponents of the block's token rows: wave w scans rows w, w + 4, ... over the
    // block's K range (16-byte units strided by lane), maximum over the wave.
    for (uint32_t r = (uint32_t)wave; r < (uint32_t)BM; r += 4) {
        const uint32_t upr = (g_end > g_begin ? g_end - g_begin : 0u) * 8u;
        uint32_t mx = 0;
        if (m0 + r < args.m) {
            const u32x4 *row = reinterpret_cast<const u32x4 *>(args.x + (size_t)(m0 + r) * args.ldx + g_begin * 64);
            for (uint32_t c = (uint32_t)lane; c < upr; c += 64) mx = max(mx, bf16_unit_max_bits(row[c]));
        }
        mx = wave_max_u32(mx);
        if (lane == 0) s_rowexp[r] = row_stage_exp(mx, -8, 15, 15);
    }
    __syncthreads();

    if (g_begin < g_end) {
        load_step(g_begin);
        store_step(0);
        __syncthreads();
        int buf = 0;
        for (uint32_t g = g_begin; g < g_end; ++g) {
            const bool more = g + 1 < g_end;
            if (more) load_step(g + 1);
            const uint16_t *base = lds_raw + buf * T::kLdsRows * kPitch;
            // two 32-wide k slices per group
#pragma unroll
            for (int kk = 0; kk < 2; ++kk) {
                const int koff = kk * 32 + 8 * (lane >> 4);
                f16x8_t af[T::kFragM];
#pragma unroll
                for (int a = 0; a < T::kFragM; ++a)
                    af[a] = *reinterpret_cast<const f16x8_t *>(base + (wm * T::kWaveM + a * 16 + (lane & 15)) * kPitch +
                                                              koff);
#pragma unroll
                for (int mi = 0; mi < NW; ++mi) {
#pragma unroll
                    for (int b = 0; b < T::kFragN; ++b) {
                        const f16x8_t bf = *reinterpret_cast<const f16x8_t *>(
                            base + (BM + mi * BN + wn * T::kWaveN + b * 16 + (lane & 15)) * kPitch + koff);
#pragma unroll
                        for (int a = 0; a < T::kFragM; ++a)
                            acc[mi][a][b] = __builtin_amdgcn_mfma_f32_16x16x32_f16(af[a], bf, acc[mi][a][b], 0, 0, 0);
                    }
                }
            }
            if (more) store_step(buf ^ 1);
            __syncthreads();
            buf ^= 1;
        }
    }

    // ---- epilogue: lane holds C[4*(lane/16) + v][lane % 16] of each 16 x 16 fragment
#pragma unroll
    for (int a = 0; a < T::kFragM; ++a) {
#pragma unroll
        for (int b = 0; b < T::kFragN; ++b) {
            const uint32_t n = n0 + wn * T::kWaveN + b * 16 + (lane & 15);
            if (n >= N) continue;
#pragma unroll
            for (int v = 0; v < 4; ++v) {
                const uint32_t m = m0 + wm * T::kWaveM + a * 16 + 4 * (lane >> 4) + v;
                if (m >= args.m) continue;
                const float unscale = exp2_int(-s_rowexp[m - m0]);  // the row's staging scale undone
                const float g0 = acc[0][a][b][v] * unscale, u0 = acc[NW - 1][a][b][v] * unscale;
                if (EPI == kMfmaPartial) {
                    // split-K partials: [split][m][NW * N]
                    float *dst = args.partial + ((size_t)ks * args.m + m) * (size_t)(NW * N) + n;
                    dst[0] = g0;
                    if (NW == 2) dst[N] = u0;
                    continue;
                }
                float val = g0;
                if (NW == 2) val = activation(val, args.act) * u0;
                if (P.bias) val += bf16_to_f32(P.bias[n]);
                const size_t o = (size_t)m * P.ldo + n;
                if (args.out_f32) {
                    float *out = reinterpret_cast<float *>(P.out);
                    out[o] = args.accumulate ? out[o] + val : val;
                } else {
                    uint16_t *out = reinterpret_cast<uint16_t *>(P.out);
                    out[o] = (uint16_t)f32_to_bf16(args.accumulate ? val + bf16_to_f32(out[o]) : val);
                }
            }
        }
    }
}

// Sum of split-K partials in split order, then the epilogue of the direct path.
__global__ __launch_bounds__(256) void q4_mfma_splitk_reduce_kernel(MfmaArgs args, int nw) {
    const MfmaProblem &P = args.p[0];
    const uint32_t N = P.w.n;
    const size_t total = (size_t)args.m * N;
    const size_t i = (size_t)blockIdx.x * 256 + threadIdx.x;
    if (i >= total) return;
    const uint32_t m = (uint32_t)(i / N), n = (uint32_t)(i % N);
    const size_t stride = (size_t)args.m * nw * N;
    const float *p0 = args.partial + (size_t)m * nw * N + n;
    float g = 0.0f, u = 0.0f;
    for (uint32_t s = 0; s < args.ksplit; ++s) {
        g += p0[s * stride];
        if (nw == 2) u += p0[s * stride + N];
    }
    float val = nw == 2 ? activation(g, args.act) * u : g;
    if (P.bias) val += bf16_to_f32(P.bias[n]);
    const size_t o = (size_t)m * P.ldo + n;
    if (args.out_f32) {
        float *out = reinterpret_cast<float *>(P.out);
        out[o] = args.accumulate ? out[o] + val : val;
    } else {
        uint16_t *out = reinterpret_cast<uint16_t *>(P.out);
        out[o] = (uint16_t)f32_to_bf16(args.accumulate ? val + bf16_to_f32(out[o]) : val);
    }
}

// The same sums and epilogue for eight consecutive outputs of a row per thread (N % 8 == 0,
// 16-byte aligned rows, partials, outputs and bias): each split's partials are two 16-byte loads,
// and up to kReduceBatch splits are requested before any of them is added (repeats of the last
// split past ksplit are loaded and ignored), so that a thread waits once per batch instead of
// once per load.  The adds run in split order from 0, as above: the bits are the same.
constexpr uint32_t kReduceBatch = 8;
template <int NW>
__global__ __launch_bounds__(256) void q4_mfma_splitk_reduce8_kernel(MfmaArgs args) {
    const MfmaProblem &P = args.p[0];
    const uint32_t N = P.w.n, units = N >> 3;
    const size_t i = (size_t)blockIdx.x * 256 + threadIdx.x;
    if (i >= (size_t)args.m * units) return;
    const uint32_t m = (uint32_t)(i / units), n = (uint32_t)(i % units) * 8;
    const size_t stride = (size_t)args.m * NW * N;
    const float *p0 = args.partial + (size_t)m * NW * N + n;
    float g[8] = {}, u[8] = {};
    for (uint32_t s0 = 0; s0 < args.ksplit; s0 += kReduceBatch) {
        f32x4 pg[kReduceBatch][2], pu[kReduceBatch][2];
#pragma unroll
        for (uint32_t j = 0; j < kReduceBatch; ++j) {
            const f32x4 *src = reinterpret_cast<const f32x4 *>(p0 + (size_t)min(s0 + j, args.ksplit - 1) * stride);
            pg[j][0] = src[0];
            pg[j][1] = src[1];
            if constexpr (NW == 2) {
                pu[j][0] = src[N / 4];
                pu[j][1] = src[N / 4 + 1];
            }
        }
#pragma unroll
        for (uint32_t j = 0; j < kReduceBatch; ++j) {
            if (s0 + j >= args.ksplit) break;
#pragma unroll
            for (int e = 0; e < 8; ++e) {
                g[e] += pg[j][e >> 2][e & 3];
                if constexpr (NW == 2) u[e] += pu[j][e >> 2][e & 3];
            }
        }
    }
    float val[8];
#pragma unroll
    for (int e = 0; e < 8; ++e) val[e] = NW == 2 ? activation(g[e], args.act) * u[e] : g[e];
    if (P.bias) {
        const u32x4 bw = *reinterpret_cast<const u32x4 *>(P.bias + n);
        const uint32_t bb[4] = {bw.x, bw.y, bw.z, bw.w};
#pragma unroll
        for (int e = 0; e < 8; ++e) val[e] += bf16_to_f32((bb[e >> 1] >> (16 * (e & 1))) & 0xFFFFu);
    }
    const size_t o = (size_t)m * P.ldo + n;
    if (args.out_f32) {
        f32x4 *out = reinterpret_cast<f32x4 *>(reinterpret_cast<float *>(P.out) + o);
        f32x4 lo = {val[0], val[1], val[2], val[3]}, hi = {val[4], val[5], val[6], val[7]};
        if (args.accumulate) {
            const f32x4 o0 = out[0], o1 = out[1];
            lo = f32x4{o0[0] + lo[0], o0[1] + lo[1], o0[2] + lo[2], o0[3] + lo[3]};
            hi = f32x4{o1[0] + hi[0], o1[1] + hi[1], o1[2] + hi[2], o1[3] + hi[3]};
        }
        out[0] = lo;
        out[1] = hi;
    } else {
        u32x4 *out = reinterpret_cast<u32x4 *>(reinterpret_cast<uint16_t *>(P.out) + o);
        if (args.accumulate) {
            const u32x4 ow = out[0];
            const uint32_t oo[4] = {ow.x, ow.y, ow.z, ow.w};
#pragma unroll
            for (int e = 0; e < 8; ++e) val[e] += bf16_to_f32((oo[e >> 1] >> (16 * (e & 1))) & 0xFFFFu);
        }
        uint32_t pk[4];
#pragma unroll
        for (int e = 0; e < 4; ++e) pk[e] = f32_to_bf16(val[2 * e]) | (f32_to_bf16(val[2 * e + 1]) << 16);
        out[0] = u32x4{pk[0], pk[1], pk[2], pk[3]};
    }
}

hipError_t launch_splitk_reduce(const MfmaArgs &a, int nw, hipStream_t s) {
    const MfmaProblem &P = a.p[0];
    const size_t total = (size_t)a.m * P.w.n;
    const bool vec = P.w.n % 8 == 0 && P.ldo % 8 == 0 && (uintptr_t)P.out % 16 == 0 &&
                     (uintptr_t)a.partial % 16 == 0 && (uintptr_t)P.bias % 16 == 0;
    if (vec) {
        const dim3 grid((unsigned)((total / 8 + 255) / 256));
        if (nw == 2)
            hipLaunchKernelGGL(q4_mfma_splitk_reduce8_kernel<2>, grid, dim3(256), 0, s, a);
        else
            hipLaunchKernelGGL(q4_mfma_splitk_reduce8_kernel<1>, grid, dim3(256), 0, s, a);
        return hipGetLastError();
    }
    hipLaunchKernelGGL(q4_mfma_splitk_reduce_kernel, dim3((unsigned)((total + 255) / 256)), dim3(256), 0, s, a, nw);
    return hipGetLastError();
}

template <int BM, int BN, int NW>
static hipError_t launch_shape(MfmaArgs &a, hipStream_t s) {
    using T = MfmaTile<BM, BN, NW>;
    uint32_t tiles = 0;
    const uint32_t tiles_m = (a.m + BM - 1) / BM;
    for (int i = 0; i < a.np; ++i) {
        a.p[i].tile_begin = tiles;
        tiles += tiles_m * ((a.p[i].w.n + BN - 1) / BN);
    }
    const dim3 grid(tiles, a.ksplit);
    if (a.ksplit > 1) {
        hipLaunchKernelGGL((q4_mfma_gemm_kernel<BM, BN, NW, kMfmaPartial>), grid, dim3(256), T::kLdsBytes, s, a);
        hipError_t e = hipGetLastError();
        if (e != hipSuccess) return e;
        return launch_splitk_reduce(a, NW, s);
    }
    hipLaunchKernelGGL((q4_mfma_gemm_kernel<BM, BN, NW, kMfmaDirect>), grid, dim3(256), T::kLdsBytes, s, a);
    return hipGetLastError();
}

hipError_t launch_mfma(MfmaArgs &a, int bm, hipStream_t s) {
    if (bm > 16 && tuning().prefill_kernel != 1 && prefill_supported(a)) return launch_prefill(a, s);
    const bool gate_up = a.p[0].w2.qw != nullptr;
    if (gate_up) {
        if (bm <= 16) return launch_shape<32, 32, 2>(a, s);
        return launch_shape<64, 64, 2>(a, s);
    }
    if (bm <= 16) return launch_shape<32, 32, 1>(a, s);
    if (bm <= 64) return launch_shape<64, 64, 1>(a, s);
    return launch_shape<128, 64, 1>(a, s);
}

}  // namespace kr
