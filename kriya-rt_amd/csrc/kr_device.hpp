// kr_device.hpp — gfx950 device helpers shared by the Q4_G64 kernels.
//
// Data layout (planar affine Q4_G64, the C ABI's kr_q4_matrix):
//   qw     u32 [n, k/8]   element 8w+j of a row in bits 4j..4j+3 of word w
//   scales bf16 [n, k/64], biases bf16 [n, k/64]
//   w = fma(q, scale, bias)   (crates/kriya-core/src/quantizer.rs:112-126)
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include <type_traits>
#include <utility>

namespace kr {

// f(integral_constant<int, 0>) ... f(integral_constant<int, N - 1>), in order: loops whose index
// must be a compile-time constant (register-array and ring-buffer positions).
template <class F, int... J>
__device__ __forceinline__ void static_for_impl(F &&f, std::integer_sequence<int, J...>) {
    (f(std::integral_constant<int, J>{}), ...);
}
template <int N, class F>
__device__ __forceinline__ void static_for(F &&f) {
    static_for_impl(f, std::make_integer_sequence<int, N>{});
}

typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef _Float16 f16x8_t __attribute__((ext_vector_type(8)));
typedef _Float16 f16x2_t __attribute__((ext_vector_type(2)));

constexpr int kWave = 64;

struct Q4Mat {
    const uint32_t *qw;
    const uint16_t *sc;
    const uint16_t *bi;
    uint32_t n, k;
};

// ---- bf16 <-> f32 (quantizer.rs:19-29: RNE with a wrapping add, exact widening)
__device__ __forceinline__ float bf16_to_f32(uint32_t bits16) { return __uint_as_float(bits16 << 16); }

__device__ __forceinline__ uint32_t f32_to_bf16(float v) {
    uint32_t u = __float_as_uint(v);
    return (u + 0x7FFFu + ((u >> 16) & 1u)) >> 16;
}

// Two values rounded to bf16 by v_cvt_pk_bf16_f32 (round to nearest even): for every input but
// NaN (whose payload it may change) the bits of f32_to_bf16 above, in one instruction.
__device__ __forceinline__ uint32_t pack_bf16_rne(float lo, float hi) {
    typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
    const bf16x2_t h = {(__bf16)lo, (__bf16)hi};
    return __builtin_bit_cast(uint32_t, h);
}

// ---- nibble unpack without conversion instructions.
// For j in 0..3, bits 4j..4j+3 and 16+4j..16+4j+3 of w (elements j and j+4 of
// the word) are placed under the bf16 pattern 0x4300 (= 128.0, ulp 1), giving
// the exact bf16 pair (128 + q_j, 128 + q_{j+4}).  The affine map is then
// applied per group: sum w*x = s * sum (128+q) x + (b - 128 s) * sum x.
__device__ __forceinline__ uint32_t q4_pair_bf16(uint32_t w, int j) {
    return ((w >> (4 * j)) & 0x000F000Fu) | 0x43004300u;
}

// Same with the f16 pattern 0x6400 (= 1024.0, ulp 1): exact (1024 + q) halves.
__device__ __forceinline__ uint32_t q4_pair_f16(uint32_t w, int j) {
    return ((w >> (4 * j)) & 0x000F000Fu) | 0x64006400u;
}

// v_dot2_f32_bf16: a.lo*b.lo + a.hi*b.hi + c in f32.
__device__ __forceinline__ float dot2_bf16(uint32_t a, uint32_t b, float c) {
    return __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2_t, a), __builtin_bit_cast(bf16x2_t, b),
                                           c, false);
}

// (a.lo16, b.lo16) and (a.hi16, b.hi16): pairs x_{i}, x_{i+4} from words (x_i, x_{i+1}), (x_{i+4}, x_{i+5}).
__device__ __forceinline__ uint32_t pack_lo(uint32_t a, uint32_t b) { return (a & 0xFFFFu) | (b << 16); }
__device__ __forceinline__ uint32_t pack_hi(uint32_t a, uint32_t b) { return (a >> 16) | (b & 0xFFFF0000u); }

// ---- loads that do not keep streamed weights in the caches
template <typename T>
__device__ __forceinline__ T ld_stream(const T *p) {
    return __builtin_nontemporal_load(p);
}

// ---- gated activations (q4_gemm_and_moe.metal:2064-2071)
// SiLU g / (1 + e^-g) on the transcendental units: e^-g = 2^(-g log2 e) by v_exp_f32 and the
// quotient as g times v_rcp_f32 (each about 1 ulp of f32, far below the bf16 rounding of the
// outputs), instead of libm's expf and an IEEE division (about 25 instructions per value; the
// prefill gate/up epilogue computes 32 per lane).  Large positive g gives g * rcp(1) = g, large
// negative g gives g * rcp(inf) = -0, as the division does.
__device__ __forceinline__ float activation(float g, int variant) {
    if (variant == 0) return g * __builtin_amdgcn_rcpf(1.0f + __builtin_amdgcn_exp2f(-1.44269504f * g));
    if (variant == 1) {
        const float kSqrt2OverPi = 0.7978845608f;
        float cubic = fmaf(0.044715f * g, g * g, g);
        return 0.5f * g * (1.0f + tanhf(kSqrt2OverPi * cubic));
    }
    return fmaxf(g, 0.0f);
}

// ---- wavefront reductions (64 lanes), without LDS
// One fixed pairing tree over the 64 lanes, level by level: lane l ^ 32 (v_permlane32_swap),
// l ^ 16 (v_permlane16_swap), l ^ 8 (DPP row_ror:8), the mirror lane of its group of 8 (DPP
// row_half_mirror), l ^ 2 and l ^ 1 (DPP quad_perm).  A reduction of R values first halves the
// value set at the top levels (each lane keeps the half it owns and adds its partner's copy of
// it), so that segment s of 64 / R lanes ends with value s; the remaining levels sum within
// the segment.  Every value is summed over the same tree whatever R is, and all lanes of a
// segment hold the same bits.
template <int kCtrl>
__device__ __forceinline__ float dpp_f32(float v) {
    return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), kCtrl, 0xF, 0xF, false));
}
// partner's copy of v at tree level L (0: l ^ 32 ... 5: l ^ 1); whether lane is the pair's upper
template <int L>
__device__ __forceinline__ float tree_partner(float v, int lane) {
    if constexpr (L == 0) {
        const auto p = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
        return __uint_as_float(lane < 32 ? p[1] : p[0]);
    } else if constexpr (L == 1) {
        const auto p = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
        return __uint_as_float((lane & 16) ? p[0] : p[1]);
    } else if constexpr (L == 2) {
        return dpp_f32<0x128>(v);  // row_ror:8, i.e. lane ^ 8 within the 16-lane row
    } else if constexpr (L == 3) {
        return dpp_f32<0x141>(v);  // row_half_mirror: lane 7 - i of its group of 8
    } else if constexpr (L == 4) {
        return dpp_f32<0x4E>(v);  // quad_perm [2, 3, 0, 1]
    } else {
        return dpp_f32<0xB1>(v);  // quad_perm [1, 0, 3, 2]
    }
}
template <int L>
__device__ __forceinline__ bool tree_upper(int lane) {
    return (lane & (32 >> L)) != 0;  // (level 3: lanes 4..7 of each group of 8)
}
// One halving level over values v[i] (i < half) and v[i + half]: the lower lane of each pair
// keeps value i, the upper value i + half, each plus its partner's copy.
template <int L, int kHalf, class V>
__device__ __forceinline__ void tree_halve(V &v, int lane) {
    constexpr int half = kHalf;
    if constexpr (L <= 1) {  // one swap instruction exchanges both values of the pair
#pragma unroll
        for (int i = 0; i < half; ++i) {
            const uint32_t a = __float_as_uint(v[i]), b = __float_as_uint(v[i + half]);
            if constexpr (L == 0) {
                const auto p = __builtin_amdgcn_permlane32_swap(a, b, false, false);
                v[i] = __uint_as_float(p[0]) + __uint_as_float(p[1]);
            } else {
                const auto p = __builtin_amdgcn_permlane16_swap(a, b, false, false);
                v[i] = __uint_as_float(p[0]) + __uint_as_float(p[1]);
            }
        }
    } else {
        // both values summed with their partner copies, then the lane's one picked: a select
        // between the two vector elements instead is turned into a run-time element index,
        // which the back end expands into a compare-and-select over the whole vector
        const bool upper = tree_upper<L>(lane);
#pragma unroll
        for (int i = 0; i < half; ++i) {
            const float lo = v[i] + tree_partner<L>(v[i], lane);
            const float hi = v[i + half] + tree_partner<L>(v[i + half], lane);
            v[i] = upper ? hi : lo;
        }
    }
}
template <int L>
__device__ __forceinline__ float tree_sum_from(float s, int lane) {
    if constexpr (L <= 5) {
        s += tree_partner<L>(s, lane);
        return tree_sum_from<L + 1>(s, lane);
    } else {
        return s;
    }
}
template <int N, class V>
__device__ __forceinline__ float tree_reduce(V &v, int lane) {
    static_assert(N >= 1 && N <= 64 && (N & (N - 1)) == 0, "a power of two of values");
    if constexpr (N >= 2) tree_halve<0, N / 2>(v, lane);
    if constexpr (N >= 4) tree_halve<1, N / 4>(v, lane);
    if constexpr (N >= 8) tree_halve<2, N / 8>(v, lane);
    if constexpr (N >= 16) tree_halve<3, N / 16>(v, lane);
    if constexpr (N >= 32) tree_halve<4, N / 32>(v, lane);
    if constexpr (N >= 64) tree_halve<5, N / 64>(v, lane);
    constexpr int kLevels = N == 1 ? 0 : N == 2 ? 1 : N == 4 ? 2 : N == 8 ? 3 : N == 16 ? 4 : N == 32 ? 5 : 6;
    return tree_sum_from<kLevels>(v[0], lane);
}

// Reduces R per-lane values at once; afterwards every lane of the 64 / R-lane segment s holds
// the total of value s.  Fixed order: the result is identical on every launch.
template <int R>
__device__ __forceinline__ float wave_reduce_rows(float (&v)[R], int lane) {
    return tree_reduce<R>(v, lane);
}

// The same over a vector of N values (an SSA value: a float array here was
// sometimes turned into a memory access with a selected index, which kept it
// out of registers).
template <int N>
struct FVec {
    typedef float type __attribute__((ext_vector_type(N)));
};
template <int N>
__device__ __forceinline__ float wave_reduce_vec(typename FVec<N>::type v, int lane) {
    return tree_reduce<N>(v, lane);
}

// Sum over all 64 lanes on the same tree, every lane holding the same bits (no LDS).
__device__ __forceinline__ float wave_total(float v, int lane) { return tree_sum_from<0>(v, lane); }
// Max over the lanes from tree level L0 on (0: all 64, 2: each row of 16); max is exact, so any
// order gives the same bits.
template <int L0>
__device__ __forceinline__ float tree_max_from(float v, int lane) {
    if constexpr (L0 <= 5) {
        v = fmaxf(v, tree_partner<L0>(v, lane));
        return tree_max_from<L0 + 1>(v, lane);
    } else {
        return v;
    }
}

// The value of lane l ^ 32 or l ^ 16 (one swap instruction, no LDS).
__device__ __forceinline__ float xchg32(float v, int lane) { return tree_partner<0>(v, lane); }
__device__ __forceinline__ float xchg16(float v, int lane) { return tree_partner<1>(v, lane); }

// ---- activations outside fp16's range on the fp16 matrix-core paths.
// fp16 holds a bf16 value exactly only within [2^-14, 65504]: a token row whose
// largest |x| lies outside a safe window is staged times 2^e and its results
// multiplied by 2^-e (both exact: powers of two).

// Largest |value| of 8 bf16 values (a 16-byte unit) as non-negative bf16 bits:
// magnitudes order as unsigned integers once the sign is cleared.
__device__ __forceinline__ uint32_t bf16_unit_max_bits(const u32x4 &v) {
    const uint32_t m = 0x7FFF7FFFu;
    const auto pmax = [](uint32_t x, uint32_t y) -> uint32_t {  // per 16-bit half
        return max(x & 0xFFFFu, y & 0xFFFFu) | (max(x >> 16, y >> 16) << 16);
    };
    const uint32_t p = pmax(pmax(v.x & m, v.y & m), pmax(v.z & m, v.w & m));
    return max(p & 0xFFFFu, p >> 16);
}

// The exponent e for a row whose largest |x| has bf16 bits mb: 0 when its unbiased
// exponent is within [lo, hi] (no scaling), else `target` - exponent, clamped so that
// 2^e and 2^-e are normal floats.  Zero rows and rows holding inf or NaN get 0.
__device__ __forceinline__ int row_stage_exp(uint32_t mb, int lo, int hi, int target) {
    const int ef = (int)(mb >> 7);  // biased exponent field of a bf16
    if (mb == 0u || ef == 0xFF) return 0;
    const int ex = ef - 127;  // bf16 subnormals count as 2^-127
    if (ex >= lo && ex <= hi) return 0;
    return max(min(target - ex, 100), -100);
}

__device__ __forceinline__ float exp2_int(int e) { return __int_as_float((127 + e) << 23); }  // |e| <= 126

// Unsigned max over aligned groups of 16 (or 8: HALF) lanes, left in every lane of the group:
// DPP quad swaps, then the half-row (and row) mirror.
template <bool HALF = false>
__device__ __forceinline__ uint32_t row16_max_u32(uint32_t v) {
    v = max(v, (uint32_t)__builtin_amdgcn_update_dpp((int)v, (int)v, 0xB1, 0xF, 0xF, false));   // quad [1,0,3,2]
    v = max(v, (uint32_t)__builtin_amdgcn_update_dpp((int)v, (int)v, 0x4E, 0xF, 0xF, false));   // quad [2,3,0,1]
    v = max(v, (uint32_t)__builtin_amdgcn_update_dpp((int)v, (int)v, 0x141, 0xF, 0xF, false));  // half-row mirror
    if (!HALF) v = max(v, (uint32_t)__builtin_amdgcn_update_dpp((int)v, (int)v, 0x140, 0xF, 0xF, false));  // row mirror
    return v;
}

// Unsigned max over the 64 lanes, as a wave-uniform value (row maxima, then the row broadcasts of
// lanes 15 and 31; lane 63 ends with the maximum).
__device__ __forceinline__ uint32_t wave_max_u32(uint32_t v) {
    v = row16_max_u32(v);
    v = max(v, (uint32_t)__builtin_amdgcn_update_dpp((int)v, (int)v, 0x142, 0xA, 0xF, false));  // row bcast 15
    v = max(v, (uint32_t)__builtin_amdgcn_update_dpp((int)v, (int)v, 0x143, 0xC, 0xF, false));  // row bcast 31
    return (uint32_t)__builtin_amdgcn_readlane((int)v, 63);
}

// Sum over the 64 lanes (the tree of wave_total), every lane holding the same bits.
__device__ __forceinline__ float wave_sum(float v) { return tree_sum_from<0>(v, (int)__lane_id()); }
__device__ __forceinline__ float wave_max(float v) { return tree_max_from<0>(v, (int)__lane_id()); }

}  // namespace kr
