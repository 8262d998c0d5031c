// moe_route.hpp — one token's softmax and top-k on one wave, shared by the
// routing kernels (moe.hip) and the routed gate/up GEMV that routes a single
// token itself (q4_gemv.hip).
#pragma once
#include <math.h>

#include "kr_internal.hpp"

namespace kr {

// Softmax over E logits and top-K selection for one token, on one wave
// (q4_gemm_and_moe.metal:2509-2568).  Lane l holds experts l + 64 i.  The
// softmax denominator is summed in increasing expert order, as the reference's
// serial loop does (the maximum does not depend on the order), so every
// probability is the reference's value.  The reference's insertion with strict '>' yields the K largest
// probabilities in descending order, ties by increasing id, NaN never taken,
// and (0, -inf) in slots left empty.  Here each expert's position in that
// order is its rank: the number of experts with a larger probability, or an
// equal one and a lower id (counted against the wave's probabilities in LDS);
// rank < K is the slot.  `pr` is this wave's LDS scratch of kMaxExperts floats;
// ti/tv receive the K slots.
constexpr int kRoutePer = (int)(kMaxExperts / 64);  // logits per lane

// This lane's logits of one token (experts lane + 64 i; -inf past E).
__device__ __forceinline__ void load_logits(const float *l, uint32_t E, uint32_t lane, float (&lv)[kRoutePer]) {
#pragma unroll
    for (int i = 0; i < kRoutePer; ++i) {
        const uint32_t e = lane + 64u * i;
        lv[i] = e < E ? l[e] : -INFINITY;
    }
}

__device__ __forceinline__ void route_token_wave(const float (&lv)[kRoutePer], uint32_t E, uint32_t K, int normalize, uint32_t lane,
                                 float *pr, uint32_t *ti, float *tv) {
    constexpr int kPer = kRoutePer;
    float mx = -INFINITY;  // the maximum does not depend on the order
#pragma unroll
    for (int i = 0; i < kPer; ++i) mx = fmaxf(mx, lv[i]);
    mx = wave_max(mx);
    float ex[kPer];
#pragma unroll
    for (int i = 0; i < kPer; ++i) ex[i] = (lane + 64u * i) < E ? expf(lv[i] - mx) : 0.0f;
    // The denominator in increasing expert order: the exponentials go through LDS (zero past E, up
    // to the next multiple of 4) and every lane adds them in order, four per 16-byte read.  Adding
    // +0 leaves the sum's bits unchanged (the sum starts at +0 and never becomes -0), so this is the
    // serial sum over e < E exactly; a cross-lane loop (one lane value per step) took ~70 cycles a
    // step, this ~4.
#pragma unroll
    for (int i = 0; i < kPer; ++i) {
        const uint32_t e = lane + 64u * i;
        if (e < ((E + 3) & ~3u)) pr[e] = ex[i];
    }
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
    float sum = 0.0f;
    {
        const f32x4 *ex4 = reinterpret_cast<const f32x4 *>(pr);
#pragma unroll 4
        for (uint32_t o4 = 0; o4 < (E + 3) / 4; ++o4) {
            const f32x4 q = ex4[o4];
            sum += q[0];
            sum += q[1];
            sum += q[2];
            sum += q[3];
        }
    }
    __builtin_amdgcn_wave_barrier();  // every lane has read the exponentials before pr is overwritten
#pragma unroll
    for (int i = 0; i < kPer; ++i) {
        const uint32_t e = lane + 64u * i;
        if (e < E) pr[e] = ex[i] / sum;
        else if (e < ((E + 3) & ~3u)) pr[e] = __int_as_float(0x7FC00000);  // NaN pads the last float4
    }
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
    uint32_t valid = 0;  // experts with a non-NaN probability
#pragma unroll
    for (int i = 0; i < kPer; ++i) {
        const uint32_t e = lane + 64u * i;
        if (64u * i >= E) break;
        const bool in = e < E;
        const float p = in ? pr[e] : 0.0f;
        valid += (uint32_t)__popcll(__ballot(in && p == p));
        if (!in || p != p) continue;
        uint32_t rank = 0;
        const f32x4 *pr4 = reinterpret_cast<const f32x4 *>(pr);
#pragma unroll 4
        for (uint32_t o4 = 0; o4 < (E + 3) / 4; ++o4) {
            const f32x4 q = pr4[o4];
#pragma unroll
            for (int c = 0; c < 4; ++c) {
                const uint32_t o = 4 * o4 + c;
                rank += (q[c] > p || (q[c] == p && o < e)) ? 1u : 0u;  // NaN pads never count
            }
        }
        if (rank < K) {
            ti[rank] = e;
            tv[rank] = p;
        }
    }
    for (uint32_t k = valid; k < K; ++k) {  // the reference leaves (0, -inf) in unfilled slots
        ti[k] = 0;
        tv[k] = -INFINITY;
    }
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
    if (normalize) {
        // slot order; the loads are independent (the slots past K add +0, which leaves the sum's
        // bits unchanged: it starts at +0 and never becomes -0)
        float t[kRouteMaxTopK];
#pragma unroll
        for (uint32_t k = 0; k < kRouteMaxTopK; ++k) t[k] = k < K ? tv[k] : 0.0f;
        float norm = 0.0f;
#pragma unroll
        for (uint32_t k = 0; k < kRouteMaxTopK; ++k) norm += t[k];
        norm = fmaxf(norm, 1e-8f);
        __builtin_amdgcn_wave_barrier();
        if (lane < K) tv[lane] = tv[lane] / norm;
    }
}

}  // namespace kr
