// moe.hip — MoE routing and combine on the device.
//
// Routing replaces moe_router_topk_and_histogram and
// moe_router_prefix_scan_and_scatter (kernels/metal/q4_gemm_and_moe.metal:2495-2624;
// dispatched at crates/kriya-backend-metal/src/encoder.rs:5275-5313) with one
// single-block launch: per-token softmax and top-k by insertion with strict '>'
// (ties go to the lower expert id), per-expert counts, their exclusive prefix
// offsets[E+1], and the expert-sorted assignment list.  The reference takes an
// assignment's slot inside its expert bucket from an atomic counter, so the
// order inside a bucket depends on thread timing (and its counts buffer is
// never reset between calls); here the slot is the assignment's rank among the
// assignments of its expert in increasing assignment id t*K + k, which is the
// order the reference's own scan test expects (crates/kriya-backend-metal/
// tests/test_shader_compile.rs:2988-3117).  The result is deterministic.
//
// Combine replaces moe_combine_routed_and_shared_bf16
// (kernels/metal/transformer_glue.metal:373-401): y[t, :] = sum_k fma(w[t, k],
// d[t*K + k, :], acc) in slot order, with the expert outputs d kept in f32.
#include <math.h>

#include "kr_internal.hpp"
#include "moe_route.hpp"

namespace kr {

// One block.  logits != nullptr: route one token per wave (writes experts,
// weights); else the assignments `experts` are given.  Then counts, offsets
// and the sorted list.
__global__ __launch_bounds__(1024) void moe_route_kernel(const float *logits, uint32_t T, uint32_t E, uint32_t K,
                                                         int normalize, uint32_t *experts, float *weights,
                                                         uint32_t *counts, uint32_t *offsets, uint32_t *sorted) {
    __shared__ uint32_t s_cnt[kMaxExperts];
    __shared__ uint32_t s_off[kMaxExperts + 1];
    __shared__ uint32_t s_ti[16][kRouteMaxTopK];
    __shared__ float s_tv[16][kRouteMaxTopK];
    __shared__ __attribute__((aligned(16))) float s_pr[16][kMaxExperts];
    __shared__ uint16_t s_exp[kRouteMaxAssign];  // expert of each assignment; 0xFFFF: id >= E
    const uint32_t tid = threadIdx.x, nthreads = blockDim.x;
    const uint32_t lane = tid & 63, wave = tid >> 6, waves = nthreads >> 6;
    const uint32_t total = T * K;
    for (uint32_t e = tid; e < E; e += nthreads) s_cnt[e] = 0;
    __syncthreads();
    if (logits) {
        // the next token's logits are requested before the current token is routed
        float lv[kRoutePer], ln[kRoutePer];
        if (wave < T) load_logits(logits + (size_t)wave * E, E, lane, ln);
        for (uint32_t t = wave; t < T; t += waves) {
#pragma unroll
            for (int i = 0; i < kRoutePer; ++i) lv[i] = ln[i];
            if (t + waves < T) load_logits(logits + (size_t)(t + waves) * E, E, lane, ln);
            route_token_wave(lv, E, K, normalize, lane, s_pr[wave], s_ti[wave], s_tv[wave]);
            __builtin_amdgcn_wave_barrier();
            __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
            __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
            if (lane < K) {
                const uint32_t e = s_ti[wave][lane];
                experts[t * K + lane] = e;
                weights[t * K + lane] = s_tv[wave][lane];
                s_exp[t * K + lane] = (uint16_t)e;
                atomicAdd(&s_cnt[e], 1u);  // counts only: the order of the adds does not matter
            }
        }
    } else {
        for (uint32_t i = tid; i < total; i += nthreads) {
            const uint32_t e = experts[i];
            // an id >= E joins no bucket, so offsets[E] < T*K reports it
            s_exp[i] = e < E ? (uint16_t)e : (uint16_t)0xFFFFu;
            if (e < E) atomicAdd(&s_cnt[e], 1u);
        }
    }
    __syncthreads();
    if (wave == 0) {  // exclusive scan: lane l owns experts 4l .. 4l+3
        uint32_t c[4], run = 0;
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const uint32_t e = 4 * lane + j;
            c[j] = e < E ? s_cnt[e] : 0u;
            run += c[j];
        }
        uint32_t incl = run;
#pragma unroll
        for (int m = 1; m < 64; m <<= 1) {
            const uint32_t o = __shfl_up(incl, m);
            if (lane >= (uint32_t)m) incl += o;
        }
        uint32_t off = incl - run;
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const uint32_t e = 4 * lane + j;
            if (e < E) s_off[e] = off;
            off += c[j];
        }
        if (lane == 63) s_off[E] = incl;
    }
    __syncthreads();
    for (uint32_t e = tid; e <= E; e += nthreads) {
        offsets[e] = s_off[e];
        if (e < E) counts[e] = s_cnt[e];
    }
    // scatter: wave w walks experts w, w + waves, ... and, for each, the
    // assignments in increasing id, 64 at a time
    const uint64_t below = (1ull << lane) - 1ull;
    for (uint32_t e = wave; e < E; e += waves) {
        uint32_t run = s_off[e];
        if (s_cnt[e] == 0) continue;
        for (uint32_t a0 = 0; a0 < total; a0 += 64) {
            const uint32_t a = a0 + lane;
            const bool hit = a < total && s_exp[a] == e;
            const uint64_t mask = __ballot(hit);
            if (hit) sorted[run + (uint32_t)__popcll(mask & below)] = a;
            run += (uint32_t)__popcll(mask);
        }
    }
}

// Softmax and top-k only, one token per wave and 16 tokens per block, for
// token counts where one block would route them in several serial rounds.
__global__ __launch_bounds__(1024) void moe_topk_kernel(const float *logits, uint32_t T, uint32_t E, uint32_t K,
                                                        int normalize, uint32_t *experts, float *weights) {
    __shared__ uint32_t s_ti[16][kRouteMaxTopK];
    __shared__ float s_tv[16][kRouteMaxTopK];
    __shared__ __attribute__((aligned(16))) float s_pr[16][kMaxExperts];
    const uint32_t lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const uint32_t t = blockIdx.x * 16 + wave;
    if (t >= T) return;
    float lv[kRoutePer];
    load_logits(logits + (size_t)t * E, E, lane, lv);
    route_token_wave(lv, E, K, normalize, lane, s_pr[wave], s_ti[wave], s_tv[wave]);
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
    if (lane < K) {
        experts[t * K + lane] = s_ti[wave][lane];
        weights[t * K + lane] = s_tv[wave][lane];
    }
}

// Tokens up to which one block routes them all (a wave per token, in rounds) rather than a top-k
// launch over 16-token blocks followed by the scan launch.  At 64 tokens (four rounds) one block
// made the cfg4 T = 64 step 106 -> 118 us.
constexpr uint32_t kRouteOneBlockTokens = 16;

hipError_t launch_moe_route(const float *logits, uint32_t T, uint32_t E, uint32_t K, int normalize,
                            uint32_t *experts, float *weights, uint32_t *counts, uint32_t *offsets, uint32_t *sorted,
                            hipStream_t s) {
    if (logits && T > kRouteOneBlockTokens) {
        // more tokens than one block routes in a round: top-k on ceil(T / 16) blocks, then the
        // counts, offsets and sorted list from the chosen experts (the same results)
        hipLaunchKernelGGL(moe_topk_kernel, dim3((T + 15) / 16), dim3(1024), 0, s, logits, T, E, K, normalize, experts,
                           weights);
        if (hipError_t e = hipGetLastError()) return e;
        logits = nullptr;
    }
    hipLaunchKernelGGL(moe_route_kernel, dim3(1), dim3(1024), 0, s, logits, T, E, K, normalize, experts, weights,
                       counts, offsets, sorted);
    return hipGetLastError();
}

// y[t, c..c+3] (+)= sum_k fma(w[t, k], d[t*K + k, c..c+3], acc), slot order.
__global__ __launch_bounds__(256) void moe_combine_kernel(const float *d, const float *w, uint32_t T, uint32_t K,
                                                          uint32_t H, void *y, int y_f32, int accumulate) {
    const uint32_t q = H / 4;
    const size_t i = (size_t)blockIdx.x * 256 + threadIdx.x;
    if (i >= (size_t)T * q) return;
    const uint32_t t = (uint32_t)(i / q), c = (uint32_t)(i % q) * 4;
    f32x4 acc = {0, 0, 0, 0};
    for (uint32_t k = 0; k < K; ++k) {
        const float wk = w[(size_t)t * K + k];
        const f32x4 dv = *reinterpret_cast<const f32x4 *>(d + ((size_t)t * K + k) * H + c);
#pragma unroll
        for (int v = 0; v < 4; ++v) acc[v] = fmaf(wk, dv[v], acc[v]);
    }
    const size_t o = (size_t)t * H + c;
    if (y_f32) {
        float *out = reinterpret_cast<float *>(y) + o;
#pragma unroll
        for (int v = 0; v < 4; ++v) out[v] = accumulate ? out[v] + acc[v] : acc[v];
    } else {
        uint16_t *out = reinterpret_cast<uint16_t *>(y) + o;
#pragma unroll
        for (int v = 0; v < 4; ++v)
            out[v] = (uint16_t)f32_to_bf16(accumulate ? bf16_to_f32(out[v]) + acc[v] : acc[v]);
    }
}

hipError_t launch_moe_combine(const float *d, const float *w, uint32_t T, uint32_t K, uint32_t H, void *y, int y_f32,
                              int accumulate, hipStream_t s) {
    const size_t n = (size_t)T * (H / 4);
    hipLaunchKernelGGL(moe_combine_kernel, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, s, d, w, T, K, H, y, y_f32,
                       accumulate);
    return hipGetLastError();
}

}  // namespace kr
