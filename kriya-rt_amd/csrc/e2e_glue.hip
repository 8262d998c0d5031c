// e2e_glue.hip — the Q4 embedding lookup and the non-Q4 glue that config 3's
// end-to-end decode needs around the Q4 matmuls: RMSNorm, RoPE + KV append,
// decode attention (GQA) and greedy argmax.  Plain, correct HIP; the Q4
// matmuls carry the time.
//
// Reference semantics:
//   embedding_lookup_q4_g64   kernels/metal/transformer_glue.metal:122-152
//   rms_norm_bf16             kernels/metal/transformer_glue.metal:158-205
//   fused_qknorm_rope_and_kv_append (no qk-norm, contiguous cache)
//                             kernels/metal/paged_gqa_and_deltanet.metal:115-222
//   RoPE table                crates/kriya-backend-metal/src/encoder.rs:1940-1950
//   gpu_token_sampler (greedy) kernels/metal/transformer_glue.metal:407-494
#include <math.h>

#include <algorithm>

#include "kr_internal.hpp"
#include "q4_dot2.hpp"

namespace kr {

// out[t, d] = bf16(fma(q, s, b)) of row tokens[t]; rows past n give zeros.
__global__ __launch_bounds__(256) void q4_embedding_kernel(Q4Mat w, const uint32_t *tokens, uint32_t count,
                                                           uint16_t *out) {
    const uint32_t t = blockIdx.y;
    const uint32_t c8 = blockIdx.x * 256 + threadIdx.x;  // 8-column unit
    if (t >= count || c8 >= (w.k >> 3)) return;
    const uint32_t row = tokens[t];
    uint16_t *dst = out + (size_t)t * w.k + 8 * c8;
    if (row >= w.n) {
#pragma unroll
        for (int j = 0; j < 8; ++j) dst[j] = 0;
        return;
    }
    const uint32_t word = w.qw[(size_t)row * (w.k >> 3) + c8];
    const size_t gi = (size_t)row * (w.k >> 6) + (c8 >> 3);
    const float s = bf16_to_f32(w.sc[gi]), b = bf16_to_f32(w.bi[gi]);
#pragma unroll
    for (int j = 0; j < 8; ++j) dst[j] = (uint16_t)f32_to_bf16(fmaf((float)((word >> (4 * j)) & 0xF), s, b));
}

// One block per row: y = bf16(x * rsqrt(mean(x^2) + eps) * w).  Rows of
// dim % 8 == 0 and dim <= 8192 take one pass: each thread holds up to four
// 8-element pieces of x and w in registers from a single round of loads.
__global__ __launch_bounds__(256) void rmsnorm_kernel(const uint16_t *x, const uint16_t *weight, uint32_t dim,
                                                      float eps, uint16_t *out) {
    __shared__ float red[4];
    const uint32_t row = blockIdx.x, tid = threadIdx.x;
    const uint16_t *xr = x + (size_t)row * dim;
    uint16_t *yr = out + (size_t)row * dim;
    const bool fast = dim % 8 == 0 && dim <= 8 * 4 * 256;
    float ss = 0.0f;
    u32x4 xv[4], wv[4];
    const uint32_t pieces = dim / 8;
    if (fast) {
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const uint32_t pc = tid + 256u * j;
            if (pc < pieces) {
                xv[j] = *reinterpret_cast<const u32x4 *>(xr + 8 * pc);
                wv[j] = *reinterpret_cast<const u32x4 *>(weight + 8 * pc);
            }
        }
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            if (tid + 256u * j < pieces) {
                const uint32_t X[4] = {xv[j].x, xv[j].y, xv[j].z, xv[j].w};
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    const float a = __uint_as_float(X[e] << 16), b = __uint_as_float(X[e] & 0xFFFF0000u);
                    ss = fmaf(a, a, ss);
                    ss = fmaf(b, b, ss);
                }
            }
        }
    } else {
        for (uint32_t d = tid; d < dim; d += 256) {
            const float v = bf16_to_f32(xr[d]);
            ss = fmaf(v, v, ss);
        }
    }
    ss = wave_sum(ss);
    if ((tid & 63) == 0) red[tid >> 6] = ss;
    __syncthreads();
    const float tot = red[0] + red[1] + red[2] + red[3];
    const float scale = 1.0f / sqrtf(tot / (float)dim + eps);
    if (fast) {
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const uint32_t pc = tid + 256u * j;
            if (pc < pieces) {
                const uint32_t X[4] = {xv[j].x, xv[j].y, xv[j].z, xv[j].w};
                const uint32_t W[4] = {wv[j].x, wv[j].y, wv[j].z, wv[j].w};
                uint32_t o[4];
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    const float lo = __uint_as_float(X[e] << 16) * scale * __uint_as_float(W[e] << 16);
                    const float hi = __uint_as_float(X[e] & 0xFFFF0000u) * scale * __uint_as_float(W[e] & 0xFFFF0000u);
                    o[e] = f32_to_bf16(lo) | (f32_to_bf16(hi) << 16);
                }
                *reinterpret_cast<u32x4 *>(yr + 8 * pc) = u32x4{o[0], o[1], o[2], o[3]};
            }
        }
    } else {
        for (uint32_t d = tid; d < dim; d += 256)
            yr[d] = (uint16_t)f32_to_bf16(bf16_to_f32(xr[d]) * scale * bf16_to_f32(weight[d]));
    }
}

// grid (q_heads + kv_heads, batch): rotate pairs (d, d + D/2) of q in place and
// of k into the cache at the sequence's position; copy v into the cache.
// cache layout [batch, max_ctx, kv_heads, D]; cos_sin [pos, D/2] (cos, sin).
__global__ __launch_bounds__(64) void rope_kv_append_kernel(uint16_t *q, const uint16_t *k, const uint16_t *v,
                                                            const float *cos_sin, const uint32_t *positions,
                                                            uint32_t q_heads, uint32_t kv_heads, uint32_t D,
                                                            uint16_t *k_cache, uint16_t *v_cache, uint32_t max_ctx) {
    const uint32_t b = blockIdx.y, head = blockIdx.x;
    const uint32_t pos = positions[b];
    if (pos >= max_ctx) return;
    const bool is_q = head < q_heads;
    const uint32_t h = is_q ? head : head - q_heads;
    const uint32_t half = D / 2;
    const uint16_t *src = is_q ? q + ((size_t)b * q_heads + h) * D : k + ((size_t)b * kv_heads + h) * D;
    const size_t cbase = (((size_t)b * max_ctx + pos) * kv_heads + h) * D;
    for (uint32_t i = threadIdx.x; i < half; i += 64) {
        const float x0 = bf16_to_f32(src[i]), x1 = bf16_to_f32(src[i + half]);
        const float c = cos_sin[2 * ((size_t)pos * half + i)], s = cos_sin[2 * ((size_t)pos * half + i) + 1];
        const float r0 = fmaf(x0, c, -x1 * s), r1 = fmaf(x0, s, x1 * c);
        if (is_q) {
            uint16_t *dst = q + ((size_t)b * q_heads + h) * D;
            dst[i] = (uint16_t)f32_to_bf16(r0);
            dst[i + half] = (uint16_t)f32_to_bf16(r1);
        } else {
            k_cache[cbase + i] = (uint16_t)f32_to_bf16(r0);
            k_cache[cbase + i + half] = (uint16_t)f32_to_bf16(r1);
            const uint16_t *vs = v + ((size_t)b * kv_heads + h) * D;
            v_cache[cbase + i] = vs[i];
            v_cache[cbase + i + half] = vs[i + half];
        }
    }
}

// grid (q_heads, batch), 1024 threads: out = softmax(q . k_p / sqrt(D)) v over
// positions p <= positions[b]; kv head = q head / (q_heads / kv_heads).
// Scores: a thread per position, its key row read in 16-byte pieces (one
// round of loads for up to 1024 positions).  Values: 512 threads, thread t
// takes 8 dims (piece t % (D/8)) over the positions p = t / (D/8) (mod
// 512 / (D/8)); the position groups are then added in a fixed order.
constexpr uint32_t kAttnMaxCtx = kGlueMaxCtx;
constexpr uint32_t kAttnMaxD = kGlueMaxHeadDim;
constexpr uint32_t kAttnThreads = 1024;
__global__ __launch_bounds__(kAttnThreads) void attention_decode_kernel(
    const uint16_t *q, const uint16_t *k_cache, const uint16_t *v_cache, const uint32_t *positions, uint32_t q_heads,
    uint32_t kv_heads, uint32_t D, uint32_t max_ctx, uint16_t *out) {
    __shared__ float qs[kAttnMaxD];
    __shared__ float sc[kAttnMaxCtx];
    __shared__ float red[kAttnThreads / 64];
    __shared__ float part[4096];  // [position group][dim], 512 threads x 8 dims
    const uint32_t b = blockIdx.y, h = blockIdx.x, tid = threadIdx.x;
    constexpr uint32_t kWaves = kAttnThreads / 64;
    const uint32_t kvh = h / (q_heads / kv_heads);
    const uint32_t n = min(positions[b], max_ctx - 1) + 1;
    const uint32_t pieces = D / 8;  // 16-byte pieces per row (D % 8 == 0)
    const float inv = 1.0f / sqrtf((float)D);
    const size_t row_stride = (size_t)kv_heads * D;  // elements between positions
    const uint16_t *kbase = k_cache + ((size_t)b * max_ctx * kv_heads + kvh) * D;
    const uint16_t *vbase = v_cache + ((size_t)b * max_ctx * kv_heads + kvh) * D;
    for (uint32_t d = tid; d < D; d += kAttnThreads) qs[d] = bf16_to_f32(q[((size_t)b * q_heads + h) * D + d]);
    __syncthreads();
    float mx = -INFINITY;
    for (uint32_t p = tid; p < n; p += kAttnThreads) {
        const u32x4 *kp = reinterpret_cast<const u32x4 *>(kbase + p * row_stride);
        u32x4 kr[kAttnMaxD / 8];
#pragma unroll
        for (uint32_t c = 0; c < kAttnMaxD / 8; ++c)
            if (c < pieces) kr[c] = kp[c];
        float dot = 0.0f;
#pragma unroll
        for (uint32_t c = 0; c < kAttnMaxD / 8; ++c) {
            if (c >= pieces) break;
            const uint32_t W[4] = {kr[c].x, kr[c].y, kr[c].z, kr[c].w};
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                dot = fmaf(qs[8 * c + 2 * e], __uint_as_float(W[e] << 16), dot);
                dot = fmaf(qs[8 * c + 2 * e + 1], __uint_as_float(W[e] & 0xFFFF0000u), dot);
            }
        }
        dot *= inv;
        sc[p] = dot;
        mx = fmaxf(mx, dot);
    }
    mx = wave_max(mx);
    if ((tid & 63) == 0) red[tid >> 6] = mx;
    __syncthreads();
    mx = red[0];
    for (uint32_t w = 1; w < kWaves; ++w) mx = fmaxf(mx, red[w]);
    __syncthreads();
    float sum = 0.0f;
    for (uint32_t p = tid; p < n; p += kAttnThreads) {
        const float e = expf(sc[p] - mx);
        sc[p] = e;
        sum += e;
    }
    sum = wave_sum(sum);
    if ((tid & 63) == 0) red[tid >> 6] = sum;
    __syncthreads();
    float tot_sum = 0.0f;
    for (uint32_t w = 0; w < kWaves; ++w) tot_sum += red[w];
    const float inv_sum = 1.0f / tot_sum;
    // values
    const uint32_t groups = 512 / pieces;
    const uint32_t pc = tid % pieces, pg = tid / pieces;
    if (pg < groups) {
        float acc[8] = {0, 0, 0, 0, 0, 0, 0, 0};
#pragma unroll 8
        for (uint32_t p = pg; p < n; p += groups) {
            const u32x4 w = *reinterpret_cast<const u32x4 *>(vbase + p * row_stride + 8 * pc);
            const uint32_t W[4] = {w.x, w.y, w.z, w.w};
            const float pr = sc[p];
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                acc[2 * e] = fmaf(pr, __uint_as_float(W[e] << 16), acc[2 * e]);
                acc[2 * e + 1] = fmaf(pr, __uint_as_float(W[e] & 0xFFFF0000u), acc[2 * e + 1]);
            }
        }
#pragma unroll
        for (int e = 0; e < 8; ++e) part[pg * D + 8 * pc + e] = acc[e];
    }
    __syncthreads();
    for (uint32_t d = tid; d < D; d += kAttnThreads) {
        float tot = 0.0f;
        for (uint32_t g = 0; g < groups; ++g) tot += part[g * D + d];
        out[((size_t)b * q_heads + h) * D + d] = (uint16_t)f32_to_bf16(tot * inv_sum);
    }
}

// ---- RoPE + KV append + decode attention, split over the context
//
// attention_split_kernel<GP>: grid (splits, kv_heads, batch), 256 threads.  The
// block owns 16 positions of one sequence and one kv head and all G <= GP
// query heads that share it (GQA: each key and value row is read once for the
// G heads).  Thread t is lane c = t % 16 of row r = t / 16.  It
//   0. requests, before anything else, its key piece in the matrix-core layout
//      (position t % 16, dims 32 (t / 64) + 8 ((t / 16) % 4)) and its value
//      piece (position c, dims 8r..) -- the rows of D > 128 in a second piece
//      each;
//   1. rotates the G query heads (bf16-rounded, as kr_rope_kv_append stores
//      them) into LDS;
//   2. if the block holds the new position, rotates k and writes k and v into
//      the cache (kr_rope_kv_append's arithmetic); its own scores take that
//      row from LDS;
//   3. scores: wave w multiplies the 32-dim steps w [and w + 4] of q (head
//      rows) with the key slice on the matrix cores (v_mfma_f32_16x16x32_bf16;
//      bf16 products are exact, sums f32); the value tile goes to LDS over q;
//   4. per head (a row of 16 lanes, one per position): the four waves' partial
//      scores added in wave order, the slice's max m and sum l of
//      exp(score - m);
//   5. values: wave w multiplies the probabilities (bf16 hi + lo) with the
//      16-dim tiles w, w + 4, ... of the LDS value tile on the matrix cores.
// The partial (m, l, acc) of each (sequence, kv head, slice) goes to the
// workspace; attention_combine_kernel merges the slices in slice order:
//   out = sum_s e^(m_s - M) acc_s / sum_s e^(m_s - M) l_s,  M = max_s m_s
// (with the running max of chunks of 64 slices rescaled as chunks are added).
constexpr uint32_t kSplitLen = 16;   // positions per slice

__device__ __forceinline__ float bf16_round(float v) { return bf16_to_f32(f32_to_bf16(v)); }

template <int GP>
__global__ __launch_bounds__(256) void attention_split_kernel(const uint16_t *q, const uint16_t *k, const uint16_t *v,
                                                              const float *cos_sin, const uint32_t *positions,
                                                              uint32_t q_heads, uint32_t kv_heads, uint32_t D,
                                                              uint16_t *k_cache, uint16_t *v_cache, uint32_t max_ctx,
                                                              float *part) {
    // rotated q [G][D]; after the scores, the value tile [kSplitLen][D] bf16 in the same memory
    constexpr uint32_t kQsFloats = GP * kGlueMaxHeadDim > kSplitLen * kGlueMaxHeadDim / 2
                                       ? GP * kGlueMaxHeadDim
                                       : kSplitLen * kGlueMaxHeadDim / 2;
    __shared__ __align__(16) float qs[kQsFloats];
    __shared__ float sc[GP][kSplitLen];                        // exp(score - m)
    __shared__ float sp[4][16][kSplitLen];                     // per-wave partial scores [wave][head][pos]
    __shared__ __align__(16) float knew[kGlueMaxHeadDim];
    __shared__ __align__(16) uint16_t vnew[kGlueMaxHeadDim];
    const uint32_t tid = threadIdx.x, r = tid >> 4, c = tid & 15;
    const uint32_t s = blockIdx.x, kvh = blockIdx.y, b = blockIdx.z, splits = gridDim.x;
    const uint32_t G = q_heads / kv_heads, half = D / 2, P = D / 8;
    const uint32_t p0 = s * kSplitLen;
    // The position first: loads complete in issue order, so it can arrive (and the RoPE table row
    // it selects be requested) while the key and value rows below are still in flight.
    const uint32_t pos = __builtin_amdgcn_readfirstlane(positions[b]);
    __builtin_amdgcn_sched_barrier(0);
    // 0. loads that do not depend on the position, all in one round trip with it: the key piece
    //    (position p0 + r, piece c [+16]) and value piece (position p0 + c, piece r [+16]) of rows
    //    below max_ctx, two query pairs per thread, and the new k and v pairs of thread < D/2.
    const size_t row_stride = (size_t)kv_heads * D;
    const uint16_t *kbase = k_cache + (((size_t)b * max_ctx + p0) * kv_heads + kvh) * D;
    const uint16_t *vbase = v_cache + (((size_t)b * max_ctx + p0) * kv_heads + kvh) * D;
    // Loads are unconditional, from clamped (in-bounds) addresses; what they should not
    // contribute is zeroed where it is used.  A conditional load merged with a default value
    // makes the compiler wait for every load in flight at the merge.
    // key pieces in the matrix-core layout of the scores: thread (wave w, lane l) takes position
    // p0 + (l & 15) and piece 4 w + (l >> 4) [+16], i.e. dims 32 w + 8 (l >> 4) [+128]
    const uint32_t kp = tid & 15, kc = 4 * (tid >> 6) + ((tid >> 4) & 3);
    const uint32_t kr_ = p0 + kp < max_ctx ? kp : 0u, vc_ = p0 + c < max_ctx ? c : 0u;
    u32x4 kw[2], vw[2];
    kw[0] = *reinterpret_cast<const u32x4 *>(kbase + kr_ * row_stride + 8 * min(kc, P - 1));
    vw[0] = *reinterpret_cast<const u32x4 *>(vbase + vc_ * row_stride + 8 * min(r, P - 1));
    kw[1] = vw[1] = u32x4{0, 0, 0, 0};
    if (P > 16) {  // rows of D > 128: a second piece (uniform)
        kw[1] = *reinterpret_cast<const u32x4 *>(kbase + kr_ * row_stride + 8 * min(kc + 16, P - 1));
        vw[1] = *reinterpret_cast<const u32x4 *>(vbase + vc_ * row_stride + 8 * min(r + 16, P - 1));
    }
    constexpr uint32_t kQPairs = GP * kGlueMaxHeadDim / 2 / 256;  // query pairs per thread: G * D/2 <= 256 max(kQPairs, 1)
    uint32_t qraw[kQPairs > 0 ? kQPairs : 1][2];
#pragma unroll
    for (uint32_t j = 0; j < (kQPairs > 0 ? kQPairs : 1); ++j) {
        const uint32_t i0 = tid + 256 * j, i = i0 < G * half ? i0 : 0u, g = i / half, d = i % half;
        const uint16_t *src = q + ((size_t)b * q_heads + kvh * G + g) * D;
        qraw[j][0] = src[d];
        qraw[j][1] = src[d + half];
    }
    uint32_t kn0, kn1, vn0, vn1;
    {
        const uint32_t tn = tid < half ? tid : 0u;
        const uint16_t *ks = k + ((size_t)b * kv_heads + kvh) * D;
        const uint16_t *vs = v + ((size_t)b * kv_heads + kvh) * D;
        kn0 = ks[tn];
        kn1 = ks[tn + half];
        vn0 = vs[tn];
        vn1 = vs[tn + half];
    }
    const bool append = pos < max_ctx;
    // the RoPE table row of the new position: requested as soon as the position is here (a
    // scalar load), not after the key and value rows issued above have arrived
    const float2 *trow = reinterpret_cast<const float2 *>(cos_sin) + (size_t)(append ? pos : 0u) * half;
    float2 tq[kQPairs > 0 ? kQPairs : 1];
#pragma unroll
    for (uint32_t j = 0; j < (kQPairs > 0 ? kQPairs : 1); ++j) {
        const uint32_t i0 = tid + 256 * j, i = i0 < G * half ? i0 : 0u;
        tq[j] = trow[i % half];
    }
    const float2 tk = trow[tid < half ? tid : 0u];
    const uint32_t n = min(pos, max_ctx - 1) + 1;
    const uint32_t p1 = min(n, p0 + kSplitLen);
    float *out = part + (((size_t)b * kv_heads + kvh) * splits + s) * (size_t)G * (D + 2);  // m[G], l[G], acc[G][D]
    if (p0 >= n) {  // nothing of this sequence in the slice
        if (tid < G) {
            out[tid] = -INFINITY;
            out[G + tid] = 0.0f;
        }
        return;
    }
    const bool has_new = append && pos >= p0 && pos < p1;
    // 1. the G query heads, rotated at the new position (the table row is the second round trip)
#pragma unroll
    for (uint32_t j = 0; j < (kQPairs > 0 ? kQPairs : 1); ++j) {
        const uint32_t i = tid + 256 * j, g = i / half, d = i % half;
        if (i < G * half) {
            float x0 = bf16_to_f32(qraw[j][0]), x1 = bf16_to_f32(qraw[j][1]);
            if (append) {
                const float2 t = tq[j];
                const float r0 = fmaf(x0, t.x, -x1 * t.y), r1 = fmaf(x0, t.y, x1 * t.x);
                x0 = bf16_round(r0);
                x1 = bf16_round(r1);
            }
            qs[g * D + d] = x0;
            qs[g * D + d + half] = x1;
        }
    }
    // rows past the sequence (loaded before its length was known) must not reach the sums
#pragma unroll
    for (uint32_t j = 0; j < 2; ++j)
        if (p0 + c >= p1) vw[j] = u32x4{0, 0, 0, 0};
    // 2. the new key (rotated) and value, into LDS for this block's own use (the cache is written at the end)
    if (has_new && tid < half) {
        const float2 t = tk;
        const float x0 = bf16_to_f32(kn0), x1 = bf16_to_f32(kn1);
        const uint32_t k0 = f32_to_bf16(fmaf(x0, t.x, -x1 * t.y)), k1 = f32_to_bf16(fmaf(x0, t.y, x1 * t.x));
        knew[tid] = bf16_to_f32(k0);
        knew[tid + half] = bf16_to_f32(k1);
        vnew[tid] = (uint16_t)vn0;
        vnew[tid + half] = (uint16_t)vn1;
        kn0 = k0;  // stored to the cache after the last barrier: a barrier waits for the
        kn1 = k1;  // block's outstanding global stores
    }
    __syncthreads();
    // 3. scores on the matrix cores: wave w multiplies the 32-dim steps w and w + 4 (D > 128) of
    //    q (16 head rows, bf16 values) with the key slice (dims x 16 positions), one
    //    v_mfma_f32_16x16x32_bf16 per step; the products are exact and sum in f32.  The four
    //    waves' partial tiles are added in wave order in step 4.
    {
        const uint32_t wv = tid >> 6, l = tid & 63, row = l & 15, kq = l >> 4;
        const bool fresh = has_new && p0 + kp == pos;
        f32x4 acc = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
        for (uint32_t j = 0; j < 2; ++j) {
            const uint32_t step = wv + 4 * j, d0 = 32 * step + 8 * kq;
            if (32 * step >= D) break;  // uniform
            uint32_t av[4] = {0, 0, 0, 0}, bv[4] = {0, 0, 0, 0};
            if (d0 < D) {
                if (row < G) {  // q values are bf16-rounded: their bf16 bits are exact
                    const f32x4 qa = *reinterpret_cast<const f32x4 *>(&qs[row * D + d0]);
                    const f32x4 qb = *reinterpret_cast<const f32x4 *>(&qs[row * D + d0 + 4]);
                    av[0] = (__float_as_uint(qa.x) >> 16) | (__float_as_uint(qa.y) & 0xFFFF0000u);
                    av[1] = (__float_as_uint(qa.z) >> 16) | (__float_as_uint(qa.w) & 0xFFFF0000u);
                    av[2] = (__float_as_uint(qb.x) >> 16) | (__float_as_uint(qb.y) & 0xFFFF0000u);
                    av[3] = (__float_as_uint(qb.z) >> 16) | (__float_as_uint(qb.w) & 0xFFFF0000u);
                }
                if (fresh) {  // the new (rotated) key, bf16-rounded in knew
                    const f32x4 ka = *reinterpret_cast<const f32x4 *>(&knew[d0]);
                    const f32x4 kb = *reinterpret_cast<const f32x4 *>(&knew[d0 + 4]);
                    bv[0] = (__float_as_uint(ka.x) >> 16) | (__float_as_uint(ka.y) & 0xFFFF0000u);
                    bv[1] = (__float_as_uint(ka.z) >> 16) | (__float_as_uint(ka.w) & 0xFFFF0000u);
                    bv[2] = (__float_as_uint(kb.x) >> 16) | (__float_as_uint(kb.y) & 0xFFFF0000u);
                    bv[3] = (__float_as_uint(kb.z) >> 16) | (__float_as_uint(kb.w) & 0xFFFF0000u);
                } else {
                    bv[0] = kw[j].x;
                    bv[1] = kw[j].y;
                    bv[2] = kw[j].z;
                    bv[3] = kw[j].w;
                }
            }
            const u32x4 a4 = {av[0], av[1], av[2], av[3]}, b4 = {bv[0], bv[1], bv[2], bv[3]};
            acc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8_t, a4),
                                                          __builtin_bit_cast(bf16x8_t, b4), acc, 0, 0, 0);
        }
        // lane l holds rows (heads) 4 (l >> 4) + e of column (position) l & 15
#pragma unroll
        for (uint32_t e = 0; e < 4; ++e) sp[wv][4 * kq + e][row] = acc[e];
    }
    __syncthreads();
    // 4a. the value tile into LDS, over q's rows (read only by the scores, done): row c =
    //     position p0 + c, the 8 dims of piece r [+16]; zero past the sequence (vw), the new
    //     value at the new position
    uint16_t *vt = reinterpret_cast<uint16_t *>(qs);
    {
        const bool vfresh = has_new && p0 + c == pos;
#pragma unroll
        for (uint32_t j = 0; j < 2; ++j) {
            const uint32_t pc = r + 16 * j;
            if (16 * j >= P) break;  // uniform: rows of D <= 128 need one round
            if (pc < P) {
                u32x4 w = vw[j];
                if (vfresh) w = *reinterpret_cast<const u32x4 *>(&vnew[8 * pc]);
                *reinterpret_cast<u32x4 *>(&vt[c * D + 8 * pc]) = w;
            }
        }
    }
    // 4b. per head: row r takes head r, lane c position p0 + c
    float m_keep = 0.0f, l_keep = 0.0f;
    if (r < G) {
        const float dot = ((sp[0][r][c] + sp[1][r][c]) + sp[2][r][c]) + sp[3][r][c];
        const float x = p0 + c < p1 ? dot * (1.0f / sqrtf((float)D)) : -INFINITY;
        float m = x;
        m = tree_max_from<2>(m, (int)__lane_id());  // over the row's 16 lanes
        const float e = x == -INFINITY ? 0.0f : expf(x - m);
        float l = e;
        l = tree_sum_from<2>(l, (int)__lane_id());
        sc[r][c] = e;
        m_keep = m;
        l_keep = l;
    }
    __syncthreads();
    // 5. values on the matrix cores, per 16-dim tile (wave w takes tiles w, w + 4, ...):
    //    out[head][dim] = sum_p P[head][p] V[p][dim] with v_mfma_f32_16x16x16_bf16.  V is bf16 in
    //    the LDS tile; P (f32) is split into bf16 hi + lo (P = hi + lo to 2^-17), two products that
    //    are exact and sum in f32.  Positions past the sequence have P = 0 and zero values.
    {
        typedef short s16x4 __attribute__((ext_vector_type(4)));
        const uint32_t wv = tid >> 6, l = tid & 63, row = l & 15, kq = l >> 4;
        s16x4 ahi, alo;  // A: P[head row][positions 4 kq .. + 3]
#pragma unroll
        for (uint32_t i = 0; i < 4; ++i) {
            const float pv = row < G ? sc[row][4 * kq + i] : 0.0f;
            const uint32_t hi = f32_to_bf16(pv);
            ahi[i] = (short)hi;
            alo[i] = (short)f32_to_bf16(pv - bf16_to_f32(hi));
        }
        const uint32_t ntile = (D + 15) / 16;
        for (uint32_t t = wv; t < ntile; t += 4) {
            const uint32_t d = 16 * t + row;  // B: V[positions 4 kq .. + 3][dim d]
            s16x4 bv;
#pragma unroll
            for (uint32_t i = 0; i < 4; ++i) bv[i] = d < D ? (short)vt[(4 * kq + i) * D + d] : (short)0;
            f32x4 acc = {0.0f, 0.0f, 0.0f, 0.0f};
            acc = __builtin_amdgcn_mfma_f32_16x16x16bf16_1k(ahi, bv, acc, 0, 0, 0);
            acc = __builtin_amdgcn_mfma_f32_16x16x16bf16_1k(alo, bv, acc, 0, 0, 0);
            // lane l holds heads 4 kq + e of dim d
#pragma unroll
            for (uint32_t e = 0; e < 4; ++e) {
                const uint32_t h = 4 * kq + e;
                if (h < G && d < D) out[2 * G + h * D + d] = acc[e];
            }
        }
    }
    // deferred global stores
    if (r < G && c == 0) {
        out[r] = m_keep;
        out[G + r] = l_keep;
    }
    if (has_new && tid < half) {
        const size_t cbase = (((size_t)b * max_ctx + pos) * kv_heads + kvh) * D;
        k_cache[cbase + tid] = (uint16_t)kn0;
        k_cache[cbase + tid + half] = (uint16_t)kn1;
        v_cache[cbase + tid] = (uint16_t)vn0;
        v_cache[cbase + tid + half] = (uint16_t)vn1;
    }
}

// attention_split64_kernel: the split kernel's job for head_dim 128 on slices of 64 positions.
// Grid (ceil(max_ctx / 64), kv_heads, batch), 256 threads: wave w takes positions p0 + 16 w ..
// p0 + 16 w + 15 of the block's slice for all G <= 16 query heads of the kv head, with every
// dimension (no partial tiles to add across waves):
//   0. loads first: its key pieces in the matrix-core layout (position p0 + 16 w + l % 16, dims
//      32 s + 8 (l / 16), s < 4) and value pieces (position p0 + 16 w + l / 16 + 4 m, dims
//      8 (l % 16)), the query pairs, the RoPE row of the new position, the new k and v;
//   1. the G query heads rotated (bf16-rounded, as kr_rope_kv_append stores them) into LDS, and
//      the new key if the slice holds the new position (its own scores take it from LDS);
//   2. scores: four v_mfma_f32_16x16x32_bf16 (query rows x key columns; bf16 products are exact,
//      sums f32), scaled by 1/sqrt(128), -inf past the sequence;
//   3. per head the wave's max m over its 16 positions, p = e^(s - m), the sum l;
//   4. values: the probabilities (bf16 hi + lo, P = hi + lo to 2^-17; transposed through the
//      wave's LDS tile) times the value tile on v_mfma_f32_16x16x16_bf16, both products exact;
//   5. the 4 waves' (m, l, acc) merged in wave order into the slice's partial
//        m = max_w m_w,  l = sum_w e^(m_w - m) l_w,  acc = sum_w e^(m_w - m) acc_w,
//      the layout the merge kernels read (a slice past the sequence publishes (-inf, 0) only).
// Against 16-position slices: a quarter of the blocks, of the query rotations and of the
// partials the merge reads.
constexpr uint32_t kSplit64 = 64;

template <uint32_t NW>  // waves per block: slices of 16 NW positions (4: the 64 of the name)
__global__ __launch_bounds__(64 * NW) void attention_split64_kernel(const uint16_t *q, const uint16_t *k, const uint16_t *v,
                                                                const float *cos_sin, const uint32_t *positions,
                                                                uint32_t q_heads, uint32_t kv_heads, uint16_t *k_cache,
                                                                uint16_t *v_cache, uint32_t max_ctx, float *part) {
    constexpr uint32_t D = 128, half = 64;
    constexpr uint32_t QS = D + 8;  // query / value tile row stride: the rows one 16-byte (or B-fragment)
    constexpr uint32_t VS = D + 8;  // read takes sit 4 (16) banks apart
    constexpr uint32_t AS = D + 4;  // merge rows: the 4 head groups of a write 16 banks apart
    typedef short s16x4 __attribute__((ext_vector_type(4)));
    __shared__ __align__(16) uint16_t qs[16 * QS];           // rotated queries, bf16 [head][dim]
    __shared__ __align__(16) uint16_t knew[D], vnew[D];      // the new key (rotated) and value
    constexpr uint32_t kLen = 16 * NW, kThreads = 64 * NW;
    __shared__ __align__(16) uint16_t vt[NW][16 * VS];       // per-wave value tile [position][dim]
    __shared__ __align__(16) float pt[NW][16 * 16];          // per-wave probability tile [head][position]
    __shared__ float mrow[NW][16], lrow[NW][16];
    __shared__ __align__(16) float accm[NW][16 * AS];        // per-wave unnormalised outputs [head][dim]
    const uint32_t tid = threadIdx.x, l = tid & 63, row = l & 15, kq = l >> 4;
    const uint32_t w = __builtin_amdgcn_readfirstlane(tid >> 6);
    const uint32_t s = blockIdx.x, kvh = blockIdx.y, b = blockIdx.z, splits = gridDim.x;
    const uint32_t G = q_heads / kv_heads;
    const uint32_t pos = __builtin_amdgcn_readfirstlane(positions[b]);
    const bool append = pos < max_ctx;
    const uint32_t n = min(pos, max_ctx - 1) + 1;  // positions attended
    const uint32_t s0 = s * kLen, p0 = s0 + 16 * w;
    float *out = part + (((size_t)b * kv_heads + kvh) * splits + s) * (size_t)G * (D + 2);  // m[G], l[G], acc[G][D]
    if (s0 >= n) {  // nothing of this sequence in the slice
        if (tid < G) {
            out[tid] = -INFINITY;
            out[G + tid] = 0.0f;
        }
        return;
    }
    const bool has_new = append && pos >= s0 && pos < s0 + kLen;
    const size_t rs = (size_t)kv_heads * D;
    const uint16_t *kb = k_cache + ((size_t)b * max_ctx * kv_heads + kvh) * D;
    const uint16_t *vb = v_cache + ((size_t)b * max_ctx * kv_heads + kvh) * D;
    // 0. loads (clamped rows; what must not contribute is masked or zeroed at use)
    u32x4 kw[4], vw[4];
    {
        const uint32_t kp = min(p0 + row, max_ctx - 1);
#pragma unroll
        for (uint32_t s2 = 0; s2 < 4; ++s2) kw[s2] = *reinterpret_cast<const u32x4 *>(kb + kp * rs + 32 * s2 + 8 * kq);
#pragma unroll
        for (uint32_t m = 0; m < 4; ++m) {
            const uint32_t vp = min(p0 + kq + 4 * m, max_ctx - 1);
            vw[m] = *reinterpret_cast<const u32x4 *>(vb + vp * rs + 8 * row);
        }
    }
    const float2 *trow = reinterpret_cast<const float2 *>(cos_sin) + (size_t)(append ? pos : 0u) * half;
    constexpr uint32_t kQP = 1024 / kThreads;  // query pairs per thread (G * 64 <= 1024)
    uint32_t qr[kQP][2];
    float2 tq[kQP];
#pragma unroll
    for (uint32_t jj = 0; jj < kQP; ++jj) {  // query pairs t, t + kThreads, ... of the G * 64
        const uint32_t i0 = tid + kThreads * jj, i = i0 < G * half ? i0 : 0u, g = i / half, d = i % half;
        const uint16_t *src = q + ((size_t)b * q_heads + kvh * G + g) * D;
        qr[jj][0] = src[d];
        qr[jj][1] = src[d + half];
        tq[jj] = trow[d];
    }
    uint32_t kn0, kn1, vn0, vn1;
    {
        const uint32_t tn = tid < half ? tid : 0u;
        const uint16_t *ks = k + ((size_t)b * kv_heads + kvh) * D;
        const uint16_t *vs = v + ((size_t)b * kv_heads + kvh) * D;
        kn0 = ks[tn];
        kn1 = ks[tn + half];
        vn0 = vs[tn];
        vn1 = vs[tn + half];
    }
    // 1. rotations into LDS
#pragma unroll
    for (uint32_t jj = 0; jj < kQP; ++jj) {
        const uint32_t i = tid + kThreads * jj, g = i / half, d = i % half;
        if (i < G * half) {
            uint32_t b0 = qr[jj][0], b1 = qr[jj][1];
            if (append) {
                const float x0 = bf16_to_f32(b0), x1 = bf16_to_f32(b1);
                const float2 t = tq[jj];
                b0 = f32_to_bf16(fmaf(x0, t.x, -x1 * t.y));
                b1 = f32_to_bf16(fmaf(x0, t.y, x1 * t.x));
            }
            qs[g * QS + d] = (uint16_t)b0;
            qs[g * QS + d + half] = (uint16_t)b1;
        }
    }
    if (has_new && tid < half) {  // tq[0] is the table row of d = tid
        const float x0 = bf16_to_f32(kn0), x1 = bf16_to_f32(kn1);
        kn0 = f32_to_bf16(fmaf(x0, tq[0].x, -x1 * tq[0].y));  // stored to the cache after the last
        kn1 = f32_to_bf16(fmaf(x0, tq[0].y, x1 * tq[0].x));   // barrier (a barrier waits for stores)
        knew[tid] = (uint16_t)kn0;
        knew[tid + half] = (uint16_t)kn1;
        vnew[tid] = (uint16_t)vn0;
        vnew[tid + half] = (uint16_t)vn1;
    }
    __syncthreads();
    // 2. scores of this wave's 16 positions
    float sc[4];
    {
        const bool fresh = has_new && p0 + row == pos;  // column `row` is the new position
        f32x4 acc = {0.0f, 0.0f, 0.0f, 0.0f};
        if (p0 < n) {  // uniform
#pragma unroll
            for (uint32_t s2 = 0; s2 < 4; ++s2) {
                const u32x4 qa = row < G ? *reinterpret_cast<const u32x4 *>(&qs[row * QS + 32 * s2 + 8 * kq])
                                         : u32x4{0, 0, 0, 0};
                const u32x4 kb4 = fresh ? *reinterpret_cast<const u32x4 *>(&knew[32 * s2 + 8 * kq]) : kw[s2];
                acc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8_t, qa),
                                                              __builtin_bit_cast(bf16x8_t, kb4), acc, 0, 0, 0);
            }
        }
        const bool valid = p0 + row < n;
        const float scale = 1.0f / sqrtf((float)D);
#pragma unroll
        for (int e = 0; e < 4; ++e) sc[e] = valid ? acc[e] * scale : -INFINITY;
    }
    // 3. the wave's softmax statistics per head (lanes 16 kq .. hold heads 4 kq + e)
    float mw[4], lw[4];
#pragma unroll
    for (int e = 0; e < 4; ++e) {
        mw[e] = tree_max_from<2>(sc[e], (int)l);
        sc[e] = sc[e] == -INFINITY ? 0.0f : expf(sc[e] - mw[e]);
        lw[e] = tree_sum_from<2>(sc[e], (int)l);
    }
    // 4. values
    f32x4 acc_o[8];
#pragma unroll
    for (int t = 0; t < 8; ++t) acc_o[t] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
    if (p0 < n) {  // uniform
#pragma unroll
        for (int e = 0; e < 4; ++e) pt[w][(4 * kq + e) * 16 + row] = sc[e];
#pragma unroll
        for (uint32_t m = 0; m < 4; ++m) {
            const uint32_t pr = kq + 4 * m;  // tile row: position p0 + pr
            u32x4 val = p0 + pr < n ? vw[m] : u32x4{0, 0, 0, 0};
            if (has_new && p0 + pr == pos) val = *reinterpret_cast<const u32x4 *>(&vnew[8 * row]);
            *reinterpret_cast<u32x4 *>(&vt[w][pr * VS + 8 * row]) = val;
        }
        __builtin_amdgcn_wave_barrier();
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
        s16x4 ahi, alo;  // P[head row][positions 4 kq .. + 3]
#pragma unroll
        for (uint32_t i = 0; i < 4; ++i) {
            const float pv = pt[w][row * 16 + 4 * kq + i];
            const uint32_t hi = f32_to_bf16(pv);
            ahi[i] = (short)hi;
            alo[i] = (short)f32_to_bf16(pv - bf16_to_f32(hi));
        }
#pragma unroll
        for (uint32_t t = 0; t < 8; ++t) {
            s16x4 bv;  // V[positions 4 kq .. + 3][dim 16 t + row]
#pragma unroll
            for (uint32_t i = 0; i < 4; ++i) bv[i] = (short)vt[w][(4 * kq + i) * VS + 16 * t + row];
            acc_o[t] = __builtin_amdgcn_mfma_f32_16x16x16bf16_1k(ahi, bv, acc_o[t], 0, 0, 0);
            acc_o[t] = __builtin_amdgcn_mfma_f32_16x16x16bf16_1k(alo, bv, acc_o[t], 0, 0, 0);
        }
    }
    // 5. the slice's partial: the waves merged in wave order
    if (row == 0) {
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            mrow[w][4 * kq + e] = mw[e];
            lrow[w][4 * kq + e] = lw[e];
        }
    }
#pragma unroll
    for (uint32_t t = 0; t < 8; ++t)
#pragma unroll
        for (int e = 0; e < 4; ++e) accm[w][(4 * kq + e) * AS + 16 * t + row] = acc_o[t][e];
    __syncthreads();
    for (uint32_t o = tid; o < G * D; o += kThreads) {
        const uint32_t h = o / D, d = o % D;
        float mv[NW], lv[NW], av[NW];
#pragma unroll
        for (uint32_t ww = 0; ww < NW; ++ww) {
            mv[ww] = mrow[ww][h];
            lv[ww] = lrow[ww][h];
            av[ww] = accm[ww][h * AS + d];
        }
        float M = mv[0];
#pragma unroll
        for (uint32_t ww = 1; ww < NW; ++ww) M = fmaxf(M, mv[ww]);
        float L = 0.0f, A = 0.0f;
#pragma unroll
        for (uint32_t ww = 0; ww < NW; ++ww) {  // a wave without positions (m = -inf) adds nothing
            const bool live = mv[ww] != -INFINITY;
            const float wt = live ? expf(mv[ww] - M) : 0.0f;
            L = live ? fmaf(wt, lv[ww], L) : L;
            A = live ? fmaf(wt, av[ww], A) : A;
        }
        out[2 * G + h * D + d] = A;
        if (d == 0) {
            out[h] = M;
            out[G + h] = L;
        }
    }
    if (has_new && tid < half) {
        const size_t cbase = (((size_t)b * max_ctx + pos) * kv_heads + kvh) * D;
        k_cache[cbase + tid] = (uint16_t)kn0;
        k_cache[cbase + tid + half] = (uint16_t)kn1;
        v_cache[cbase + tid] = (uint16_t)vn0;
        v_cache[cbase + tid + half] = (uint16_t)vn1;
    }
}

// attention_merge_oproj_kernel: one sequence's attention slices merged and multiplied by the output
// projection in one launch: h[row] (+)= x . W[row] with
//   x[head, d] = bf16(sum_s w_hs acc_s[head, d] / L_h),  w_hs = e^(m_s - M_h),  M_h = max_s m_s,
//   L_h = sum_s w_hs l_s   (slices in order; a slice of weight 0 is skipped, not multiplied),
// over the partials (m, l, acc) the split kernels write.  Grid ceil(n / 8), 256 threads: every block
// merges all of x into LDS (each output row needs all of it), then wave w computes rows 8 b + 2 w and
// 8 b + 2 w + 1 with the m == 1 GEMV's arithmetic (one 16-byte chunk per lane, chunk_dot, the fixed
// reduction tree).  The weights, the partials and the old outputs are all requested first.  head_dim
// 128; n = rows of W, k = q_heads * 128 <= 2048; splits <= kMergeMaxSlices.
constexpr uint32_t kMergeMaxSlices = kMergeOprojMaxSlices;

template <uint32_t NS>  // slices held in registers (>= splits)
__global__ __launch_bounds__(256) void attention_merge_oproj_kernel(const float *part, uint32_t q_heads,
                                                                    uint32_t kv_heads, uint32_t splits, Q4Mat W,
                                                                    void *h, int h_f32) {
    constexpr uint32_t D = 128;
    __shared__ float s_m[16][kMergeMaxSlices], s_l[16][kMergeMaxSlices];
    __shared__ float s_w[16][kMergeMaxSlices], s_L[16];
    __shared__ u32x4 s_x[256];  // x, bf16, 8 values per unit
    const uint32_t tid = threadIdx.x, lane = tid & 63;
    const uint32_t wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const uint32_t G = q_heads / kv_heads, K = W.k, nchunks = K >> 5, wpr = K >> 3, groups = K >> 6;
    const size_t slice = (size_t)G * (D + 2);  // floats of one (kv head, slice) partial
    // 1. requests: the wave's two weight rows (chunk `lane`), the old outputs, the partials
    const bool live = lane < nchunks;
    const uint32_t c = live ? lane : 0u;
    const uint32_t r0 = blockIdx.x * 8 + 2 * wave;
    u32x4 wv[2];
    uint32_t sv[2], bv[2];
#pragma unroll
    for (uint32_t r = 0; r < 2; ++r) {
        const size_t row = min(r0 + r, W.n - 1);  // a tail row is never stored
        wv[r] = ld_stream(reinterpret_cast<const u32x4 *>(W.qw + row * wpr) + c);
        sv[r] = ld_stream(W.sc + row * groups + (c >> 1));
        bv[r] = ld_stream(W.bi + row * groups + (c >> 1));
    }
    float pre = 0.0f;  // lanes 0 and 32 store rows r0, r0 + 1
    if ((lane & 31) == 0 && r0 + (lane >> 5) < W.n) {
        const uint32_t row = r0 + (lane >> 5);
        pre = h_f32 ? reinterpret_cast<const float *>(h)[row] : bf16_to_f32(reinterpret_cast<const uint16_t *>(h)[row]);
    }
    // (m, l) of (head, slice) for thread t < q_heads * splits
    float mt = -INFINITY, lt = 0.0f;
    {
        const uint32_t t = tid < q_heads * splits ? tid : 0u, hh = t / splits, sl = t % splits;
        const float *pb = part + ((size_t)(hh / G) * splits + sl) * slice;
        mt = pb[hh % G];
        lt = pb[G + hh % G];
    }
    // the acc units of thread t < K / 8: head t / 16, dims 8 (t % 16) .. + 7, every slice
    const uint32_t units = K >> 3;
    const uint32_t ut = tid < units ? tid : 0u, uh = ut >> 4, ud = 8 * (ut & 15);
    f32x4 av[NS][2];
    {
        const float *pb = part + (size_t)(uh / G) * splits * slice + 2 * G + (uh % G) * D + ud;
#pragma unroll
        for (uint32_t sl = 0; sl < NS; ++sl) {
            const float *ps = pb + (size_t)min(sl, splits - 1) * slice;
            av[sl][0] = *reinterpret_cast<const f32x4 *>(ps);
            av[sl][1] = *reinterpret_cast<const f32x4 *>(ps + 4);
        }
    }
    // 2. per head: M, the slice weights and L (one thread per head, slices in order)
    if (tid < q_heads * splits) {
        s_m[tid / splits][tid % splits] = mt;
        s_l[tid / splits][tid % splits] = lt;
    }
    __syncthreads();
    if (tid < q_heads) {
        float M = -INFINITY;
        for (uint32_t sl = 0; sl < splits; ++sl) M = fmaxf(M, s_m[tid][sl]);
        float L = 0.0f;
        for (uint32_t sl = 0; sl < splits; ++sl) {
            const float m = s_m[tid][sl];
            const float w = m == -INFINITY ? 0.0f : expf(m - M);
            s_w[tid][sl] = w;
            L = fmaf(w, s_l[tid][sl], L);
        }
        s_L[tid] = L;
    }
    __syncthreads();
    // 3. x units into LDS
    if (tid < units) {
        f32x4 a0 = {0.0f, 0.0f, 0.0f, 0.0f}, a1 = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
        for (uint32_t sl = 0; sl < NS; ++sl) {
            const float w = sl < splits ? s_w[uh][sl] : 0.0f;
            if (w != 0.0f) {  // an empty slice's acc is never read
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    a0[e] = fmaf(w, av[sl][0][e], a0[e]);
                    a1[e] = fmaf(w, av[sl][1][e], a1[e]);
                }
            }
        }
        const float L = s_L[uh];
        s_x[tid] = u32x4{pack_bf16_rne(a0[0] / L, a0[1] / L), pack_bf16_rne(a0[2] / L, a0[3] / L),
                         pack_bf16_rne(a1[0] / L, a1[1] / L), pack_bf16_rne(a1[2] / L, a1[3] / L)};
    }
    __syncthreads();
    // 4. the wave's two rows
    uint32_t X[16];
#pragma unroll
    for (int qd = 0; qd < 4; ++qd) {
        const u32x4 u = s_x[4 * c + qd];
        X[4 * qd] = u.x;
        X[4 * qd + 1] = u.y;
        X[4 * qd + 2] = u.z;
        X[4 * qd + 3] = u.w;
    }
    XChunk xc;
    build_xchunk(xc, X, sgpr_const(0x05040100u), sgpr_const(0x07060302u));
    const uint32_t kMask = sgpr_const(0x000F000Fu);
    const uint32_t kMagic = vgpr_const(0x43004300u);
    float acc[2];
#pragma unroll
    for (uint32_t r = 0; r < 2; ++r) {
        const float d = chunk_dot(wv[r], sv[r], bv[r], xc, 0.0f, kMask, kMagic);
        acc[r] = live ? d : 0.0f;
    }
    const float tot = wave_reduce_rows<2>(acc, (int)lane);  // lanes 0..31 row r0, 32..63 row r0 + 1
    if ((lane & 31) == 0 && r0 + (lane >> 5) < W.n) {
        const uint32_t row = r0 + (lane >> 5);
        if (h_f32) reinterpret_cast<float *>(h)[row] = pre + tot;
        else reinterpret_cast<uint16_t *>(h)[row] = (uint16_t)f32_to_bf16(tot + pre);
    }
}

hipError_t launch_attention_merge_oproj(const float *part, uint32_t q_heads, uint32_t kv_heads, uint32_t splits,
                                        const Q4Mat &w, void *h, int h_f32, hipStream_t s) {
    if (splits == 0 || splits > kMergeMaxSlices || w.k != q_heads * 128 || w.k > 2048 || q_heads > 16)
        return hipErrorInvalidValue;
    const dim3 grid((w.n + 7) / 8);
    if (splits <= 4) hipLaunchKernelGGL(attention_merge_oproj_kernel<4>, grid, dim3(256), 0, s, part, q_heads, kv_heads, splits, w, h, h_f32);
    else if (splits <= 8) hipLaunchKernelGGL(attention_merge_oproj_kernel<8>, grid, dim3(256), 0, s, part, q_heads, kv_heads, splits, w, h, h_f32);
    else if (splits <= 12) hipLaunchKernelGGL(attention_merge_oproj_kernel<12>, grid, dim3(256), 0, s, part, q_heads, kv_heads, splits, w, h, h_f32);
    else hipLaunchKernelGGL(attention_merge_oproj_kernel<16>, grid, dim3(256), 0, s, part, q_heads, kv_heads, splits, w, h, h_f32);
    return hipGetLastError();
}

uint32_t attention_slices64(uint32_t max_ctx) { return (max_ctx + kSplit64 - 1) / kSplit64; }

hipError_t launch_rope_attention_partials64(const uint16_t *q, const uint16_t *k, const uint16_t *v,
                                            const float *cos_sin, const uint32_t *positions, uint32_t batch,
                                            uint32_t q_heads, uint32_t kv_heads, uint16_t *k_cache,
                                            uint16_t *v_cache, uint32_t max_ctx, float *part, hipStream_t s) {
    hipLaunchKernelGGL(attention_split64_kernel<4>, dim3(attention_slices64(max_ctx), kv_heads, batch), dim3(256), 0, s,
                       q, k, v, cos_sin, positions, q_heads, kv_heads, k_cache, v_cache, max_ctx, part);
    return hipGetLastError();
}

// grid (q_heads, batch), 256 threads: merge the slices of one head in slice order.  Every slice
// publishes (m, l) -- empty slices (-inf, 0) -- so the merge needs no slice count.  Slices are
// taken in rounds of NI * 32 (NI = 256 / D interleaves): thread t reads (m, l) of slice t of the
// round and thread (d = t % D, i = t / D) the values of dim d of slices i, i + NI, ... -- all of a
// round's loads at once.  The round's max, the weights e^(m_s - M) (one slice per thread) and
// sum_s w_s l_s are block reductions in a fixed order; the value sums run in slice order per
// interleave, interleaves added in order; earlier rounds are rescaled to the new max.
__device__ __forceinline__ float block_max256(float v, float *red) {
    v = wave_max(v);
    if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = v;
    __syncthreads();
    v = fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3]));
    __syncthreads();
    return v;
}
__device__ __forceinline__ float block_sum256(float v, float *red) {
    v = wave_sum(v);
    if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = v;
    __syncthreads();
    v = ((red[0] + red[1]) + red[2]) + red[3];
    __syncthreads();
    return v;
}

__global__ __launch_bounds__(256) void attention_combine_kernel(const float *part, uint32_t q_heads,
                                                                uint32_t kv_heads, uint32_t D, uint32_t splits,
                                                                uint16_t *out) {
    constexpr uint32_t kPer = 32;
    __shared__ float sw[256];
    __shared__ float red[256];
    __shared__ float r4[4];
    const uint32_t h = blockIdx.x, b = blockIdx.y, tid = threadIdx.x;
    const uint32_t G = q_heads / kv_heads, kvh = h / G, g = h % G;
    const float *base = part + ((size_t)b * kv_heads + kvh) * splits * (size_t)G * (D + 2);
    const size_t stride = (size_t)G * (D + 2);
    const uint32_t NI = 256 / D, d = tid % D, il = tid / D;
    const uint32_t round = min(256u, NI * kPer);
    float M = -INFINITY, L = 0.0f, acc = 0.0f;
    for (uint32_t s0 = 0; s0 < splits; s0 += round) {
        const uint32_t cnt = min(round, splits - s0);
        const float *rb = base + (size_t)s0 * stride;
        // (m, l) first and unconditional (clamped row; what it should not contribute is dropped
        // below): a conditional load merged with a default value after the value loads would make
        // the compiler wait for all of them before issuing it -- a second round trip.
        const float mraw = rb[min(tid, cnt - 1) * stride + g];
        const float lraw = rb[min(tid, cnt - 1) * stride + G + g];
        float a[kPer];
#pragma unroll
        for (uint32_t j = 0; j < kPer; ++j) {
            const uint32_t sj = il + j * NI;
            a[j] = (il < NI && sj < cnt) ? rb[sj * stride + 2 * G + g * D + d] : 0.0f;
        }
        const float mt = tid < cnt ? mraw : -INFINITY;
        const float lt = tid < cnt ? lraw : 0.0f;
        const float Mc = fmaxf(M, block_max256(mt, r4));
        const float wt = mt == -INFINITY ? 0.0f : expf(mt - Mc);
        sw[tid] = wt;
        const float Lr = block_sum256(wt * lt, r4);  // also publishes sw
        // A slice with weight 0 is skipped, not multiplied: an empty slice (past the sequence) writes
        // only its (m, l), so its acc holds whatever the workspace held (possibly NaN or inf).
        // Skipping leaves finite sums bit-identical (fmaf(0, a, acc) == acc).
        float part_acc = 0.0f;
#pragma unroll
        for (uint32_t j = 0; j < kPer; ++j) {
            const uint32_t sj = il + j * NI;
            if (il < NI && sj < cnt && sw[sj] != 0.0f) part_acc = fmaf(sw[sj], a[j], part_acc);
        }
        if (il < NI) red[tid] = part_acc;
        __syncthreads();
        float racc = 0.0f;
        for (uint32_t i = 0; i < NI; ++i) racc += red[i * D + d];  // interleaves in order
        const float scale = M == -INFINITY ? 0.0f : expf(M - Mc);
        acc = fmaf(acc, scale, racc);
        L = fmaf(L, scale, Lr);
        M = Mc;
        __syncthreads();  // sw, red are rewritten by the next round
    }
    if (tid < D) out[((size_t)b * q_heads + h) * D + tid] = (uint16_t)f32_to_bf16(acc / L);
}

// grid (q_heads, batch), 256 threads: the merge of at most 64 slices for D = 4 DW with DW | 64.
// Wave w takes dims [w DW, (w + 1) DW) of head h; lane (d = l % DW, i = l / DW) the values of
// slices i, i + NI, ... (NI = 64 / DW interleaves).  Each wave forms every slice's weight itself
// (lane s holds slice s: max, e^(m_s - M) and sum_s w_s l_s are wave reductions), so there is no
// block barrier; the weights reach the value lanes through the wave's own LDS row.  The sums run
// in the order of attention_combine_kernel (one round): the same bits.
template <uint32_t DW>
__global__ __launch_bounds__(256) void attention_combine_wave_kernel(const float *part, uint32_t q_heads,
                                                                     uint32_t kv_heads, uint32_t D, uint32_t splits,
                                                                     uint16_t *out) {
    constexpr uint32_t NI = kWave / DW;
    constexpr uint32_t J = kWave / NI;  // slices per lane at most
    __shared__ float sw[4][kWave];
    const uint32_t h = blockIdx.x, b = blockIdx.y, lane = threadIdx.x & (kWave - 1);
    const uint32_t w = __builtin_amdgcn_readfirstlane(threadIdx.x / kWave);
    const uint32_t G = q_heads / kv_heads, kvh = h / G, g = h % G;
    const size_t stride = (size_t)G * (D + 2);
    const float *base = part + ((size_t)b * kv_heads + kvh) * splits * stride;
    const uint32_t d = w * DW + lane % DW, il = lane / DW;
    // all loads unconditional, from clamped slices (what they should not contribute is dropped below)
    const uint32_t sl = min(lane, splits - 1);
    const float mraw = base[sl * stride + g];
    const float lraw = base[sl * stride + G + g];
    float a[J];
#pragma unroll
    for (uint32_t j = 0; j < J; ++j) a[j] = base[min(il + NI * j, splits - 1) * stride + 2 * G + g * D + d];
    const float mt = lane < splits ? mraw : -INFINITY;
    float M = mt;
    M = wave_max(M);
    const float wt = mt == -INFINITY ? 0.0f : expf(mt - M);
    const float L = wave_sum(wt * (lane < splits ? lraw : 0.0f));
    sw[w][lane] = wt;
    __builtin_amdgcn_wave_barrier();
    float acc = 0.0f;
#pragma unroll
    for (uint32_t j = 0; j < J; ++j) {  // weight-0 slices skipped, as in attention_combine_kernel
        const uint32_t sj = il + NI * j;
        if (sj < splits && sw[w][sj] != 0.0f) acc = fmaf(sw[w][sj], a[j], acc);
    }
    float tot = 0.0f;
#pragma unroll
    for (uint32_t i = 0; i < NI; ++i) tot += __shfl(acc, (int)(lane % DW + i * DW));  // interleaves in order
    if (il == 0) out[((size_t)b * q_heads + h) * D + d] = (uint16_t)f32_to_bf16(tot / L);
}

// One block (1024 threads) per row: index of the largest logit, ties to the
// lowest index (NaN never wins).  Rows of n % 4 == 0 are read as float4,
// eight loads in flight per thread.
__global__ __launch_bounds__(1024) void argmax_kernel(const float *logits, uint32_t n, uint32_t *out) {
    __shared__ float bv[16];
    __shared__ uint32_t bi[16];
    const float *row = logits + (size_t)blockIdx.x * n;
    const uint32_t tid = threadIdx.x;
    float v = -INFINITY;
    uint32_t idx = 0xFFFFFFFFu;
    auto take = [&](float x, uint32_t i) {  // i increases along a thread's scan
        if (x > v || (idx == 0xFFFFFFFFu && x == x)) {
            v = x;
            idx = i;
        }
    };
    if (n % 4 == 0) {
        // Per float4 a cheap max first (fmaxf drops NaN); only a quad that can win is searched
        // for its first lane holding that max -- the order of `take` within the quad.
        // Eight quads are requested before any is scanned (clamped, unconditional loads): with a
        // load per scan step the branch keeps the compiler from hoisting the next loads, and each
        // quad costs a round trip.
        const f32x4 *r4 = reinterpret_cast<const f32x4 *>(row);
        const uint32_t n4 = n / 4;
        constexpr uint32_t kBatch = 8;
        for (uint32_t i0 = tid; i0 < n4; i0 += 1024 * kBatch) {
            f32x4 xq[kBatch];
#pragma unroll
            for (uint32_t j = 0; j < kBatch; ++j) xq[j] = r4[min(i0 + 1024 * j, n4 - 1)];
#pragma unroll
            for (uint32_t j = 0; j < kBatch; ++j) {
                const uint32_t i = i0 + 1024 * j;
                const f32x4 x = xq[j];
                const float m = fmaxf(fmaxf(x[0], x[1]), fmaxf(x[2], x[3]));
                if (i < n4 && (m > v || (idx == 0xFFFFFFFFu && m == m))) {
                    const uint32_t c = x[0] == m ? 0u : x[1] == m ? 1u : x[2] == m ? 2u : 3u;
                    v = m;
                    idx = 4 * i + c;
                }
            }
        }
    } else {
        for (uint32_t i = tid; i < n; i += 1024) take(row[i], i);
    }
#pragma unroll
    for (int m = 32; m >= 1; m >>= 1) {
        const float ov = __shfl_xor(v, m);
        const uint32_t oi = __shfl_xor(idx, m);
        if (ov > v || (ov == v && oi < idx) || (idx == 0xFFFFFFFFu && oi != 0xFFFFFFFFu)) {
            v = ov;
            idx = oi;
        }
    }
    if ((tid & 63) == 0) {
        bv[tid >> 6] = v;
        bi[tid >> 6] = idx;
    }
    __syncthreads();
    if (tid == 0) {
        v = bv[0];
        idx = bi[0];
        for (int w = 1; w < 16; ++w)
            if (bv[w] > v || (bv[w] == v && bi[w] < idx) || (idx == 0xFFFFFFFFu && bi[w] != 0xFFFFFFFFu)) {
                v = bv[w];
                idx = bi[w];
            }
        out[blockIdx.x] = idx == 0xFFFFFFFFu ? 0u : idx;
    }
}

// Greedy argmax over a row spread across several blocks (rows with many logits: one block reads
// a row at about 54 GB/s whatever its depth).  Block (j, r) takes logits [j per, (j + 1) per) of row
// r and publishes (largest value, its first index) -- index kNoArg when it saw only NaN -- to
// part[r][j]; argmax_merge_kernel then picks, per row, the largest value and among equal values the
// lowest index.  Max-then-lowest-index is associative and commutative, so the result is the row's
// first maximum (NaN never taken, a row of NaN gives 0) for any split: kr_argmax's result.
constexpr uint32_t kNoArg = 0xFFFFFFFFu;

struct ArgPart {
    float v;
    uint32_t i;
};

__device__ __forceinline__ void arg_take(float &v, uint32_t &idx, float ov, uint32_t oi) {
    if (ov > v || (ov == v && oi < idx) || (idx == kNoArg && oi != kNoArg)) {
        v = ov;
        idx = oi;
    }
}

// grid (P, rows), 256 threads; per % 4 == 0 when vec (rows of n % 4 == 0, 16-byte aligned)
__global__ __launch_bounds__(256) void argmax_partial_kernel(const float *logits, uint32_t n, uint32_t per, int vec,
                                                             ArgPart *part) {
    __shared__ float bv[4];
    __shared__ uint32_t bi[4];
    const uint32_t tid = threadIdx.x, j = blockIdx.x, r = blockIdx.y;
    const float *row = logits + (size_t)r * n;
    const uint32_t e0 = j * per, e1 = min(e0 + per, n);
    float v = -INFINITY;
    uint32_t idx = kNoArg;
    if (vec) {
        // a cheap max per quad first (fmaxf drops NaN); a quad that can win is searched for its
        // first lane holding that max; two quads requested before either is scanned
        const f32x4 *r4 = reinterpret_cast<const f32x4 *>(row);
        const uint32_t u0 = e0 / 4, u1 = (e1 + 3) / 4;
        for (uint32_t i0 = u0 + tid; i0 < u1; i0 += 512) {
            const uint32_t i1 = i0 + 256;
            const f32x4 xa = r4[i0], xb = r4[min(i1, u1 - 1)];
#pragma unroll
            for (int h = 0; h < 2; ++h) {
                const uint32_t i = h ? i1 : i0;
                const f32x4 x = h ? xb : xa;
                const float m = fmaxf(fmaxf(x[0], x[1]), fmaxf(x[2], x[3]));
                if (i < u1 && (m > v || (idx == kNoArg && m == m))) {
                    const uint32_t c = x[0] == m ? 0u : x[1] == m ? 1u : x[2] == m ? 2u : 3u;
                    v = m;
                    idx = 4 * i + c;
                }
            }
        }
    } else {
        for (uint32_t i = e0 + tid; i < e1; i += 256) {
            const float x = row[i];
            if (x > v || (idx == kNoArg && x == x)) {
                v = x;
                idx = i;
            }
        }
    }
#pragma unroll
    for (int m = 32; m >= 1; m >>= 1) arg_take(v, idx, __shfl_xor(v, m), __shfl_xor(idx, m));
    if ((tid & 63) == 0) {
        bv[tid >> 6] = v;
        bi[tid >> 6] = idx;
    }
    __syncthreads();
    if (tid == 0) {
        v = bv[0];
        idx = bi[0];
        for (int w = 1; w < 4; ++w) arg_take(v, idx, bv[w], bi[w]);
        part[(size_t)r * gridDim.x + j] = ArgPart{v, idx};
    }
}

// grid rows, one wave: the row's P partials merged
__global__ __launch_bounds__(64) void argmax_merge_kernel(const ArgPart *part, uint32_t P, uint32_t *out) {
    const uint32_t lane = threadIdx.x, r = blockIdx.x;
    float v = -INFINITY;
    uint32_t idx = kNoArg;
    for (uint32_t j = lane; j < P; j += 64) {
        const ArgPart a = part[(size_t)r * P + j];
        arg_take(v, idx, a.v, a.i);
    }
#pragma unroll
    for (int m = 32; m >= 1; m >>= 1) arg_take(v, idx, __shfl_xor(v, m), __shfl_xor(idx, m));
    if (lane == 0) out[r] = idx == kNoArg ? 0u : idx;
}

hipError_t launch_q4_embedding(const Q4Mat &w, const uint32_t *tokens, uint32_t count, uint16_t *out, hipStream_t s) {
    const dim3 grid((w.k / 8 + 255) / 256, count);
    hipLaunchKernelGGL(q4_embedding_kernel, grid, dim3(256), 0, s, w, tokens, count, out);
    return hipGetLastError();
}

hipError_t launch_rmsnorm(const uint16_t *x, const uint16_t *weight, uint32_t rows, uint32_t dim, float eps,
                          uint16_t *out, hipStream_t s) {
    hipLaunchKernelGGL(rmsnorm_kernel, dim3(rows), dim3(256), 0, s, x, weight, dim, eps, out);
    return hipGetLastError();
}

hipError_t launch_rope_kv_append(uint16_t *q, const uint16_t *k, const uint16_t *v, const float *cos_sin,
                                 const uint32_t *positions, uint32_t batch, uint32_t q_heads, uint32_t kv_heads,
                                 uint32_t D, uint16_t *k_cache, uint16_t *v_cache, uint32_t max_ctx, hipStream_t s) {
    hipLaunchKernelGGL(rope_kv_append_kernel, dim3(q_heads + kv_heads, batch), dim3(64), 0, s, q, k, v, cos_sin,
                       positions, q_heads, kv_heads, D, k_cache, v_cache, max_ctx);
    return hipGetLastError();
}

hipError_t launch_attention_decode(const uint16_t *q, const uint16_t *k_cache, const uint16_t *v_cache,
                                   const uint32_t *positions, uint32_t batch, uint32_t q_heads, uint32_t kv_heads,
                                   uint32_t D, uint32_t max_ctx, uint16_t *out, hipStream_t s) {
    hipLaunchKernelGGL(attention_decode_kernel, dim3(q_heads, batch), dim3(kAttnThreads), 0, s, q, k_cache, v_cache,
                       positions,
                       q_heads, kv_heads, D, max_ctx, out);
    return hipGetLastError();
}

uint32_t attention_splits(uint32_t max_ctx) { return (max_ctx + kSplitLen - 1) / kSplitLen; }

size_t attention_workspace_bytes(uint32_t batch, uint32_t q_heads, uint32_t D, uint32_t max_ctx) {
    return (size_t)batch * attention_splits(max_ctx) * q_heads * (D + 2) * sizeof(float);
}

hipError_t launch_rope_attention(const uint16_t *q, const uint16_t *k, const uint16_t *v, const float *cos_sin,
                                 const uint32_t *positions, uint32_t batch, uint32_t q_heads, uint32_t kv_heads,
                                 uint32_t D, uint16_t *k_cache, uint16_t *v_cache, uint32_t max_ctx, uint16_t *out,
                                 float *part, hipStream_t s) {
    const uint32_t G = q_heads / kv_heads;
    // 64-position slices (head_dim 128): when they still give about one block per compute unit
    // (16-position slices spread a short batch over more of them)
    const uint32_t s64 = (max_ctx + kSplit64 - 1) / kSplit64;
    const bool wide = D == 128 && G <= 16 &&
                      (tuning().attn_slice64 == 2 ||
                       (tuning().attn_slice64 == 1 && (uint64_t)batch * kv_heads * s64 >= (uint64_t)device_cus()));
    const uint32_t splits = wide ? s64 : attention_splits(max_ctx);
    const dim3 grid(splits, kv_heads, batch);
#define KR_SPLIT(GP)                                                                                           \
    hipLaunchKernelGGL(attention_split_kernel<GP>, grid, dim3(256), 0, s, q, k, v, cos_sin, positions, q_heads, \
                       kv_heads, D, k_cache, v_cache, max_ctx, part)
    if (wide)
        hipLaunchKernelGGL(attention_split64_kernel<4>, grid, dim3(256), 0, s, q, k, v, cos_sin, positions, q_heads,
                           kv_heads, k_cache, v_cache, max_ctx, part);
    else if (G <= 1)
        KR_SPLIT(1);
    else if (G <= 2)
        KR_SPLIT(2);
    else if (G <= 4)
        KR_SPLIT(4);
    else if (G <= 8)
        KR_SPLIT(8);
    else
        KR_SPLIT(16);
#undef KR_SPLIT
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return e;
    const dim3 mgrid(q_heads, batch);
#define KR_MERGE(DW)                                                                                           \
    hipLaunchKernelGGL(attention_combine_wave_kernel<DW>, mgrid, dim3(256), 0, s, part, q_heads, kv_heads, D, \
                       splits, out)
    const bool wave_merge = tuning().attn_merge_wave && splits <= kWave;
    if (wave_merge && D == 256) KR_MERGE(64);
    else if (wave_merge && D == 128) KR_MERGE(32);
    else if (wave_merge && D == 64) KR_MERGE(16);
    else if (wave_merge && D == 32) KR_MERGE(8);
    else if (wave_merge && D == 16) KR_MERGE(4);
    else if (wave_merge && D == 8) KR_MERGE(2);
    else
        hipLaunchKernelGGL(attention_combine_kernel, mgrid, dim3(256), 0, s, part, q_heads, kv_heads, D, splits, out);
#undef KR_MERGE
    return hipGetLastError();
}

// Blocks per row of the split argmax: about 512 blocks in all, at least 1024 logits each (so a
// thread has a quad or more), at most kArgmaxMaxParts.
uint32_t argmax_parts(uint32_t rows, uint32_t n) {
    const uint32_t by_size = std::max<uint32_t>(1, n / 1024);
    const uint32_t by_grid = std::max<uint32_t>(1, (512 + rows - 1) / std::max<uint32_t>(rows, 1));
    return std::min<uint32_t>(std::min(by_size, by_grid), kArgmaxMaxParts);
}

size_t argmax_workspace_bytes(uint32_t rows, uint32_t n) { return (size_t)rows * argmax_parts(rows, n) * sizeof(ArgPart); }

hipError_t launch_argmax_split(const float *logits, uint32_t rows, uint32_t n, uint32_t *out, void *ws, hipStream_t s) {
    const uint32_t P = argmax_parts(rows, n);
    const int vec = n % 4 == 0 && (uintptr_t)logits % 16 == 0;
    uint32_t per = (n + P - 1) / P;
    if (vec) per = (per + 3) / 4 * 4;
    ArgPart *part = reinterpret_cast<ArgPart *>(ws);
    hipLaunchKernelGGL(argmax_partial_kernel, dim3(P, rows), dim3(256), 0, s, logits, n, per, vec, part);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return e;
    hipLaunchKernelGGL(argmax_merge_kernel, dim3(rows), dim3(64), 0, s, part, P, out);
    return hipGetLastError();
}

hipError_t launch_argmax(const float *logits, uint32_t rows, uint32_t n, uint32_t *out, hipStream_t s) {
    hipLaunchKernelGGL(argmax_kernel, dim3(rows), dim3(1024), 0, s, logits, n, out);
    return hipGetLastError();
}

}  // namespace kr
