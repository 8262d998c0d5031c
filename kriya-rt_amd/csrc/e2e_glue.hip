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

#include "kr_internal.hpp"

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
#pragma unroll
    for (int m = 32; m >= 1; m >>= 1) mx = fmaxf(mx, __shfl_xor(mx, m));
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
        const f32x4 *r4 = reinterpret_cast<const f32x4 *>(row);
#pragma unroll 8
        for (uint32_t i = tid; i < n / 4; i += 1024) {
            const f32x4 x = r4[i];
#pragma unroll
            for (int c = 0; c < 4; ++c) take(x[c], 4 * i + c);
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

hipError_t launch_argmax(const float *logits, uint32_t rows, uint32_t n, uint32_t *out, hipStream_t s) {
    hipLaunchKernelGGL(argmax_kernel, dim3(rows), dim3(1024), 0, s, logits, n, out);
    return hipGetLastError();
}

}  // namespace kr
