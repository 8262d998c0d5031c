// q4_gemv.hip — single-token (m == 1) Q4_G64 GEMV family for gfx950.
//
// Replaces the decode kernels of kernels/metal/q4_gemm_and_moe.metal:
//   q4_g64_decode_gemv[_2row,_4row,_sub16]           :932-1076, 1162-1215, 1280-1344
//   q4_g64_decode_gemv_accumulate[_2row,_4row,_sub16] :1081-1157, 1220-1275, 1349-1423
//   q4_g64_decode_gate_up_swiglu_gemv[_2chan,_sub16]  :1850-1901, 2003-2158
//
// Bound: HBM.  Per output row the kernel streams k/2 bytes of nibbles and
// k/16 bytes of scales+biases once; x (2k bytes) is shared by all rows and
// stays in L2.
//
// Mapping.  One wavefront owns R rows (R in {1,2,4,8}).  Lane l reads the
// 16-byte chunks c = l, l+64, ... of every row: one global_load_dwordx4 per
// row per chunk, 64 consecutive chunks per wave instruction, so a wave
// instruction reads 1 KiB of one row contiguously.  A chunk is 32 elements =
// half a 64-group, so each lane needs one scale/bias pair per row per chunk.
//
// Arithmetic per 8 nibbles (one u32 word): 4 AND-OR + 3 shifts turn nibble
// pairs into exact bf16 values (128+q) (kr_device.hpp), and 4 v_dot2_f32_bf16
// multiply them with the matching x pairs.  x is re-paired once per chunk
// (shared by the R rows) and its chunk sum is taken once; per row and chunk
// the affine map costs two FMAs:  acc += s * D + (b - 128 s) * sum(x).
// The R row sums are reduced across the wavefront with the transposing
// butterfly of wave_reduce_rows (R-1 + 6-log2(R) shuffles for R rows).
#include "kr_internal.hpp"

namespace kr {

template <int R, int EPI>
__global__ __launch_bounds__(256) void q4_gemv_dot2_kernel(Q4Mat A, Q4Mat B, const uint16_t *__restrict__ x,
                                                           void *__restrict__ out, int act, uint32_t tiles) {
    constexpr bool kGateUp = (EPI == kGateUpF32 || EPI == kGateUpBF16);
    constexpr int kSeg = kWave / R;  // lanes per row after the reduction
    const int lane = threadIdx.x & (kWave - 1);
    const uint32_t wave = threadIdx.x / kWave;
    const uint32_t K = A.k;
    const uint32_t nchunks = K >> 5;
    const uint32_t words_per_row = K >> 3;
    const uint32_t groups = K >> 6;
    const u32x4 *__restrict__ xv = reinterpret_cast<const u32x4 *>(x);

    for (uint32_t t = blockIdx.x * 4 + wave; t < tiles; t += gridDim.x * 4) {
        const u32x4 *rq[R];
        const uint16_t *rs[R];
        const uint16_t *rb[R];
#pragma unroll
        for (int r = 0; r < R; ++r) {
            uint32_t row;
            const Q4Mat *m = &A;
            if (kGateUp) {
                row = t * (R / 2) + (r >> 1);
                if (r & 1) m = &B;
            } else {
                row = t * R + r;
            }
            row = row < A.n ? row : A.n - 1;  // tail rows re-read a valid row, never stored
            rq[r] = reinterpret_cast<const u32x4 *>(m->qw + (size_t)row * words_per_row);
            rs[r] = m->sc + (size_t)row * groups;
            rb[r] = m->bi + (size_t)row * groups;
        }

        float acc[R];
#pragma unroll
        for (int r = 0; r < R; ++r) acc[r] = 0.0f;

        for (uint32_t c = lane; c < nchunks; c += kWave) {
            u32x4 wv[R];
            uint32_t sraw[R], braw[R];
#pragma unroll
            for (int r = 0; r < R; ++r) {
                wv[r] = ld_stream(rq[r] + c);
                sraw[r] = ld_stream(rs[r] + (c >> 1));
                braw[r] = ld_stream(rb[r] + (c >> 1));
            }
            const u32x4 x0 = xv[4 * c + 0], x1 = xv[4 * c + 1], x2 = xv[4 * c + 2], x3 = xv[4 * c + 3];
            const uint32_t X[16] = {x0.x, x0.y, x0.z, x0.w, x1.x, x1.y, x1.z, x1.w,
                                    x2.x, x2.y, x2.z, x2.w, x3.x, x3.y, x3.z, x3.w};
            uint32_t P[16];
            float xs = 0.0f;
#pragma unroll
            for (int w = 0; w < 4; ++w) {
                P[4 * w + 0] = pack_lo(X[4 * w + 0], X[4 * w + 2]);
                P[4 * w + 1] = pack_hi(X[4 * w + 0], X[4 * w + 2]);
                P[4 * w + 2] = pack_lo(X[4 * w + 1], X[4 * w + 3]);
                P[4 * w + 3] = pack_hi(X[4 * w + 1], X[4 * w + 3]);
            }
#pragma unroll
            for (int i = 0; i < 16; ++i) xs = dot2_bf16(X[i], 0x3F803F80u, xs);

#pragma unroll
            for (int r = 0; r < R; ++r) {
                const float s = bf16_to_f32(sraw[r]);
                const float b = bf16_to_f32(braw[r]);
                float d = 0.0f;
                const uint32_t wd[4] = {wv[r].x, wv[r].y, wv[r].z, wv[r].w};
#pragma unroll
                for (int w = 0; w < 4; ++w) {
#pragma unroll
                    for (int j = 0; j < 4; ++j) d = dot2_bf16(q4_pair_bf16(wd[w], j), P[4 * w + j], d);
                }
                acc[r] = fmaf(s, d, fmaf(fmaf(-128.0f, s, b), xs, acc[r]));
            }
        }

        const float tot = wave_reduce_rows<R>(acc, lane);
        const int slot = lane / kSeg;
        if (kGateUp) {
            const float up = __shfl_xor(tot, kSeg);
            if ((lane % kSeg) == 0 && (slot & 1) == 0) {
                const uint32_t ch = t * (R / 2) + (slot >> 1);
                if (ch < A.n) {
                    const float v = activation(tot, act) * up;
                    if (EPI == kGateUpF32)
                        reinterpret_cast<float *>(out)[ch] = v;
                    else
                        reinterpret_cast<uint16_t *>(out)[ch] = (uint16_t)f32_to_bf16(v);
                }
            }
        } else if ((lane % kSeg) == 0) {
            const uint32_t row = t * R + slot;
            if (row < A.n) {
                if (EPI == kStoreF32) {
                    reinterpret_cast<float *>(out)[row] = tot;
                } else if (EPI == kStoreBF16) {
                    reinterpret_cast<uint16_t *>(out)[row] = (uint16_t)f32_to_bf16(tot);
                } else if (EPI == kAccF32) {
                    reinterpret_cast<float *>(out)[row] += tot;
                } else {  // kAccBF16: res = bf16(f32(res) + y), q4_gemm_and_moe.metal:1407-1420
                    uint16_t *o = reinterpret_cast<uint16_t *>(out);
                    o[row] = (uint16_t)f32_to_bf16(tot + bf16_to_f32(o[row]));
                }
            }
        }
    }
}

template <int R, int EPI>
static hipError_t launch_rows(const Q4Mat &a, const Q4Mat &b, const uint16_t *x, void *out, int act,
                              hipStream_t s) {
    constexpr bool kGateUp = (EPI == kGateUpF32 || EPI == kGateUpBF16);
    const uint32_t per_tile = kGateUp ? R / 2 : R;
    const uint32_t tiles = (a.n + per_tile - 1) / per_tile;
    uint32_t blocks = (tiles + 3) / 4;
    const int cap = tuning().gemv_max_blocks;
    if (cap > 0 && blocks > (uint32_t)cap) blocks = (uint32_t)cap;
    hipLaunchKernelGGL((q4_gemv_dot2_kernel<R, EPI>), dim3(blocks), dim3(256), 0, s, a, b, x, out, act, tiles);
    return hipGetLastError();
}

template <int EPI>
static hipError_t launch_epi(const Q4Mat &a, const Q4Mat &b, const uint16_t *x, void *out, int act,
                             hipStream_t s) {
    constexpr bool kGateUp = (EPI == kGateUpF32 || EPI == kGateUpBF16);
    switch (tuning().gemv_rows_per_wave) {
        case 1:
            if constexpr (!kGateUp) return launch_rows<1, EPI>(a, b, x, out, act, s);
            else return launch_rows<2, EPI>(a, b, x, out, act, s);
        case 2: return launch_rows<2, EPI>(a, b, x, out, act, s);
        case 8: return launch_rows<8, EPI>(a, b, x, out, act, s);
        default: return launch_rows<4, EPI>(a, b, x, out, act, s);
    }
}

hipError_t launch_gemv(const Q4Mat &a, const Q4Mat *b, const uint16_t *x, void *out, int epilogue, int act,
                       hipStream_t s) {
    const Q4Mat &bb = b ? *b : a;
    switch (epilogue) {
        case kStoreF32: return launch_epi<kStoreF32>(a, bb, x, out, act, s);
        case kStoreBF16: return launch_epi<kStoreBF16>(a, bb, x, out, act, s);
        case kAccF32: return launch_epi<kAccF32>(a, bb, x, out, act, s);
        case kAccBF16: return launch_epi<kAccBF16>(a, bb, x, out, act, s);
        case kGateUpF32: return launch_epi<kGateUpF32>(a, bb, x, out, act, s);
        case kGateUpBF16: return launch_epi<kGateUpBF16>(a, bb, x, out, act, s);
        default: return hipErrorInvalidValue;
    }
}

}  // namespace kr
