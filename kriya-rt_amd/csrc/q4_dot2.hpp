// q4_dot2.hpp — the shared inner step of the m == 1 Q4_G64 kernels (GEMV
// family and fused MLP): nibble unpack by bit patterns + v_dot2_f32_bf16.
//
// Arithmetic per 8 nibbles (one u32 word): 3 shifts + 4 v_and_or_b32 turn the
// nibble pairs (j, j+4) into exact bf16 values (128+q) (kr_device.hpp), and
// 4 v_dot2_f32_bf16 multiply them with the matching x pairs.  A chunk is 16
// bytes = 32 elements = half a 64-group; per row and chunk the affine map
// costs two FMAs:  acc += s * D + (b - 128 s) * sum(x).
#pragma once

#include "kr_internal.hpp"

namespace kr {

// Constants placed in registers through an opaque move, so that the compiler
// cannot fold them into literals: gfx9 VOP3 encodings (v_and_or_b32,
// v_perm_b32) take no literal operand, and with literals the unpack splits
// into separate AND and OR instructions.
__device__ __forceinline__ uint32_t sgpr_const(uint32_t v) {
    uint32_t r;
    asm volatile("s_mov_b32 %0, %1" : "=s"(r) : "i"(v));
    return r;
}
__device__ __forceinline__ uint32_t vgpr_const(uint32_t v) {
    uint32_t r;
    asm volatile("v_mov_b32 %0, %1" : "=v"(r) : "i"(v));
    return r;
}

// x operand of one chunk: the 16 dot2 pairs P[4w + j] = (x_{8w+j}, x_{8w+j+4})
// and the chunk sum.
struct XChunk {
    uint32_t p[16];
    float sum;
};

// x pairs of one chunk from its 16 words (32 bf16 values, element order).
__device__ __forceinline__ void build_xchunk(XChunk &xc, const uint32_t (&X)[16], uint32_t sel_lo, uint32_t sel_hi) {
#pragma unroll
    for (int w = 0; w < 4; ++w) {
        xc.p[4 * w + 0] = __builtin_amdgcn_perm(X[4 * w + 2], X[4 * w + 0], sel_lo);
        xc.p[4 * w + 1] = __builtin_amdgcn_perm(X[4 * w + 2], X[4 * w + 0], sel_hi);
        xc.p[4 * w + 2] = __builtin_amdgcn_perm(X[4 * w + 3], X[4 * w + 1], sel_lo);
        xc.p[4 * w + 3] = __builtin_amdgcn_perm(X[4 * w + 3], X[4 * w + 1], sel_hi);
    }
    float s = 0.0f;
#pragma unroll
    for (int i = 0; i < 16; ++i) s = dot2_bf16(X[i], 0x3F803F80u, s);
    xc.sum = s;
}

__device__ __forceinline__ void load_xwords(uint32_t (&X)[16], const uint16_t *__restrict__ x, uint32_t c) {
    const u32x4 *xv = reinterpret_cast<const u32x4 *>(x) + 4 * c;
    const u32x4 v0 = xv[0], v1 = xv[1], v2 = xv[2], v3 = xv[3];
    const uint32_t W[16] = {v0.x, v0.y, v0.z, v0.w, v1.x, v1.y, v1.z, v1.w,
                            v2.x, v2.y, v2.z, v2.w, v3.x, v3.y, v3.z, v3.w};
#pragma unroll
    for (int i = 0; i < 16; ++i) X[i] = W[i];
}

__device__ __forceinline__ void load_xchunk(XChunk &xc, const uint16_t *__restrict__ x, uint32_t c, uint32_t sel_lo,
                                            uint32_t sel_hi) {
    uint32_t X[16];
    load_xwords(X, x, c);
    build_xchunk(xc, X, sel_lo, sel_hi);
}

// acc += s * sum_j (128 + q_j) x_j + (b - 128 s) * sum(x) over one chunk of one row.
__device__ __forceinline__ float chunk_dot(const u32x4 &wv, uint32_t sraw, uint32_t braw, const XChunk &xc, float acc,
                                           uint32_t mask, uint32_t magic) {
    const float s = bf16_to_f32(sraw);
    const float b = bf16_to_f32(braw);
    const uint32_t wd[4] = {wv.x, wv.y, wv.z, wv.w};
    float d = 0.0f;
#pragma unroll
    for (int w = 0; w < 4; ++w) {
#pragma unroll
        for (int j = 0; j < 4; ++j) d = dot2_bf16(((wd[w] >> (4 * j)) & mask) | magic, xc.p[4 * w + j], d);
    }
    return fmaf(s, d, fmaf(fmaf(-128.0f, s, b), xc.sum, acc));
}

// The same for M tokens (x rows of `xc`) sharing the chunk's unpacked words:
// acc[base + t] += s * D_t + (b - 128 s) * sum(x_t).  M == 1 is chunk_dot.
// The accumulators are a vector value (a float array here ended up in LDS).
template <int M, typename V>
__device__ __forceinline__ void chunk_dot_m(const u32x4 &wv, uint32_t sraw, uint32_t braw, const XChunk (&xc)[M],
                                            V &acc, int base, uint32_t mask, uint32_t magic) {
    const float s = bf16_to_f32(sraw);
    const float b = bf16_to_f32(braw);
    const float c0 = fmaf(-128.0f, s, b);
    const uint32_t wd[4] = {wv.x, wv.y, wv.z, wv.w};
    uint32_t u[16];
#pragma unroll
    for (int w = 0; w < 4; ++w) {
#pragma unroll
        for (int j = 0; j < 4; ++j) u[4 * w + j] = ((wd[w] >> (4 * j)) & mask) | magic;
    }
#pragma unroll
    for (int t = 0; t < M; ++t) {
        float d = 0.0f;
#pragma unroll
        for (int i = 0; i < 16; ++i) d = dot2_bf16(u[i], xc[t].p[i], d);
        acc[base + t] = fmaf(s, d, fmaf(c0, xc[t].sum, acc[base + t]));
    }
}

// Epilogue operands of the m <= 4 kernels.
struct GemvOut {
    void *out;              // [n] (or [channels] for gate/up); token t's row at out + t * ldo
    const uint16_t *bias;   // bf16 [n] added by the store epilogues, or nullptr
    int act;                // activation of the gate/up epilogues
    uint32_t ldo;           // elements between the output rows of consecutive tokens (M > 1)
};

template <int EPI>
// `pre` is the row's bias (store epilogues) or its old output value
// (accumulate epilogues), read by tile_prefetch when the tile's weights were
// requested, so that the store does not wait for a read.
__device__ __forceinline__ void store_row(const GemvOut &o, uint32_t row, float v, float pre) {
    void *out = o.out;
    if (EPI == kStoreF32 || EPI == kStoreBF16) {
        if (o.bias) v += pre;
    }
    if (EPI == kStoreF32) {
        reinterpret_cast<float *>(out)[row] = v;
    } else if (EPI == kStoreBF16) {
        reinterpret_cast<uint16_t *>(out)[row] = (uint16_t)f32_to_bf16(v);
    } else if (EPI == kAccF32) {
        reinterpret_cast<float *>(out)[row] = pre + v;
    } else if (EPI == kAccBF16) {  // res = bf16(f32(res) + y), q4_gemm_and_moe.metal:1407-1420
        reinterpret_cast<uint16_t *>(out)[row] = (uint16_t)f32_to_bf16(v + pre);
    } else if (EPI == kGateUpF32) {
        reinterpret_cast<float *>(out)[row] = v;
    } else {
        reinterpret_cast<uint16_t *>(out)[row] = (uint16_t)f32_to_bf16(v);
    }
}

// Row r of tile t: plain rows t*R + r, or (gate, up) rows of channel t*R/2 + r/2.
template <int R, bool kGateUp>
__device__ __forceinline__ void tile_rows(const Q4Mat &A, const Q4Mat &B, uint32_t t, const u32x4 *(&rq)[R],
                                          const uint16_t *(&rs)[R], const uint16_t *(&rb)[R]) {
    const uint32_t wpr = A.k >> 3, groups = A.k >> 6;
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
        row = row < A.n ? row : A.n - 1;  // tail rows re-read a valid row and are never stored
        rq[r] = reinterpret_cast<const u32x4 *>(m->qw + (size_t)row * wpr);
        rs[r] = m->sc + (size_t)row * groups;
        rb[r] = m->bi + (size_t)row * groups;
    }
}

// Tokens rounded up to a power of two: the transposing butterfly reduces a
// power-of-two count of values.
template <int M>
constexpr int tokens_pow2() {
    return M <= 1 ? 1 : M <= 2 ? 2 : M <= 4 ? 4 : 8;
}

// After wave_reduce_rows<R * MP> over values v = r * MP + token (MP =
// tokens_pow2<M>(), padded tokens hold zeros), the lanes of segment
// v = lane / (64 / (R MP)) hold the total of (row r, token).
// The value store_row needs besides the dot product (bias or old output) of
// the output this lane stores for tile t; 0 when none.
template <int R, int EPI, int M = 1>
__device__ __forceinline__ float tile_prefetch(int lane, uint32_t t, uint32_t nrows, const GemvOut &o) {
    constexpr int MP = tokens_pow2<M>();
    constexpr int kSeg = kWave / (R * MP);
    const uint32_t v = (uint32_t)(lane / kSeg);
    const uint32_t row = t * R + v / MP, tok = v % MP;
    if ((lane % kSeg) != 0 || row >= nrows || tok >= (uint32_t)M) return 0.0f;
    const size_t idx = (size_t)tok * o.ldo + row;
    if (EPI == kAccF32) return reinterpret_cast<const float *>(o.out)[idx];
    if (EPI == kAccBF16) return bf16_to_f32(reinterpret_cast<const uint16_t *>(o.out)[idx]);
    if ((EPI == kStoreF32 || EPI == kStoreBF16) && o.bias) return bf16_to_f32(o.bias[row]);
    return 0.0f;
}

template <int R, int EPI, int M = 1>
__device__ __forceinline__ void tile_epilogue(float tot, int lane, uint32_t t, uint32_t nrows, const GemvOut &o,
                                              float pre) {
    constexpr bool kGateUp = (EPI == kGateUpF32 || EPI == kGateUpBF16);
    constexpr int MP = tokens_pow2<M>();
    constexpr int kSeg = kWave / (R * MP);
    const uint32_t v = (uint32_t)(lane / kSeg);
    const uint32_t r = v / MP, tok = v % MP;
    if (tok >= (uint32_t)M) return;
    if (kGateUp) {
        // row r + 1 of the same token, from the lane that holds it
        const float up = kWave / R == 32 ? xchg32(tot, lane) : kWave / R == 16 ? xchg16(tot, lane) : __shfl_xor(tot, kWave / R);
        if ((lane % kSeg) == 0 && (r & 1) == 0) {
            const uint32_t ch = t * (R / 2) + (r >> 1);
            if (ch < nrows) store_row<EPI>(o, tok * o.ldo + ch, activation(tot, o.act) * up, 0.0f);
        }
    } else if ((lane % kSeg) == 0) {
        const uint32_t row = t * R + r;
        if (row < nrows) store_row<EPI>(o, tok * o.ldo + row, tot, pre);
    }
}

// Up to three problems that share x and k in one launch of the wave kernel
// (the Q, K and V projections): tile t belongs to problem i when
// p[i].tile_begin <= t < p[i + 1].tile_begin.  ln_w != nullptr: x is first
// RMS-normalised, y = bf16(x * rsqrt(mean(x^2) + eps) * ln_w) as kr_rmsnorm
// computes it (the wave holds all of x when k <= 64 * 32 * C, so the mean is
// one wave reduction).
struct GemvProblem {
    Q4Mat A, B;          // B: the up matrix of the gate/up epilogues (= A otherwise)
    GemvOut o;
    uint32_t tile_begin;
};
struct GemvBatch {
    GemvProblem p[3];
    int np;
    uint32_t tiles;
    const uint16_t *ln_w;
    float eps;
};

template <typename T>
__device__ __forceinline__ T pick3(int i, T a, T b, T c) {
    return i == 2 ? c : (i == 1 ? b : a);
}

// Problem `pi` of the batch (wave-uniform) and tile t's index inside it.
__device__ __forceinline__ GemvProblem pick_problem(const GemvBatch &gb, int pi, uint32_t t, uint32_t &lt) {
    const GemvProblem &p0 = gb.p[0], &p1 = gb.p[1], &p2 = gb.p[2];
    GemvProblem P;
    P.A.qw = pick3(pi, p0.A.qw, p1.A.qw, p2.A.qw);
    P.A.sc = pick3(pi, p0.A.sc, p1.A.sc, p2.A.sc);
    P.A.bi = pick3(pi, p0.A.bi, p1.A.bi, p2.A.bi);
    P.A.n = pick3(pi, p0.A.n, p1.A.n, p2.A.n);
    P.A.k = p0.A.k;
    P.B.qw = pick3(pi, p0.B.qw, p1.B.qw, p2.B.qw);
    P.B.sc = pick3(pi, p0.B.sc, p1.B.sc, p2.B.sc);
    P.B.bi = pick3(pi, p0.B.bi, p1.B.bi, p2.B.bi);
    P.B.n = pick3(pi, p0.B.n, p1.B.n, p2.B.n);
    P.B.k = p0.A.k;
    P.o.out = pick3(pi, p0.o.out, p1.o.out, p2.o.out);
    P.o.bias = pick3(pi, p0.o.bias, p1.o.bias, p2.o.bias);
    P.o.act = pick3(pi, p0.o.act, p1.o.act, p2.o.act);
    P.tile_begin = pick3(pi, p0.tile_begin, p1.tile_begin, p2.tile_begin);
    lt = t - P.tile_begin;
    return P;
}

// The persistent wave loop of the m == 1 wave kernel: wave `t0` of `nwaves`
// takes tiles t0, t0 + nwaves, ...; lane l owns the 16-byte chunks l, l + 64
// of every row (k <= 64 * 32 * C).  The x operand pairs of the lane's chunks
// are built once, and the next tile's weights (and the value its epilogue
// needs) are requested before the current tile is reduced and stored.
// M > 1: x holds M token rows of k elements; every unpacked word is
// multiplied with all of them (no RMSNorm, single problem).
template <int R, int C, int EPI, bool kMulti, int M = 1, bool kNorm = false>
__device__ __forceinline__ void gemv_wave_loop(const GemvBatch &gb, const uint16_t *__restrict__ x, uint32_t t0,
                                               uint32_t nwaves) {
    constexpr bool kGateUp = (EPI == kGateUpF32 || EPI == kGateUpBF16);
    static_assert(M == 1 || !kMulti, "several tokens: one problem per launch");
    const int lane = threadIdx.x & (kWave - 1);
    uint32_t t = t0;
    const uint32_t tiles = gb.tiles;
    const uint32_t K = gb.p[0].A.k;
    const uint32_t nchunks = K >> 5;
    const uint32_t kMask = sgpr_const(0x000F000Fu);
    const uint32_t kMagic = vgpr_const(0x43004300u);
    const uint32_t kSelLo = sgpr_const(0x05040100u);
    const uint32_t kSelHi = sgpr_const(0x07060302u);
    // (the norm-fused kernel returns after its block-wide prologue: every wave of the block
    // reaches that prologue's barriers)
    if (!kNorm && t >= tiles) return;

    // lane's chunks (c < nchunks is lane-dependent only through c = lane + 64 i)
    bool live[C];
#pragma unroll
    for (int i = 0; i < C; ++i) live[i] = lane + kWave * i < nchunks;

    // The problem is selected field by field from constant-index reads
    // (scalar loads and selects).  Indexing the table with a run-time index,
    // or selecting whole structs, went through per-lane or scratch loads whose
    // vmcnt waits also waited for the weight prefetch in flight.
    const int np = gb.np;
    auto locate = [&](uint32_t tt, uint32_t &lt) -> GemvProblem {
        if (!kMulti) {
            lt = tt;
            return gb.p[0];
        }
        const int pi = (np > 2 && tt >= gb.p[2].tile_begin) ? 2 : (np > 1 && tt >= gb.p[1].tile_begin) ? 1 : 0;
        return pick_problem(gb, pi, tt, lt);
    };

    const u32x4 *rq[R];
    const uint16_t *rs[R];
    const uint16_t *rb[R];
    u32x4 wv[C][R];
    uint32_t sv[C][R], bv[C][R];
    auto fetch = [&](uint32_t tt) -> float {
        uint32_t lt;
        const GemvProblem P = locate(tt, lt);
        tile_rows<R, kGateUp>(P.A, P.B, lt, rq, rs, rb);
#pragma unroll
        for (int i = 0; i < C; ++i) {
            const uint32_t c = lane + kWave * i;
            if (live[i]) {
#pragma unroll
                for (int r = 0; r < R; ++r) {
                    wv[i][r] = ld_stream(rq[r] + c);
                    sv[i][r] = ld_stream(rs[r] + (c >> 1));
                    bv[i][r] = ld_stream(rb[r] + (c >> 1));
                }
            }
        }
        return tile_prefetch<R, EPI, M>(lane, lt, P.A.n, P.o);
    };

    XChunk xc[C][M];
    float pre = 0.0f;
    if constexpr (M > 1) {
        // the first tile's words, then every token's x words, all in flight before the first conversion
        pre = fetch(t);
        uint32_t X[M][C][16];
#pragma unroll
        for (int tk = 0; tk < M; ++tk) {
#pragma unroll
            for (int i = 0; i < C; ++i)
                if (live[i]) load_xwords(X[tk][i], x + (size_t)tk * K, lane + kWave * i);
        }
#pragma unroll
        for (int tk = 0; tk < M; ++tk) {
#pragma unroll
            for (int i = 0; i < C; ++i)
                if (live[i]) build_xchunk(xc[i][tk], X[tk][i], kSelLo, kSelHi);
        }
    } else {
        uint32_t X[C][16];
        if constexpr (kNorm) {
            // The block RMS-normalises x once, into LDS (bf16(x * rsqrt(mean(x^2) + eps) * w),
            // kr_rmsnorm's arithmetic): thread t loads 16-byte units t and t + 256 of x and ln_w,
            // the four waves' sums of squares meet in LDS (added in wave order), each thread
            // scales its units, and every lane reads its chunks back.  Per-wave norms read x and
            // ln_w once per wave and repeated the arithmetic.  The first tile's words are
            // requested before the norm waits for x.  Every wave runs this prologue (its loads
            // depend only on the thread and K; a wave without a tile requests a valid tile it
            // never uses) and so reaches both barriers; such a wave returns after them.
            static_assert(C <= 2, "k <= 4096: at most two 16-byte units per thread");
            __shared__ u32x4 s_xn[2 * 256];
            __shared__ float s_ss[4];
            const uint32_t tid = threadIdx.x, units = K >> 3;
            u32x4 xu[2], wu[2];
#pragma unroll
            for (int j = 0; j < 2; ++j) {
                const uint32_t uu = min(tid + 256u * j, units - 1);
                xu[j] = *reinterpret_cast<const u32x4 *>(x + 8 * (size_t)uu);
                wu[j] = *reinterpret_cast<const u32x4 *>(gb.ln_w + 8 * (size_t)uu);
            }
            pre = fetch(t < tiles ? t : tiles - 1);
            __builtin_amdgcn_sched_barrier(0);  // the norm's arithmetic stays after the requests
            float ss = 0.0f;
#pragma unroll
            for (int j = 0; j < 2; ++j) {
                if (tid + 256u * j < units) {
                    const uint32_t W4[4] = {xu[j].x, xu[j].y, xu[j].z, xu[j].w};
#pragma unroll
                    for (int e = 0; e < 4; ++e) {
                        const float a = __uint_as_float(W4[e] << 16), b = __uint_as_float(W4[e] & 0xFFFF0000u);
                        ss = fmaf(a, a, ss);
                        ss = fmaf(b, b, ss);
                    }
                }
            }
            ss = wave_total(ss, lane);
            if (lane == 0) s_ss[tid >> 6] = ss;
            asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");  // LDS only: the words stay in flight
            const float scale = 1.0f / sqrtf((((s_ss[0] + s_ss[1]) + s_ss[2]) + s_ss[3]) / (float)K + gb.eps);
#pragma unroll
            for (int j = 0; j < 2; ++j) {
                if (tid + 256u * j < units) {
                    const uint32_t X4[4] = {xu[j].x, xu[j].y, xu[j].z, xu[j].w};
                    const uint32_t L4[4] = {wu[j].x, wu[j].y, wu[j].z, wu[j].w};
                    uint32_t o[4];
#pragma unroll
                    for (int e = 0; e < 4; ++e) {
                        const float lo = __uint_as_float(X4[e] << 16) * scale * __uint_as_float(L4[e] << 16);
                        const float hi =
                            __uint_as_float(X4[e] & 0xFFFF0000u) * scale * __uint_as_float(L4[e] & 0xFFFF0000u);
                        o[e] = pack_bf16_rne(lo, hi);
                    }
                    s_xn[tid + 256u * j] = u32x4{o[0], o[1], o[2], o[3]};
                }
            }
            asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
            if (t >= tiles) return;
#pragma unroll
            for (int i = 0; i < C; ++i) {
                if (live[i]) {
                    const uint32_t c = lane + kWave * i;
#pragma unroll
                    for (int q = 0; q < 4; ++q) {
                        const u32x4 v = s_xn[4 * c + q];
                        X[i][4 * q] = v.x;
                        X[i][4 * q + 1] = v.y;
                        X[i][4 * q + 2] = v.z;
                        X[i][4 * q + 3] = v.w;
                    }
                    build_xchunk(xc[i][0], X[i], kSelLo, kSelHi);
                }
            }
        } else {
#pragma unroll
            for (int i = 0; i < C; ++i)
                if (live[i]) load_xwords(X[i], x, lane + kWave * i);
#pragma unroll
            for (int i = 0; i < C; ++i)
                if (live[i]) build_xchunk(xc[i][0], X[i], kSelLo, kSelHi);
            pre = fetch(t);
        }
    }

    for (;;) {
        // consume the fetched tile into accumulators, then prefetch the next one
        constexpr int MP = tokens_pow2<M>();
        typename FVec<R * MP>::type acc = {};
#pragma unroll
        for (int i = 0; i < C; ++i) {
            if (live[i]) {
#pragma unroll
                for (int r = 0; r < R; ++r)
                    chunk_dot_m<M>(wv[i][r], sv[i][r], bv[i][r], xc[i], acc, r * MP, kMask, kMagic);
            }
        }
        const uint32_t tn = t + nwaves;
        float pre_n = 0.0f;
        if (tn < tiles) pre_n = fetch(tn);
        const float tot = wave_reduce_vec<R * MP>(acc, lane);
        uint32_t lt;
        const GemvProblem P = locate(t, lt);
        tile_epilogue<R, EPI, M>(tot, lane, lt, P.A.n, P.o, pre);
        if (tn >= tiles) break;
        t = tn;
        pre = pre_n;
    }
}

}  // namespace kr
