// q4_gemv.hip — single-token (m == 1) Q4_G64 GEMV family for gfx950.
//
// Replaces the decode kernels of kernels/metal/q4_gemm_and_moe.metal:
//   q4_g64_decode_gemv[_2row,_4row,_sub16]           :932-1076, 1162-1215, 1280-1344
//   q4_g64_decode_gemv_accumulate[_2row,_4row,_sub16] :1081-1157, 1220-1275, 1349-1423
//   q4_g64_decode_gate_up_swiglu_gemv[_2chan,_sub16]  :1850-1901, 2003-2158
//
// Bound: HBM.  Per output row the kernels stream k/2 bytes of nibbles and
// k/16 bytes of scales+biases once.
//
// Three kernels share one inner step (chunk_dot):
//   * wave kernel, k <= 64 * 32 * C (C = chunks per lane, 1 or 2): a
//     wavefront owns a tile of R rows; lane l reads the 16-byte chunks l,
//     l+64 of every row (one global_load_dwordx4 per row per chunk, so a wave
//     instruction reads 1 KiB of a row contiguously).  Waves are persistent:
//     the x operand pairs of the lane's chunks are built once, and the next
//     tile's weights are loaded while the current tile is reduced.
//   * long-row kernel, 4096 < k <= 24576 (the down projection, k = 11008):
//     one block per RB rows (4 by default) with a wave per 64 chunks of the
//     row (512 threads up to k = 16384, 768 beyond); thread c
//     requests chunk c of all the block's rows at once and builds the x pairs
//     of chunk c once for all of them, so x is read once per RB rows (the
//     split-K block kernel reads it once per R = 2 rows: 22 KB per 12 KB of
//     weights).
//   * block kernel (split-K), the gate/up pairs over k > 4096, or any rows when a split-K threshold is set:
//     the 256 threads of a block share the chunks of R rows; thread i reads
//     chunks i, i+256, i+512; the four wave partials are added through LDS.
//
// Arithmetic per 8 nibbles (one u32 word): 3 shifts + 4 v_and_or_b32 turn the
// nibble pairs (j, j+4) into exact bf16 values (128+q) (kr_device.hpp), and
// 4 v_dot2_f32_bf16 multiply them with the matching x pairs.  A chunk is 32
// elements = half a 64-group; per row and chunk the affine map costs two
// FMAs:  acc += s * D + (b - 128 s) * sum(x).
// Reductions run in a fixed order (transposing butterfly, then wave order),
// so results are bitwise reproducible and independent of the grid size.
#include "moe_route.hpp"
#include "q4_dot2.hpp"

namespace kr {

// ---------------------------------------------------------------- wave kernel

// kMulti: the batch may hold several problems (np > 1); single-problem
// launches skip the per-tile problem selection.
template <int R, int C, int EPI, bool kMulti, bool kNorm = false>
__global__ __launch_bounds__(256) void q4_gemv_wave_kernel(GemvBatch gb, const uint16_t *__restrict__ x) {
    gemv_wave_loop<R, C, EPI, kMulti, 1, kNorm>(gb, x, blockIdx.x * 4 + __builtin_amdgcn_readfirstlane(threadIdx.x / kWave),
                                              gridDim.x * 4);
}

// The wave kernel for M = 2..4 tokens (x holds M rows), two rows per tile,
// k <= 2048; at most 128 VGPRs so that four waves fit per SIMD.
template <int EPI, int M>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(4))) void q4_gemv_tokens_kernel(
    GemvBatch gb, const uint16_t *__restrict__ x) {
    gemv_wave_loop<2, 1, EPI, false, M>(gb, x, blockIdx.x * 4 + __builtin_amdgcn_readfirstlane(threadIdx.x / kWave),
                                        gridDim.x * 4);
}

// ---------------------------------------------------------------- block (split-K) kernel

template <int R, int C, int EPI>
__global__ __launch_bounds__(256) void q4_gemv_block_kernel(Q4Mat A, Q4Mat B, const uint16_t *__restrict__ x,
                                                            GemvOut o, uint32_t tiles) {
    constexpr bool kGateUp = (EPI == kGateUpF32 || EPI == kGateUpBF16);
    constexpr int kSeg = kWave / R;
    __shared__ float red[4][R];
    const int tid = threadIdx.x;
    const int lane = tid & (kWave - 1);
    const uint32_t wave = __builtin_amdgcn_readfirstlane(tid / kWave);
    const uint32_t nchunks = A.k >> 5;
    const uint32_t kMask = sgpr_const(0x000F000Fu);
    const uint32_t kMagic = vgpr_const(0x43004300u);
    const uint32_t kSelLo = sgpr_const(0x05040100u);
    const uint32_t kSelHi = sgpr_const(0x07060302u);
    uint32_t t = blockIdx.x;
    if (t >= tiles) return;

    const u32x4 *rq[R];
    const uint16_t *rs[R];
    const uint16_t *rb[R];
    u32x4 wv[C][R];
    uint32_t sv[C][R], bv[C][R];
    bool live[C];
    auto fetch = [&](uint32_t tt) {
        tile_rows<R, kGateUp>(A, B, tt, rq, rs, rb);
#pragma unroll
        for (int i = 0; i < C; ++i) {
            const uint32_t c = tid + 256 * i;
            if (live[i]) {
#pragma unroll
                for (int r = 0; r < R; ++r) {
                    wv[i][r] = ld_stream(rq[r] + c);
                    sv[i][r] = ld_stream(rs[r] + (c >> 1));
                    bv[i][r] = ld_stream(rb[r] + (c >> 1));
                }
            }
        }
    };
#pragma unroll
    for (int i = 0; i < C; ++i) live[i] = (tid + 256u * i) < nchunks;
    fetch(t);  // weights first: they do not depend on x
    float pre = wave == 0 ? tile_prefetch<R, EPI>(lane, t, A.n, o) : 0.0f;
    XChunk xc[C];
#pragma unroll
    for (int i = 0; i < C; ++i)
        if (live[i]) load_xchunk(xc[i], x, tid + 256 * i, kSelLo, kSelHi);

    for (;;) {
        float acc[R];
#pragma unroll
        for (int r = 0; r < R; ++r) acc[r] = 0.0f;
#pragma unroll
        for (int i = 0; i < C; ++i) {
            if (live[i]) {
#pragma unroll
                for (int r = 0; r < R; ++r) acc[r] = chunk_dot(wv[i][r], sv[i][r], bv[i][r], xc[i], acc[r], kMask, kMagic);
            }
        }
        const uint32_t tn = t + gridDim.x;
        float pre_n = 0.0f;
        if (tn < tiles) {
            fetch(tn);
            if (wave == 0) pre_n = tile_prefetch<R, EPI>(lane, tn, A.n, o);
        }
        float tot = wave_reduce_rows<R>(acc, lane);
        const int slot = lane / kSeg;
        if ((lane % kSeg) == 0) red[wave][slot] = tot;
        __syncthreads();
        if (wave == 0) {
            tot = ((red[0][slot] + red[1][slot]) + red[2][slot]) + red[3][slot];
            tile_epilogue<R, EPI>(tot, lane, t, A.n, o, pre);
        }
        if (tn >= tiles) break;
        __syncthreads();  // red is rewritten by the next tile
        t = tn;
        pre = pre_n;
    }
}

// ---------------------------------------------------------------- long-row kernel

// Rows longer than the wave kernel covers (the down projection, k = 11008), up
// to 64 W chunks: one block of NG row groups of W waves per RB rows (W = 8: up to
// 512 chunks, k <= 16384; W = 12, one row group, up to 768 chunks: k <= 24576,
// the largest k the library takes).  Thread (g, c) with row group g = wave / W (rows g,
// g + NG, ..., of the block) and chunk c = 64 (wave mod W) + lane requests the
// chunk c of all its rows at once, builds the x pairs of chunk c once and
// reuses them for those rows -- x is read once per block, not once per row
// pair -- then the rows are reduced in a fixed order (butterfly, then the W
// waves of the group in order).
// M > 1: x holds M token rows; thread (g, c) multiplies its words with the
// chunk c of every token and the block stores M rows of outputs.
template <int RB, int EPI, int M = 1, int NG = 2, int W = 8>
__global__ __launch_bounds__(NG * W * 64) void q4_gemv_rows_kernel(Q4Mat A, const uint16_t *__restrict__ x, GemvOut o) {
    constexpr int RPG = RB / NG;
    constexpr int MP = tokens_pow2<M>();
    constexpr int kVals = RPG * MP;  // values per thread: (row i of the group, token), tokens padded
    constexpr int kSeg = kWave / kVals;
    __shared__ float red[NG][W][kVals];
    const int tid = threadIdx.x;
    const int lane = tid & (kWave - 1);
    const uint32_t wave = __builtin_amdgcn_readfirstlane(tid / kWave);
    const uint32_t g = NG == 1 ? 0u : wave / W, c = (wave % W) * kWave + lane;
    const uint32_t r0 = blockIdx.x * RB;
    const uint32_t nchunks = A.k >> 5, wpr = A.k >> 3, groups = A.k >> 6;
    const uint32_t kMask = sgpr_const(0x000F000Fu);
    const uint32_t kMagic = vgpr_const(0x43004300u);
    const uint32_t kSelLo = sgpr_const(0x05040100u);
    const uint32_t kSelHi = sgpr_const(0x07060302u);
    typename FVec<kVals>::type acc = {};
    // the epilogue's operand (old output or bias) of output tid = (token tid / RB, row tid % RB),
    // requested with the weights
    const uint32_t out_row = r0 + (uint32_t)tid % RB, out_tok = (uint32_t)tid / RB;
    const size_t out_idx = (size_t)out_tok * o.ldo + out_row;
    float pre = 0.0f;
    if (tid < RB * M && out_row < A.n) {
        if (EPI == kAccF32) pre = reinterpret_cast<const float *>(o.out)[out_idx];
        if (EPI == kAccBF16) pre = bf16_to_f32(reinterpret_cast<const uint16_t *>(o.out)[out_idx]);
        if ((EPI == kStoreF32 || EPI == kStoreBF16) && o.bias) pre = bf16_to_f32(o.bias[out_row]);
    }
    if (c < nchunks) {
        u32x4 wv[RPG];
        uint32_t sv[RPG], bv[RPG];
#pragma unroll
        for (int i = 0; i < RPG; ++i) {
            uint32_t row = r0 + g + NG * i;
            row = row < A.n ? row : A.n - 1;  // tail rows re-read a valid row and are never stored
            wv[i] = ld_stream(reinterpret_cast<const u32x4 *>(A.qw + (size_t)row * wpr) + c);
            sv[i] = ld_stream(A.sc + (size_t)row * groups + (c >> 1));
            bv[i] = ld_stream(A.bi + (size_t)row * groups + (c >> 1));
        }
        XChunk xc[M];
        uint32_t X[M][16];
#pragma unroll
        for (int tk = 0; tk < M; ++tk) load_xwords(X[tk], x + (size_t)tk * A.k, c);
#pragma unroll
        for (int tk = 0; tk < M; ++tk) build_xchunk(xc[tk], X[tk], kSelLo, kSelHi);
#pragma unroll
        for (int i = 0; i < RPG; ++i) chunk_dot_m<M>(wv[i], sv[i], bv[i], xc, acc, i * MP, kMask, kMagic);
    }
    const float tot = wave_reduce_vec<kVals>(acc, lane);
    if ((lane % kSeg) == 0) red[g][wave % W][lane / kSeg] = tot;
    __syncthreads();
    if (tid < RB * M && out_row < A.n) {
        const uint32_t rr = (uint32_t)tid % RB;
        const uint32_t gg = rr % NG, v = (rr / NG) * MP + out_tok;
        float sum = 0.0f;
#pragma unroll
        for (int w = 0; w < W; ++w) sum += red[gg][w][v];
        store_row<EPI>(o, out_idx, sum, pre);
    }
}

// ---------------------------------------------------------------- launch

template <int EPI>
static uint32_t tiles_for(uint32_t n, int R) {
    constexpr bool kGateUp = (EPI == kGateUpF32 || EPI == kGateUpBF16);
    const uint32_t per_tile = kGateUp ? R / 2 : R;
    return (n + per_tile - 1) / per_tile;
}

static uint32_t cap_blocks(uint32_t blocks, uint32_t persistent_default) {
    const int cap = tuning().gemv_max_blocks;
    if (cap > 0) return blocks < (uint32_t)cap ? blocks : (uint32_t)cap;
    return blocks < persistent_default ? blocks : persistent_default;
}

template <int R, int EPI>
static hipError_t launch_wave_batch(GemvBatch &gb, const uint16_t *x, hipStream_t s) {
    uint32_t tiles = 0;
    for (int i = 0; i < gb.np; ++i) {
        gb.p[i].tile_begin = tiles;
        tiles += tiles_for<EPI>(gb.p[i].A.n, R);
    }
    gb.tiles = tiles;
    if (tiles == 0) return hipSuccess;  // (the norm-fused kernel requests tile min(t, tiles - 1))
    const uint32_t blocks = cap_blocks((tiles + 3) / 4, (uint32_t)tuning().gemv_persistent_blocks);
    const bool c1 = gb.p[0].A.k <= 64 * 32;
    // the norm-fused kernels (x RMS-normalised in the kernel) exist for the epilogues the fused
    // norms use: gate/up (kr_rmsnorm_q4_mlp) and the stores (kr_rmsnorm_q4_qkv)
    constexpr bool kNormable = EPI == kGateUpBF16 || EPI == kStoreF32 || EPI == kStoreBF16;
    if (gb.ln_w && !kNormable) return hipErrorInvalidValue;
#define KR_WAVE(CC, MULTI)                                                                                       \
    do {                                                                                                         \
        if constexpr (kNormable) {                                                                               \
            if (gb.ln_w) {                                                                                       \
                hipLaunchKernelGGL((q4_gemv_wave_kernel<R, CC, EPI, MULTI, true>), dim3(blocks), dim3(256), 0, s, \
                                   gb, x);                                                                       \
                break;                                                                                           \
            }                                                                                                    \
        }                                                                                                        \
        hipLaunchKernelGGL((q4_gemv_wave_kernel<R, CC, EPI, MULTI, false>), dim3(blocks), dim3(256), 0, s, gb, x); \
    } while (0)
    if (gb.np == 1) {
        if (c1)
            KR_WAVE(1, false);
        else
            KR_WAVE(2, false);
    } else if constexpr (EPI == kStoreF32 || EPI == kStoreBF16) {
        if (c1)
            KR_WAVE(1, true);
        else
            KR_WAVE(2, true);
    } else {
        return hipErrorInvalidValue;  // batches of several problems use the store epilogues only
    }
#undef KR_WAVE
    return hipGetLastError();
}

template <int R, int EPI>
static hipError_t launch_wave(const Q4Mat &a, const Q4Mat &b, const uint16_t *x, const GemvOut &o, hipStream_t s) {
    GemvBatch gb{};
    gb.p[0] = GemvProblem{a, b, o, 0};
    gb.np = 1;
    return launch_wave_batch<R, EPI>(gb, x, s);
}

template <int R, int EPI>
static hipError_t launch_block(const Q4Mat &a, const Q4Mat &b, const uint16_t *x, const GemvOut &o, hipStream_t s) {
    const uint32_t tiles = tiles_for<EPI>(a.n, R);
    const uint32_t blocks = cap_blocks(tiles, 1u << 30);
    const uint32_t nchunks = a.k >> 5;
    if (nchunks <= 256)
        hipLaunchKernelGGL((q4_gemv_block_kernel<R, 1, EPI>), dim3(blocks), dim3(256), 0, s, a, b, x, o, tiles);
    else if (nchunks <= 512)
        hipLaunchKernelGGL((q4_gemv_block_kernel<R, 2, EPI>), dim3(blocks), dim3(256), 0, s, a, b, x, o, tiles);
    else
        hipLaunchKernelGGL((q4_gemv_block_kernel<R, 3, EPI>), dim3(blocks), dim3(256), 0, s, a, b, x, o, tiles);
    return hipGetLastError();
}

template <int EPI>
static hipError_t launch_epi(const Q4Mat &a, const Q4Mat &b, const uint16_t *x, const GemvOut &o, hipStream_t s) {
    constexpr bool kGateUp = (EPI == kGateUpF32 || EPI == kGateUpBF16);
    const uint32_t chunks = a.k >> 5;
    const int lr = tuning().gemv_long_rows;
    if constexpr (!kGateUp) {
        if (lr > 0 && chunks > 128 && chunks <= 768 && tuning().gemv_split_k_chunks == 0) {
            const uint32_t blocks = (a.n + lr - 1) / lr;
#define KR_ROWS(RB, NG) \
    hipLaunchKernelGGL((q4_gemv_rows_kernel<RB, EPI, 1, NG>), dim3(blocks), dim3(NG * 512), 0, s, a, x, o)
#define KR_ROWS_W(RB, W) \
    hipLaunchKernelGGL((q4_gemv_rows_kernel<RB, EPI, 1, 1, W>), dim3(blocks), dim3(W * 64), 0, s, a, x, o)
            if (chunks > 512) {  // 16384 < k <= kMaxGemvK: 12 waves per row group, one group
                if (lr == 4) KR_ROWS_W(4, 12);
                else if (lr == 16) KR_ROWS_W(16, 12);
                else KR_ROWS_W(8, 12);
            } else if (tuning().gemv_long_groups == 1) {
                if (lr == 4) KR_ROWS(4, 1);
                else if (lr == 16) KR_ROWS(16, 1);
                else KR_ROWS(8, 1);
            } else {
                if (lr == 4) KR_ROWS(4, 2);
                else if (lr == 16) KR_ROWS(16, 2);
                else KR_ROWS(8, 2);
            }
#undef KR_ROWS
#undef KR_ROWS_W
            return hipGetLastError();
        }
    }
    const int split = tuning().gemv_split_k_chunks;
    const bool use_block = chunks > 128 || (split > 0 && chunks >= (uint32_t)split);
    const int rw = use_block ? tuning().gemv_block_rows : tuning().gemv_rows_per_wave;
    switch (rw) {
        case 1:
            if constexpr (!kGateUp)
                return use_block ? launch_block<1, EPI>(a, b, x, o, s) : launch_wave<1, EPI>(a, b, x, o, s);
            else
                return use_block ? launch_block<2, EPI>(a, b, x, o, s) : launch_wave<2, EPI>(a, b, x, o, s);
        case 2:
            return use_block ? launch_block<2, EPI>(a, b, x, o, s) : launch_wave<2, EPI>(a, b, x, o, s);
        case 8:
            return use_block ? launch_block<8, EPI>(a, b, x, o, s) : launch_wave<8, EPI>(a, b, x, o, s);
        default:
            return use_block ? launch_block<4, EPI>(a, b, x, o, s) : launch_wave<4, EPI>(a, b, x, o, s);
    }
}

template <int EPI>
static hipError_t launch_batch_epi(GemvBatch &gb, const uint16_t *x, hipStream_t s) {
    switch (tuning().gemv_rows_per_wave) {
        case 1:
            if constexpr (EPI == kGateUpF32 || EPI == kGateUpBF16) return launch_wave_batch<2, EPI>(gb, x, s);
            else return launch_wave_batch<1, EPI>(gb, x, s);
        case 2: return launch_wave_batch<2, EPI>(gb, x, s);
        case 8: return launch_wave_batch<8, EPI>(gb, x, s);
        default: return launch_wave_batch<4, EPI>(gb, x, s);
    }
}

bool gemv_batch_supported(uint32_t k) { return k % 64 == 0 && k <= 2 * 64 * 32; }

// ---------------------------------------------------------------- routed MoE GEMV

// Items are (sorted position p, row tile) pairs, p-major; wave w takes the
// contiguous run [w * per, (w + 1) * per), so that its items mostly share one
// position: the expert lookup and the x pairs are redone only when p changes.
// Expert of p: the number of bucket ends offsets[1..E] <= p (one ballot per 64
// experts).  The next item's words are requested before the current item is
// reduced and stored, as in the wave kernel.
//
// kRoute (one token, gate/up): the routing is part of the launch.  Every wave routes the token
// itself (route_token_wave, the routing kernel's arithmetic, so the same experts and weights): the
// K slots' experts e_k, and their positions p_k = #{k' : e_k' < e_k} + #{k' < k : e_k' == e_k} in
// the expert-sorted order (offsets[e] + rank inside the bucket, as the routing kernel assigns
// them).  Wave 0 of block 0 writes selected, weights, counts, offsets and sorted.
template <int EPI, bool kRoute>
__global__ __launch_bounds__(256) void q4_moe_gemv_kernel(MoeGemvArgs a) {
    constexpr int R = 2;
    constexpr bool kGateUp = (EPI == kGateUpF32 || EPI == kGateUpBF16);
    const int lane = threadIdx.x & (kWave - 1);
    const uint32_t wid = __builtin_amdgcn_readfirstlane(threadIdx.x / kWave);
    const uint32_t wave = blockIdx.x * 4 + wid;
    const uint32_t nwaves = gridDim.x * 4;
    const uint32_t total = a.assign * a.tiles_per;
    const uint32_t per = (total + nwaves - 1) / nwaves;
    const uint32_t t_begin = wave * per, t_end = min(t_begin + per, total);
    uint32_t r_e = 0, r_p = 0;  // lane k < K: slot k's expert and sorted position (kRoute)
    if constexpr (kRoute) {
        // wave 0 of the block routes the token and hands (e_k, p_k) to the block's waves through LDS;
        // wave 0 of block 0 also writes the routing arrays.  A block whose waves have no items
        // (items go to waves in order) leaves at once, unless it is block 0.
        __shared__ __attribute__((aligned(16))) float s_pr[kMaxExperts];
        __shared__ __attribute__((aligned(16))) uint32_t s_ti[kRouteMaxTopK];
        __shared__ uint32_t s_e[kRouteMaxTopK], s_p[kRouteMaxTopK];
        __shared__ float s_tv[kRouteMaxTopK];
        if (blockIdx.x * 4 * per >= total && blockIdx.x != 0) return;
        if (wid == 0) {
            float lv[kRoutePer];
            load_logits(a.logits, a.experts, (uint32_t)lane, lv);
            route_token_wave(lv, a.experts, a.topk, a.normalize, (uint32_t)lane, s_pr, s_ti, s_tv);
            __builtin_amdgcn_wave_barrier();
            __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
            __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
            const bool slot = (uint32_t)lane < a.topk;
            uint32_t ek[kRouteMaxTopK];  // every slot's expert in every lane (16-byte LDS reads)
#pragma unroll
            for (uint32_t q = 0; q < kRouteMaxTopK / 4; ++q) {
                const u32x4 v = reinterpret_cast<const u32x4 *>(s_ti)[q];
                ek[4 * q] = v.x;
                ek[4 * q + 1] = v.y;
                ek[4 * q + 2] = v.z;
                ek[4 * q + 3] = v.w;
            }
            r_e = s_ti[slot ? lane : 0];
#pragma unroll
            for (uint32_t k = 0; k < kRouteMaxTopK; ++k)
                r_p += (k < a.topk && (ek[k] < r_e || (ek[k] == r_e && k < (uint32_t)lane))) ? 1u : 0u;
            if (slot) {
                s_e[lane] = r_e;
                s_p[lane] = r_p;
            }
            if (blockIdx.x == 0) {
                if (slot) {
                    a.r_selected[lane] = r_e;
                    a.r_weights[lane] = s_tv[lane];
                    const_cast<uint32_t *>(a.sorted)[r_p] = (uint32_t)lane;
                }
                for (uint32_t e = (uint32_t)lane; e < a.experts; e += kWave) {
                    uint32_t cnt = 0, below = 0;
#pragma unroll
                    for (uint32_t k = 0; k < kRouteMaxTopK; ++k) {
                        cnt += (k < a.topk && ek[k] == e) ? 1u : 0u;
                        below += (k < a.topk && ek[k] < e) ? 1u : 0u;
                    }
                    a.r_counts[e] = cnt;
                    const_cast<uint32_t *>(a.offsets)[e] = below;
                }
                if (lane == 0) const_cast<uint32_t *>(a.offsets)[a.experts] = a.topk;
            }
        }
        __syncthreads();
        if (t_begin >= t_end) return;
        const uint32_t k = (uint32_t)lane < a.topk ? (uint32_t)lane : 0u;
        r_e = s_e[k];
        r_p = s_p[k];
    } else {
        if (t_begin >= t_end) return;
    }
    const uint32_t K = a.w.k, nchunks = K >> 5, wpr = K >> 3, groups = K >> 6;
    const uint32_t kMask = sgpr_const(0x000F000Fu);
    const uint32_t kMagic = vgpr_const(0x43004300u);
    const uint32_t kSelLo = sgpr_const(0x05040100u);
    const uint32_t kSelHi = sgpr_const(0x07060302u);
    const bool live = (uint32_t)lane < nchunks;
    const uint32_t c = live ? (uint32_t)lane : 0u;

    // A fixed, unrolled sequence with uniform guards and clamped loads, not a loop: the compiler
    // waits for every load in flight before entering a loop, which would serialise this lookup
    // behind sorted[p].
    auto expert_of = [&](uint32_t p) -> uint32_t {
        uint32_t e = 0;
#pragma unroll
        for (uint32_t i = 0; i < kMaxExperts / kWave; ++i) {
            if (i * kWave < a.experts) {
                const uint32_t j = i * kWave + (uint32_t)lane;
                const uint32_t end = a.offsets[min(j, a.experts - 1) + 1];
                e += (uint32_t)__popcll(__ballot(j < a.experts && end <= p));
            }
        }
        return e;
    };
    // per-position state: views of the expert's matrices, the x pairs, the output row base.
    // Only the views depend on the expert; a position change requests sorted[p] with the
    // expert lookup, then the tile's words, then the x words, and the x pairs are built just
    // before the next dot: the chain to the first words is one round trip, not three.
    Q4Mat A = a.w, B = a.w2;
    GemvOut o{nullptr, nullptr, a.act, 0};
    XChunk xc;
    uint32_t X[16];
    uint32_t cur_p = 0xFFFFFFFFu, cur_xr = 0;
    auto enter = [&](uint32_t p) {
        uint32_t sp, e;
        if constexpr (kRoute) {
            // the slot at position p (positions of the K slots are distinct, 0 .. K-1)
            const uint64_t m = __ballot((uint32_t)lane < a.topk && r_p == p);
            sp = m ? (uint32_t)__builtin_ctzll(m) : 0u;
            e = min(__builtin_amdgcn_readlane(r_e, sp), a.experts - 1);
        } else {
            // sorted[p] through a lane-varying zero: a uniform load is moved to a scalar register
            // right away (a wait before the expert lookup is even requested); this one stays in a
            // vector register until its use
            // Both are clamped: a position at or past offsets[E] (an id >= E that joined no bucket)
            // has no expert and an unwritten sorted[p].  Its rows are then some expert's result for
            // some assignment (unspecified), but every access stays inside the arrays.
            sp = min(a.sorted[p + __builtin_amdgcn_mbcnt_lo(0u, 0u)], a.assign - 1);
            e = min(expert_of(p), a.experts - 1);
        }
        const size_t r0 = (size_t)e * a.rows;
        A.qw = a.w.qw + r0 * wpr;
        A.sc = a.w.sc + r0 * groups;
        A.bi = a.w.bi + r0 * groups;
        B.qw = a.w2.qw + r0 * wpr;
        B.sc = a.w2.sc + r0 * groups;
        B.bi = a.w2.bi + r0 * groups;
        A.n = B.n = a.rows;
        cur_xr = a.x_div ? sp / a.x_div : p;
        const uint32_t orow = a.out_scatter ? sp : p;
        const size_t esz = (EPI == kStoreF32 || EPI == kAccF32 || EPI == kGateUpF32) ? 4 : 2;
        o.out = reinterpret_cast<char *>(a.out) + (size_t)orow * a.ldo * esz;
        cur_p = p;
    };
    auto load_x = [&] { load_xwords(X, a.x + (size_t)cur_xr * K, c); };

    const u32x4 *rq[R];
    const uint16_t *rs[R];
    const uint16_t *rb[R];
    u32x4 wv[R];
    uint32_t sv[R], bv[R];
    auto fetch = [&](uint32_t lt) {
        tile_rows<R, kGateUp>(A, B, lt, rq, rs, rb);
#pragma unroll
        for (int r = 0; r < R; ++r) {
            wv[r] = ld_stream(rq[r] + c);
            sv[r] = ld_stream(rs[r] + (c >> 1));
            bv[r] = ld_stream(rb[r] + (c >> 1));
        }
    };
    uint32_t t = t_begin;
    enter(t / a.tiles_per);
    fetch(t % a.tiles_per);
    load_x();
    bool x_new = true;
    for (;;) {
        if (x_new) build_xchunk(xc, X, kSelLo, kSelHi);
        x_new = false;
        float acc[R];
#pragma unroll
        for (int r = 0; r < R; ++r) {
            const float d = chunk_dot(wv[r], sv[r], bv[r], xc, 0.0f, kMask, kMagic);
            acc[r] = live ? d : 0.0f;
        }
        const uint32_t lt = t % a.tiles_per;
        const GemvOut oc = o;
        const uint32_t tn = t + 1;
        if (tn < t_end) {
            const uint32_t pn = tn / a.tiles_per;
            if (pn != cur_p) {
                enter(pn);
                fetch(tn % a.tiles_per);
                load_x();
                x_new = true;
            } else {
                fetch(tn % a.tiles_per);
            }
        }
        const float tot = wave_reduce_rows<R>(acc, lane);
        tile_epilogue<R, EPI>(tot, lane, lt, a.rows, oc, 0.0f);
        if (tn >= t_end) break;
        t = tn;
    }
}

// The routed down projection with the combine folded in (few assignments, topk <= 4; replaces the
// down GEMV + moe_combine_kernel pair, transformer_glue.metal:373-401).  Items are (token t, row
// pair i), token-major; wave w takes the contiguous run [w * per, (w + 1) * per).  For every slot
// k < KS of t (slots >= topk repeat the last one and are not summed) the slot's position p_k in the
// expert-sorted list (the lane j < assign holding sorted[j] == t * topk + k) and its expert e_k
// (bucket ends <= p_k) select rows e_k * rows + 2i, 2i + 1 of the stacked matrices and h row p_k.
// The 2 * KS dots are reduced at once on the fixed tree, on which each value is summed exactly as
// the two-row reduction of the routed GEMV sums it, so every d_k has the bits of the down GEMV's f32
// output; then y[t, row] (+)= sum_k fma(w[t, k], d_k, acc) in slot order, moe_combine_kernel's
// arithmetic.  The results are those of the three-launch path bit for bit.
template <int KS>
__global__ __launch_bounds__(256) void q4_moe_down_combine_kernel(MoeDownArgs a) {
    constexpr int R = 2, NV = R * KS, kSeg = kWave / NV;
    const int lane = threadIdx.x & (kWave - 1);
    const uint32_t wave = blockIdx.x * 4 + __builtin_amdgcn_readfirstlane(threadIdx.x / kWave);
    const uint32_t nwaves = gridDim.x * 4;
    const uint32_t tiles = (a.rows + 1) / 2;
    const uint32_t total = a.tokens * tiles;
    const uint32_t per = (total + nwaves - 1) / nwaves;
    const uint32_t t_begin = wave * per, t_end = min(t_begin + per, total);
    if (t_begin >= t_end) return;
    const uint32_t K = a.w.k, nchunks = K >> 5, wpr = K >> 3, groups = K >> 6;
    const uint32_t kMask = sgpr_const(0x000F000Fu);
    const uint32_t kMagic = vgpr_const(0x43004300u);
    const uint32_t kSelLo = sgpr_const(0x05040100u);
    const uint32_t kSelHi = sgpr_const(0x07060302u);
    const bool live = (uint32_t)lane < nchunks;
    const uint32_t c = live ? (uint32_t)lane : 0u;
    const uint32_t assign = a.tokens * a.topk;
    // the routing state, requested once: lane j < assign holds sorted[j], lane j of round i the bucket
    // end offsets[64 i + j + 1] (unrolled with uniform guards and clamped loads: no loop waits)
    const uint32_t srt = a.sorted[min((uint32_t)lane, assign - 1)];
    uint32_t ends[kMaxExperts / kWave];
#pragma unroll
    for (uint32_t i = 0; i < kMaxExperts / kWave; ++i)
        ends[i] = i * kWave < a.experts ? a.offsets[min(i * kWave + (uint32_t)lane, a.experts - 1) + 1] : 0u;

    uint32_t xrow[KS];
    size_t rbase[KS];
    float wk[KS];
    uint32_t cur_t = 0xFFFFFFFFu;
    auto enter = [&](uint32_t tok) {
#pragma unroll
        for (int k = 0; k < KS; ++k) {
            const uint32_t aid = tok * a.topk + min((uint32_t)k, a.topk - 1);
            const uint64_t m = __ballot((uint32_t)lane < assign && srt == aid);
            // an assignment that joined no bucket (expert id >= E) has no position: its rows are some
            // expert's (unspecified), every access in bounds
            const uint32_t p = m ? (uint32_t)__builtin_ctzll(m) : 0u;
            uint32_t e = 0;
#pragma unroll
            for (uint32_t i = 0; i < kMaxExperts / kWave; ++i) {
                if (i * kWave < a.experts) {
                    const uint32_t j = i * kWave + (uint32_t)lane;
                    e += (uint32_t)__popcll(__ballot(j < a.experts && ends[i] <= p));
                }
            }
            e = min(e, a.experts - 1);
            xrow[k] = p;
            rbase[k] = (size_t)e * a.rows;
            wk[k] = a.weights[aid];
        }
        cur_t = tok;
    };

    u32x4 wv[KS][R];
    uint32_t sv[KS][R], bv[KS][R];
    auto fetch = [&](uint32_t i) {
#pragma unroll
        for (int k = 0; k < KS; ++k) {
#pragma unroll
            for (int r = 0; r < R; ++r) {
                const size_t row = rbase[k] + min(2 * i + (uint32_t)r, a.rows - 1);  // a tail row is never stored
                wv[k][r] = ld_stream(reinterpret_cast<const u32x4 *>(a.w.qw + row * wpr) + c);
                sv[k][r] = ld_stream(a.w.sc + row * groups + (c >> 1));
                bv[k][r] = ld_stream(a.w.bi + row * groups + (c >> 1));
            }
        }
    };
    uint32_t X[KS][16];
    XChunk xc[KS];
    auto load_x = [&] {
#pragma unroll
        for (int k = 0; k < KS; ++k) load_xwords(X[k], a.h + (size_t)xrow[k] * K, c);
    };
    uint32_t t = t_begin;
    enter(t / tiles);
    fetch(t % tiles);
    load_x();
    bool x_new = true;
    for (;;) {
        if (x_new) {
#pragma unroll
            for (int k = 0; k < KS; ++k) build_xchunk(xc[k], X[k], kSelLo, kSelHi);
        }
        x_new = false;
        float acc[NV];
#pragma unroll
        for (int k = 0; k < KS; ++k) {
#pragma unroll
            for (int r = 0; r < R; ++r) {
                const float d = chunk_dot(wv[k][r], sv[k][r], bv[k][r], xc[k], 0.0f, kMask, kMagic);
                acc[k * R + r] = live ? d : 0.0f;
            }
        }
        const uint32_t i = t % tiles, tok = cur_t;
        float w[KS];
#pragma unroll
        for (int k = 0; k < KS; ++k) w[k] = wk[k];
        const uint32_t tn = t + 1;
        if (tn < t_end) {
            if (tn / tiles != cur_t) {
                enter(tn / tiles);
                fetch(tn % tiles);
                load_x();
                x_new = true;
            } else {
                fetch(tn % tiles);
            }
        }
        const float tot = wave_reduce_rows<NV>(acc, lane);  // segment v = k * R + r holds d_k of row r
#pragma unroll
        for (int r = 0; r < R; ++r) {
            float y = 0.0f;
#pragma unroll
            for (int k = 0; k < KS; ++k) {
                const float d = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(tot), (k * R + r) * kSeg));
                if ((uint32_t)k < a.topk) y = fmaf(w[k], d, y);
            }
            const uint32_t row = 2 * i + r;
            if (lane == r && row < a.rows) {
                const size_t o = (size_t)tok * a.rows + row;
                if (a.y_f32) {
                    float *out = reinterpret_cast<float *>(a.y) + o;
                    *out = a.accumulate ? *out + y : y;
                } else {
                    uint16_t *out = reinterpret_cast<uint16_t *>(a.y) + o;
                    *out = (uint16_t)f32_to_bf16(a.accumulate ? bf16_to_f32(*out) + y : y);
                }
            }
        }
        if (tn >= t_end) break;
        t = tn;
    }
}

bool moe_gemv_fits(uint32_t k) { return k % 64 == 0 && k <= 2048; }
bool moe_gemv_route_fits(uint32_t experts, uint32_t topk) {
    return experts >= 1 && experts <= kMaxExperts && topk >= 1 && topk <= kRouteMaxTopK && topk <= experts;
}

hipError_t launch_moe_gemv(MoeGemvArgs &a, int epilogue, hipStream_t s) {
    if (!moe_gemv_fits(a.w.k) || a.assign == 0) return hipErrorInvalidValue;
    const bool gate_up = epilogue == kGateUpBF16 || epilogue == kGateUpF32;
    if (a.logits && (!gate_up || a.assign != a.topk || !moe_gemv_route_fits(a.experts, a.topk)))
        return hipErrorInvalidValue;  // in-launch routing: one token, gate/up
    a.tiles_per = gate_up ? a.rows : (a.rows + 1) / 2;  // two rows per tile: (gate, up) or a row pair
    const uint32_t total = a.assign * a.tiles_per;
    const uint32_t blocks = cap_blocks((total + 3) / 4, (uint32_t)tuning().gemv_persistent_blocks);
    switch (epilogue) {
        case kGateUpBF16:
            if (a.logits) hipLaunchKernelGGL((q4_moe_gemv_kernel<kGateUpBF16, true>), dim3(blocks), dim3(256), 0, s, a);
            else hipLaunchKernelGGL((q4_moe_gemv_kernel<kGateUpBF16, false>), dim3(blocks), dim3(256), 0, s, a);
            break;
        case kStoreF32:
            hipLaunchKernelGGL((q4_moe_gemv_kernel<kStoreF32, false>), dim3(blocks), dim3(256), 0, s, a);
            break;
        default: return hipErrorInvalidValue;
    }
    return hipGetLastError();
}

bool moe_down_combine_fits(uint32_t k, uint32_t topk) { return moe_gemv_fits(k) && topk >= 1 && topk <= 4; }

hipError_t launch_moe_down_combine(const MoeDownArgs &a, hipStream_t s) {
    if (!moe_down_combine_fits(a.w.k, a.topk) || a.tokens == 0 || a.rows == 0) return hipErrorInvalidValue;
    const uint32_t total = a.tokens * ((a.rows + 1) / 2);
    const uint32_t blocks = cap_blocks((total + 3) / 4, (uint32_t)tuning().gemv_persistent_blocks);
    switch (a.topk) {
        case 1: hipLaunchKernelGGL((q4_moe_down_combine_kernel<1>), dim3(blocks), dim3(256), 0, s, a); break;
        case 2: hipLaunchKernelGGL((q4_moe_down_combine_kernel<2>), dim3(blocks), dim3(256), 0, s, a); break;
        default: hipLaunchKernelGGL((q4_moe_down_combine_kernel<4>), dim3(blocks), dim3(256), 0, s, a); break;
    }
    return hipGetLastError();
}

// ---------------------------------------------------------------- 2 <= m <= 4 tokens

template <int EPI, int M>
static hipError_t launch_tokens_m(const Q4Mat &a, const Q4Mat &b, const uint16_t *x, const GemvOut &o, hipStream_t s) {
    constexpr bool kGateUp = (EPI == kGateUpF32 || EPI == kGateUpBF16);
    const uint32_t chunks = a.k >> 5;
    if (chunks <= 64) {  // one chunk per lane: the wave kernel, two rows per tile
        GemvBatch gb{};
        gb.p[0] = GemvProblem{a, b, o, 0};
        gb.np = 1;
        gb.tiles = tiles_for<EPI>(a.n, 2);
        const uint32_t blocks = cap_blocks((gb.tiles + 3) / 4, (uint32_t)tuning().gemv_persistent_blocks);
        hipLaunchKernelGGL((q4_gemv_tokens_kernel<EPI, M>), dim3(blocks), dim3(256), 0, s, gb, x);
        return hipGetLastError();
    }
    if constexpr (!kGateUp) {
        if (chunks <= 512) {
            const uint32_t blocks = (a.n + 7) / 8;
            // one row group of 512 threads: each thread's x words serve all 8 rows of the block
            // (x is M times the weight bytes per chunk here; measured 3-4 % faster than two groups)
            hipLaunchKernelGGL((q4_gemv_rows_kernel<8, EPI, M, 1>), dim3(blocks), dim3(512), 0, s, a, x, o);
            return hipGetLastError();
        }
    }
    return hipErrorInvalidValue;
}

template <int EPI>
static hipError_t launch_tokens_epi(const Q4Mat &a, const Q4Mat &b, const uint16_t *x, uint32_t m, const GemvOut &o,
                                    hipStream_t s) {
    switch (m) {
        case 2: return launch_tokens_m<EPI, 2>(a, b, x, o, s);
        case 3: return launch_tokens_m<EPI, 3>(a, b, x, o, s);
        case 4: return launch_tokens_m<EPI, 4>(a, b, x, o, s);
        default: return hipErrorInvalidValue;
    }
}

bool gemv_tokens_supported(uint32_t m, uint32_t k, bool gate_up) {
    return m >= 2 && m <= kGemvMaxTokens && k % 64 == 0 && (k <= 2048 || (!gate_up && k <= 16384));
}

hipError_t launch_gemv_tokens(const Q4Mat &a, const Q4Mat *b, const uint16_t *x, uint32_t m, void *out, uint32_t ldo,
                              int epilogue, int act, const uint16_t *bias, hipStream_t s) {
    const Q4Mat &bb = b ? *b : a;
    const GemvOut o{out, bias, act, ldo};
    switch (epilogue) {
        case kStoreF32: return launch_tokens_epi<kStoreF32>(a, bb, x, m, o, s);
        case kStoreBF16: return launch_tokens_epi<kStoreBF16>(a, bb, x, m, o, s);
        case kAccF32: return launch_tokens_epi<kAccF32>(a, bb, x, m, o, s);
        case kAccBF16: return launch_tokens_epi<kAccBF16>(a, bb, x, m, o, s);
        case kGateUpF32: return launch_tokens_epi<kGateUpF32>(a, bb, x, m, o, s);
        case kGateUpBF16: return launch_tokens_epi<kGateUpBF16>(a, bb, x, m, o, s);
        default: return hipErrorInvalidValue;
    }
}

hipError_t launch_gemv_batch(const Q4Mat *mats, const Q4Mat *up, const uint16_t *x, void *const *outs,
                             const uint16_t *const *biases, int np, int epilogue, int act, const uint16_t *ln_w,
                             float eps, hipStream_t s) {
    GemvBatch gb{};
    gb.np = np;
    gb.ln_w = ln_w;
    gb.eps = eps;
    for (int i = 0; i < np; ++i) gb.p[i] = GemvProblem{mats[i], up ? up[i] : mats[i], GemvOut{outs[i], biases[i], act, 0}, 0};
    switch (epilogue) {
        case kStoreF32: return launch_batch_epi<kStoreF32>(gb, x, s);
        case kStoreBF16: return launch_batch_epi<kStoreBF16>(gb, x, s);
        case kAccF32: return launch_batch_epi<kAccF32>(gb, x, s);
        case kAccBF16: return launch_batch_epi<kAccBF16>(gb, x, s);
        case kGateUpF32: return launch_batch_epi<kGateUpF32>(gb, x, s);
        case kGateUpBF16: return launch_batch_epi<kGateUpBF16>(gb, x, s);
        default: return hipErrorInvalidValue;
    }
}

hipError_t launch_gemv(const Q4Mat &a, const Q4Mat *b, const uint16_t *x, void *out, int epilogue, int act,
                       const uint16_t *bias, hipStream_t s) {
    const Q4Mat &bb = b ? *b : a;
    const GemvOut o{out, bias, act, 0};
    switch (epilogue) {
        case kStoreF32: return launch_epi<kStoreF32>(a, bb, x, o, s);
        case kStoreBF16: return launch_epi<kStoreBF16>(a, bb, x, o, s);
        case kAccF32: return launch_epi<kAccF32>(a, bb, x, o, s);
        case kAccBF16: return launch_epi<kAccBF16>(a, bb, x, o, s);
        case kGateUpF32: return launch_epi<kGateUpF32>(a, bb, x, o, s);
        case kGateUpBF16: return launch_epi<kGateUpBF16>(a, bb, x, o, s);
        default: return hipErrorInvalidValue;
    }
}

}  // namespace kr
