// q4_skinny.hip — Q4_G64 matmul for a few tokens per weight tile on the matrix
// cores: batched decode (config 1 B = 4, 16) and the routed MoE experts
// (config 4), where every expert sees only the few tokens routed to it.
// Replaces the reference's small-M path q4_g64_prefill_gemm / _gate_up_gemm
// (kernels/metal/q4_gemm_and_moe.metal:2173-2486) and the routed expert GEMV
// q4_g64_routed_moe_gemv (:2642-2698), which re-reads an expert's weights once
// per routed (token, slot) pair.
//
// Bound: HBM (the weights are read once per launch; 16 tokens give AI <= 57 FLOP/B).
//
// Mapping.  v_mfma_f32_16x16x32_f16 with A = X (16 token rows, zero-padded)
// and B = W^T (16 weight rows).  A wave owns a K range of 4 L columns: lane
// group g = lane / 16 covers [k0 + g L, k0 + (g + 1) L) and lane l % 16 its
// token row (A) or weight row (B).  The X fragments of the range stay in
// registers while the wave walks its weight tiles; per tile each lane loads
// L/8 consecutive u32 words of one weight row straight into registers (a wave
// instruction reads 16 rows x 64 contiguous bytes), and the next tile's words
// are requested before the current tile is multiplied (two register buffers).
// Dequantisation in registers: nibble pairs (j, j+4) under the fp16 pattern
// 0x6400 -> exact (1024+q) halves, v_pk_add_f16 -1024, v_pk_fma_f16 (s, b); the
// resulting order e0 e4 e1 e5 e2 e6 e3 e7 is applied to the X fragments too,
// so it cancels in the dot product.
// Gate/up: a tile holds 8 gate rows (lanes 0-7) and the same 8 up rows (lanes
// 8-15), so one MFMA chain yields both dot products of 8 features and the
// epilogue pairs lane c with lane c + 8.
// A block of NWAVES waves covers NWAVES consecutive K ranges; the wave partials
// are added through LDS in wave order.  When K needs more ranges than a block
// has, K is also split over blocks and f32 partials are reduced in split order
// by q4_mfma_splitk_reduce_kernel.
// Grouped mode (MoE): the weight matrix stacks E experts of expert_rows rows;
// offsets[E+1] and the expert-sorted assignment list select, per expert, the
// token rows to gather (X row = sorted[p] / x_div, or p) and where each result
// row goes (sorted[p], or p).  Work items are (active expert, tile) pairs in
// expert order; each block takes a contiguous run of them, so X is reloaded
// only when the expert changes.  Experts with more than 16 routed rows loop
// over 16-row chunks with the weight tile held in registers.
#include <algorithm>

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

__device__ __forceinline__ uint32_t word_of(const u32x4 &v, int i) {
    return i == 0 ? v.x : i == 1 ? v.y : i == 2 ? v.z : v.w;
}

// One lane's share of a weight tile: L/8 words of one row plus its scales/biases.
template <int L>
struct WTile {
    u32x4 w[L / 32];
    uint32_t s[L / 64], b[L / 64];
};

}  // namespace

// L: columns per lane group (64 or 128); NWAVES: K ranges per block (4 or 8);
// kGateUp: interleaved gate/up tiles with the activation epilogue;
// kGrouped: MoE expert groups.
template <int L, int NWAVES, bool kGateUp, bool kGrouped>
__global__ __launch_bounds__(NWAVES * 64) void q4_skinny_kernel(SkinnyArgs a) {
    constexpr int kSlices = L / 8;  // MFMA k-slices per tile (8 columns per lane each)
    constexpr int kVec = L / 32;    // dwordx4 loads per lane per tile
    constexpr int kGroups = L / 64; // quantisation groups per lane per tile
    constexpr uint32_t kTileRows = kGateUp ? 8 : 16;  // output features per tile
    constexpr int kLists = kGrouped ? (int)kMaxExperts : 1;
    __shared__ f32x4 red[2][NWAVES][64];
    __shared__ uint32_t s_active[kLists], s_base[kLists], s_cnt[kLists];
    __shared__ uint32_t s_nactive;

    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int g = lane >> 4, r16 = lane & 15;
    const uint32_t K = a.k;
    const uint32_t split = blockIdx.x % a.ksplit;
    const uint32_t k_lane = (split * NWAVES + wave) * (4 * L) + g * L;  // first column of this lane group
    const bool k_live = k_lane < K;  // K % L == 0: a lane group is all in or all out
    const uint32_t k_col = k_live ? k_lane : 0;  // dead lane groups read column 0 and zero it
    const uint32_t kMask = opq_s(0x000F000Fu);
    const uint32_t kMagic = opq_v(0x64006400u);

    // ---- active experts (grouped mode): non-empty buckets in increasing id, with base and count
    uint32_t nactive = 1;
    if constexpr (kGrouped) {
        if (wave == 0) {
            uint32_t n = 0;
            for (uint32_t e0 = 0; e0 < a.experts; e0 += 64) {
                const uint32_t e = e0 + lane;
                uint32_t lo = 0, hi = 0;
                if (e < a.experts) {
                    lo = a.offsets[e];
                    hi = a.offsets[e + 1];
                }
                const bool live = hi > lo;
                const uint64_t mask = __ballot(live);
                if (live) {
                    const uint32_t slot = n + (uint32_t)__popcll(mask & ((1ull << lane) - 1ull));
                    s_active[slot] = e;
                    s_base[slot] = lo;
                    s_cnt[slot] = hi - lo;
                }
                n += (uint32_t)__popcll(mask);
            }
            if (lane == 0) s_nactive = n;
        }
        __syncthreads();
        nactive = s_nactive;
    }

    // ---- this block's contiguous run of work items (active expert, tile)
    const uint32_t tiles_per_expert = (a.expert_rows + kTileRows - 1) / kTileRows;
    const uint32_t total = nactive * tiles_per_expert;
    const uint32_t nblk = gridDim.x / a.ksplit;
    const uint32_t per = (total + nblk - 1) / nblk;
    uint32_t it = (blockIdx.x / a.ksplit) * per;
    const uint32_t end = min(it + per, total);
    if (it >= end) return;

    // weight rows: lanes 0-7 gate, 8-15 up (gate/up tiles); lane r16 otherwise
    const bool up_lane = kGateUp && r16 >= 8;
    const uint32_t *qw_base = up_lane ? a.w2.qw : a.w.qw;
    const uint16_t *sc_base = up_lane ? a.w2.sc : a.w.sc;
    const uint16_t *bi_base = up_lane ? a.w2.bi : a.w.bi;
    const uint32_t kw = K >> 3, kg = K >> 6;

    auto fetch = [&](WTile<L> &B, uint32_t item) {
        const uint32_t j = item / tiles_per_expert, t = item - j * tiles_per_expert;
        const uint32_t e = kGrouped ? s_active[j] : 0;
        uint32_t f = kGateUp ? t * 8 + (r16 & 7) : t * 16 + r16;
        f = f < a.expert_rows ? f : a.expert_rows - 1;  // tail rows re-read a valid row and are never stored
        const size_t row = (size_t)e * a.expert_rows + f;
        const u32x4 *src = reinterpret_cast<const u32x4 *>(qw_base + row * kw + (k_col >> 3));
#pragma unroll
        for (int i = 0; i < kVec; ++i) B.w[i] = ld_stream(src + i);
#pragma unroll
        for (int q = 0; q < kGroups; ++q) {
            B.s[q] = sc_base[row * kg + (k_col >> 6) + q];
            B.b[q] = bi_base[row * kg + (k_col >> 6) + q];
        }
    };

    // ---- X fragments of this lane: token row r16 of a 16-row chunk, columns k_lane .. k_lane + L
    f16x8_t xf[kSlices];
    uint32_t x_key = 0xFFFFFFFFu;
    auto load_x = [&](uint32_t base, uint32_t rows) {
        const bool live = (uint32_t)r16 < rows && k_live;
        const uint32_t p = base + (live ? (uint32_t)r16 : 0u);
        uint32_t xr = p;
        if constexpr (kGrouped) {
            if (a.x_div) xr = a.sorted[p] / a.x_div;
        }
        const uint16_t *xrow = a.x + (size_t)xr * a.ldx + k_col;
        u32x4 raw[kSlices];
#pragma unroll
        for (int s = 0; s < kSlices; ++s) raw[s] = *reinterpret_cast<const u32x4 *>(xrow + 8 * s);
#pragma unroll
        for (int s = 0; s < kSlices; ++s) {
            const u32x4 z = {0, 0, 0, 0};
            xf[s] = x_frag(live ? raw[s] : z);
        }
    };

    auto multiply = [&](const WTile<L> &B) {
        f32x4 acc = {0, 0, 0, 0};
#pragma unroll
        for (int q = 0; q < kGroups; ++q) {
            // zero scale and bias: a dead lane group contributes exact zeros
            const f16x2_t s2 = half2_of_bf16(k_live ? B.s[q] : 0u), b2 = half2_of_bf16(k_live ? B.b[q] : 0u);
#pragma unroll
            for (int s = 0; s < 8; ++s) {  // 8 slices of 8 columns = one group
                const int widx = q * 8 + s;
                acc = __builtin_amdgcn_mfma_f32_16x16x32_f16(
                    xf[widx], w_frag(word_of(B.w[widx / 4], widx % 4), s2, b2, kMask, kMagic), acc, 0, 0, 0);
            }
        }
        return acc;
    };

    // ---- block reduction over the NWAVES K ranges (wave order) and the epilogue of wave 0.
    // Two LDS slots: a slot is rewritten two tiles later, after a barrier that
    // wave 0 reaches only once it has read the slot.
    int slot = 0;
    auto finish = [&](const f32x4 &acc, uint32_t e, uint32_t t, uint32_t base, uint32_t rows) {
        red[slot][wave][lane] = acc;
        __syncthreads();
        if (wave == 0) {
            f32x4 tot = red[slot][0][lane];
#pragma unroll
            for (int w = 1; w < NWAVES; ++w) tot += red[slot][w][lane];
            float up[4] = {0, 0, 0, 0};
            if (kGateUp && !a.partial) {
#pragma unroll
                for (int v = 0; v < 4; ++v) up[v] = __shfl_xor(tot[v], 8);
            }
            const uint32_t f = kGateUp ? t * 8 + (r16 & 7) : t * 16 + r16;
            const bool col_live = f < a.expert_rows && (!kGateUp || a.partial || r16 < 8);
            if (col_live) {
#pragma unroll
                for (int v = 0; v < 4; ++v) {
                    const uint32_t row = 4 * g + v;
                    if (row >= rows) continue;
                    if (a.partial) {  // dense split-K: [ksplit, m, nw * n], gate at f, up at n + f
                        const uint32_t nw = kGateUp ? 2 : 1;
                        float *dst = a.partial + ((size_t)split * a.m + row) * (size_t)(nw * a.expert_rows);
                        dst[(up_lane ? a.expert_rows : 0u) + f] = tot[v];
                        continue;
                    }
                    float val = tot[v];
                    if (kGateUp) val = activation(val, a.act) * up[v];
                    if (a.bias) val += bf16_to_f32(a.bias[(size_t)e * a.expert_rows + f]);
                    uint32_t orow = base + row;
                    if constexpr (kGrouped) {
                        if (a.out_scatter) orow = a.sorted[orow];
                    }
                    const size_t o = (size_t)orow * a.ldo + f;
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
        slot ^= 1;
    };

    // One work item on the words in `cur`, after requesting the next item's
    // words into `nxt`.  The prefetch is unconditional (the last item of a run
    // re-requests its own tile, which L2 still holds) so that the wait for
    // `cur` never has to cover it.
    auto run_item = [&](WTile<L> &cur, WTile<L> &nxt, uint32_t item) {
        const uint32_t j = item / tiles_per_expert, t = item - j * tiles_per_expert;
        uint32_t e = 0, base = 0, cnt = a.m;
        if constexpr (kGrouped) {
            e = s_active[j];
            base = s_base[j];
            cnt = s_cnt[j];
            // X of the first chunk is requested before the next tile's words, so
            // that waiting for X does not wait for the prefetch.
            const uint32_t key = j << 16;
            if (key != x_key) {
                load_x(base, min(cnt, 16u));
                x_key = key;
            }
        }
        fetch(nxt, min(item + 1, end - 1));
        __builtin_amdgcn_sched_barrier(0);  // keep uses of `cur` below the prefetch
        if constexpr (kGrouped) {
            for (uint32_t c0 = 0; c0 < cnt; c0 += 16) {
                if (c0 > 0) {
                    load_x(base + c0, min(cnt - c0, 16u));
                    x_key = (j << 16) | (c0 >> 4);
                }
                const f32x4 acc = multiply(cur);
                finish(acc, e, t, base + c0, min(cnt - c0, 16u));
            }
        } else {  // dense: m <= 16 rows, X loaded once
            const f32x4 acc = multiply(cur);
            finish(acc, e, t, 0, cnt);
        }
    };

    {  // X of the first item, then its weight tile
        const uint32_t j = it / tiles_per_expert;
        if constexpr (kGrouped) {
            load_x(s_base[j], min(s_cnt[j], 16u));
        } else {
            load_x(0, min(a.m, 16u));
        }
        x_key = j << 16;
    }
    WTile<L> A, B;
    fetch(A, it);
    for (;;) {
        run_item(A, B, it);
        if (++it >= end) break;
        run_item(B, A, it);
        if (++it >= end) break;
    }
}

namespace {

struct SkinnyShape {
    int lane_cols;  // L
    int waves;      // NWAVES
};

// Lane columns and waves per block for rows of k columns.  L = 128 needs
// k % 128 == 0 (whole lane groups); the grouped path needs one block to cover k.
SkinnyShape skinny_shape(uint32_t k, bool grouped) {
    int L = tuning().skinny_lane_cols;
    int W = tuning().skinny_waves;
    if (k % (uint32_t)L != 0) L = 64;
    if (grouped) {
        while ((uint32_t)(W * 4 * L) < k && W < 8) W *= 2;
        if ((uint32_t)(W * 4 * L) < k && L == 64 && k % 128 == 0) L = 128;
    }
    return {L, W};
}

uint32_t ksplit_of(uint32_t k, SkinnyShape sh) {
    const uint32_t ranges = (k + 4 * sh.lane_cols - 1) / (4 * sh.lane_cols);
    return (ranges + sh.waves - 1) / sh.waves;
}

template <int L, int NW, bool GU, bool G>
hipError_t launch_t(SkinnyArgs &a, uint32_t items, hipStream_t s) {
    uint32_t nblk = items;
    const uint32_t cap = std::max<uint32_t>(1, (uint32_t)tuning().skinny_max_blocks / a.ksplit);
    if (nblk > cap) nblk = cap;
    hipLaunchKernelGGL((q4_skinny_kernel<L, NW, GU, G>), dim3(nblk * a.ksplit), dim3(NW * 64), 0, s, a);
    return hipGetLastError();
}

template <bool GU, bool G>
hipError_t launch_shape(SkinnyArgs &a, SkinnyShape sh, uint32_t items, hipStream_t s) {
    if (sh.lane_cols == 128)
        return sh.waves == 8 ? launch_t<128, 8, GU, G>(a, items, s) : launch_t<128, 4, GU, G>(a, items, s);
    return sh.waves == 8 ? launch_t<64, 8, GU, G>(a, items, s) : launch_t<64, 4, GU, G>(a, items, s);
}

}  // namespace

hipError_t launch_skinny(SkinnyArgs &a, hipStream_t s) {
    const bool gate_up = a.w2.qw != nullptr;
    const bool grouped = a.offsets != nullptr;
    const SkinnyShape sh = skinny_shape(a.k, grouped);
    a.ksplit = ksplit_of(a.k, sh);
    if (grouped && a.ksplit != 1) return hipErrorInvalidValue;
    if (!grouped) {
        a.experts = 1;
        a.expert_rows = a.w.n;
        a.max_active = 1;
    }
    const uint32_t tile_rows = gate_up ? 8 : 16;
    const uint32_t items = a.max_active * ((a.expert_rows + tile_rows - 1) / tile_rows);
    if (gate_up) return grouped ? launch_shape<true, true>(a, sh, items, s) : launch_shape<true, false>(a, sh, items, s);
    return grouped ? launch_shape<false, true>(a, sh, items, s) : launch_shape<false, false>(a, sh, items, s);
}

uint32_t skinny_ksplit(uint32_t k) { return ksplit_of(k, skinny_shape(k, false)); }

bool skinny_grouped_fits(uint32_t k) { return ksplit_of(k, skinny_shape(k, true)) == 1; }

}  // namespace kr
