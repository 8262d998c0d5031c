// q4_skinny.hip — Q4_G64 matmul for a few tokens per weight tile on the matrix
// cores: batched decode (config 1 B = 4, 16) and the routed MoE experts
// (config 4), where every expert sees only the few tokens routed to it.
// Replaces the reference's small-M path q4_g64_prefill_gemm / _gate_up_gemm
// (kernels/metal/q4_gemm_and_moe.metal:2173-2486) and the routed expert GEMV
// q4_g64_routed_moe_gemv (:2642-2698), which re-reads an expert's weights once
// per routed (token, slot) pair.
//
// Bound: HBM (each weight is read once per launch; 16 tokens give AI <= 57 FLOP/B).
//
// Mapping.  v_mfma_f32_16x16x32_f16 with A = X (16 token rows, zero-padded)
// and B = W^T (16 weight rows).  A wave owns whole weight tiles: 16 rows over
// a K slab of up to NLOAD * 128 columns.  It requests all of a tile's words at
// once (NLOAD dwordx4 per lane) and multiplies them as they arrive.  Load i of
// lane group g = lane / 16 reads the 16 bytes of piece 4 i + g of the row
// (lane l % 16), so one wave instruction reads 64 contiguous bytes of each of
// 16 rows.  Word j of a piece holds columns 32 (4 i + g) + 8 j .. + 7: that
// lane's k-block of MFMA slice (i, j).  The matching X fragment comes from LDS,
// where the block staged the slab's X rows once as fp16 in the order e0 e4 e1
// e5 e2 e6 e3 e7 of every 8 columns (the order the nibble pairs unpack in), in
// 16-byte units XOR-swizzled by row so that the 16 rows of a read hit distinct
// banks.  Scales and biases: lane group g loads the bf16 pairs of groups
// (2 i, 2 i + 1) for i = 4 g .. 4 g + 3, and slice i takes its pair from lane
// group i / 4 by a lane shuffle.
// Dequantisation in registers: nibble pairs (j, j+4) under the fp16 pattern
// 0x6400 -> exact (1024+q) halves, v_pk_add_f16 -1024, v_pk_fma_f16 (s, b).
// Waves work independently after the staging barrier: no per-tile barrier, no
// cross-wave reduction; each lane stores its 4 outputs (rows 4 g + v, column
// l % 16) directly.
// Gate/up: a tile holds 8 gate rows (lanes 0-7) and the same 8 up rows (lanes
// 8-15); the epilogue pairs lane c with lane c + 8.
// K longer than one slab is split over blocks (one slab each) and the f32
// partials are reduced in slab order by q4_mfma_splitk_reduce_kernel.
// Grouped mode (MoE): the weight matrix stacks E experts of expert_rows rows;
// offsets[E+1] and the expert-sorted assignment list select, per expert, the
// token rows to gather (X row = sorted[p] / x_div, or p) and where each result
// row goes (sorted[p], or p).  Work items are (active expert, tile) pairs in
// expert order; a block takes a contiguous run of them and restages X when
// the expert changes.  Experts with more than 16 routed rows are processed in
// 16-row chunks.
#include <algorithm>

#include "kr_internal.hpp"

namespace kr {

namespace {

constexpr int kSkinnyWaves = 8;

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
__device__ __forceinline__ u32x4 x_unit(const u32x4 &v) {
    const uint32_t X[4] = {v.x, v.y, v.z, v.w};
    _Float16 e[8];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        e[2 * i] = (_Float16)__uint_as_float(X[i] << 16);
        e[2 * i + 1] = (_Float16)__uint_as_float(X[i] & 0xFFFF0000u);
    }
    const f16x8_t r = {e[0], e[4], e[1], e[5], e[2], e[6], e[3], e[7]};
    return __builtin_bit_cast(u32x4, r);
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

// (bf16 lo, bf16 hi) -> (fp16 lo, fp16 hi), round to nearest even
__device__ __forceinline__ uint32_t f16_pair_of_bf16_pair(uint32_t p) {
    const f16x2_t h = {(_Float16)__uint_as_float(p << 16), (_Float16)__uint_as_float(p & 0xFFFF0000u)};
    return __builtin_bit_cast(uint32_t, h);
}

__device__ __forceinline__ uint32_t word_of(const u32x4 &v, int i) {
    return i == 0 ? v.x : i == 1 ? v.y : i == 2 ? v.z : v.w;
}

// LDS position of 16-byte X unit u (8 columns) of row r (XOR swizzle by row).
template <int NLOAD>
__device__ __forceinline__ uint32_t xs_index(uint32_t r, uint32_t u) {
    return r * (NLOAD * 16) + (u ^ r);
}

}  // namespace

// NLOAD: dwordx4 loads per lane per tile (slab of NLOAD * 128 columns);
// kGateUp: interleaved gate/up tiles with the activation epilogue;
// kGrouped: MoE expert groups.
template <int NLOAD, bool kGateUp, bool kGrouped>
__global__ __launch_bounds__(kSkinnyWaves * 64) __attribute__((amdgpu_waves_per_eu(4, 4))) void q4_skinny_kernel(
    SkinnyArgs a) {
    constexpr int NW = kSkinnyWaves;
    constexpr uint32_t kTileRows = kGateUp ? 8 : 16;  // output features per tile
    constexpr int kUnits = NLOAD * 16;                // 16-byte X units per LDS row
    constexpr int kStage = 16 * kUnits / (NW * 64);   // X units staged per thread
    __shared__ u32x4 xs[16 * kUnits];                 // X slab: 16 rows x NLOAD*128 fp16

    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int g = lane >> 4, r16 = lane & 15;
    const uint32_t K = a.k;
    const uint32_t slab = blockIdx.x % a.ksplit;
    const uint32_t k0 = slab * (NLOAD * 128u);
    const uint32_t nld = min((uint32_t)NLOAD, (K - k0) >> 7);  // live loads (K % 128 == 0)
    const uint32_t kMask = opq_s(0x000F000Fu);
    const uint32_t kMagic = opq_v(0x64006400u);

    // ---- active experts (grouped mode), held in registers: lane l covers experts l + 64 i
    constexpr int kEPer = kGrouped ? (int)(kMaxExperts / 64) : 1;
    uint32_t e_lo[kEPer], e_cnt[kEPer];
    uint32_t nactive = 1;
    if constexpr (kGrouped) {
        nactive = 0;
#pragma unroll
        for (int i = 0; i < kEPer; ++i) {
            const uint32_t e = lane + 64u * i;
            uint32_t lo = 0, hi = 0;
            if (e < a.experts) {
                lo = a.offsets[e];
                hi = a.offsets[e + 1];
            }
            e_lo[i] = lo;
            e_cnt[i] = hi - lo;
            nactive += (uint32_t)__popcll(__ballot(hi > lo));
        }
    }
    // j-th non-empty bucket -> (expert, base, count); uniform
    auto expert_of = [&](uint32_t j, uint32_t &e, uint32_t &base, uint32_t &cnt) {
        e = 0;
        base = 0;
        cnt = a.m;
        if constexpr (kGrouped) {
#pragma unroll
            for (int i = 0; i < kEPer; ++i) {
                const bool live = e_cnt[i] > 0;
                const uint64_t mask = __ballot(live);
                const uint32_t n = (uint32_t)__popcll(mask);
                if (j < n) {
                    const uint32_t rank = (uint32_t)__popcll(mask & ((1ull << lane) - 1ull));
                    const uint64_t hit = __ballot(live && rank == j);
                    const int src = __builtin_ctzll(hit);
                    e = 64u * i + (uint32_t)src;
                    base = __builtin_amdgcn_readlane(e_lo[i], src);
                    cnt = __builtin_amdgcn_readlane(e_cnt[i], src);
                    return;
                }
                j -= n;
            }
        }
    };

    // ---- this block's contiguous run of work items (active expert, tile)
    const uint32_t tiles_per_expert = (a.expert_rows + kTileRows - 1) / kTileRows;
    const uint32_t total = nactive * tiles_per_expert;
    const uint32_t nblk = gridDim.x / a.ksplit;
    const uint32_t per = (total + nblk - 1) / nblk;
    const uint32_t run_begin = (blockIdx.x / a.ksplit) * per;
    const uint32_t run_end = min(run_begin + per, total);
    if (run_begin >= run_end) return;

    // weight rows: lanes 0-7 gate, 8-15 up (gate/up tiles); lane r16 otherwise
    const bool up_lane = kGateUp && r16 >= 8;
    const uint32_t *qw_base = up_lane ? a.w2.qw : a.w.qw;
    const uint16_t *sc_base = up_lane ? a.w2.sc : a.w.sc;
    const uint16_t *bi_base = up_lane ? a.w2.bi : a.w.bi;
    const uint32_t kw = K >> 3, kg = K >> 6;

    u32x4 wv[NLOAD];
    uint32_t sp[4], bp[4];
    // Words of tile t of expert e.  Loads past the slab (i >= nld) re-read a
    // live piece and are never multiplied; issuing them keeps every wait on
    // the words independent of the slab width.
    auto fetch = [&](uint32_t e, uint32_t t) {
        uint32_t f = kGateUp ? t * 8 + (r16 & 7) : t * 16 + r16;
        f = f < a.expert_rows ? f : a.expert_rows - 1;  // tail rows re-read a valid row and are never stored
        const size_t row = (size_t)e * a.expert_rows + f;
        // scales first: their shuffles then never wait for the words
        // bf16 pairs (groups 2i, 2i+1) for i = 4g .. 4g+3; 4-byte aligned (kg even, scales 4-byte aligned)
        const uint32_t *s32 = reinterpret_cast<const uint32_t *>(sc_base + row * kg + (k0 >> 6));
        const uint32_t *b32 = reinterpret_cast<const uint32_t *>(bi_base + row * kg + (k0 >> 6));
#pragma unroll
        for (int q = 0; q < 4; ++q) {
            uint32_t i = 4u * (uint32_t)g + (uint32_t)q;
            i = i < nld ? i : nld - 1;
            sp[q] = s32[i];
            bp[q] = b32[i];
        }
        const u32x4 *src = reinterpret_cast<const u32x4 *>(qw_base + row * kw + (k0 >> 3));
#pragma unroll
        for (int i = 0; i < NLOAD; ++i) {
            const uint32_t ii = (uint32_t)i < nld ? (uint32_t)i : nld - 1;
            wv[i] = ld_stream(src + 4 * ii + g);
        }
    };

    // X rows [base, base + rows) of the slab -> LDS (zeros beyond `rows` and beyond the slab).
    // All loads are issued before the first conversion.
    auto stage_x = [&](uint32_t base, uint32_t rows) {
        uint32_t tid_v = (uint32_t)tid;
        asm volatile("" : "+v"(tid_v));  // recompute the staging addresses here rather than keep them live
        // Loads are unconditional (dead units re-read row `base`, unit 0) and
        // zeroed after, so that no branch splits the batch of loads.
        u32x4 raw[kStage];
#pragma unroll
        for (int s = 0; s < kStage; ++s) {
            const uint32_t idx = tid_v + (uint32_t)s * (NW * 64);
            const uint32_t r = idx / kUnits, u = idx % kUnits;
            const bool live = r < rows && u < nld * 16;
            uint32_t xr = base + (live ? r : 0u);
            if constexpr (kGrouped) {
                if (a.x_div) xr = a.sorted[xr] / a.x_div;
            }
            raw[s] = *reinterpret_cast<const u32x4 *>(a.x + (size_t)xr * a.ldx + k0 + 8 * (live ? u : 0u));
        }
#pragma unroll
        for (int s = 0; s < kStage; ++s) {
            const uint32_t idx = tid_v + (uint32_t)s * (NW * 64);
            const uint32_t r = idx / kUnits, u = idx % kUnits;
            const bool live = r < rows && u < nld * 16;
            const u32x4 z = {0, 0, 0, 0};
            xs[xs_index<NLOAD>(r, u)] = x_unit(live ? raw[s] : z);
        }
    };

    // X fragment of MFMA slice s = 4 i + j for this lane: unit 16 i + 4 g + j of
    // row r16, i.e. (swizzle) r16 * kUnits + 16 i + ((4 g + j) ^ r16): one base
    // per j, and i as an immediate offset.
    uint32_t xbase[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) xbase[j] = (uint32_t)r16 * kUnits + ((4u * (uint32_t)g + (uint32_t)j) ^ (uint32_t)r16);
    // LDS byte addresses of the four bases (the low 32 bits of a generic LDS
    // pointer are its LDS offset).  The reads are issued from inline asm that
    // waits for them: the compiler cannot hoist all 64 of a tile's reads ahead
    // of the MFMAs and run out of registers; other waves hide the latency.
    uint32_t xaddr[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) xaddr[j] = (uint32_t)reinterpret_cast<uintptr_t>(&xs[xbase[j]]);
    // The four X fragments of piece i (slices 4i .. 4i+3) in one batch: four
    // reads in flight, one wait.
    auto xread4 = [&](int i, f16x8_t (&x)[4]) {
        u32x4 v0, v1, v2, v3;
        asm volatile(
            "ds_read_b128 %0, %4 offset:%8\n\t"
            "ds_read_b128 %1, %5 offset:%8\n\t"
            "ds_read_b128 %2, %6 offset:%8\n\t"
            "ds_read_b128 %3, %7 offset:%8\n\t"
            "s_waitcnt lgkmcnt(0)"
            : "=&v"(v0), "=&v"(v1), "=&v"(v2), "=&v"(v3)
            : "v"(xaddr[0]), "v"(xaddr[1]), "v"(xaddr[2]), "v"(xaddr[3]), "i"(256 * i)
            : "memory");
        x[0] = __builtin_bit_cast(f16x8_t, v0);
        x[1] = __builtin_bit_cast(f16x8_t, v1);
        x[2] = __builtin_bit_cast(f16x8_t, v2);
        x[3] = __builtin_bit_cast(f16x8_t, v3);
    };

    auto tile = [&](uint32_t e, uint32_t t, uint32_t base, uint32_t rows) {
        constexpr int kSlices = NLOAD * 4;
        f32x4 acc = {0, 0, 0, 0};
        // this lane's bf16 scale/bias pairs (groups 2i, 2i+1 of i = 4g + q) as fp16
        // pairs; pairs past the slab (i >= nld) become zero, so that those pieces,
        // which are multiplied too, add exact zeros against zero X (a branch here
        // would let the compiler sink each piece's load down to its use)
        uint32_t sh[4], bh[4];
#pragma unroll
        for (int q = 0; q < 4; ++q) {
            const bool live = 4u * (uint32_t)g + (uint32_t)q < nld;
            sh[q] = live ? f16_pair_of_bf16_pair(sp[q]) : 0u;
            bh[q] = live ? f16_pair_of_bf16_pair(bp[q]) : 0u;
        }
        // v_perm selector broadcasting this lane's half (group 2i + g/2) of the
        // second operand to both halves (selector bytes 0-3 pick that operand's bytes)
        const uint32_t half_sel = (g >> 1) ? 0x03020302u : 0x01000100u;
        f16x2_t s2 = {}, b2 = {};
        f16x8_t xp[4];
#pragma unroll
        for (int s = 0; s < kSlices; ++s) {
            const int i = s / 4, j = s % 4;
            if (j == 0) xread4(i, xp);
            if (j == 0) {  // the pairs of piece i live in lane group i / 4
                const int src = 16 * (i / 4) + r16;
                const uint32_t spair = __shfl(sh[i % 4], src);
                const uint32_t bpair = __shfl(bh[i % 4], src);
                s2 = __builtin_bit_cast(f16x2_t, __builtin_amdgcn_perm(0u, spair, half_sel));
                b2 = __builtin_bit_cast(f16x2_t, __builtin_amdgcn_perm(0u, bpair, half_sel));
            }
            acc = __builtin_amdgcn_mfma_f32_16x16x32_f16(xp[j], w_frag(word_of(wv[i], j), s2, b2, kMask, kMagic), acc,
                                                         0, 0, 0);
        }
        // ---- epilogue: lane holds rows 4g + v of column r16
        float up[4] = {0, 0, 0, 0};
        if (kGateUp && !a.partial) {
#pragma unroll
            for (int v = 0; v < 4; ++v) up[v] = __shfl_xor(acc[v], 8);
        }
        const uint32_t f = kGateUp ? t * 8 + (r16 & 7) : t * 16 + r16;
        const bool col_live = f < a.expert_rows && (!kGateUp || a.partial || r16 < 8);
        if (!col_live) return;
#pragma unroll
        for (int v = 0; v < 4; ++v) {
            const uint32_t row = 4 * g + v;
            if (row >= rows) continue;
            if (a.partial) {  // dense split-K: [ksplit, m, nw * n], gate at f, up at n + f
                const uint32_t nw = kGateUp ? 2 : 1;
                float *dst = a.partial + ((size_t)slab * a.m + row) * (size_t)(nw * a.expert_rows);
                dst[(up_lane ? a.expert_rows : 0u) + f] = acc[v];
                continue;
            }
            float val = acc[v];
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
    };

    // X is staged before the first tile is requested: holding a tile's words
    // through the staging spills registers, which costs more than the overlap
    // would save.
    if constexpr (!kGrouped) {  // dense: one X for the whole run
        stage_x(0, min(a.m, 16u));
        __syncthreads();
        for (uint32_t t = run_begin + (uint32_t)wave; t < run_end; t += NW) {
            fetch(0, t);
            tile(0, t, 0, a.m);
        }
        return;
    }

    // ---- grouped: segments of the run that share an expert
    uint32_t item = run_begin;
    while (item < run_end) {
        const uint32_t j = item / tiles_per_expert;
        const uint32_t seg_end = min(run_end, (j + 1) * tiles_per_expert);
        uint32_t e, base, cnt;
        expert_of(j, e, base, cnt);
        for (uint32_t c0 = 0; c0 < cnt; c0 += 16) {
            const uint32_t rows = min(cnt - c0, 16u);
            __syncthreads();  // the previous segment's readers are done with xs
            stage_x(base + c0, rows);
            __syncthreads();
            for (uint32_t my = item + (uint32_t)wave; my < seg_end; my += NW) {
                const uint32_t t = my - j * tiles_per_expert;
                fetch(e, t);
                tile(e, t, base + c0, rows);
            }
        }
        item = seg_end;
    }
}

namespace {

template <int NLOAD, bool GU, bool G>
hipError_t launch_t(SkinnyArgs &a, uint32_t items, hipStream_t s) {
    // blocks per slab: every CU busy, each block a contiguous run of ceil(items / nblk) tiles
    const uint32_t cap = std::max<uint32_t>(1, (uint32_t)tuning().skinny_max_blocks / a.ksplit);
    const uint32_t nblk = std::max<uint32_t>(1, std::min(items, cap));
    const dim3 grid(nblk * a.ksplit), block(kSkinnyWaves * 64);
    hipLaunchKernelGGL((q4_skinny_kernel<NLOAD, GU, G>), grid, block, 0, s, a);
    return hipGetLastError();
}

template <bool GU, bool G>
hipError_t launch_nload(SkinnyArgs &a, int nload, uint32_t items, hipStream_t s) {
    switch (nload) {
        case 4: return launch_t<4, GU, G>(a, items, s);
        case 8: return launch_t<8, GU, G>(a, items, s);
        case 12: return launch_t<12, GU, G>(a, items, s);
        default: return launch_t<16, GU, G>(a, items, s);
    }
}

// Slab width in loads (128 columns each): the smallest instantiated width that
// covers k, else 16 (2048 columns) with K split over blocks.
int slab_loads(uint32_t k) {
    const uint32_t need = k / 128;
    for (int n : {4, 8, 12, 16})
        if (need <= (uint32_t)n) return n;
    return 16;
}

}  // namespace

bool skinny_supported(const Q4Mat &w) {
    return w.k % 128 == 0 && (uintptr_t)w.sc % 4 == 0 && (uintptr_t)w.bi % 4 == 0;
}

hipError_t launch_skinny(SkinnyArgs &a, hipStream_t s) {
    const bool gate_up = a.w2.qw != nullptr;
    if (!skinny_supported(a.w) || (gate_up && !skinny_supported(a.w2))) return hipErrorInvalidValue;
    const bool grouped = a.offsets != nullptr;
    const int nload = slab_loads(a.k);
    a.ksplit = (a.k + nload * 128 - 1) / (nload * 128);
    if (grouped && a.ksplit != 1) return hipErrorInvalidValue;
    if (!grouped) {
        a.experts = 1;
        a.expert_rows = a.w.n;
        a.max_active = 1;
    }
    const uint32_t tile_rows = gate_up ? 8 : 16;
    const uint32_t items = a.max_active * ((a.expert_rows + tile_rows - 1) / tile_rows);
    if (gate_up)
        return grouped ? launch_nload<true, true>(a, nload, items, s) : launch_nload<true, false>(a, nload, items, s);
    return grouped ? launch_nload<false, true>(a, nload, items, s) : launch_nload<false, false>(a, nload, items, s);
}

uint32_t skinny_ksplit(uint32_t k) {
    const int nload = slab_loads(k);
    return (k + nload * 128 - 1) / (nload * 128);
}

bool skinny_grouped_fits(uint32_t k) { return k % 128 == 0 && skinny_ksplit(k) == 1; }

}  // namespace kr
