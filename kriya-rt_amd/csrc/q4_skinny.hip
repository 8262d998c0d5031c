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
// Mapping.  v_mfma_f32_16x16x32_bf16 with A = X (16 token rows, zero-padded)
// and B = the exact integers 128 + q (16 weight rows); the affine map of each
// 64-column group is applied to the f32 results, as the GEMV does:
//   sum_c x_c (s q_c + b) = s * D + (b - 128 s) * S,  D = sum_c x_c (128 + q_c),  S = sum_c x_c
// (the reference's distributive block dot, q4_gemm_and_moe.metal:414-473).  Both
// products are exact in bf16 (bf16 x, integers below 256) and sum in f32, so x
// keeps its full bf16 range: there is no fp16 conversion of x or of w.  S comes
// from the same X fragments times a fragment of ones on the matrix cores.
// A block takes a tile of 16 weight rows over a K slab of 2048 columns; wave w
// multiplies the slab's 128-column pieces 2w, 2w + 1 and the 8 waves' 16 x 16
// partial tiles are summed through LDS in wave order (fixed order: results do
// not depend on timing).  The next tile's words are requested before the
// current tile is multiplied (two register buffers), and the epilogue's
// operands (bias, old output) with them, so that no wait on them also waits for
// the prefetch in flight.  Barriers are LDS-only (s_barrier after an lgkmcnt
// wait): a fenced barrier would wait for the prefetch.
// Loads: lane (r16, g) reads 16 bytes of piece p of row r16 (columns 128 p +
// 32 g .. + 31), so one wave instruction reads 64 contiguous bytes of each of
// 16 rows: lanes 0-31 hold group 2p, lanes 32-63 group 2p + 1.  Words 2q and
// 2q + 1 are swapped across the lane halves (v_permlane32_swap), after which
// one register holds group 2p in every lane and the other group 2p + 1: each
// matrix instruction contracts within one group.  The matching X fragments
// come from LDS, where the block staged the slab's X rows once, bf16, in the
// order e0 e4 e1 e5 e2 e6 e3 e7 of every 8 columns (the order the nibble pairs
// unpack in), in 16-byte units XOR-swizzled by row so that the 16 rows of a read
// hit distinct banks.
// Scales and biases: every lane loads the bf16 pair (groups 2p, 2p + 1) of its
// row and piece; the results of lane (r16, .) belong to weight row r16.
// Unpacking: nibble pairs (j, j + 4) of a word under the bf16 pattern 0x4300
// -> the exact values (128 + q_j, 128 + q_{j+4}), one v_and_or_b32 each.
// Gate/up: a tile holds 8 gate rows (lanes 0-7) and the same 8 up rows (lanes
// 8-15); the epilogue pairs column c with column c + 8.
// K longer than one slab is split over blocks (one slab each) and the f32
// partials are reduced in slab order, by the last block of each run (tickets)
// or by a second launch (launch_splitk_reduce).
// Grouped mode (MoE): the weight matrix stacks E experts of expert_rows rows;
// offsets[E+1] and the expert-sorted assignment list select, per expert, the
// token rows to gather (X row = sorted[p] / x_div, or p) and where each result
// row goes (sorted[p], or p).  Work items are (active expert, tile) pairs in
// expert order; a block takes a contiguous run of them and restages X when
// the expert changes.  Experts with more than 16 routed rows are processed in
// 16-row chunks.
#include <algorithm>
#include <type_traits>

#include "kr_internal.hpp"

namespace kr {

namespace {

constexpr int kSkinnyWaves = 8;
constexpr int kSkinnyPieces = 2;                                // 128-column pieces per wave
constexpr int kSlabCols = kSkinnyWaves * kSkinnyPieces * 128;  // K columns per block

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

// 8 bf16 x values (4 u32 words, element order) -> the same 8 bf16 in the order e0 e4 e1 e5 e2 e6 e3 e7.
__device__ __forceinline__ u32x4 x_unit(const u32x4 &v) {
    return u32x4{__builtin_amdgcn_perm(v.z, v.x, 0x05040100u), __builtin_amdgcn_perm(v.z, v.x, 0x07060302u),
                 __builtin_amdgcn_perm(v.w, v.y, 0x05040100u), __builtin_amdgcn_perm(v.w, v.y, 0x07060302u)};
}

// one word of 8 nibbles -> B fragment (128 + q) in the order (w0 w4 w1 w5 w2 w6 w3 w7), bf16
__device__ __forceinline__ bf16x8_t q_frag(uint32_t w, uint32_t mask, uint32_t magic) {
    const u32x4 r = {(w & mask) | magic, ((w >> 4) & mask) | magic, ((w >> 8) & mask) | magic,
                     ((w >> 12) & mask) | magic};
    return __builtin_bit_cast(bf16x8_t, r);
}

// XOR swizzle of row r's 16-byte units: the 16 rows of a fragment read hit distinct banks
// (r & 15 alone measured 35-42 % bank-conflict cycles for these reads; this order, none).
__device__ __forceinline__ uint32_t xs_swz(uint32_t r) { return ((r & 7u) << 1) | ((r >> 3) & 1u); }

// LDS position of 16-byte X unit u (8 columns) of row r (r < 16).
template <int kUnits>
__device__ __forceinline__ uint32_t xs_index(uint32_t r, uint32_t u) {
    return r * kUnits + (u ^ xs_swz(r));
}

}  // namespace

// A block takes a tile of 16 weight rows (gate/up: 8 gate + the same 8 up
// rows) over a K slab of kSlabCols columns; wave w multiplies the slab's
// 128-column pieces w * kPieces .. + kPieces - 1 and the 8 waves' 16 x 16
// partial products are summed through LDS in wave order.
// kGateUp: interleaved gate/up tiles with the activation epilogue;
// kGrouped: MoE expert groups;
// MG: groups of 16 token rows per launch (dense mode: 1 or 2).  With two, every unpacked weight
// word is multiplied with both groups' X fragments (32 rows for the price of little more than 16);
// kPre: the epilogue reads a bias or the old output (dense mode, no split-K partials).  Launches
// without either issue no such loads: the memory instructions per tile, not their bytes, set this
// kernel's pace (measured: two dummy loads per tile cost 0.7 us of 13.8 at cfg1 B = 16 gate/up).
// D: register buffers of tile words, i.e. D - 1 tiles in flight while one is multiplied (2, or 3
// for dense runs of at least 6 tiles: the launcher's choice).
// kOdd: K is an odd number of 64-groups (K % 128 == 64; dense mode): the last piece of the last slab
// holds one group.  Its other half re-reads the live half's words (in the row, never past it), meets
// zero X and a zero scale and bias, and the scale/bias pairs come in two 2-byte loads (a row's pairs
// are not 4-byte aligned when K / 64 is odd).
template <bool kGateUp, bool kGrouped, int MG, bool kPre, int D, bool kOdd>
__global__ __launch_bounds__(kSkinnyWaves * 64) __attribute__((amdgpu_waves_per_eu(kGrouped ? 4 : 2))) void q4_skinny_kernel(
    SkinnyArgs a) {
    static_assert(MG == 1 || (MG == 2 && !kGrouped), "two row groups in dense mode only");
    static_assert(!(kOdd && kGrouped), "odd group counts in dense mode only");
    static_assert(!(kPre && (kGrouped || kGateUp)), "bias and accumulation: dense plain tiles only");
    static_assert(D == 2 || (D == 3 && !kGrouped), "a deeper ring in dense mode only");
    static_assert(!kPre || D == 2, "epilogue operands with one tile in flight only");
    constexpr int NW = kSkinnyWaves;
    constexpr int KW = kSkinnyPieces;                  // 128-column pieces per wave
    constexpr uint32_t kTileRows = kGateUp ? 8 : 16;  // output features per tile
    constexpr int kUnits = NW * KW * 16;               // 16-byte X units per LDS row
    constexpr int kStage = 16 * kUnits / (NW * 64);    // X units staged per thread
    __shared__ u32x4 xs[16 * kUnits];                  // X slab: 16 rows x kSlabCols bf16
    __shared__ float red[2][MG][NW][4][64];            // per-wave partial tiles, double buffered

    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int g = lane >> 4, r16 = lane & 15;
    const uint32_t K = a.k;
    const uint32_t slab = blockIdx.x % a.ksplit;
    const uint32_t k0 = slab * (uint32_t)kSlabCols;
    // live pieces of the slab (the last one half when K % 128 == 64) and live 8-column X units
    const uint32_t npieces = min((uint32_t)(NW * KW), (K - k0 + 127) >> 7);
    const uint32_t kunits = min((uint32_t)(NW * KW * 16), (K - k0) >> 3);
    const uint32_t p0 = (uint32_t)wave * KW;                           // this wave's first piece
    const uint32_t kMask = opq_s(0x000F000Fu);
    const uint32_t kMagic = opq_v(0x43004300u);  // bf16 128.0 in both halves

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

    // ---- this block's contiguous run of work items (active expert, tile); dense mode: the
    // tiles of the problems one after the other
    const uint32_t tiles_per_expert = (a.expert_rows + kTileRows - 1) / kTileRows;
    const uint32_t total = kGrouped ? nactive * tiles_per_expert : a.tile_begin[a.nmore + 1];
    const uint32_t nblk = gridDim.x / a.ksplit;
    const uint32_t per = (total + nblk - 1) / nblk;
    const uint32_t run_begin = (blockIdx.x / a.ksplit) * per;
    const uint32_t run_end = min(run_begin + per, total);
    if (run_begin >= run_end) return;

    // The current problem (dense mode: one of up to three sharing x; its fields
    // are selected by value, uniform).  Weight rows: lanes 0-7 gate, 8-15 up
    // (gate/up tiles); lane r16 otherwise.
    Q4Mat cw = a.w, cw2 = a.w2;
    void *cout = a.out;
    const uint16_t *cbias = a.bias;
    uint32_t cldo = a.ldo, crows = a.expert_rows;
    const bool up_lane = kGateUp && r16 >= 8;
    const uint32_t kw = K >> 3, kg = K >> 6;

    // Tile words, double buffered (the buffer index is a compile-time
    // constant: a run-time index into register arrays becomes moves and
    // waits).  Pieces past the slab re-read the last live piece and are
    // multiplied with zero scales and zero X, so that every wait on the words
    // is independent of the slab width.
    // The epilogue's operands (bias, old output) of the tile are requested
    // with its words, so that the epilogue never waits for the next tile's
    // words in flight.
    using B0 = std::integral_constant<int, 0>;
    using B1 = std::integral_constant<int, 1>;
    u32x4 wv[D][KW];
    static_assert(KW == 2, "one scale/bias load per lane covers two pieces");
    uint32_t sb[D];  // the lane's scale or bias word (see fetch_words)
    // The epilogue's operands as raw bits (a bf16 in the low half, or an f32), converted at use.
    // Only launches with one tile in flight have them (kPre implies D = 2).
    uint32_t pre_b[D] = {}, pre_o[D] = {};
    // epilogue output (token row erow, column ecol) of threads < 256 MG: row group tid / 256; the 64
    // threads of a wave read one v row of the reduction buffer (64 consecutive floats: no bank
    // conflicts)
    const uint32_t erow = 16u * ((uint32_t)tid >> 8) + 4u * (((uint32_t)tid >> 4) & 3u) + (((uint32_t)tid >> 6) & 3u),
                   ecol = (uint32_t)tid & 15u;
    uint32_t orow = 0;                                                      // its output row (per segment)
    bool eout = false;                                                      // it stores an output
    // The epilogue's operands of tile t (dense mode; grouped launches have no bias and do not
    // accumulate): loads of exactly the element, unconditional (threads without an operand read
    // x[0], or the first weight word for an f32), so that no branch on the thread makes the
    // compiler wait for them before its join.  The old output is an f32 or a bf16 load under a
    // launch-uniform branch, one load either way.
    auto fetch_pre = [&](auto BUF, uint32_t e, uint32_t t) {
        constexpr int b = decltype(BUF)::value;
        const uint32_t ef = kGateUp ? t * 8 + (ecol & 7) : t * 16 + ecol;
        const bool ok = eout && ef < crows;
        pre_b[b] = *((cbias && ok) ? cbias + (size_t)e * crows + ef : a.x);
        const size_t o = (size_t)orow * cldo + ef;
        const bool acc_ok = a.accumulate && ok;
        if (a.out_f32)
            pre_o[b] = *(acc_ok ? reinterpret_cast<const uint32_t *>(cout) + o : cw.qw);
        else
            pre_o[b] = *(acc_ok ? reinterpret_cast<const uint16_t *>(cout) + o : a.x);
    };
    // The words (and scale/bias pairs) of tile t.
    auto fetch_words = [&](auto BUF, uint32_t e, uint32_t t) {
        constexpr int b = decltype(BUF)::value;
        const uint32_t *qw_base = up_lane ? cw2.qw : cw.qw;
        const uint16_t *sc_base = up_lane ? cw2.sc : cw.sc;
        const uint16_t *bi_base = up_lane ? cw2.bi : cw.bi;
        uint32_t f = kGateUp ? t * 8 + (r16 & 7) : t * 16 + r16;
        f = f < crows ? f : crows - 1;  // tail rows re-read a valid row and are never stored
        const size_t row = (size_t)e * crows + f;
        const u32x4 *src = reinterpret_cast<const u32x4 *>(qw_base + row * kw + (k0 >> 3));
#pragma unroll
        for (int i = 0; i < KW; ++i) {
            uint32_t p = p0 + (uint32_t)i;
            p = p < npieces ? p : npieces - 1;
            uint32_t gw = (uint32_t)g;
            if constexpr (kOdd) {  // the half piece: lane groups 2, 3 re-read groups 0, 1 of it
                if (k0 + 128u * p + 32u * gw >= K) gw -= 2u;
            }
            wv[b][i] = ld_stream(src + 4 * p + gw);
        }
        // The scales and biases of the wave's two pieces in one load: lane group g reads the bf16
        // pair (groups 2p, 2p + 1) of piece p = p0 + (g >> 1), scales for even g, biases for odd g
        // (4-byte aligned: kg even, scales and biases 4-byte aligned); tile_mma spreads them.
        {
            uint32_t p = p0 + ((uint32_t)g >> 1);
            p = p < npieces ? p : npieces - 1;
            const uint16_t *base = ((uint32_t)g & 1u) ? bi_base : sc_base;
            if constexpr (kOdd) {  // groups 2p, 2p + 1 (clamped to the row's last; tile_mma masks it)
                const uint16_t *rg = base + row * kg;
                const uint32_t i0 = (k0 >> 6) + 2u * p, i1 = min(i0 + 1u, kg - 1u);
                sb[b] = (uint32_t)rg[i0] | ((uint32_t)rg[i1] << 16);
            } else {
                sb[b] = reinterpret_cast<const uint32_t *>(base + row * kg + (k0 >> 6))[p];
            }
        }
    };
    // The epilogue's operands (when the launch has any) are requested first: loads complete in
    // issue order, so a wait for them (an epilogue, or a register copy the compiler places at the
    // loop's back edge) then does not also wait for the tile's words (measured: MLP at B = 16
    // 27.5 -> 26.8 us).
    auto fetch = [&](auto BUF, uint32_t e, uint32_t t) {
        if constexpr (kPre) fetch_pre(BUF, e, t);
        fetch_words(BUF, e, t);
    };

    // X rows [base, base + rows) of the slab -> LDS (zeros beyond `rows` and
    // beyond the slab), in two halves: the loads, then (after the caller has
    // requested the first tile's words) the conversion and LDS stores.
    // Loads are unconditional (dead units re-read row `base`, unit 0) and
    // zeroed after, so that no branch splits the batch of loads.
    // Unit s of a thread: row 2 wave + s / 4, column block lane + 64 (s % 4) -- a wave holds two whole
    // rows, so the RMSNorm below needs no other wave.
    static_assert(kStage == 8 && kUnits == 4 * 64 && NW * 2 == 16, "two 256-unit rows per wave");
    auto unit_of = [&](int s, uint32_t &r, uint32_t &u) {
        r = 2u * (uint32_t)wave + ((uint32_t)s >> 2);
        u = (uint32_t)lane + 64u * ((uint32_t)s & 3u);
    };
    u32x4 raw[MG][kStage];  // [row group]
    auto stage_load = [&](u32x4(&rw)[kStage], uint32_t base, uint32_t rows) {
#pragma unroll
        for (int s = 0; s < kStage; ++s) {
            uint32_t r, u;
            unit_of(s, r, u);
            const bool live = r < rows && u < kunits;
            uint32_t xr = base + (live ? r : 0u);
            if constexpr (kGrouped) {
                if (a.x_div) xr = a.sorted[xr] / a.x_div;
            }
            rw[s] = *reinterpret_cast<const u32x4 *>(a.x + (size_t)xr * a.ldx + k0 + 8 * (live ? u : 0u));
        }
    };
    auto stage_store = [&](const u32x4(&rw)[kStage], uint32_t rows) {
#pragma unroll
        for (int s = 0; s < kStage; ++s) {
            uint32_t r, u;
            unit_of(s, r, u);
            const bool live = r < rows && u < kunits;
            const u32x4 z = {0, 0, 0, 0};
            xs[xs_index<kUnits>(r, u)] = x_unit(live ? rw[s] : z);
        }
    };

    // LDS-only barrier: the weight prefetch stays in flight across it (a
    // barrier with a memory fence would wait for every outstanding load).
    auto lds_barrier = [] { asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory"); };
    // RMSNorm of the staged rows (dense mode, the whole row in this slab), kr_rmsnorm's arithmetic and
    // order: per 8-column unit a sequential sum of squares, per 64 units (lanes) the wave tree, the four
    // quarters of the row added in order; then bf16(x * (1 / sqrt(mean + eps)) * w).  The wave holds its
    // two rows whole, so every lane forms the scales itself: no LDS, no barrier.
    auto norm_x = [&](u32x4(&rw)[kStage], uint32_t rows) {
        u32x4 wl[4];
#pragma unroll
        for (int q = 0; q < 4; ++q) {
            const uint32_t u = (uint32_t)lane + 64u * (uint32_t)q;
            wl[q] = *reinterpret_cast<const u32x4 *>(a.ln_w + k0 + 8 * (u < kunits ? u : 0u));
        }
        float scale[2];
#pragma unroll
        for (int h = 0; h < 2; ++h) {
            float tot = 0.0f;
#pragma unroll
            for (int q = 0; q < 4; ++q) {
                uint32_t r, u;
                unit_of(4 * h + q, r, u);
                float ss = 0.0f;
                if (u < kunits && r < rows) {
                    const u32x4 v = rw[4 * h + q];
                    const uint32_t X[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
                    for (int i = 0; i < 4; ++i) {
                        const float lo = __uint_as_float(X[i] << 16), hi = __uint_as_float(X[i] & 0xFFFF0000u);
                        ss = fmaf(lo, lo, ss);
                        ss = fmaf(hi, hi, ss);
                    }
                }
                ss = wave_total(ss, lane);
                tot = q == 0 ? ss : tot + ss;
            }
            scale[h] = 1.0f / sqrtf(tot / (float)K + a.eps);
        }
#pragma unroll
        for (int st = 0; st < kStage; ++st) {
            const float sc = scale[st >> 2];
            const u32x4 wq = wl[st & 3];
            const uint32_t W[4] = {wq.x, wq.y, wq.z, wq.w};
            uint32_t X[4] = {rw[st].x, rw[st].y, rw[st].z, rw[st].w};
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const float lo = __uint_as_float(X[i] << 16) * sc * __uint_as_float(W[i] << 16);
                const float hi = __uint_as_float(X[i] & 0xFFFF0000u) * sc * __uint_as_float(W[i] & 0xFFFF0000u);
                X[i] = pack_bf16_rne(lo, hi);
            }
            rw[st] = u32x4{X[0], X[1], X[2], X[3]};
        }
    };

    // X fragments of piece i for its four matrix instructions (h = group 2p + h, q = words 2q, 2q + 1):
    // lane group g reads unit 16 (p0 + i) + 4 (g & 1) + (g >> 1) + 2 q + 8 h of row r16, i.e.
    // (swizzle) r16 * kUnits + 16 (p0 + i) + (unit ^ xs_swz(r16)): one base per (h, q), and i as an immediate
    // offset.  The low 32 bits of a generic LDS pointer are its LDS offset.
    uint32_t xaddr[4];  // [2 h + q]
#pragma unroll
    for (uint32_t hq = 0; hq < 4; ++hq) {
        const uint32_t unit = 4u * ((uint32_t)g & 1u) + ((uint32_t)g >> 1) + 2u * (hq & 1u) + 8u * (hq >> 1);
        xaddr[hq] = (uint32_t)reinterpret_cast<uintptr_t>(&xs[(uint32_t)r16 * kUnits + 16u * p0 + (unit ^ xs_swz(r16))]);
    }
    // The two X fragments of group 2p + h of piece i: two reads in flight, one wait.
    auto xread2 = [&](int i, int h, bf16x8_t (&x)[2]) {
        u32x4 v0, v1;
        asm volatile(
            "ds_read_b128 %0, %2 offset:%4\n\t"
            "ds_read_b128 %1, %3 offset:%4\n\t"
            "s_waitcnt lgkmcnt(0)"
            : "=&v"(v0), "=&v"(v1)
            : "v"(xaddr[2 * h]), "v"(xaddr[2 * h + 1]), "i"(256 * i)
            : "memory");
        x[0] = __builtin_bit_cast(bf16x8_t, v0);
        x[1] = __builtin_bit_cast(bf16x8_t, v1);
    };

    const bf16x8_t ones = __builtin_bit_cast(bf16x8_t, u32x4{0x3F803F80u, 0x3F803F80u, 0x3F803F80u, 0x3F803F80u});
    // Dense mode: the wave's X fragments do not change between the tiles of the run, so they are
    // read from LDS once, with their group sums S (the same X fragments times a fragment of ones):
    // 48 more registers (2 waves per SIMD), cfg1 B = 16 MLP 26.4 -> 24.9 us.  Grouped mode stages X
    // per expert and keeps 4 waves per SIMD: it reads them per tile (119 against 129 us at T = 64).
    constexpr bool kXRegs = !kGrouped;
    bf16x8_t xf[MG][KW][2][2];
    f32x4 xsum[MG][KW][2];
    auto load_x_frags = [&](auto GI) {  // into row group GI's registers
        constexpr int gi = decltype(GI)::value;
        const f32x4 zero = {0, 0, 0, 0};
#pragma unroll
        for (int i = 0; i < KW; ++i)
#pragma unroll
            for (int h = 0; h < 2; ++h) {
                xread2(i, h, xf[gi][i][h]);
                f32x4 sx = __builtin_amdgcn_mfma_f32_16x16x32_bf16(xf[gi][i][h][0], ones, zero, 0, 0, 0);
                xsum[gi][i][h] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(xf[gi][i][h][1], ones, sx, 0, 0, 0);
            }
    };
    struct Acc {
        f32x4 v[MG];
    };
    auto tile_mma = [&](auto BUF) -> Acc {
        constexpr int b = decltype(BUF)::value;
        Acc acc;
#pragma unroll
        for (int gi = 0; gi < MG; ++gi) acc.v[gi] = f32x4{0, 0, 0, 0};
        const f32x4 zero = {0, 0, 0, 0};
        // scale (even rows of lanes) and bias (odd rows) words, each then from lanes 0-31 (piece
        // p0) and lanes 32-63 (piece p0 + 1) in every lane
        const auto sbp = __builtin_amdgcn_permlane16_swap(sb[b], sb[b], false, false);
        const auto spp = __builtin_amdgcn_permlane32_swap(sbp[0], sbp[0], false, false);
        const auto bpp = __builtin_amdgcn_permlane32_swap(sbp[1], sbp[1], false, false);
#pragma unroll
        for (int i = 0; i < KW; ++i) {
            // past the slab: the re-read words meet zero X; zero scales keep the products at 0
            const bool live = p0 + (uint32_t)i < npieces;
            uint32_t sv = live ? spp[i] : 0u, bv = live ? bpp[i] : 0u;
            if constexpr (kOdd) {  // the half piece's missing group: zero scale and bias
                if (k0 + 128u * (p0 + (uint32_t)i) + 64u >= K) {
                    sv &= 0xFFFFu;
                    bv &= 0xFFFFu;
                }
            }
            // swap words (0, 1) and (2, 3) across the lane halves: [0] holds group 2p, [1] group 2p + 1
            const auto p01 = __builtin_amdgcn_permlane32_swap(wv[b][i].x, wv[b][i].y, false, false);
            const auto p23 = __builtin_amdgcn_permlane32_swap(wv[b][i].z, wv[b][i].w, false, false);
#pragma unroll
            for (int h = 0; h < 2; ++h) {  // one group at a time: fewer registers live
                const float sg = __uint_as_float(h ? (sv & 0xFFFF0000u) : (sv << 16));
                const float cg = fmaf(-128.0f, sg, __uint_as_float(h ? (bv & 0xFFFF0000u) : (bv << 16)));
                const bf16x8_t q01 = q_frag(p01[h], kMask, kMagic), q23 = q_frag(p23[h], kMask, kMagic);
#pragma unroll
                for (int gi = 0; gi < MG; ++gi) {  // the unpacked words serve every row group
                    bf16x8_t xp[2];
                    f32x4 sx;
                    if constexpr (kXRegs) {
                        xp[0] = xf[gi][i][h][0];
                        xp[1] = xf[gi][i][h][1];
                    } else {
                        xread2(i, h, xp);
                    }
                    f32x4 d = __builtin_amdgcn_mfma_f32_16x16x32_bf16(xp[0], q01, zero, 0, 0, 0);
                    if constexpr (!kXRegs) sx = __builtin_amdgcn_mfma_f32_16x16x32_bf16(xp[0], ones, zero, 0, 0, 0);
                    d = __builtin_amdgcn_mfma_f32_16x16x32_bf16(xp[1], q23, d, 0, 0, 0);
                    if constexpr (kXRegs) {
                        sx = xsum[gi][i][h];
                    } else {
                        sx = __builtin_amdgcn_mfma_f32_16x16x32_bf16(xp[1], ones, sx, 0, 0, 0);
                    }
#pragma unroll
                    for (int v = 0; v < 4; ++v) acc.v[gi][v] = fmaf(cg, sx[v], fmaf(sg, d[v], acc.v[gi][v]));
                    // pinned here: otherwise the compiler sinks the arithmetic into the epilogue's
                    // conditional block and keeps every matrix result alive until then
                    asm volatile("" : "+v"(acc.v[gi]));
                }
            }
        }
        return acc;
    };

    // ---- epilogue: output (erow, ecol) of the tile, summed over the waves in order
    int par = 0;
    auto finish = [&](auto BUF, const Acc &acc, uint32_t t) {
        constexpr int b = decltype(BUF)::value;
#pragma unroll
        for (int gi = 0; gi < MG; ++gi)
#pragma unroll
            for (int v = 0; v < 4; ++v) red[par][gi][wave][v][lane] = acc.v[gi][v];
        lds_barrier();
        const uint32_t f = kGateUp ? t * 8 + (ecol & 7) : t * 16 + ecol;
        if (eout && f < crows) {
            const uint32_t L = 16u * ((erow & 15u) >> 2) + ecol, v = erow & 3u, eg = MG > 1 ? erow >> 4 : 0u;
            float val = 0.0f;
#pragma unroll
            for (int w = 0; w < NW; ++w) val += red[par][eg][w][v][L];
            if (a.partial) {  // dense split-K: [ksplit, m, nw * n], gate at f, up at n + f
                const uint32_t nw = kGateUp ? 2 : 1;
                float *dst = a.partial + ((size_t)slab * a.m + erow) * (size_t)(nw * crows);
                // device-coherent store (written through, not held in this XCD's L2), so that the
                // block reducing the run reads it without a cache write-back or invalidate
                __hip_atomic_store(dst + ((kGateUp && ecol >= 8) ? crows : 0u) + f, val, __ATOMIC_RELAXED,
                                   __HIP_MEMORY_SCOPE_AGENT);
            } else {
                if constexpr (kGateUp) {
                    float up = 0.0f;
#pragma unroll
                    for (int w = 0; w < NW; ++w) up += red[par][eg][w][v][L + 8];
                    val = activation(val, a.act) * up;
                }
                const size_t o = (size_t)orow * cldo + f;
                if constexpr (kPre) {
                    if (cbias) val += __uint_as_float(pre_b[b] << 16);
                    if (a.out_f32) {
                        reinterpret_cast<float *>(cout)[o] = a.accumulate ? __uint_as_float(pre_o[b]) + val : val;
                    } else {
                        uint16_t *dst = reinterpret_cast<uint16_t *>(cout) + o;
                        *dst = (uint16_t)f32_to_bf16(a.accumulate ? val + __uint_as_float(pre_o[b] << 16) : val);
                    }
                } else if (a.out_f32) {
                    reinterpret_cast<float *>(cout)[o] = val;
                } else {
                    reinterpret_cast<uint16_t *>(cout)[o] = (uint16_t)f32_to_bf16(val);
                }
            }
        }
        par ^= 1;
    };
    // Tiles t_begin .. t_end - 1, the first already requested into buffer 0;
    // each tile's successor is requested before it is multiplied.  The loop
    // body requests unconditionally and the last one or two tiles are peeled,
    // so that the compiler's wait counts never assume a skipped request.
    // Deeper ring (dense mode, D > 2): tiles t + 1 .. t + D - 1 are in flight while tile t is
    // multiplied; tile t_begin + j lives in buffer j % D.  Requests past the run's end re-request
    // its last tile (the same addresses: cache hits, never stored), so that every request is
    // unconditional: a request under a branch leaves the compiler's wait counts conservative (it
    // then waits for every tile in flight).  The launcher takes this ring for runs of at least
    // 6 tiles, where such repeats are few (cfg1 gate/up at B = 16: 11.0 -> 9.9 us; at runs of 4
    // tiles the repeats cost more than the depth gains).  prefetch_ring requests tiles
    // t_begin + 1 .. t_begin + D - 2 (the caller requested t_begin into buffer 0).
    auto prefetch_ring = [&](uint32_t e, uint32_t t_begin, uint32_t t_end) {
        if constexpr (D > 2)
            static_for<D - 2>([&](auto J) {
                fetch(std::integral_constant<int, J + 1>{}, e, min(t_begin + (uint32_t)J + 1u, t_end - 1u));
            });
    };
    auto run_tiles = [&](uint32_t e, uint32_t t_begin, uint32_t t_end) {
        if constexpr (D > 2) {
            for (uint32_t t = t_begin; t < t_end; t += D) {
                static_for<D>([&](auto J) {
                    constexpr int j = J;
                    fetch(std::integral_constant<int, (j + D - 1) % D>{}, e, min(t + (uint32_t)(j + D - 1), t_end - 1u));
                    if (t + (uint32_t)j < t_end) finish(J, tile_mma(J), t + (uint32_t)j);
                });
            }
            return;
        }
        uint32_t t = t_begin;
        for (; t + 2 < t_end; t += 2) {
            fetch(B1{}, e, t + 1);
            finish(B0{}, tile_mma(B0{}), t);
            fetch(B0{}, e, t + 2);
            finish(B1{}, tile_mma(B1{}), t + 1);
        }
        if (t + 1 < t_end) {
            fetch(B1{}, e, t + 1);
            finish(B0{}, tile_mma(B0{}), t);
            finish(B1{}, tile_mma(B1{}), t + 1);
        } else {
            finish(B0{}, tile_mma(B0{}), t);
        }
    };

    // ---- split K without a second launch (dense mode, a.tickets set): the ksplit blocks of a
    // run publish their partials and take a ticket; the last one sums the run's partials in slab
    // order (as q4_mfma_splitk_reduce_kernel does), applies the epilogue and leaves the ticket at
    // zero.  No block waits for another.  The partials are device-coherent stores and loads, so
    // the only ordering needed is that this block's stores have completed before its ticket
    // (a fence would write back and invalidate whole L2s, which costs far more at this scale).
    auto reduce_run = [&]() {
        asm volatile("s_waitcnt vmcnt(0)" ::: "memory");  // this thread's partial stores are done
        __syncthreads();
        uint32_t *s_ticket = reinterpret_cast<uint32_t *>(&red[0][0][0][0][0]);  // red is free here
        const uint32_t rb = blockIdx.x / a.ksplit;
        // Ordering argument (a hardware one, not a C++ release/acquire pair).  The partials were
        // written with agent-scope relaxed atomic stores: on gfx950 these are global stores with
        // the sc1 cache policy, written through this XCD's L2 to the device-coherent level.  The
        // s_waitcnt vmcnt(0) above returns only once every such store is acknowledged at that
        // level, and the barrier orders all threads' waits before this ticket.  The reducer reads
        // the partials with agent-scope relaxed atomic loads (sc1: never served from a stale
        // non-coherent cache line), issued after its ticket came back.  A release/acquire pair at
        // agent scope would add an L2 write-back (buffer_wbl2) on every block and an invalidate on
        // the reducers: the MLP step at m = 16 took 126 us that way against 27 us.  If the store
        // path changes, KR_OPT_SPLITK_TICKETS = 0 (a second reduction launch, ordered by the
        // stream) is the fallback; tests compare the two bit for bit.
        if (tid == 0) s_ticket[0] = atomicAdd(&a.tickets[rb], 1u);
        __syncthreads();
        if (s_ticket[0] != a.ksplit - 1) return;
        constexpr uint32_t nw = kGateUp ? 2 : 1;
        const uint32_t n = a.w.n;
        const uint32_t f0 = run_begin * kTileRows, f1 = min(run_end * kTileRows, n);
        const uint32_t nrows = f1 - f0, items = nrows * a.m;
        const size_t stride = (size_t)a.m * nw * n;
        // Four consecutive features per thread (16-byte loads of every slab's partials and one
        // load of the old outputs, all issued before any store: one round trip) when the run's
        // features and the rows stay 16-byte aligned; else one feature per thread.
        const bool vec = nrows % 4 == 0 && n % 4 == 0 && a.ldo % 4 == 0 && (uintptr_t)a.partial % 16 == 0 &&
                         (uintptr_t)a.out % 16 == 0 && !a.bias && (size_t)a.ksplit * stride * 4 < (1ull << 31);
        const uint32_t width = vec ? 4u : 1u, vitems = items / width, vrows = nrows / width;
        for (uint32_t it = (uint32_t)tid; it < vitems; it += NW * 64) {
            const uint32_t tok = it / vrows, f = f0 + (it % vrows) * width;
            const float *p = a.partial + (size_t)tok * nw * n + f;
            const size_t o = (size_t)tok * a.ldo + f;
            f32x4 gsum = {0, 0, 0, 0}, usum = {0, 0, 0, 0}, old = {0, 0, 0, 0};
            if (vec) {
                // device-coherent 16-byte loads (the sc1 policy of the scalar path's agent-scope atomic
                // loads: never served from a stale line of this XCD's L2), through a buffer resource
                // over the partials; offsets below 2^32 bytes (the launcher checks)
                const __amdgpu_buffer_rsrc_t rp = __builtin_amdgcn_make_buffer_rsrc(
                    a.partial, (short)0, (int)((size_t)a.ksplit * stride * 4), 0x00020000);
                const uint32_t pb = (uint32_t)((size_t)tok * nw * n + f) * 4u;
                f32x4 gs[kSkinnyMaxTicketSplit], us[kSkinnyMaxTicketSplit];
#pragma unroll
                for (uint32_t sl = 0; sl < kSkinnyMaxTicketSplit; ++sl) {  // unconditional (clamped) loads
                    const uint32_t off = pb + (uint32_t)(min(sl, a.ksplit - 1) * stride) * 4u;
                    gs[sl] = __builtin_bit_cast(f32x4, __builtin_amdgcn_raw_buffer_load_b128(rp, off, 0, 16));
                    if (nw == 2) us[sl] = __builtin_bit_cast(f32x4, __builtin_amdgcn_raw_buffer_load_b128(rp, off + n * 4u, 0, 16));
                }
                if (a.accumulate) {
                    if (a.out_f32) {
                        old = *reinterpret_cast<const f32x4 *>(reinterpret_cast<const float *>(a.out) + o);
                    } else {
                        const uint2 ob = *reinterpret_cast<const uint2 *>(reinterpret_cast<const uint16_t *>(a.out) + o);
                        old = f32x4{__uint_as_float(ob.x << 16), __uint_as_float(ob.x & 0xFFFF0000u),
                                    __uint_as_float(ob.y << 16), __uint_as_float(ob.y & 0xFFFF0000u)};
                    }
                }
#pragma unroll
                for (uint32_t sl = 0; sl < kSkinnyMaxTicketSplit; ++sl) {
                    if (sl < a.ksplit) {
                        gsum += gs[sl];
                        if (nw == 2) usum += us[sl];
                    }
                }
            } else {
                float gs[kSkinnyMaxTicketSplit], us[kSkinnyMaxTicketSplit];
#pragma unroll
                for (uint32_t sl = 0; sl < kSkinnyMaxTicketSplit; ++sl) {
                    const size_t off = (size_t)min(sl, a.ksplit - 1) * stride;
                    gs[sl] = __hip_atomic_load(p + off, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                    us[sl] = nw == 2 ? __hip_atomic_load(p + off + n, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) : 0.0f;
                }
                if (a.accumulate)
                    old[0] = a.out_f32 ? reinterpret_cast<const float *>(a.out)[o]
                                       : bf16_to_f32(reinterpret_cast<const uint16_t *>(a.out)[o]);
#pragma unroll
                for (uint32_t sl = 0; sl < kSkinnyMaxTicketSplit; ++sl) {
                    if (sl < a.ksplit) {
                        gsum[0] += gs[sl];
                        usum[0] += us[sl];
                    }
                }
            }
            float val[4];
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                val[e] = kGateUp ? activation(gsum[e], a.act) * usum[e] : gsum[e];
                if (a.bias) val[e] += bf16_to_f32(a.bias[f + e]);  // (scalar path only)
                if (a.accumulate) val[e] = a.out_f32 ? old[e] + val[e] : val[e] + old[e];
            }
            if (a.out_f32) {
                float *out = reinterpret_cast<float *>(a.out) + o;
                if (vec)
                    *reinterpret_cast<f32x4 *>(out) = f32x4{val[0], val[1], val[2], val[3]};
                else
                    out[0] = val[0];
            } else {
                uint16_t *out = reinterpret_cast<uint16_t *>(a.out) + o;
                if (vec)
                    *reinterpret_cast<uint2 *>(out) = uint2{f32_to_bf16(val[0]) | (f32_to_bf16(val[1]) << 16),
                                                            f32_to_bf16(val[2]) | (f32_to_bf16(val[3]) << 16)};
                else
                    out[0] = (uint16_t)f32_to_bf16(val[0]);
            }
        }
        if (tid == 0) __hip_atomic_store(&a.tickets[rb], 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    };

    if constexpr (!kGrouped) {  // dense: one X for the whole run
        const uint32_t rows = min(a.m, 16u * MG);
        eout = tid < 256 * MG && erow < rows && (!kGateUp || a.partial || ecol < 8);
        orow = erow;
        // the problem holding tile t: its fields, by value; returns its first tile
        auto select = [&](uint32_t t) -> uint32_t {
            const int pi = (a.nmore > 1 && t >= a.tile_begin[2]) ? 2 : (a.nmore > 0 && t >= a.tile_begin[1]) ? 1 : 0;
            if (pi == 0) {
                cw = a.w;
                cout = a.out;
                cbias = a.bias;
                cldo = a.ldo;
            } else {
                const SkinnyArgs::More &mp = pi == 1 ? a.more[0] : a.more[1];
                cw.qw = mp.w.qw;
                cw.sc = mp.w.sc;
                cw.bi = mp.w.bi;
                cw.n = mp.w.n;
                cout = mp.out;
                cbias = mp.bias;
                cldo = mp.ldo;
            }
            crows = cw.n;
            return a.tile_begin[pi];
        };
        // first tile of the problem after the one holding t (constant kernel-argument indices)
        auto next_begin = [&](uint32_t t) -> uint32_t {
            if (a.nmore > 0 && t < a.tile_begin[1]) return a.tile_begin[1];
            if (a.nmore > 1 && t < a.tile_begin[2]) return a.tile_begin[2];
            return a.nmore == 0 ? a.tile_begin[1] : a.nmore == 1 ? a.tile_begin[2] : a.tile_begin[3];
        };
        uint32_t tb = select(run_begin);
        // X loads first (every row group's), then the first tile's words: the conversion waits for
        // X only.  The row groups pass through the one LDS slab in turn (the launcher gives a
        // two-group launch more than 16 rows, so row 16 exists).
        const uint32_t rows0 = min(rows, 16u), rows1 = rows - rows0;
        stage_load(raw[0], 0, rows0);
        if constexpr (MG == 2) stage_load(raw[MG - 1], 16, rows1);
        fetch(B0{}, 0, run_begin - tb);
        prefetch_ring(0, run_begin - tb, min(run_end, next_begin(run_begin)) - tb);
        __builtin_amdgcn_sched_barrier(0);
        if (a.ln_w) norm_x(raw[0], rows0);
        stage_store(raw[0], rows0);
        lds_barrier();
        load_x_frags(std::integral_constant<int, 0>{});
        if constexpr (MG == 2) {
            lds_barrier();  // every wave has read group 0's fragments
            if (a.ln_w) norm_x(raw[MG - 1], rows1);
            stage_store(raw[MG - 1], rows1);
            lds_barrier();
            load_x_frags(std::integral_constant<int, MG - 1>{});
        }
        uint32_t t = run_begin;
        for (;;) {
            const uint32_t seg_end = min(run_end, next_begin(t));
            run_tiles(0, t - tb, seg_end - tb);
            t = seg_end;
            if (t >= run_end) break;
            tb = select(t);
            fetch(B0{}, 0, t - tb);
            prefetch_ring(0, t - tb, min(run_end, next_begin(t)) - tb);
        }
        if (a.tickets) reduce_run();
        return;
    }

    // ---- grouped: segments of the run that share an expert
    uint32_t item = run_begin;
    while (item < run_end) {
        const uint32_t j = item / tiles_per_expert;
        const uint32_t seg_end = min(run_end, (j + 1) * tiles_per_expert);
        uint32_t e, base, cnt;
        expert_of(j, e, base, cnt);
        const uint32_t t_begin = item - j * tiles_per_expert, t_end = seg_end - j * tiles_per_expert;
        for (uint32_t c0 = 0; c0 < cnt; c0 += 16) {
            const uint32_t rows = min(cnt - c0, 16u);
            eout = tid < 256 && erow < rows && (!kGateUp || a.partial || ecol < 8);
            orow = base + c0 + erow;
            if (eout && a.out_scatter) orow = a.sorted[orow];
            stage_load(raw[0], base + c0, rows);
            fetch(B0{}, e, t_begin);
            __builtin_amdgcn_sched_barrier(0);
            lds_barrier();  // the previous segment's readers are done with xs
            stage_store(raw[0], rows);
            lds_barrier();
            run_tiles(e, t_begin, t_end);
        }
        item = seg_end;
    }
}

namespace {

template <bool GU, bool G, int MG, bool P, int D, bool O>
hipError_t launch_d(SkinnyArgs &a, uint32_t nblk, hipStream_t s) {
    const dim3 grid(nblk * a.ksplit), block(kSkinnyWaves * 64);
    hipLaunchKernelGGL((q4_skinny_kernel<GU, G, MG, P, D, O>), grid, block, 0, s, a);
    return hipGetLastError();
}

template <bool GU, bool G, int MG, bool P, bool O>
hipError_t launch_t(SkinnyArgs &a, uint32_t items, hipStream_t s) {
    // blocks per slab: every CU busy, each block a contiguous run of ceil(items / nblk) tiles
    // grouped (MoE) launches take twice the cap: cfg4 T = 64 is 1.3 % faster at 512 blocks, the dense
    // cfg1 B = 16 step 2 % faster at 256
    const uint32_t cap_all = (uint32_t)tuning().skinny_max_blocks * (G ? 2u : 1u);
    uint32_t cap = std::max<uint32_t>(1, cap_all / a.ksplit);
    if (a.tickets) cap = std::min(cap, kSkinnyTickets);  // one ticket word per run
    const uint32_t nblk = std::max<uint32_t>(1, std::min(items, cap));
    // the deeper ring for dense launches without epilogue operands whose runs hold >= 6 tiles
    if constexpr (!G && !P) {
        const int depth = tuning().skinny_depth;
        const uint32_t per = (items + nblk - 1) / nblk;
        if (depth == 3 || (depth == 0 && per >= 6)) return launch_d<GU, G, MG, P, 3, O>(a, nblk, s);
    }
    return launch_d<GU, G, MG, P, 2, O>(a, nblk, s);
}

// dense launches: the even or the odd group-count kernels
template <bool GU, int MG, bool P>
hipError_t launch_dense(SkinnyArgs &a, uint32_t items, hipStream_t s) {
    return a.k % 128 == 0 ? launch_t<GU, false, MG, P, false>(a, items, s) : launch_t<GU, false, MG, P, true>(a, items, s);
}

}  // namespace

bool skinny_supported(const Q4Mat &w) {
    if (w.k == 0 || w.k % 64 != 0) return false;
    // even group counts load each scale/bias pair as one 4-byte word
    return w.k % 128 != 0 || ((uintptr_t)w.sc % 4 == 0 && (uintptr_t)w.bi % 4 == 0);
}

hipError_t launch_skinny(SkinnyArgs &a, hipStream_t s) {
    const bool gate_up = a.w2.qw != nullptr;
    if (!skinny_supported(a.w) || (gate_up && !skinny_supported(a.w2))) return hipErrorInvalidValue;
    const bool grouped = a.offsets != nullptr;
    a.ksplit = skinny_ksplit(a.k);
    if (grouped && (a.ksplit != 1 || a.k % 128 != 0)) return hipErrorInvalidValue;
    if (grouped && (a.nmore > 0 || a.ln_w || a.bias || a.accumulate)) return hipErrorInvalidValue;
    if (a.nmore < 0 || a.nmore > 2 || (a.nmore > 0 && (gate_up || a.partial))) return hipErrorInvalidValue;
    if (!grouped && (a.m == 0 || a.m > kSkinnyMaxM)) return hipErrorInvalidValue;
    if (a.ln_w && a.ksplit != 1) return hipErrorInvalidValue;  // the norm needs the whole row in the slab
    if (a.tickets && (grouped || a.nmore > 0 || !a.partial || a.ksplit < 2 || a.ksplit > kSkinnyMaxTicketSplit))
        return hipErrorInvalidValue;
    for (int i = 0; i < a.nmore; ++i)
        if (!skinny_supported(a.more[i].w) || a.more[i].w.k != a.k) return hipErrorInvalidValue;
    const uint32_t tile_rows = gate_up ? 8 : 16;
    if (!grouped) {
        a.experts = 1;
        a.expert_rows = a.w.n;
        a.max_active = 1;
        a.tile_begin[0] = 0;
        a.tile_begin[1] = (a.w.n + tile_rows - 1) / tile_rows;
        for (int i = 0; i < a.nmore; ++i) a.tile_begin[i + 2] = a.tile_begin[i + 1] + (a.more[i].w.n + 15) / 16;
    }
    const uint32_t items =
        grouped ? a.max_active * ((a.expert_rows + tile_rows - 1) / tile_rows) : a.tile_begin[a.nmore + 1];
    // the epilogue reads a bias or the old output (never with split-K partials: their reduction does)
    bool pre = false;
    if (!a.partial) {
        pre = a.bias != nullptr || a.accumulate;
        for (int i = 0; i < a.nmore; ++i) pre = pre || a.more[i].bias != nullptr;
    }
    if (grouped)
        return gate_up ? launch_t<true, true, 1, false, false>(a, items, s)
                       : launch_t<false, true, 1, false, false>(a, items, s);
    if (gate_up && pre) return hipErrorInvalidValue;  // gate/up launches have neither
    if (a.m > 16) {  // two row groups per launch
        if (gate_up) return launch_dense<true, 2, false>(a, items, s);
        return pre ? launch_dense<false, 2, true>(a, items, s) : launch_dense<false, 2, false>(a, items, s);
    }
    if (gate_up) return launch_dense<true, 1, false>(a, items, s);
    return pre ? launch_dense<false, 1, true>(a, items, s) : launch_dense<false, 1, false>(a, items, s);
}

uint32_t skinny_ksplit(uint32_t k) { return (k + kSlabCols - 1) / kSlabCols; }

bool skinny_grouped_fits(uint32_t k) { return k % 128 == 0 && skinny_ksplit(k) == 1; }  // even group counts only

}  // namespace kr
