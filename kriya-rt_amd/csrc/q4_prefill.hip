// q4_prefill.hip — prefill-sized (m > 16) Q4_G64 matmul on the gfx950 matrix cores.
//
// Replaces the reference's M >= 64 simdgroup kernels (kernels/metal/q4_gemm_and_moe.metal):
//   q4_g64_batched_simdgroup_gemm_m64                     :2708-2851
//   q4_g64_batched_simdgroup_qkv_gemm_m64                 :2853-3022
//   q4_g64_batched_simdgroup_gate_up_swiglu_gemm_m64      :3024-3215
// and the 1 < M < 64 prefill kernels (:2173-2486) for m > 16.
//
// Y[M, N] = X[M, K] . W[N, K]^T, X bf16, W planar Q4_G64, f32 accumulation on
// v_mfma_f32_16x16x32_f16.  Operand numerics are those of the reference's M >= 64
// kernels (half operands, q4_gemm_and_moe.metal:2722-2724, 2761-2764):
//   * w = fma(q, s, b) rounded once to fp16 (s, b: bf16 -> fp16 RNE);
//   * x: bf16 -> fp16 RNE, exact for |x| in [2^-14, 65504]; smaller values become
//     fp16 subnormals (the reference's M >= 64 kernels stage half as well).  A value
//     beyond 65504 turns into inf, and so does its block's result: a block whose
//     accumulators come out non-finite computes its tile again in plain f32
//     arithmetic (dequantised weights times bf16 x, exact products of the inputs'
//     values), which writes the outputs itself.  Ordinary data never takes that
//     path.  The few-token kernel, exact in bf16, serves m < 64 (q4_skinny.hip).
//
// Where the time goes at these shapes (M = 512, K = 2048 .. 11008): dequantising
// a nibble costs ~2 VALU lane-ops, converting an X element ~1.5, and the matrix
// cores need 2 * M_reuse FLOP per weight element to stay ahead of the VALU.  So:
//   * each wave owns MF x 16 token rows by NF x 16 weight rows and dequantises
//     its weight rows itself, straight from global memory into the MFMA B
//     fragments (no LDS round trip for W, no barrier between dequant and use);
//     one dequantised word feeds MF matrix instructions;
//   * X is staged in LDS by direct-to-LDS buffer loads (no VGPRs held across
//     the step; shapes with wave groups load it into registers and write it
//     after the step's products), converted to fp16 once per block unless the caller
//     converted it beforehand (double buffered, two 64-column quantisation
//     groups per step, one barrier per step) and shared by the WAVES waves of
//     the block, which split the weight rows;
//   * scales and biases arrive in 16-byte blocks that cover four steps of a
//     row: the kernel is paced by memory requests more than by bytes, and a
//     4-byte load per row and step was one request for 4 bytes;
//   * the k order inside each 8-column unit is the nibble-pair order of the
//     dequantiser, (e0 e4 e1 e5 e2 e6 e3 e7), applied to X when it is staged,
//     so neither side permutes in the inner loop (a dot product does not depend
//     on the order of its terms);
//   * LDS rows of 8 units are XOR-swizzled by row so that the 16-byte reads of
//     16 rows x 4 units and the staging writes are bank-conflict free;
//   * weights, scales and X are read through buffer resources with the block-
//     and step-uniform part of every offset in an SGPR; every offset is kept in
//     range on the host side of the check (tail rows are clamped, never stored).
//   * the A fragments of the next 32-column slice are read from LDS before the
//     current slice's dequantisation and matrix instructions;
//   * the epilogue stages the block's tile in LDS, so each thread stores 8
//     consecutive columns of a row (16-byte stores) instead of 2- or 4-byte pieces;
//   * shapes with fewer tiles than two per CU run two groups of waves per tile
//     that split its steps and add their accumulators through LDS.
// Gate/up: a wave's fragments are FPM gate fragments followed by FPM up
// fragments of the same rows, so act(g) * u is formed lane-locally.
// Block ids are remapped so that the M tiles of one N tile run on one XCD and
// share its L2; split-K (grid.y) writes f32 partials that the reduction
// launch (launch_splitk_reduce) sums in split order.
#include <type_traits>

#include "kr_internal.hpp"


namespace kr {

namespace {

using rsrc_t = __amdgpu_buffer_rsrc_t;

__device__ __forceinline__ rsrc_t make_rsrc(const void *p, uint32_t bytes) {
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<void *>(p), (short)0, (int)bytes, 0x00020000);
}

__device__ __forceinline__ uint32_t opaque_v(uint32_t v) {
    uint32_t r;
    asm volatile("v_mov_b32 %0, %1" : "=v"(r) : "i"(v));
    return r;
}

__device__ __forceinline__ f16x2_t f16_pair(uint32_t bf16_bits) {
    const _Float16 h = (_Float16)bf16_to_f32(bf16_bits);
    return f16x2_t{h, h};
}

// LDS row swizzle of the X slice: 16 consecutive rows x one unit hit 16
// distinct 16-byte slots modulo 256 bytes, and 8 consecutive rows distinct
// slots modulo 128 bytes.
__device__ __forceinline__ uint32_t swz(uint32_t r) { return (r & 7) ^ ((r >> 3) & 1); }

// 16 bytes per lane from a buffer straight into LDS: lane l writes lds[16 l, 16 l + 16).
// `lds` must be wave-uniform (it goes to M0).
__device__ __forceinline__ void dma16(rsrc_t r, char *lds, uint32_t voffset, uint32_t soffset) {
    __builtin_amdgcn_raw_ptr_buffer_load_lds(r, (__attribute__((address_space(3))) void *)lds, 16, voffset, soffset, 0,
                                             0);
}

// 8 nibbles of one word -> the B fragment (w0 w4)(w1 w5)(w2 w6)(w3 w7), w = fma(q, s, b).
__device__ __forceinline__ f16x8_t dequant_pairs(uint32_t w, f16x2_t s2, f16x2_t b2, uint32_t mask, uint32_t magic) {
    const f16x2_t k1024 = {(_Float16)-1024.0f, (_Float16)-1024.0f};
    f16x2_t pr[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        const uint32_t h = ((w >> (4 * j)) & mask) | magic;           // (1024 + q_j, 1024 + q_{j+4})
        pr[j] = __builtin_elementwise_fma(__builtin_bit_cast(f16x2_t, h) + k1024, s2, b2);
    }
    return f16x8_t{pr[0].x, pr[0].y, pr[1].x, pr[1].y, pr[2].x, pr[2].y, pr[3].x, pr[3].y};
}

// 8 bf16 columns (x0 x1)(x2 x3)(x4 x5)(x6 x7) -> fp16 (x0 x4)(x1 x5)(x2 x6)(x3 x7).
__device__ __forceinline__ u32x4 x_unit_f16(u32x4 d) {
    auto lo = [](uint32_t v) { return __uint_as_float(v << 16); };
    auto hi = [](uint32_t v) { return __uint_as_float(v & 0xFFFF0000u); };
    const f16x2_t o0 = {(_Float16)lo(d.x), (_Float16)lo(d.z)};
    const f16x2_t o1 = {(_Float16)hi(d.x), (_Float16)hi(d.z)};
    const f16x2_t o2 = {(_Float16)lo(d.y), (_Float16)lo(d.w)};
    const f16x2_t o3 = {(_Float16)hi(d.y), (_Float16)hi(d.w)};
    return u32x4{__builtin_bit_cast(uint32_t, o0), __builtin_bit_cast(uint32_t, o1),
                 __builtin_bit_cast(uint32_t, o2), __builtin_bit_cast(uint32_t, o3)};
}

}  // namespace

template <int MF, int NF, int WAVES, int NW, int KW = 1>
struct PrefillTile {
    static constexpr int kBM = MF * 16;                 // token rows per block
    static constexpr int kThreads = 64 * WAVES * KW;
    static constexpr int kFPM = NF / NW;                // fragments per matrix per wave
    static constexpr int kWaveRows = kFPM * 16;         // output columns per wave
    static constexpr int kBN = WAVES * kWaveRows;       // output columns per block
    static constexpr int kBufBytes = kBM * 128;         // one 64-column X slice in fp16
    static_assert(NF % NW == 0, "gate/up needs pairs of fragments");
};

// D: steps of look-ahead.  The X slice and the weights of step g + D are
// requested at step g (ring of D + 1 X buffers and weight register sets).
// vmcnt completes in issue order, so waiting for the X slice of step g + 1 at
// the end of step g also waits for every load issued before it: with X and
// weights requested together D steps ahead, both get D steps of latency.
// SW: quantisation groups (64 columns) per step.  With SW = 2 a lane's
// weights of a step are one 16-byte load (32 nibbles: four MFMA slices) and
// its scales and biases come in 16-byte blocks of four steps (below): far
// fewer load instructions and memory requests than SW = 1, whose lanes load
// 8 bytes and two 2-byte values per 64 columns.
// KW: groups of WAVES waves that split the block's steps (each group has its
// own X ring) and add their accumulators through LDS in group order at the
// end.  With SW = 2 and D = 1 group k takes the k-th contiguous part of the
// steps; otherwise steps k, k + KW, ....  Shapes with few tiles (N = 2048)
// get KW waves per tile instead of one: more waves per SIMD to overlap the
// latencies of each wave's step, with no workspace.
template <int MF, int NF, int WAVES, int NW, int OCC, int EPI, int D, int SW, int KW>
__global__ __launch_bounds__(64 * WAVES * KW, OCC) void q4_prefill_kernel(MfmaArgs args) {
    using T = PrefillTile<MF, NF, WAVES, NW, KW>;
    constexpr int FPM = T::kFPM;
    constexpr int kUnits = 8 * SW;                  // 16-byte X units per LDS row
    constexpr int kBuf = T::kBM * 16 * kUnits;      // bytes of one X slice
    constexpr int kSlices = 2 * SW;                 // 32-column MFMA slices per step
    static_assert(SW == 1 || SW == 2, "one or two groups per step");
    extern __shared__ __align__(16) char lds[];
    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wid = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int wave = wid % WAVES, kg = wid / WAVES;  // wave within its K group, the group
    const int c = lane & 15, kq = lane >> 4;
    char *const xring = lds + kg * (D + 1) * kBuf;  // this group's X buffers

    // ---- block -> (problem, n tile, m tile, K split).  Workgroups go to the 8 XCDs (each with its own
    // L2) round-robin in launch order.  Unsplit: the M tiles of one N tile share an XCD, so each
    // weight tile is read into one L2.  Split K (xcd_tiles > 0, one problem): the blocks of K split
    // ks go to XCDs ks * 8 / ksplit ..; XCD j takes the xcd_tiles consecutive tiles (whole N tiles
    // with all their M tiles) of part j % (8 / ksplit), so an L2 holds one K range of X and of the
    // weights instead of all of X.  Any grid maps one-to-one; only locality depends on the order.
    const uint32_t nblk = gridDim.x;
    uint32_t bid = blockIdx.x, ks = blockIdx.y;
    if (args.xcd_tiles) {
        const uint32_t L = blockIdx.x + blockIdx.y * nblk, j = L & 7, g = 8 / gridDim.y;
        ks = j / g;
        bid = (j % g) * args.xcd_tiles + (L >> 3);
    } else if (nblk >= 8 && (nblk & 7) == 0) {
        bid = (bid & 7) * (nblk >> 3) + (bid >> 3);
    }
    int pi = 0;
#pragma unroll
    for (int i = 1; i < kMaxMfmaProblems; ++i)
        if (i < args.np && bid >= args.p[i].tile_begin) pi = i;
    const MfmaProblem &P = args.p[pi];
    const uint32_t local = bid - P.tile_begin;
    const uint32_t tiles_m = (args.m + T::kBM - 1) / T::kBM;
    const uint32_t mt = local % tiles_m, nt = local / tiles_m;
    const uint32_t m0 = mt * T::kBM;
    const uint32_t N = P.w.n, M = args.m, K = args.k, G = K >> 6;
    const uint32_t GS = G / SW;                                // steps over the whole row
    const uint32_t row0 = nt * T::kBN + wave * T::kWaveRows;  // first weight row of this wave
    const uint32_t g_begin = ks * (args.groups_per_split / SW);  // in steps (groups_per_split % SW == 0)
    const uint32_t g_end = min(GS, g_begin + args.groups_per_split / SW);

    const uint32_t kMask = opaque_v(0x000F000Fu);
    const uint32_t kMagic = opaque_v(0x64006400u);

    // ---- buffer resources and per-lane offsets (the step-uniform part goes in soffset)
    const uint32_t rowbytes = K >> 1;
    rsrc_t rq[NW], rs[NW], rb[NW];
    rq[0] = make_rsrc(P.w.qw, N * rowbytes);
    rs[0] = make_rsrc(P.w.sc, N * G * 2);
    rb[0] = make_rsrc(P.w.bi, N * G * 2);
    if constexpr (NW == 2) {
        rq[1] = make_rsrc(P.w2.qw, N * rowbytes);
        rs[1] = make_rsrc(P.w2.sc, N * G * 2);
        rb[1] = make_rsrc(P.w2.bi, N * G * 2);
    }
    uint32_t oq[FPM], os[FPM];
#pragma unroll
    for (int f = 0; f < FPM; ++f) {
        const uint32_t row = min(row0 + f * 16 + c, N - 1);  // tail rows re-read row N-1; never stored
        oq[f] = row * rowbytes + kq * (8 * SW);
        os[f] = row * G * 2;
    }
    // ---- X staging: direct-to-LDS loads (no VGPR round trip), converted in place.
    // A buffer holds the block's BM rows x kUnits units (16 B) of one step's columns;
    // row r, unit u lives in slot r * kUnits + (u ^ swizzle(r)).  DMA instruction i of a
    // wave writes 64 consecutive slots (lane l -> slot base + l), so each lane
    // loads the global unit that belongs in its slot and later converts exactly
    // the slots it loaded (its own data: no barrier between load and convert).
    auto swizzle = [](uint32_t r) -> uint32_t { return SW == 1 ? swz(r) : (((r & 7) << 1) | ((r >> 3) & 1)); };
    constexpr int XI = T::kBM * kUnits / 64 / WAVES;  // DMA instructions per wave per step
    static_assert(T::kBM * kUnits % (64 * WAVES) == 0, "X slice must split into whole DMA instructions");
    // x in bf16, converted here; or (args.xh) converted once beforehand, staged as it is
    const bool cvt = args.xh == nullptr;
    const rsrc_t rx = make_rsrc(cvt ? args.x : args.xh, (M - 1) * args.ldx * 2 + K * 2);
    uint32_t xo[XI];
#pragma unroll
    for (int i = 0; i < XI; ++i) {
        const uint32_t slot = (wave * XI + i) * 64 + lane;
        const uint32_t r = slot / kUnits, u = (slot % kUnits) ^ swizzle(r);
        xo[i] = min(m0 + r, M - 1) * args.ldx * 2 + u * 16;  // tail rows re-read row M-1; never stored
    }
    auto dma_x = [&](uint32_t g, int buf) {
#pragma unroll
        for (int i = 0; i < XI; ++i) dma16(rx, xring + buf * kBuf + (wave * XI + i) * 1024, xo[i], g * (128 * SW));
    };
    auto convert_x = [&](int buf) {
        if (!cvt) return;
#pragma unroll
        for (int i = 0; i < XI; ++i) {
            u32x4 *p = reinterpret_cast<u32x4 *>(xring + buf * kBuf + (wave * XI + i) * 1024 + lane * 16);
            *p = x_unit_f16(*p);
        }
    };
    // Block-wide OR without LDS of its own (a static LDS array would cost the 64-row shape one of
    // its five blocks per CU): each wave's ballot goes to a flag byte in X buffer 0 (inside wave 0's
    // slice of it), a barrier, then every lane reads the WAVES flags.  Only after the last step.  The
    // 64-column path's last step requests a clamped look-ahead slice that nothing waits for, and it
    // may land in buffer 0: every wave waits for its direct-to-LDS loads, and a barrier makes sure all
    // have landed, before any flag byte is written.
    auto block_any = [&](bool pred) -> bool {
        int8_t *flags = reinterpret_cast<int8_t *>(lds);
        const bool wave_any = __ballot(pred) != 0ull;
        asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
        __syncthreads();
        if (lane == 0) flags[wid] = wave_any ? 1 : 0;
        __syncthreads();
        bool any = false;
#pragma unroll
        for (int w = 0; w < WAVES * KW; ++w) any |= flags[w] != 0;
        return any;
    };
    // A fragment of slice j: row r = 16 * a + c (the swizzle depends on c only), unit
    // 2 kq + j (SW = 1) or 4 kq + j (SW = 2): the lane's 8 columns of that slice
    uint32_t xa[kSlices];
#pragma unroll
    for (int j = 0; j < kSlices; ++j)
        xa[j] = ((c * kUnits) + (((uint32_t)kSlices * kq + j) ^ swizzle(c))) * 16;

    struct WRegs {
        uint32_t q[NF][kSlices];
        uint32_t s[NF], b[NF];
    };
    auto load_w = [&](uint32_t g, WRegs &r) {
#pragma unroll
        for (int f = 0; f < NF; ++f) {
            const int mi = f / FPM, fi = f % FPM;
            if constexpr (SW == 1) {
                const u32x2 v = __builtin_bit_cast(u32x2, __builtin_amdgcn_raw_buffer_load_b64(rq[mi], oq[fi], g * 32, 0));
                r.q[f][0] = v.x;
                r.q[f][1] = v.y;
                r.s[f] = __builtin_amdgcn_raw_buffer_load_b16(rs[mi], os[fi], g * 2, 0);
                r.b[f] = __builtin_amdgcn_raw_buffer_load_b16(rb[mi], os[fi], g * 2, 0);
            } else {
                const u32x4 v = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(rq[mi], oq[fi], g * 64, 0));
                r.q[f][0] = v.x;
                r.q[f][1] = v.y;
                r.q[f][2] = v.z;
                r.q[f][3] = v.w;
                r.s[f] = __builtin_amdgcn_raw_buffer_load_b32(rs[mi], os[fi], g * 4, 0);  // groups 2g, 2g + 1
                r.b[f] = __builtin_amdgcn_raw_buffer_load_b32(rb[mi], os[fi], g * 4, 0);
            }
        }
    };

    f32x4 acc[MF][NF];
#pragma unroll
    for (int a = 0; a < MF; ++a)
#pragma unroll
        for (int f = 0; f < NF; ++f) acc[a][f] = f32x4{0, 0, 0, 0};

    auto compute = [&](int buf, WRegs &w) {
        f16x2_t s2[NF], b2[NF];
#pragma unroll
        for (int f = 0; f < NF; ++f) {
            // SW = 2: lane groups kq = 0, 1 hold columns of group 2g, kq = 2, 3 of group 2g + 1
            const uint32_t sb = SW == 1 ? w.s[f] : (kq >= 2 ? w.s[f] >> 16 : w.s[f] & 0xFFFFu);
            const uint32_t bb = SW == 1 ? w.b[f] : (kq >= 2 ? w.b[f] >> 16 : w.b[f] & 0xFFFFu);
            s2[f] = f16_pair(sb);
            b2[f] = f16_pair(bb);
        }
        // The A fragments of slice j + 1 are requested before slice j's dequantisation and matrix
        // instructions (two register sets), so that LDS latency overlaps them instead of stalling
        // every instruction on its own read.  The 64-column shapes (more waves per SIMD) have
        // no registers for the second set and read each fragment where it is used.
        if constexpr (SW == 1) {
#pragma unroll
            for (int j = 0; j < kSlices; ++j) {
                f16x8_t bf[NF];
#pragma unroll
                for (int f = 0; f < NF; ++f) bf[f] = dequant_pairs(w.q[f][j], s2[f], b2[f], kMask, kMagic);
                const char *ab = xring + buf * kBuf + xa[j];
#pragma unroll
                for (int a = 0; a < MF; ++a) {
                    const f16x8_t af = *reinterpret_cast<const f16x8_t *>(ab + a * 16 * kUnits * 16);
#pragma unroll
                    for (int f = 0; f < NF; ++f)
                        acc[a][f] = __builtin_amdgcn_mfma_f32_16x16x32_f16(af, bf[f], acc[a][f], 0, 0, 0);
                }
            }
            return;
        }
        f16x8_t af[2][MF];
        auto read_a = [&](int j, f16x8_t *dst) {
            const char *ab = xring + buf * kBuf + xa[j];
#pragma unroll
            for (int a = 0; a < MF; ++a) dst[a] = *reinterpret_cast<const f16x8_t *>(ab + a * 16 * kUnits * 16);
        };
        // Software pipeline: slice j + 1's A reads and dequantisation are interleaved with slice
        // j's matrix instructions, one MFMA then two VALU (the wave's dequantisation runs while its
        // own matrix instructions execute): gate/up 71.8 -> 69.7 us (1 or 3 VALU: 71.1, 70.8).
        f16x8_t bq[2][NF];
        read_a(0, af[0]);
#pragma unroll
        for (int f = 0; f < NF; ++f) bq[0][f] = dequant_pairs(w.q[f][0], s2[f], b2[f], kMask, kMagic);
        __builtin_amdgcn_sched_barrier(0);
#pragma unroll
        for (int j = 0; j < kSlices; ++j) {
            if (j + 1 < kSlices) {
                read_a(j + 1, af[(j + 1) & 1]);
#pragma unroll
                for (int f = 0; f < NF; ++f) bq[(j + 1) & 1][f] = dequant_pairs(w.q[f][j + 1], s2[f], b2[f], kMask, kMagic);
            }
#pragma unroll
            for (int a = 0; a < MF; ++a)
#pragma unroll
                for (int f = 0; f < NF; ++f)
                    acc[a][f] = __builtin_amdgcn_mfma_f32_16x16x32_f16(af[j & 1][a], bq[j & 1][f], acc[a][f], 0, 0, 0);
            if (j + 1 < kSlices) {
                __builtin_amdgcn_sched_group_barrier(0x100, MF, 0);  // the A reads first
#pragma unroll
                for (int i = 0; i < MF * NF; ++i) {
                    __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);  // one MFMA
                    __builtin_amdgcn_sched_group_barrier(0x002, 2, 0);  // then two VALU
                }
            }
            __builtin_amdgcn_sched_barrier(0);
        }
    };

    if constexpr (SW == 2 && D == 1) {
      if (g_begin < g_end) {
        // 128-column steps, one step of look-ahead, scales and biases in blocks of four steps: a
        // lane's 16-byte load holds the scale (or bias) words of four consecutive steps of its row
        // (groups 2 g .. 2 g + 7), the same 16 bytes for the row's four lanes, so a row costs one
        // memory request per four steps instead of one per step (per-step 4-byte loads were 12 %
        // of the gate/up time: the kernel is paced by requests, not bytes).  The block of steps
        // i + 1 .. i + 4 is requested at step i = 3 mod 4 (one step ahead, as the words), after
        // that step's words were taken from the previous block; reads past the end of the scale
        // arrays return zeros (buffer range check) and are never used.  A group's steps are
        // contiguous (group k takes the k-th part of the range), and the loop runs whole blocks
        // of four: steps past the group's part load (clamped) and wait but do not compute.
        constexpr int NB = 2;
        constexpr int kQLoads = NF, kSBLoads = 2 * NF;
        WRegs w[NB];
        u32x4 sblk[NF], bblk[NF];
        const uint32_t nsteps = (g_end - g_begin + KW - 1) / KW;
        const uint32_t gfirst = g_begin + kg * nsteps;
        auto gstep = [&](uint32_t i) { return gfirst + i; };
        auto gc = [&](uint32_t g) { return min(g, GS - 1); };
        auto load_q = [&](uint32_t g, WRegs &r) {
#pragma unroll
            for (int f = 0; f < NF; ++f) {
                const int mi = f / FPM, fi = f % FPM;
                const u32x4 v = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(rq[mi], oq[fi], g * 64, 0));
                r.q[f][0] = v.x;
                r.q[f][1] = v.y;
                r.q[f][2] = v.z;
                r.q[f][3] = v.w;
            }
        };
        auto load_sb = [&](uint32_t g) {
#pragma unroll
            for (int f = 0; f < NF; ++f) {
                const int mi = f / FPM, fi = f % FPM;
                sblk[f] = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(rs[mi], os[fi], g * 4, 0));
                bblk[f] = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(rb[mi], os[fi], g * 4, 0));
            }
        };
        // X slices: direct-to-LDS loads, or (shapes with wave groups, whose few tiles leave each step's
        // latency exposed) loads into registers written to LDS after the step's products: q/k/v
        // 17.8 -> 16.6 us per call that way, while gate/up (63.9 against 58.6 us) and the split-K
        // down projection (40.2 against 36.6 us) are faster with the direct-to-LDS loads.
        constexpr bool kXViaRegs = KW > 1;
        u32x4 xv[kXViaRegs ? XI : 1];
        auto request_x = [&](uint32_t g, int buf) {
            if constexpr (kXViaRegs) {
#pragma unroll
                for (int q = 0; q < XI; ++q)
                    xv[q] = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(rx, xo[q], g * (128 * SW), 0));
            } else {
                dma_x(g, buf);
            }
        };
        // the slice requested into buffer buf is in LDS, converted (vmcnt completes in issue order:
        // the direct-to-LDS loads are followed by `after` loads)
        auto land_x = [&](int buf, auto AFTER) {
            if constexpr (kXViaRegs) {
#pragma unroll
                for (int q = 0; q < XI; ++q) {
                    u32x4 *p = reinterpret_cast<u32x4 *>(xring + buf * kBuf + (wave * XI + q) * 1024 + lane * 16);
                    *p = cvt ? x_unit_f16(xv[q]) : xv[q];
                }
            } else {
                asm volatile("s_waitcnt vmcnt(%0)" ::"n"(decltype(AFTER)::value) : "memory");
                convert_x(buf);
            }
        };
        request_x(gc(gstep(0)), 0);
        __builtin_amdgcn_sched_barrier(0);
        load_q(gc(gstep(0)), w[0]);
        load_sb(gc(gstep(0)));
        __builtin_amdgcn_sched_barrier(0);
        land_x(0, std::integral_constant<int, kQLoads + kSBLoads>{});
        __syncthreads();
        for (uint32_t i0 = 0; i0 < nsteps; i0 += 4) {
            static_for<4>([&](auto U) {
                constexpr int u = U;
                constexpr int b = u & 1;
                const uint32_t i = i0 + (uint32_t)u;
                request_x(gc(gstep(i + 1)), b ^ 1);
                __builtin_amdgcn_sched_barrier(0);
                load_q(gc(gstep(i + 1)), w[b ^ 1]);
#pragma unroll
                for (int f = 0; f < NF; ++f) {
                    w[b].s[f] = sblk[f][u];
                    w[b].b[f] = bblk[f][u];
                }
                if constexpr (u == 3) load_sb(gc(gstep(i + 1)));
                __builtin_amdgcn_sched_barrier(0);  // keep the loads at the top of the step
                if (i < nsteps && gstep(i) < g_end) compute(b, w[b]);
                land_x(b ^ 1, std::integral_constant<int, kQLoads + (u == 3 ? kSBLoads : 0)>{});
                __syncthreads();
            });
        }
      }
    } else if (g_begin < g_end) {
        constexpr int NB = D + 1;
        constexpr int kWLoads = 3 * NF;
        // loads issued after the X slice of a step: its weights and the later D - 1 (X, weights) pairs
        constexpr int kAfterX = kWLoads + (D - 1) * (XI + kWLoads);
        WRegs w[NB];
        // Step i of this group is g_begin + kg + i * KW.  Requests past the last step are clamped
        // to step GS - 1 (in bounds, never used), so that every step issues the same loads and the
        // waits are fixed counts; all groups run the same number of steps (barriers), a group
        // whose step lies beyond the range skips its compute.
        const uint32_t nsteps = (g_end - g_begin + KW - 1) / KW;
        auto gstep = [&](uint32_t i) { return g_begin + kg + i * KW; };
        auto gc = [&](uint32_t g) { return min(g, GS - 1); };
#pragma unroll
        for (int d = 0; d < D; ++d) {
            dma_x(gc(gstep(d)), d);
            __builtin_amdgcn_sched_barrier(0);  // X before the weights (vmcnt order)
            load_w(gc(gstep(d)), w[d]);
            __builtin_amdgcn_sched_barrier(0);
        }
        asm volatile("s_waitcnt vmcnt(%0)" ::"n"(kAfterX) : "memory");
        convert_x(0);
        __syncthreads();
        auto step = [&](auto I, uint32_t i) {
            constexpr int b = decltype(I)::value;
            constexpr int pf = (b + D) % NB;
            dma_x(gc(gstep(i + D)), pf);
            __builtin_amdgcn_sched_barrier(0);
            load_w(gc(gstep(i + D)), w[pf]);
            __builtin_amdgcn_sched_barrier(0);  // keep the loads at the top of the step
            if (KW == 1 || gstep(i) < g_end) compute(b, w[b]);
            asm volatile("s_waitcnt vmcnt(%0)" ::"n"(kAfterX) : "memory");  // X slice of the next step
            convert_x((b + 1) % NB);
            __syncthreads();
        };
        using S0 = std::integral_constant<int, 0>;
        using S1 = std::integral_constant<int, 1>;
        using S2 = std::integral_constant<int, 2>;
        using S3 = std::integral_constant<int, 3>;
        static_assert(NB >= 2 && NB <= 4, "look-ahead of 1 to 3 steps");
        uint32_t i = 0;
        for (; i + NB <= nsteps; i += NB) {
            step(S0{}, i);
            step(S1{}, i + 1);
            if constexpr (NB > 2) step(S2{}, i + 2);
            if constexpr (NB > 3) step(S3{}, i + 3);
        }
        if (i < nsteps) step(S0{}, i);
        if constexpr (NB > 2) {
            if (i + 1 < nsteps) step(S1{}, i + 1);
        }
        if constexpr (NB > 3) {
            if (i + 2 < nsteps) step(S2{}, i + 2);
        }
    }
    if constexpr (KW > 1) {
        // Groups 1 .. KW-1 hand their accumulators to group 0 through LDS (past the flag bytes of
        // block_any; the last step's barrier ended every read of the X buffers), which adds them
        // in group order.
        constexpr int kAccBytes = MF * NF * 64 * 16;  // one wave's accumulators
        static_assert(256 + (KW - 1) * WAVES * kAccBytes <= KW * (D + 1) * kBuf, "reduction area");
        f32x4 *red = reinterpret_cast<f32x4 *>(lds + 256);
        if (kg > 0) {
#pragma unroll
            for (int a = 0; a < MF; ++a)
#pragma unroll
                for (int f = 0; f < NF; ++f) red[(((kg - 1) * WAVES + wave) * MF * NF + a * NF + f) * 64 + lane] = acc[a][f];
        }
        __syncthreads();
        if (kg == 0) {
#pragma unroll
            for (int k = 1; k < KW; ++k)
#pragma unroll
                for (int a = 0; a < MF; ++a)
#pragma unroll
                    for (int f = 0; f < NF; ++f) acc[a][f] += red[(((k - 1) * WAVES + wave) * MF * NF + a * NF + f) * 64 + lane];
        }
    }
    // Exact fallback (see the top of the file): a non-finite accumulator sends the block to a plain f32
    // computation of its tile (rows beyond M and columns beyond N skipped), which writes the outputs.
    bool bad = false;
#pragma unroll
    for (int a = 0; a < MF; ++a)
#pragma unroll
        for (int f = 0; f < NF; ++f)
#pragma unroll
            for (int v = 0; v < 4; ++v) bad |= !__builtin_isfinite(acc[a][f][v]);
    bad = bad && kg == 0;  // group 0 holds the sums
    if (block_any(bad)) {
        const uint32_t c0 = g_begin * 64 * SW, c1 = min(g_end * SW, G) * 64;
        const uint32_t outs = T::kBM * T::kBN;
        for (uint32_t o = (uint32_t)tid; o < outs; o += T::kThreads) {
            const uint32_t mi = o / T::kBN, ni = o % T::kBN;
            const uint32_t m = m0 + mi;
            const uint32_t fw = ni / T::kWaveRows, fr = ni % T::kWaveRows;  // wave, row of its fragments
            const uint32_t n = nt * T::kBN + fw * T::kWaveRows + fr;
            if (m >= M || n >= N) continue;
            float gsum = 0.0f, usum = 0.0f;
            const uint16_t *xr = args.x + (size_t)m * args.ldx;
            for (uint32_t c = c0; c < c1; c += 8) {
                const uint32_t wq = P.w.qw[(size_t)n * (K >> 3) + (c >> 3)];
                const float sc = bf16_to_f32(P.w.sc[(size_t)n * G + (c >> 6)]), bi = bf16_to_f32(P.w.bi[(size_t)n * G + (c >> 6)]);
                uint32_t uq = 0;
                float usc = 0.0f, ubi = 0.0f;
                if (NW == 2) {
                    uq = P.w2.qw[(size_t)n * (K >> 3) + (c >> 3)];
                    usc = bf16_to_f32(P.w2.sc[(size_t)n * G + (c >> 6)]);
                    ubi = bf16_to_f32(P.w2.bi[(size_t)n * G + (c >> 6)]);
                }
#pragma unroll
                for (int j = 0; j < 8; ++j) {
                    const float x = bf16_to_f32(xr[c + j]);
                    gsum = fmaf(fmaf((float)((wq >> (4 * j)) & 15u), sc, bi), x, gsum);
                    if (NW == 2) usum = fmaf(fmaf((float)((uq >> (4 * j)) & 15u), usc, ubi), x, usum);
                }
            }
            if (EPI == kMfmaPartial) {
                float *dst = args.partial + ((size_t)ks * M + m) * (size_t)(NW * N) + n;
                dst[0] = gsum;
                if (NW == 2) dst[N] = usum;
                continue;
            }
            float val = gsum;
            if (NW == 2) val = activation(val, args.act) * usum;
            if (EPI == kMfmaDirect && P.bias) val += bf16_to_f32(P.bias[n]);
            const size_t oo = (size_t)m * P.ldo + n;
            if (args.out_f32) {
                float *out = reinterpret_cast<float *>(P.out);
                out[oo] = args.accumulate ? out[oo] + val : val;
            } else {
                uint16_t *out = reinterpret_cast<uint16_t *>(P.out);
                const uint32_t b = f32_to_bf16(args.accumulate ? val + bf16_to_f32(out[oo]) : val);
                out[oo] = (uint16_t)b;
                if (NW == 2 && args.out_h) {  // column n of its 8-column unit goes to 2 (n % 4) + (n % 8) / 4
                    const _Float16 hv = (_Float16)bf16_to_f32(b);
                    args.out_h[oo - n + (n & ~7u) + 2 * (n & 3u) + ((n & 7u) >> 2)] = __builtin_bit_cast(uint16_t, hv);
                }
            }
        }
        return;
    }

    // ---- epilogue.  A lane holds C[4 kq + v][c] of each 16 x 16 fragment: column pieces of 2 or 4
    // bytes.  The block's tile goes through LDS (past block_any's flag bytes; every read of the X
    // buffers and of the group reduction ended at a barrier) so that each thread then stores 8
    // consecutive columns of one row: one 16-byte store for bf16, two for f32.
    constexpr int kPitch = T::kBN + 4;  // floats per LDS row: 4 rows of a 16-column write hit distinct banks
    constexpr bool kPartial = EPI == kMfmaPartial;
    constexpr int kRows = (kPartial && NW == 2) ? 2 * T::kBM : T::kBM;  // partials: gate rows, then up rows
    float *tile = reinterpret_cast<float *>(lds + 256);
    if (kg == 0) {
#pragma unroll
        for (int fo = 0; fo < FPM; ++fo) {
            const int col = wave * T::kWaveRows + fo * 16 + c;
#pragma unroll
            for (int a = 0; a < MF; ++a)
#pragma unroll
                for (int v = 0; v < 4; ++v) {
                    const int row = a * 16 + 4 * kq + v;
                    const float g0 = acc[a][fo][v];
                    if constexpr (kPartial) {
                        tile[row * kPitch + col] = g0;
                        if constexpr (NW == 2) tile[(T::kBM + row) * kPitch + col] = acc[a][fo + FPM][v];
                    } else {
                        tile[row * kPitch + col] = NW == 2 ? activation(g0, args.act) * acc[a][fo + FPM][v] : g0;
                    }
                }
        }
    }
    __syncthreads();
    const uint32_t n_base = nt * T::kBN;
    const bool vec_out = kPartial ? ((uintptr_t)args.partial % 16 == 0 && N % 8 == 0)
                                  : ((uintptr_t)P.out % 16 == 0 && P.ldo % 8 == 0 &&
                                     (!(EPI == kMfmaDirect && P.bias) || (uintptr_t)P.bias % 16 == 0));
    constexpr int kUnitsPerRow = T::kBN / 8;
    for (uint32_t it = (uint32_t)tid; it < (uint32_t)(kRows * kUnitsPerRow); it += T::kThreads) {
        const uint32_t r = it / kUnitsPerRow, cu = it % kUnitsPerRow;
        const uint32_t row = r % T::kBM;
        const uint32_t m = m0 + row, n = n_base + cu * 8;
        if (m >= M || n >= N) continue;
        const float *src = tile + r * kPitch + cu * 8;
        float val[8];
#pragma unroll
        for (int e = 0; e < 8; ++e) val[e] = src[e];
        const bool full = vec_out && n + 8 <= N;
        if constexpr (kPartial) {
            float *dst = args.partial + ((size_t)ks * M + m) * (size_t)(NW * N) + (r / T::kBM) * N + n;
            if (full) {
                reinterpret_cast<f32x4 *>(dst)[0] = f32x4{val[0], val[1], val[2], val[3]};
                reinterpret_cast<f32x4 *>(dst)[1] = f32x4{val[4], val[5], val[6], val[7]};
            } else {
                for (int e = 0; e < 8 && n + e < N; ++e) dst[e] = val[e];
            }
            continue;
        }
        const size_t o = (size_t)m * P.ldo + n;
        if (full) {
            if (EPI == kMfmaDirect && P.bias) {
                const u32x4 bw = *reinterpret_cast<const u32x4 *>(P.bias + n);
                const uint32_t bb[4] = {bw.x, bw.y, bw.z, bw.w};
#pragma unroll
                for (int e = 0; e < 8; ++e) val[e] += bf16_to_f32((bb[e >> 1] >> (16 * (e & 1))) & 0xFFFFu);
            }
            if (args.out_f32) {
                f32x4 *out = reinterpret_cast<f32x4 *>(reinterpret_cast<float *>(P.out) + o);
                f32x4 lo = {val[0], val[1], val[2], val[3]}, hi = {val[4], val[5], val[6], val[7]};
                if (args.accumulate) {
                    lo += out[0];
                    hi += out[1];
                }
                out[0] = lo;
                out[1] = hi;
            } else {
                u32x4 *out = reinterpret_cast<u32x4 *>(reinterpret_cast<uint16_t *>(P.out) + o);
                if (args.accumulate) {
                    const u32x4 ow = out[0];
                    const uint32_t oo[4] = {ow.x, ow.y, ow.z, ow.w};
#pragma unroll
                    for (int e = 0; e < 8; ++e) val[e] += bf16_to_f32((oo[e >> 1] >> (16 * (e & 1))) & 0xFFFFu);
                }
                uint32_t pk[4];
#pragma unroll
                for (int e = 0; e < 4; ++e) pk[e] = f32_to_bf16(val[2 * e]) | (f32_to_bf16(val[2 * e + 1]) << 16);
                out[0] = u32x4{pk[0], pk[1], pk[2], pk[3]};
                if (NW == 2 && args.out_h)  // the same 8 values as the next projection's fp16 operand
                    *reinterpret_cast<u32x4 *>(args.out_h + o) = x_unit_f16(u32x4{pk[0], pk[1], pk[2], pk[3]});
            }
            continue;
        }
        for (int e = 0; e < 8 && n + e < N; ++e) {
            float x = val[e];
            if (EPI == kMfmaDirect && P.bias) x += bf16_to_f32(P.bias[n + e]);
            if (args.out_f32) {
                float *out = reinterpret_cast<float *>(P.out);
                out[o + e] = args.accumulate ? out[o + e] + x : x;
            } else {
                uint16_t *out = reinterpret_cast<uint16_t *>(P.out);
                const uint32_t b = f32_to_bf16(args.accumulate ? x + bf16_to_f32(out[o + e]) : x);
                out[o + e] = (uint16_t)b;
                if (NW == 2 && args.out_h) {  // element e of its 8-column unit goes to 2 (e % 4) + e / 4
                    const _Float16 hv = (_Float16)bf16_to_f32(b);
                    const uint32_t c = n + e;
                    args.out_h[o - n + (c & ~7u) + 2 * (c & 3u) + ((c & 7u) >> 2)] = __builtin_bit_cast(uint16_t, hv);
                }
            }
        }
    }
}

// One 16-byte unit (8 columns) per thread.
__global__ __launch_bounds__(256) void x_to_f16_kernel(const u32x4 *x, u32x4 *xh, uint32_t units) {
    const uint32_t i = blockIdx.x * 256u + threadIdx.x;
    if (i < units) xh[i] = x_unit_f16(x[i]);
}

hipError_t launch_x_to_f16(const uint16_t *x, uint32_t m, uint32_t k, uint16_t *xh, hipStream_t s) {
    if (k % 8 != 0 || (uintptr_t)x % 16 != 0 || (uintptr_t)xh % 16 != 0) return hipErrorInvalidValue;
    const uint64_t units = (uint64_t)m * (k / 8);
    if (units == 0) return hipSuccess;
    if (units >= (1ull << 32)) return hipErrorInvalidValue;
    hipLaunchKernelGGL(x_to_f16_kernel, dim3((uint32_t)((units + 255) / 256)), dim3(256), 0, s,
                       reinterpret_cast<const u32x4 *>(x), reinterpret_cast<u32x4 *>(xh), (uint32_t)units);
    return hipGetLastError();
}

template <int MF, int NF, int WAVES, int NW, int OCC, int D, int SW, int KW = 1>
static hipError_t launch_prefill_shape(MfmaArgs &a, hipStream_t s) {
    using T = PrefillTile<MF, NF, WAVES, NW, KW>;
    constexpr int kRing = KW * (D + 1) * T::kBM * 128 * SW;
    constexpr int kTile = 256 + T::kBM * (T::kBN + 4) * 4;  // the epilogue's tile (gate/up partials: two)
    constexpr int kLds = kRing > kTile ? kRing : kTile;
    constexpr int kLdsPartial = kRing > kTile + (NW - 1) * (kTile - 256) ? kRing : kTile + (NW - 1) * (kTile - 256);
    uint32_t tiles = 0;
    const uint32_t tiles_m = (a.m + T::kBM - 1) / T::kBM;
    for (int i = 0; i < a.np; ++i) {
        a.p[i].tile_begin = tiles;
        tiles += tiles_m * ((a.p[i].w.n + T::kBN - 1) / T::kBN);
    }
    if (a.ksplit <= 1) a.groups_per_split = a.k / 64;
    if (a.groups_per_split % SW != 0) return hipErrorInvalidValue;
    const dim3 grid(tiles, a.ksplit > 1 ? a.ksplit : 1);
    // split K over XCDs (q4_prefill_kernel): one problem, 8 % ksplit == 0 and whole tile ranges per XCD
    a.xcd_tiles = 0;
    if (tuning().prefill_xcd_split && a.np == 1 && (a.ksplit == 2 || a.ksplit == 4 || a.ksplit == 8) &&
        tiles % (8 / a.ksplit) == 0)
        a.xcd_tiles = tiles / (8 / a.ksplit);
    if (a.ksplit > 1) {
        hipLaunchKernelGGL((q4_prefill_kernel<MF, NF, WAVES, NW, OCC, kMfmaPartial, D, SW, KW>), grid, dim3(T::kThreads),
                           kLdsPartial, s, a);
        hipError_t e = hipGetLastError();
        if (e != hipSuccess) return e;
        return launch_splitk_reduce(a, NW, s);
    }
    hipLaunchKernelGGL((q4_prefill_kernel<MF, NF, WAVES, NW, OCC, kMfmaDirect, D, SW, KW>), grid, dim3(T::kThreads), kLds, s,
                       a);
    return hipGetLastError();
}

// Launch shapes (measured on MI355X at M = 512, K = 2048 / 11008) with
// 128-column steps (64-column steps where k / 64 is odd):
//   gate/up: 128 token rows x (4 waves x 16 gate + 16 up rows), one step of
//            look-ahead, 2 waves per SIMD (the 32 KB X slices fill the LDS);
//   plain:    64 token rows x (4 waves x 16 rows), one step of look-ahead, 4
//             waves per SIMD: the N = 2048 projections are short of blocks with
//             larger tiles (96 x 128: down 145 us, o 33 us; 64 x 64: 72 / 17.6 us);
//   split K: 128 token rows x (4 waves x 32 rows), one step of look-ahead, when
//             the MLP's workspace lets the down projection split K over blocks
//             (K split to about one block per CU: cfg2 down 4 ways, 37.0 us + 5.3 us
//             of reduction, against 96-row tiles split 8 ways, 38.9 + 7.2 us).
using GateUpShape = PrefillTile<8, 2, 4, 2>;
using PlainShape = PrefillTile<4, 1, 4, 1>;
using SplitShape = PrefillTile<8, 2, 4, 1>;  // plain projections whose K is split over blocks

uint32_t prefill_block_m(bool gate_up) { return gate_up ? GateUpShape::kBM : SplitShape::kBM; }
uint32_t prefill_block_rows(bool gate_up) { return gate_up ? GateUpShape::kBN : SplitShape::kBN; }

bool prefill_supported(const MfmaArgs &a) {
    // 32-bit buffer offsets: every operand must span < 4 GiB
    const uint64_t xbytes = (uint64_t)a.m * a.ldx * 2;
    if (xbytes >= (1ull << 32)) return false;
    for (int i = 0; i < a.np; ++i) {
        const uint64_t qbytes = (uint64_t)a.p[i].w.n * (a.k / 2);
        if (qbytes >= (1ull << 32)) return false;
    }
    return a.m > 16 && a.k % 64 == 0;
}

hipError_t launch_prefill(MfmaArgs &a, hipStream_t s) {
    const bool gate_up = a.p[0].w2.qw != nullptr;
    const uint32_t gps = a.ksplit > 1 ? a.groups_per_split : a.k / 64;
    if (tuning().prefill_kernel == 2 || a.k % 128 != 0 || gps % 2 != 0) {  // 64 columns per step
        if (gate_up) return launch_prefill_shape<8, 2, 4, 2, 3, 2, 1>(a, s);
        if (a.ksplit > 1) return launch_prefill_shape<8, 2, 4, 1, 3, 2, 1>(a, s);
        return launch_prefill_shape<4, 1, 4, 1, 4, 2, 1>(a, s);
    }
    if (gate_up) return launch_prefill_shape<8, 2, 4, 2, 2, 1, 2>(a, s);
    if (a.ksplit > 1) return launch_prefill_shape<8, 2, 4, 1, 2, 1, 2>(a, s);
    // Fewer tiles than two per compute unit (the N = 2048 .. 2560 projections at M = 512): two
    // groups of waves per tile split its steps (qkv 20.2 -> 19.0 us; four groups: 21.8 us).
    uint32_t tiles = 0;
    for (int i = 0; i < a.np; ++i) tiles += ((a.m + 63) / 64) * ((a.p[i].w.n + 63) / 64);
    if (tiles < 2u * (uint32_t)device_cus()) return launch_prefill_shape<4, 1, 4, 1, 2, 1, 2, 2>(a, s);
    return launch_prefill_shape<4, 1, 4, 1, 4, 1, 2>(a, s);
}

}  // namespace kr
