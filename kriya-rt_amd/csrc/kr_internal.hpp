// kr_internal.hpp — host-side launchers shared between the kernel files and
// the C ABI (kr_api.cpp).  Launchers assume validated arguments.
#pragma once

#include <hip/hip_runtime.h>
#include <stddef.h>
#include <stdint.h>

#include "kr_device.hpp"

namespace kr {

// Epilogues of the m == 1 GEMV.
enum GemvEpilogue : int {
    kStoreF32 = 0,
    kStoreBF16 = 1,
    kAccF32 = 2,
    kAccBF16 = 3,
    kGateUpF32 = 4,   // rows come from (gate, up) pairs, out = act(g) * u
    kGateUpBF16 = 5,
};

// Runtime tuning knobs (set through kr_set_option for sweeps; defaults are the
// measured best on MI355X).
struct Tuning {
    int gemv_rows_per_wave = 2;        // rows per wave tile: 1, 2, 4 or 8
    int gemv_block_rows = 2;           // rows per split-K block tile: 1, 2, 4 or 8
    int gemv_max_blocks = 0;           // > 0: cap on the grid (tests use it for grid invariance)
    int gemv_persistent_blocks = 1024; // grid of the persistent wave kernel
    int gemv_split_k_chunks = 0;       // rows of >= this many 16-byte chunks use the block kernel
                                       // (always beyond 128 chunks); 0 = default
    int skinny_max_blocks = 256;       // grid cap of the few-token kernel (blocks walk runs of tiles);
                                       // grouped MoE launches take twice this
    int prefill_kernel = 0;            // m > 16: 0 = register-dequant prefill kernel,
                                       // 1 = LDS-dequant tiled kernel
    int gemv_long_rows = 4;            // k > 4096: rows per block of the long-row kernels (4, 8, 16);
                                       // 0 = split-K block kernel
    int gemv_long_groups = 1;          // long-row kernel: row groups of 512 threads per block (1, 2)
    int gemv_tokens = 1;               // 2 <= m <= 4: GEMV kernels over the tokens (1) or the few-token
                                       // MFMA kernel (0)
    int moe_gemv = 1;                  // MoE with <= 16 assignments: routed GEMV (1) or grouped MFMA kernel (0)
    int moe_combine = 1;               // routed GEMV path, topk <= 4: combine folded into the down
                                       // projection (1) or a launch of its own (0)
    int moe_route_fused = 1;           // kr_q4_moe_route_experts with one token on the routed GEMV path:
                                       // routing inside the gate/up launch (1) or a launch of its own (0)
    int splitk_tickets = 1;            // few-token split K: 1 the last block of a run reduces, 0 a second launch
    int prefill_xcd_split = 1;         // prefill split K: each K split on its own XCDs (1) or the tile
                                       // grouping of unsplit launches (0)
    int attn_slice64 = 1;              // decode attention, head_dim 128: slices of 64 positions when they give
                                       // >= 1 block per CU (1), always (2), never: 16 (0)
    int attn_merge_oproj = 1;          // kr_rope_attention_q4_out, one sequence: the merge inside the output
                                       // projection's launch (1) or kr_rope_attention_decode + kr_q4_linear (0)
    int attn_merge_wave = 1;           // decode attention merge of <= 64 slices, D a power of two 8..256:
                                       // 1 the barrier-free wave kernel, 0 the general block kernel
    int prefill_operands = 1;          // kr_q4_mlp at m >= 64: 1 fp16 operands converted once per call
    int skinny_groups = 2;             // dense few-token launches: 16-row groups per launch (1 or 2)
    int skinny_depth = 0;              // dense few-token launches without epilogue operands: tiles
                                       // in flight + 1; 0 = 3 for runs of >= 6 tiles, else 2
};
Tuning &tuning();

// Largest k of the m == 1 kernels (three 16-byte chunks per thread of a 256-thread block).
constexpr uint32_t kMaxGemvK = 3 * 256 * 32;

hipError_t launch_format_dequant(const Q4Mat &w, float *out, hipStream_t s);
size_t stream_read_pieces(size_t bytes);
hipError_t launch_stream_read(const void *buf, size_t bytes, uint32_t match, uint32_t *hits, hipStream_t s);
hipError_t launch_from_blocks36(const void *blocks, uint32_t n, uint32_t k, uint32_t *qw, uint16_t *sc,
                                uint16_t *bi, hipStream_t s);
hipError_t launch_to_blocks36(const Q4Mat &w, void *blocks, hipStream_t s);
hipError_t launch_from_split(const void *qs, const void *sb, uint32_t n, uint32_t k, uint32_t *qw, uint16_t *sc,
                             uint16_t *bi, hipStream_t s);
hipError_t launch_to_split(const Q4Mat &w, void *qs, void *sb, hipStream_t s);
hipError_t launch_f16_to_bf16(const uint16_t *in, uint16_t *out, size_t count, hipStream_t s);

// ---- batched (m > 1) matrix-core path (q4_mfma.hip)
constexpr int kMaxMfmaProblems = 3;
enum MfmaEpilogue : int { kMfmaDirect = 0, kMfmaPartial = 1 };

struct MfmaProblem {
    Q4Mat w;                // N = w.n rows, k = MfmaArgs::k
    Q4Mat w2;               // up matrix for the gate/up epilogue (qw == nullptr otherwise)
    void *out;              // [m, ldo] bf16 or f32
    const uint16_t *bias;   // bf16 [N] added before the store, or nullptr
    uint32_t ldo;           // output row stride in elements
    uint32_t tile_begin;    // set by the launcher
};

struct MfmaArgs {
    MfmaProblem p[kMaxMfmaProblems];
    int np;
    const uint16_t *x;      // bf16 [m, ldx]
    uint32_t m, k, ldx;
    int act;                // activation of the gate/up epilogue
    int out_f32;            // 1: f32 outputs, 0: bf16
    int accumulate;         // 1: out += result (bf16: RNE of the f32 sum)
    float *partial;         // split-K partials [ksplit, m, nw * N] (ksplit > 1)
    uint32_t ksplit;
    uint32_t groups_per_split;
    // prefill kernel only (ignored elsewhere): x already converted to fp16 in the kernel's column
    // order (launch_x_to_f16), read instead of converting x per block; x stays the exact operand
    // of the overflow fallback
    const uint16_t *xh;
    // prefill gate/up with bf16 output only: also write the output converted the same way (the
    // next projection's xh), [m, ldo] fp16
    uint16_t *out_h;
    // prefill split K, set by the launcher: > 0 places each K split on 8 / ksplit XCDs, each taking
    // `xcd_tiles` consecutive tiles (see q4_prefill_kernel); 0 the default tile grouping
    uint32_t xcd_tiles;
};

// bm: the M tile class (16, 64 or 128) chosen by the caller from m.
hipError_t launch_mfma(MfmaArgs &a, int bm, hipStream_t s);
// Prefill kernel (q4_prefill.hip): m > 16, k % 64 == 0, operands < 4 GiB.
bool prefill_supported(const MfmaArgs &a);
hipError_t launch_prefill(MfmaArgs &a, hipStream_t s);
// xh[m, k] = fp16 of bf16 x[m, k] (RNE; beyond 65504 -> inf), each 8 columns in the order
// e0 e4 e1 e5 e2 e6 e3 e7 of the prefill kernel's operands.  k % 8 == 0, 16-byte aligned rows.
hipError_t launch_x_to_f16(const uint16_t *x, uint32_t m, uint32_t k, uint16_t *xh, hipStream_t s);
int device_cus();                               // compute units of the current device
uint32_t prefill_block_m(bool gate_up);         // token rows per block
uint32_t prefill_block_rows(bool gate_up);      // weight rows (per matrix) per block
// Fixed-order sum of split-K partials [ksplit, m, nw * N] + the epilogue of p[0].
hipError_t launch_splitk_reduce(const MfmaArgs &a, int nw, hipStream_t s);

// ---- few-token (m <= 16) and grouped MoE matrix-core path (q4_skinny.hip)
constexpr uint32_t kSkinnyMaxM = 32;       // rows of one dense launch (two groups of 16)
constexpr uint32_t kSkinnyChunkMaxM = 63;  // the host runs 33..63 rows as 32-row chunks
// Rows of one dense few-token launch under the current tuning.
inline uint32_t skinny_chunk_rows() { return tuning().skinny_groups == 1 ? 16u : kSkinnyMaxM; }
constexpr uint32_t kMaxExperts = 256;
struct SkinnyArgs {
    Q4Mat w, w2;            // w2: up matrix for the gate/up epilogue (qw == nullptr otherwise)
    const uint16_t *x;      // bf16 [rows, ldx]
    uint32_t m, k, ldx;     // m: token rows (dense mode)
    void *out;              // [rows, ldo]
    const uint16_t *bias;   // bf16 [n] or nullptr (dense mode)
    uint32_t ldo;
    int act, out_f32, accumulate;
    float *partial;         // [ksplit, m, nw * n] when the K split exceeds one block, else nullptr
    uint32_t *tickets;      // dense split K: kSkinnyTickets words, zero on entry and on return; the
                            // last block of each run reduces it (no second launch); nullptr: caller reduces
    uint32_t ksplit;        // set by the launcher
    // grouped (MoE) mode; offsets == nullptr selects dense mode
    const uint32_t *offsets;  // [experts + 1] bucket offsets into `sorted`
    const uint32_t *sorted;   // expert-sorted assignment ids
    uint32_t experts;         // E; w (and w2) stack E matrices of expert_rows rows
    uint32_t expert_rows;
    uint32_t x_div;           // > 0: X row of sorted position p is sorted[p] / x_div; 0: row p
    int out_scatter;          // 1: result row of sorted position p goes to row sorted[p]; 0: row p
    uint32_t max_active;      // upper bound of non-empty buckets (sizes the grid)
    // dense mode only: up to two more problems sharing x and k (the K and V
    // projections next to Q), each with its own weights, output and bias
    struct More {
        Q4Mat w;
        void *out;
        const uint16_t *bias;
        uint32_t ldo;
    } more[2];
    int nmore;
    uint32_t tile_begin[4];   // set by the launcher: problem i's first tile; [nmore + 1] = all tiles
    // dense mode, k <= 2048: x rows are RMS-normalised while staged,
    // bf16(x * rsqrt(mean(x^2) + eps) * ln_w) as kr_rmsnorm computes it
    const uint16_t *ln_w;
    float eps;
};
constexpr uint32_t kSkinnyTickets = 512;        // ticket words of a split-K skinny launch (runs per slab)
constexpr uint32_t kSkinnyMaxTicketSplit = 8;   // K slabs the in-kernel reduction takes (k <= 16384)
hipError_t launch_skinny(SkinnyArgs &a, hipStream_t s);

// Routed MoE GEMV: one token per (expert, sorted position) pair on the m = 1
// wave kernel, for few assignments.  Position p of the expert-sorted list
// belongs to the expert whose bucket [offsets[e], offsets[e+1]) holds it; its
// x row is sorted[p] / x_div (x_div > 0) or p, its output row sorted[p]
// (out_scatter) or p.  k <= 2048.
struct MoeGemvArgs {
    Q4Mat w, w2;                // stacked experts (w2: up matrix of the gate/up epilogue, else == w)
    uint32_t rows;              // rows per expert
    const uint16_t *x;          // bf16 [.., k]
    uint32_t x_div;
    const uint32_t *offsets;    // [experts + 1]
    const uint32_t *sorted;     // [assign]
    uint32_t experts, assign;
    void *out;                  // [.., ldo]
    uint32_t ldo;
    int out_scatter, act;
    uint32_t tiles_per;         // set by the launcher
    // One token routed inside the launch (logits != nullptr; gate/up only): every wave takes the
    // token's softmax and top-k itself, and wave 0 of block 0 writes the routing arrays as the
    // routing kernel does.  offsets/sorted above are then outputs, not inputs.
    const float *logits;        // f32 [experts]
    int normalize;
    uint32_t topk;
    uint32_t *r_selected, *r_counts;
    float *r_weights;
};
constexpr uint32_t kMoeGemvMaxAssign = 16;  // the routed GEMV is used up to this many assignments
// The routed down projection with the combine folded in (topk <= 4, rows of k <= 2048 columns).
struct MoeDownArgs {
    Q4Mat w;                    // stacked down matrices [experts * rows, k]
    uint32_t rows;              // rows per expert (hidden)
    const uint16_t *h;          // bf16 [assign, k], expert-sorted order
    const uint32_t *offsets;    // [experts + 1]
    const uint32_t *sorted;     // [assign]
    const float *weights;       // [tokens * topk]
    uint32_t experts, tokens, topk;
    void *y;                    // [tokens, rows], f32 or bf16
    int y_f32, accumulate;
};
bool moe_down_combine_fits(uint32_t k, uint32_t topk);
hipError_t launch_moe_down_combine(const MoeDownArgs &a, hipStream_t s);
bool moe_gemv_fits(uint32_t k);
hipError_t launch_moe_gemv(MoeGemvArgs &a, int epilogue, hipStream_t s);
// True when launch_moe_gemv can route the (single) token inside the gate/up launch.
bool moe_gemv_route_fits(uint32_t experts, uint32_t topk);

// ---- MoE routing and combine (moe.hip)
constexpr uint32_t kRouteMaxTopK = 16;      // top-k list length of the routing kernel
constexpr uint32_t kRouteMaxAssign = 16384; // T * K held in the routing block's LDS
// logits == nullptr: `experts` [T*K] are given and only counts/offsets/sorted are produced.
hipError_t launch_moe_route(const float *logits, uint32_t T, uint32_t E, uint32_t K, int normalize,
                            uint32_t *experts, float *weights, uint32_t *counts, uint32_t *offsets, uint32_t *sorted,
                            hipStream_t s);
hipError_t launch_moe_combine(const float *d, const float *w, uint32_t T, uint32_t K, uint32_t H, void *y, int y_f32,
                              int accumulate, hipStream_t s);
// Number of K splits (blocks per N tile) the dense skinny launcher uses for rows of k columns.
uint32_t skinny_ksplit(uint32_t k);
// True when one block of the grouped kernel covers rows of k columns (no K split).
bool skinny_grouped_fits(uint32_t k);
// The few-token kernel needs k % 64 == 0, and 4-byte aligned scales/biases when k % 128 == 0
// (an odd group count loads them 2 bytes at a time); its grouped (MoE) mode needs k % 128 == 0.
bool skinny_supported(const Q4Mat &w);

// ---- embedding and end-to-end glue (e2e_glue.hip)
constexpr uint32_t kGlueMaxCtx = 8192;
constexpr uint32_t kGlueMaxHeadDim = 256;
hipError_t launch_q4_embedding(const Q4Mat &w, const uint32_t *tokens, uint32_t count, uint16_t *out, hipStream_t s);
hipError_t launch_rmsnorm(const uint16_t *x, const uint16_t *weight, uint32_t rows, uint32_t dim, float eps,
                          uint16_t *out, hipStream_t s);
hipError_t launch_rope_kv_append(uint16_t *q, const uint16_t *k, const uint16_t *v, const float *cos_sin,
                                 const uint32_t *positions, uint32_t batch, uint32_t q_heads, uint32_t kv_heads,
                                 uint32_t D, uint16_t *k_cache, uint16_t *v_cache, uint32_t max_ctx, hipStream_t s);
hipError_t launch_attention_decode(const uint16_t *q, const uint16_t *k_cache, const uint16_t *v_cache,
                                   const uint32_t *positions, uint32_t batch, uint32_t q_heads, uint32_t kv_heads,
                                   uint32_t D, uint32_t max_ctx, uint16_t *out, hipStream_t s);
hipError_t launch_argmax(const float *logits, uint32_t rows, uint32_t n, uint32_t *out, hipStream_t s);
// The same result from P blocks per row and a merge launch (workspace: argmax_workspace_bytes).
constexpr uint32_t kArgmaxMaxParts = 512;
uint32_t argmax_parts(uint32_t rows, uint32_t n);
size_t argmax_workspace_bytes(uint32_t rows, uint32_t n);
hipError_t launch_argmax_split(const float *logits, uint32_t rows, uint32_t n, uint32_t *out, void *ws, hipStream_t s);
constexpr uint32_t kGlueMaxGroup = 16;  // query heads per kv head of the split attention
size_t attention_workspace_bytes(uint32_t batch, uint32_t q_heads, uint32_t D, uint32_t max_ctx);
// One sequence: the 64-position-slice partials of kr_rope_attention_decode (head_dim 128, G <= 16)
// and their merge fused into the output projection h (+)= x . W^T (w.k = q_heads * 128 <= 2048,
// at most 16 slices).
constexpr uint32_t kMergeOprojMaxSlices = 16;
uint32_t attention_slices64(uint32_t max_ctx);
hipError_t launch_rope_attention_partials64(const uint16_t *q, const uint16_t *k, const uint16_t *v,
                                            const float *cos_sin, const uint32_t *positions, uint32_t batch,
                                            uint32_t q_heads, uint32_t kv_heads, uint16_t *k_cache,
                                            uint16_t *v_cache, uint32_t max_ctx, float *part, hipStream_t s);
hipError_t launch_attention_merge_oproj(const float *part, uint32_t q_heads, uint32_t kv_heads, uint32_t splits,
                                        const Q4Mat &w, void *h, int h_f32, hipStream_t s);
hipError_t launch_rope_attention(const uint16_t *q, const uint16_t *k, const uint16_t *v, const float *cos_sin,
                                 const uint32_t *positions, uint32_t batch, uint32_t q_heads, uint32_t kv_heads,
                                 uint32_t D, uint16_t *k_cache, uint16_t *v_cache, uint32_t max_ctx, uint16_t *out,
                                 float *part, hipStream_t s);

// One launch of the m == 1 wave kernel over up to three problems sharing x and
// k (k <= 4096): mats[i] (with up[i] for the gate/up epilogues) -> outs[i]
// (+ biases[i] for the store epilogues).  ln_w != nullptr: x is RMS-normalised
// first (kr_rmsnorm's arithmetic).
bool gemv_batch_supported(uint32_t k);
hipError_t launch_gemv_batch(const Q4Mat *mats, const Q4Mat *up, const uint16_t *x, void *const *outs,
                             const uint16_t *const *biases, int np, int epilogue, int act, const uint16_t *ln_w,
                             float eps, hipStream_t s);

// y = W x for one token; `b` is the up matrix for the gate/up epilogues;
// `bias` (bf16 [n] or nullptr) is added by the store epilogues.
// 2 <= m <= kGemvMaxTokens tokens on the GEMV kernels (every unpacked word
// multiplied with all tokens): k <= 2048, or k <= 16384 without the gate/up
// epilogue.  Output row t at out + t * ldo elements.
constexpr uint32_t kGemvMaxTokens = 4;
bool gemv_tokens_supported(uint32_t m, uint32_t k, bool gate_up);
hipError_t launch_gemv_tokens(const Q4Mat &a, const Q4Mat *b, const uint16_t *x, uint32_t m, void *out, uint32_t ldo,
                              int epilogue, int act, const uint16_t *bias, hipStream_t s);
hipError_t launch_gemv(const Q4Mat &a, const Q4Mat *b, const uint16_t *x, void *out, int epilogue,
                       int activation, const uint16_t *bias, hipStream_t s);

}  // namespace kr
