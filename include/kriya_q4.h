/*
 * kriya_q4.h — C ABI of the MI355X (gfx950) Q4_G64 matmul path.
 *
 * Drop-in boundary for kriya-rt's Q4 operator surface
 * (crates/kriya-backend-metal/src/encoder.rs, MetalExecutor::encode_q4_*).
 * Each entry point names the reference function it replaces.
 *
 * Conventions
 *   - The caller owns all device memory.  Pointers are device pointers unless
 *     a comment says otherwise.  No entry point allocates device memory.
 *   - Calls enqueue work on `stream` (a hipStream_t; NULL = the null stream)
 *     and return at once.  0 on success, a negative KR_E* code on failure;
 *     kr_last_error() returns the message (thread-local).
 *   - Shapes and alignment are checked on the host before any launch; a call
 *     that fails a check enqueues nothing.  (The reference performs no shape
 *     checks in its encode functions, encoder.rs:2361-2536.)
 *   - Calls on distinct streams are independent; the library keeps no
 *     per-call state on the device (except kr_q4_mlp_noalloc, whose device
 *     scratch array is shared by every call on one GPU).
 *   - Results do not depend on the launch grid: every output element is
 *     reduced by one wavefront in a fixed order (no atomics on data).
 *   - Activation range.  For m < 64 token rows (the GEMV and few-token
 *     kernels) every bf16 x is multiplied exactly (bf16 products, f32 sums).
 *     For m >= 64 (the prefill kernel) x is staged in fp16, as the reference's
 *     M >= 64 kernels stage half (q4_gemm_and_moe.metal:2722-2724): exact for
 *     |x| in [2^-14, 65504]; a tile whose sums overflow fp16 is recomputed in
 *     f32 (exact), and values below 2^-14 keep fp16's subnormal precision
 *     (absolute error <= 2^-25 per element).  Weights are rounded once to fp16
 *     there (w = fma(q, s, b)); elsewhere they are exact.
 *
 * Weight format (kr_q4_matrix): the planar affine Q4_G64 triplet
 *   qw     u32  [n, k/8]   word w of row r holds elements 8w..8w+7 of that
 *                          row, element 8w+j in bits 4j..4j+3
 *   scales bf16 [n, k/64]  raw bits
 *   biases bf16 [n, k/64]  raw bits
 *   w[r, c] = fma(q, scale, bias)            (quantizer.rs:112-126)
 * Its nibble plane is byte-identical to the `qs` bytes of kriya's 36-byte
 * BlockQ4Group64 (tensor.rs:104-115): kr_q4_from_blocks36() converts.
 */
#ifndef KRIYA_Q4_H
#define KRIYA_Q4_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define KR_ABI_VERSION 1

/* ---- error codes ---- */
#define KR_OK 0
#define KR_E_INVALID (-1)     /* null pointer, bad enum, bad count            */
#define KR_E_SHAPE (-2)       /* k % 64 != 0, mismatched matrices, too large  */
#define KR_E_ALIGN (-3)       /* a pointer is not aligned as documented        */
#define KR_E_HIP (-4)         /* the HIP runtime reported an error             */
#define KR_E_WORKSPACE (-5)   /* workspace missing or smaller than required    */
#define KR_E_UNSUPPORTED (-6) /* no kernel for this combination                */

/* ---- element types of activations / outputs ---- */
#define KR_DTYPE_BF16 0
#define KR_DTYPE_F32 1

/* ---- gated activations (descriptor.rs ActivationVariant; encoder.rs:2718-2722) ---- */
#define KR_ACT_SWIGLU 0 /* silu(g) * u; silu(g) = g / (1 + e^-g) computed as g * rcp(1 + exp2(-g log2 e))
                         * on the hardware exp2 and reciprocal (about 1 ulp of f32 each)               */
#define KR_ACT_GEGLU 1  /* gelu_tanh(g) * u                 */
#define KR_ACT_RELU 2   /* max(g, 0) * u                    */

typedef struct kr_q4_matrix {
    const uint32_t *qw;     /* [n, k/8], 16-byte aligned            */
    const uint16_t *scales; /* [n, k/64] bf16 bits, 2-byte aligned  */
    const uint16_t *biases; /* [n, k/64] bf16 bits, 2-byte aligned  */
    uint32_t n;             /* rows = output features               */
    uint32_t k;             /* columns = input features, k % 64 == 0 */
} kr_q4_matrix;

/* ---- library ---- */
int kr_abi_version(void);
/* Message of the last failed call on this thread ("" if none). */
const char *kr_last_error(void);

/* Process-wide launch tuning (no counterpart in the reference, whose launch
 * shapes are fixed in encoder.rs).  Not synchronised with calls in flight on
 * other threads.  Results never depend on these values. */
#define KR_OPT_GEMV_ROWS_PER_WAVE 1     /* rows per wave tile: 1, 2 (default), 4 or 8     */
#define KR_OPT_GEMV_MAX_BLOCKS 2        /* 0 (default): no cap; > 0: cap on the grid       */
#define KR_OPT_GEMV_SPLIT_K_CHUNKS 3    /* m == 1 rows of >= value 16-byte chunks use the
                                           split-K block kernel (always for k > 4096);
                                           0 (default): only beyond k = 4096               */
#define KR_OPT_GEMV_BLOCK_ROWS 4        /* rows per split-K block tile: 1, 2 (default), 4, 8 */
#define KR_OPT_GEMV_PERSISTENT_BLOCKS 5 /* grid of the persistent wave kernel (1024)       */
#define KR_OPT_SKINNY_MAX_BLOCKS 6      /* grid cap of the few-token kernel (256; grouped
                                           MoE launches take twice this)                  */
#define KR_OPT_PREFILL_KERNEL 7         /* m > 16: 0 register-dequant (default), 1 tiled, 2 register-dequant
                                           with 64-column steps (0 takes 128 where k allows) */
#define KR_OPT_GEMV_LONG_ROWS 8         /* k > 4096 rows per long-row block: 4 (default), 8, 16; 0 split-K */
#define KR_OPT_GEMV_TOKENS 9            /* 2 <= m <= 4: 1 (default) the GEMV kernels take all tokens per
                                           unpacked word (k <= 2048, or k <= 16384 without gate/up);
                                           0 the few-token MFMA kernel */
#define KR_OPT_MOE_GEMV 10              /* kr_q4_moe_experts with tokens * topk <= 16: 1 (default) one GEMV
                                           per (expert, token) pair, 0 the grouped MFMA kernel */
#define KR_OPT_GEMV_LONG_GROUPS 11      /* long-row kernel: row groups of 512 threads per block, each
                                           taking rows / groups of the block's rows: 1 (default) or 2 */
#define KR_OPT_SPLITK_TICKETS 12        /* kr_q4_mlp at 2 <= m <= 16: 1 (default) the down projection's
                                           K split is reduced by the last block of each run (one launch),
                                           0 by a second launch */
#define KR_OPT_ATTN_MERGE_WAVE 13       /* kr_rope_attention_decode: 1 (default) the slices of a head are merged
                                           by a kernel without block barriers when there are <= 64 of
                                           them and D is a power of two from 8 to 256, 0 always by the
                                           general kernel (same bits) */
#define KR_OPT_PREFILL_OPERANDS 14      /* kr_q4_mlp at m >= 64: 1 (default) x is converted to the prefill
                                         * kernel's fp16 operand once per call and the gate/up launch writes
                                         * the activation in that form as well; 0 every block converts its
                                         * own X slices.  Bitwise the same results either way. */
#define KR_OPT_SKINNY_GROUPS 15         /* few-token kernel, 17 <= m <= 63: 2 (default) 32-row launches, each
                                         * multiplying every unpacked weight word with two 16-row groups
                                         * of x; 1 16-row launches.  Bitwise the same results either way. */
#define KR_OPT_SKINNY_DEPTH 16          /* few-token kernel, launches with no bias and no accumulation:
                                         * 0 (default) three register buffers of tile words (two tiles
                                         * in flight) when a block's run holds >= 6 tiles, else two;
                                         * 2 or 3 forces that depth.  Bitwise the same results. */
#define KR_OPT_MOE_COMBINE 17          /* kr_q4_moe_experts on the routed GEMV path (option 10) with
                                         * topk <= 4: 1 (default) the combine is folded into the down
                                         * projection's launch; 0 a launch of its own.  Bitwise the same. */
#define KR_OPT_MOE_ROUTE_FUSED 18      /* kr_q4_moe_route_experts / kr_q4_moe_block with one token on the
                                         * routed GEMV path: 1 (default) the routing runs inside the gate/up
                                         * launch; 0 the routing kernel first.  Bitwise the same. */
#define KR_OPT_PREFILL_XCD_SPLIT 19     /* prefill kernel with K split over blocks (kr_q4_mlp's down
                                         * projection at m >= 64): 1 (default) the blocks of each K split
                                         * are placed on their own XCDs, so that an L2 holds one K range
                                         * of x; 0 the tile grouping of unsplit launches.  Bitwise the same. */
#define KR_OPT_ATTN_SLICE64 20          /* kr_rope_attention_decode with head_dim 128: slices of 64 positions
                                         * (one wave per 16 of them, all dims) instead of 16 (four waves
                                         * over the dims): 1 (default) when batch * kv_heads * slices still
                                         * gives one block per compute unit, 2 always, 0 never.  The f32
                                         * sums differ in order. */
#define KR_OPT_ATTN_MERGE_OPROJ 21      /* kr_rope_attention_q4_out with one sequence, head_dim 128: 1 (default)
                                         * the slices' merge runs inside the output projection's launch;
                                         * 0 kr_rope_attention_decode, then kr_q4_linear (accumulate). */
int kr_set_option(int option, int value);
int kr_get_option(int option);

/* ---- format boundary ---- */

/* Bit-exact dequantisation: out[r, c] = fma(q, scale, bias) as f32 [n, k].
 * Replaces dequantize_q4_group64_to_f32 (crates/kriya-core/src/quantizer.rs:112-126)
 * for on-device checks.  out 16-byte aligned. */
int kr_q4_dequant(const kr_q4_matrix *w, float *out, void *stream);

/* 36-byte BlockQ4Group64 blocks [n, k/64] (tensor.rs:104-115; block (r, g) at
 * index r*(k/64)+g, q4_gemm_and_moe.metal:951) -> planar triplet.  The nibble
 * bytes are copied verbatim.  blocks 4-byte aligned, qw 16-byte aligned.
 * Replaces the bind-time repack of encoder.rs:651-703 / safetensors_loader.rs:221-273. */
int kr_q4_from_blocks36(const void *blocks, uint32_t n, uint32_t k,
                        uint32_t *qw, uint16_t *scales, uint16_t *biases, void *stream);
/* Planar triplet -> 36-byte blocks (inverse of the above, byte-identical). */
int kr_q4_to_blocks36(const kr_q4_matrix *w, void *blocks, void *stream);

/* Split planes (tensor.rs:117-211: ScaledAlignedQ4Block [n * k/64] of 32
 * nibble bytes, 16-byte aligned, and BlockQ4ScaleBias [n * k/64] {scale_bf16,
 * bias_bf16}; block (r, g) at index r*(k/64)+g, the layout split_slice makes for
 * the consolidated QKV, encoder.rs:998-1015) -> planar triplet.  The nibble
 * plane holds the planar qw bytes unchanged, so qw may equal qs (then only the
 * pairs are split); otherwise it is copied.  qs, qw 16-byte aligned, sb 4-byte.
 * Replaces BlockQ4Group64::from_split (tensor.rs:172-187) feeding a planar bind. */
int kr_q4_from_split(const void *qs, const void *sb, uint32_t n, uint32_t k,
                     uint32_t *qw, uint16_t *scales, uint16_t *biases, void *stream);
/* Planar triplet -> split planes (inverse of the above; qs may equal w->qw).
 * Replaces BlockQ4Group64::split_slice (tensor.rs:156-170). */
int kr_q4_to_split(const kr_q4_matrix *w, void *qs, void *sb, void *stream);

/* MLX scale/bias planes stored as IEEE half -> bf16 bits, element-wise:
 * bf16_rne(f16_to_f32(h)).  Replaces parse_half_endian(is_f16 = true)
 * (safetensors_loader.rs:310-318; quantizer.rs:19-57).  in may equal out. */
int kr_f16_to_bf16(const uint16_t *in, uint16_t *out, size_t count, void *stream);

/* ---- Q4 linear: encoder.rs:2361-2420 (encode_q4_linear) and
 *      encoder.rs:2497-2536 (encode_q4_linear_accumulate) ----
 * y[i, r] = sum_c x[i, c] * w[r, c] for i < m, accumulated in f32.
 *   x: bf16 [m, w->k], 16-byte aligned (the reference's input_byte_offset is
 *      folded into the pointer by the caller).
 *   y: [m, w->n] of y_dtype.
 *   accumulate = 0: y = result (bf16 outputs are RNE of the f32 result).
 *   accumulate = 1: y = y + result, in place; for KR_DTYPE_BF16 the stored
 *      value is bf16(f32(y) + result) (q4_gemm_and_moe.metal:1407-1420).
 * m == 1 runs the decode GEMV; m > 1 runs the batched kernels. */
int kr_q4_linear(const kr_q4_matrix *w, const uint16_t *x, uint32_t m,
                 void *y, int y_dtype, int accumulate, void *stream);

/* The same Q4 linear (encoder.rs:2361-2420, 2497-2536; the same y and the
 * same accumulate semantics) with a caller workspace.  The workspace lets
 * 5 <= m rows over a long K (more than 2048 columns, and at m >= 64 few
 * output tiles) split K over blocks into f32 partials, summed in a fixed
 * order.  kr_q4_linear has no such buffer: there a few tokens over a long row
 * take the token GEMV in chunks, and more take the unsplit tiled kernel.
 * Results are within f32 summation order of kr_q4_linear's, and the same
 * bits from run to run.
 * workspace: kr_q4_linear_workspace_bytes(m, w->n, w->k) bytes, 16-byte
 * aligned, zero-filled once before its first use.  It holds the counters
 * that pick the block that sums a tile's partials, and every call leaves
 * them at zero.  Calls sharing a workspace must not overlap in time.  A
 * workspace sized for (m, n, k) serves every smaller m with the same n and k.
 * m <= 1 needs none (0 bytes; workspace may be NULL). */
size_t kr_q4_linear_workspace_bytes(uint32_t m, uint32_t n, uint32_t k);
int kr_q4_linear_ws(const kr_q4_matrix *w, const uint16_t *x, uint32_t m,
                    void *y, int y_dtype, int accumulate,
                    void *workspace, size_t workspace_bytes, void *stream);

/* ---- fused gate+up+activation: encoder.rs:2703-2848 (encode_fused_gate_up) ----
 * a[i, j] = act(gate_j . x_i) * (up_j . x_i) for j < gate->n, both dots in f32.
 *   gate, up: same n (intermediate) and k (hidden).
 *   act_out: [m, gate->n] of act_dtype (bf16 = RNE of the f32 value, as the
 *   reference kernels store it, q4_gemm_and_moe.metal:2076). */
int kr_q4_gate_up_act(const kr_q4_matrix *gate, const kr_q4_matrix *up,
                      const uint16_t *x, uint32_t m, void *act_out, int act_dtype,
                      int activation, void *stream);

/* ---- fused Q/K/V projections: encoder.rs:2539-2619 (encode_fused_qkv;
 *      kernels q4_g64_decode_qkv_gemv* and q4_g64_batched_simdgroup_qkv_gemm_m64,
 *      q4_gemm_and_moe.metal:1564-1793, 2853-3022) ----
 * q_out[i] = x_i . q^T (+ q_bias), same for k and v; q, k, v share k (hidden).
 * Biases are bf16 [n] or NULL (Qwen2 has them, quantizer.rs:395).  Outputs are
 * [m, n] of out_dtype; for bf16 the stored value is RNE(f32 dot + f32 bias).
 * m > 1 runs the three projections in one launch. */
int kr_q4_qkv(const kr_q4_matrix *q, const kr_q4_matrix *k, const kr_q4_matrix *v,
              const uint16_t *q_bias, const uint16_t *k_bias, const uint16_t *v_bias,
              const uint16_t *x, uint32_t m, void *q_out, void *k_out, void *v_out,
              int out_dtype, void *stream);

/* ---- dense MLP: encoder.rs:2851-2906 (encode_dense_mlp) ----
 * h[i, :] += down . bf16(act(gate . h_i) * (up . h_i))   for i < m
 * The residual h is read as bf16 and updated in place (h_dtype bf16: stored
 * RNE of f32(h) + f32 sum; f32: f32 += sum).  The MLP input is the bf16 view
 * of h; for h_dtype f32 a separate bf16 input x must be given (x may be NULL
 * when h_dtype is bf16, then x = h).  The intermediate activation is kept in
 * bf16 in the workspace, as the reference stores it.
 * workspace: device memory of at least
 * kr_q4_mlp_workspace_bytes(m, gate->k, gate->n), 16-byte aligned; calls that
 * share a workspace must not overlap in time.  For m > 1 the workspace also
 * holds split-K partial sums of the down projection, reduced in a fixed order,
 * and the counters that pick the block that reduces them (at its start, the
 * same place for every m): zero-fill the workspace once before its first use
 * (every call leaves them zero); a workspace sized for the largest m serves
 * every smaller one. */
size_t kr_q4_mlp_workspace_bytes(uint32_t m, uint32_t hidden, uint32_t intermediate);
int kr_q4_mlp(const kr_q4_matrix *gate, const kr_q4_matrix *up, const kr_q4_matrix *down,
              const uint16_t *x, void *h, int h_dtype, uint32_t m, int activation,
              void *workspace, size_t workspace_bytes, void *stream);

/* ---- dense MLP without a workspace (no counterpart in the reference) ----
 * For callers that cannot allocate device memory: code under HIP graph capture,
 * tight serving loops, harnesses that forbid hipMalloc.  Same arguments, results
 * and kernels as kr_q4_mlp, but the workspace is a device array inside the
 * library: kr_q4_mlp_noalloc_max_bytes() (4 MiB) on each GPU, held until the
 * process ends.  A call whose kr_q4_mlp_workspace_bytes(m, hidden, inter)
 * exceeds it fails with KR_E_WORKSPACE and enqueues nothing (cfg-1 shape
 * hidden 2048, inter 11008: m <= 37).  Allocates nothing, on the device or the
 * host.  The first call on a device also enqueues a small kernel that zeroes
 * the array's split-K counters.  All calls on one GPU share its array: calls
 * that overlap in time on one GPU (other streams, other threads) race. */
size_t kr_q4_mlp_noalloc_max_bytes(void);
int kr_q4_mlp_noalloc(const kr_q4_matrix *gate, const kr_q4_matrix *up, const kr_q4_matrix *down,
                      const uint16_t *x, void *h, int h_dtype, uint32_t m, int activation, void *stream);

/* ---- MoE routing: q4_gemm_and_moe.metal:2495-2624 (moe_router_topk_and_histogram
 *      + moe_router_prefix_scan_and_scatter, dispatched at encoder.rs:5275-5313) ----
 * logits: f32 [tokens, experts].  Per token: softmax, then the top `topk`
 * probabilities by insertion with strict '>' (ties go to the lower expert id),
 * renormalised by their sum (floored at 1e-8) when normalize != 0.
 * Outputs (device):
 *   selected      u32 [tokens, topk]  expert ids, descending probability
 *   weights       f32 [tokens, topk]
 *   counts        u32 [experts]
 *   offsets       u32 [experts + 1]   exclusive prefix sum of counts
 *   sorted_assign u32 [tokens * topk] assignment ids a = t * topk + k grouped by
 *                 expert: bucket e is sorted_assign[offsets[e] .. offsets[e+1]),
 *                 increasing a inside a bucket.
 * Deterministic (the reference's bucket order depends on atomic timing).
 * Limits: experts <= 256, topk <= min(experts, 16), tokens * topk <= 16384. */
int kr_moe_route(const float *logits, uint32_t tokens, uint32_t experts, uint32_t topk, int normalize,
                 uint32_t *selected, float *weights, uint32_t *counts, uint32_t *offsets,
                 uint32_t *sorted_assign, void *stream);

/* The scan/scatter stage alone (q4_gemm_and_moe.metal:2578-2624) for given
 * assignments selected[num_assign]: counts, offsets and sorted_assign as above.
 * An id >= experts joins no bucket, so offsets[experts] < num_assign reports it.
 * Limits: experts <= 256, num_assign <= 16384. */
int kr_moe_scan_scatter(const uint32_t *selected, uint32_t num_assign, uint32_t experts,
                        uint32_t *counts, uint32_t *offsets, uint32_t *sorted_assign, void *stream);

/* ---- routed Q4 experts + combine: encoder.rs:5316-5445 (q4_g64_routed_moe_gemv
 *      for gate, up and down, q4_gemm_and_moe.metal:2642-2698;
 *      fused_gated_activation_bf16 and moe_combine_routed_and_shared_bf16,
 *      transformer_glue.metal:307-336, 373-401) ----
 * gate, up: `experts` stacked matrices, n = experts * inter, k = hidden
 * (expert e owns rows e*inter .. (e+1)*inter); down: n = experts * hidden, k = inter.
 * For each assignment a = t * topk + k with expert e:
 *   h_a = bf16(act(gate_e . x_t) * (up_e . x_t)),   d_a = down_e . h_a  (f32),
 *   y[t] = sum over k = 0 .. topk-1 of fma(weights[a], d_a, acc), in slot order,
 * stored as y_dtype; accumulate = 1 adds it to y as kr_q4_linear does.  A
 * shared expert (moe_combine_routed_and_shared_bf16 with has_shared_expert,
 * transformer_glue.metal:396-398) is this form with y holding the shared
 * expert's bf16 output: the routed sum, then + shared, rounded once to bf16.
 * offsets and sorted_assign are kr_moe_route's: every assignment in a bucket,
 * offsets[experts] == tokens * topk.  Routing from kr_moe_scan_scatter with ids
 * >= experts breaks that; then the outputs are unspecified, but every memory
 * access stays inside the given arrays.  Every expert's weights are read
 * once per call for all the tokens routed to it (grouped matmul; the reference
 * re-reads them per routed token).  The reference also rounds gate.x, up.x and
 * d_a to bf16; here they stay f32.
 * workspace: kr_q4_moe_workspace_bytes(tokens, topk, hidden, inter) bytes,
 * 16-byte aligned; calls sharing it must not overlap in time.
 * Limits: experts <= 256; hidden and inter multiples of 128 and <= 2048;
 * scales and biases 4-byte aligned. */
size_t kr_q4_moe_workspace_bytes(uint32_t tokens, uint32_t topk, uint32_t hidden, uint32_t inter);
int kr_q4_moe_experts(const kr_q4_matrix *gate, const kr_q4_matrix *up, const kr_q4_matrix *down,
                      uint32_t experts, const uint16_t *x, uint32_t tokens, uint32_t topk,
                      const float *weights, const uint32_t *offsets, const uint32_t *sorted_assign,
                      int activation, void *y, int y_dtype, int accumulate,
                      void *workspace, size_t workspace_bytes, void *stream);

/* ---- routing from logits and the routed experts in one call: the topk, scan
 *      and expert dispatches the reference encodes back to back into one command
 *      buffer (encoder.rs:5275-5445) ----
 * kr_moe_route(logits, tokens, experts, topk, normalize, selected, weights,
 * counts, offsets, sorted_assign) followed by kr_q4_moe_experts(..., weights,
 * offsets, sorted_assign, ...): the same arguments, limits, routing arrays and
 * y bit for bit.  With one token on the routed GEMV path (KR_OPT_MOE_GEMV = 1)
 * the routing runs inside the experts' first launch: every wavefront takes the
 * token's softmax and top-k itself, one of them writes the routing arrays
 * (KR_OPT_MOE_ROUTE_FUSED = 0 launches the routing kernel instead).  All checks
 * of both stages run before anything is enqueued. */
int kr_q4_moe_route_experts(const kr_q4_matrix *gate, const kr_q4_matrix *up, const kr_q4_matrix *down,
                            uint32_t experts, const uint16_t *x, uint32_t tokens, uint32_t topk,
                            const float *logits, int normalize, uint32_t *selected, float *weights,
                            uint32_t *counts, uint32_t *offsets, uint32_t *sorted_assign,
                            int activation, void *y, int y_dtype, int accumulate,
                            void *workspace, size_t workspace_bytes, void *stream);

/* ---- the whole routed MoE stage on the device: the SparseMoE channel mixer of
 *      forward_and_sample_impl / forward_prefill_batch (encoder.rs:5246-5445 and
 *      4425-4625): router Q4 GEMV -> top-k routing -> experts -> combine ----
 * logits = x . router^T in f32 (router: Q4 [experts, hidden]), then
 * kr_q4_moe_route_experts(logits, normalize, ...) as above, all on
 * `stream` with nothing returned to the host.  The reference writes the router
 * logits as bf16 and reads them as f32, and never resets its expert counters
 * (encoder.rs:4435-4445, 5255-5265, 1982); here the logits stay f32 and the
 * routing keeps no state between calls.
 * x: bf16 [tokens, hidden] (the normed hidden state); y as kr_q4_moe_experts'.
 * workspace: kr_q4_moe_block_workspace_bytes(tokens, experts, topk, hidden, inter)
 * bytes, 16-byte aligned; calls sharing it must not overlap in time.
 * Limits: those of kr_moe_route and kr_q4_moe_experts. */
size_t kr_q4_moe_block_workspace_bytes(uint32_t tokens, uint32_t experts, uint32_t topk, uint32_t hidden,
                                       uint32_t inter);
int kr_q4_moe_block(const kr_q4_matrix *router, const kr_q4_matrix *gate, const kr_q4_matrix *up,
                    const kr_q4_matrix *down, uint32_t experts, const uint16_t *x, uint32_t tokens, uint32_t topk,
                    int normalize, int activation, void *y, int y_dtype, int accumulate, void *workspace,
                    size_t workspace_bytes, void *stream);

/* ---- Q4 embedding lookup: transformer_glue.metal:122-152 (embedding_lookup_q4_g64),
 *      dispatched at encoder.rs:4803-4846 ----
 * out[t, :] = bf16(fma(q, s, b)) of row tokens[t] of w (the tied Q4 embedding
 * [vocab, hidden]).  tokens: device u32 [count]; ids >= w->n give zero rows.
 * out: bf16 [count, w->k], 2-byte aligned. */
int kr_q4_embedding(const kr_q4_matrix *w, const uint32_t *tokens, uint32_t count, uint16_t *out,
                    void *stream);

/* ---- measurement helper (no counterpart in the reference) ----
 * A plain read of `bytes` bytes of device memory, the floor the GEMV kernels are
 * compared with at the same byte count.  hits[i] = 1 where some 16-byte unit
 * of the i-th 1 KB of buf (the last piece may be shorter) has its four 32-bit
 * words xor to `match`; other words of hits are not written.  hits holds
 * kr_stream_read_pieces(bytes) words.  buf 16-byte aligned, bytes a positive
 * multiple of 16. */
size_t kr_stream_read_pieces(size_t bytes);
int kr_stream_read(const void *buf, size_t bytes, uint32_t match, uint32_t *hits, void *stream);

#ifdef __cplusplus
}
#endif
#endif /* KRIYA_Q4_H */
