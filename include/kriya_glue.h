/*
 * kriya_glue.h — the non-Q4 steps of config 3's end-to-end decode, as a C ABI
 * beside kriya_q4.h: RMSNorm, RoPE with KV-cache append, decode attention
 * (GQA) and greedy argmax.  Conventions as in kriya_q4.h (device pointers,
 * stream-ordered, 0 or a negative KR_E* code, message in kr_last_error()).
 * These are simple, correct kernels; the Q4 matmuls carry the time.
 */
#ifndef KRIYA_GLUE_H
#define KRIYA_GLUE_H

#include <stddef.h>
#include <stdint.h>

#include "kriya_q4.h"

#ifdef __cplusplus
extern "C" {
#endif

/* rms_norm_bf16 (transformer_glue.metal:158-205):
 * out[r, :] = bf16(x * rsqrt(mean(x^2) + eps) * w), x/out bf16 [rows, dim], w bf16 [dim].
 * out may equal x. */
int kr_rmsnorm(const uint16_t *x, const uint16_t *weight, uint32_t rows, uint32_t dim, float eps,
               uint16_t *out, void *stream);

/* fused_qknorm_rope_and_kv_append without q/k norm (paged_gqa_and_deltanet.metal:115-222),
 * on a contiguous cache:
 *   q   bf16 [batch, q_heads, head_dim], rotated in place;
 *   k,v bf16 [batch, kv_heads, head_dim]; k rotated, both written to
 *   k_cache/v_cache bf16 [batch, max_ctx, kv_heads, head_dim] at row positions[b].
 * Rotation of pairs (d, d + head_dim/2): (x0 c - x1 s, x0 s + x1 c) with
 * cos_sin f32 [max_ctx, head_dim/2, 2] (encoder.rs:1940-1950).  positions: device
 * u32 [batch]; a position >= max_ctx leaves that sequence untouched.
 * Limits: q_heads % kv_heads == 0, head_dim a multiple of 8 and <= 256, max_ctx <= 8192. */
int kr_rope_kv_append(uint16_t *q, const uint16_t *k, const uint16_t *v, const float *cos_sin,
                      const uint32_t *positions, uint32_t batch, uint32_t q_heads, uint32_t kv_heads,
                      uint32_t head_dim, uint16_t *k_cache, uint16_t *v_cache, uint32_t max_ctx,
                      void *stream);

/* Decode attention: out[b, h] = softmax_p(q[b,h] . k[b,p,kvh] / sqrt(head_dim)) v[b,p,kvh]
 * over p <= positions[b], kvh = h / (q_heads / kv_heads).  out bf16 [batch, q_heads, head_dim].
 * Limits: q_heads % kv_heads == 0, head_dim <= 256 and a multiple of 8, max_ctx <= 8192;
 * q, k_cache, v_cache 16-byte aligned. */
int kr_attention_decode(const uint16_t *q, const uint16_t *k_cache, const uint16_t *v_cache,
                        const uint32_t *positions, uint32_t batch, uint32_t q_heads, uint32_t kv_heads,
                        uint32_t head_dim, uint32_t max_ctx, uint16_t *out, void *stream);

/* RMSNorm fused into the consumers of its output (the two per-layer norms of a
 * decode step).  Results are those of kr_rmsnorm into a bf16 buffer followed by
 * the Q4 call, up to the f32 summation order of mean(x^2).
 *
 * qkv(rmsnorm(h)): arguments as kr_q4_qkv, with h bf16 [m, k] and ln_weight bf16
 * [k].  One launch when m == 1 with k <= 4096 (each block of the GEMV normalises
 * h into its LDS) and for the few-token kernel (2 <= m <= 63 with k <= 2048;
 * each wave normalises the rows it stages); xnorm is then not written.
 * Otherwise the norm goes to xnorm (bf16 [m, k], 16-byte aligned; may be NULL
 * in the one-launch cases) first. */
int kr_rmsnorm_q4_qkv(const uint16_t *h, const uint16_t *ln_weight, float eps, const kr_q4_matrix *q,
                      const kr_q4_matrix *k, const kr_q4_matrix *v, const uint16_t *q_bias, const uint16_t *k_bias,
                      const uint16_t *v_bias, uint32_t m, void *q_out, void *k_out, void *v_out, int out_dtype,
                      uint16_t *xnorm, void *stream);

/* h += mlp(rmsnorm(h)) for bf16 h [m, hidden] updated in place (kr_q4_mlp with
 * x = rmsnorm(h)).  m == 1 with hidden <= 4096: the norm is fused into the
 * gate/up GEMV.  workspace: kr_rmsnorm_q4_mlp_workspace_bytes(m, hidden, inter),
 * zero-filled once before its first use, as kr_q4_mlp's. */
size_t kr_rmsnorm_q4_mlp_workspace_bytes(uint32_t m, uint32_t hidden, uint32_t intermediate);
int kr_rmsnorm_q4_mlp(const kr_q4_matrix *gate, const kr_q4_matrix *up, const kr_q4_matrix *down, uint16_t *h,
                      const uint16_t *ln_weight, float eps, uint32_t m, int activation, void *workspace,
                      size_t workspace_bytes, void *stream);

/* RoPE + KV append + decode attention in two launches: the results of
 * kr_rope_kv_append followed by kr_attention_decode (up to f32 summation
 * order), except that q is only read (its rotated copy is not written back).
 * The context is split into slices of 16 positions (64 with head_dim 128 when
 * the 64-position slices still give a block per compute unit,
 * KR_OPT_ATTN_SLICE64); one block takes a slice of one sequence for one kv head
 * and all the query heads that share it (GQA), and a second launch merges the
 * slices in a fixed order.
 * workspace: kr_attention_workspace_bytes(batch, q_heads, head_dim, max_ctx)
 * bytes, 16-byte aligned (per-slice partial sums); calls sharing a workspace
 * must not overlap in time.
 * Limits: those of kr_attention_decode and q_heads / kv_heads <= 16. */
size_t kr_attention_workspace_bytes(uint32_t batch, uint32_t q_heads, uint32_t head_dim, uint32_t max_ctx);
int kr_rope_attention_decode(const uint16_t *q, const uint16_t *k, const uint16_t *v, const float *cos_sin,
                             const uint32_t *positions, uint32_t batch, uint32_t q_heads, uint32_t kv_heads,
                             uint32_t head_dim, uint16_t *k_cache, uint16_t *v_cache, uint32_t max_ctx,
                             uint16_t *out, void *workspace, size_t workspace_bytes, void *stream);

/* The attention block's tail: RoPE + KV append + decode attention, then the
 * output projection accumulated into the residual,
 *   h[b] (+)= attention(q, k, v, ...)[b] . o_proj^T,
 * i.e. kr_rope_attention_decode followed by kr_q4_linear(o_proj, attn, h,
 * accumulate = 1) (the o_proj step of the reference's decode layer,
 * encoder.rs:4880-5484).  With one sequence, head_dim 128, q_heads <= 16 and at
 * most 16 slices of 64 positions (max_ctx <= 1024), the slices' merge runs
 * inside the projection's launch (every block merges the partials into x
 * itself): two launches instead of three (KR_OPT_ATTN_MERGE_OPROJ).  Results
 * within f32 summation order of the two calls.  o_proj: Q4 [n, q_heads *
 * head_dim]; h: [batch, n] bf16 or f32 (h_dtype), updated in place.
 * workspace: kr_attention_q4_out_workspace_bytes(batch, q_heads, head_dim,
 * max_ctx) bytes, 16-byte aligned; calls sharing it must not overlap in time.
 * Limits: those of kr_rope_attention_decode and kr_q4_linear. */
size_t kr_attention_q4_out_workspace_bytes(uint32_t batch, uint32_t q_heads, uint32_t head_dim, uint32_t max_ctx);
int kr_rope_attention_q4_out(const uint16_t *q, const uint16_t *k, const uint16_t *v, const float *cos_sin,
                             const uint32_t *positions, uint32_t batch, uint32_t q_heads, uint32_t kv_heads,
                             uint32_t head_dim, uint16_t *k_cache, uint16_t *v_cache, uint32_t max_ctx,
                             const kr_q4_matrix *o_proj, void *h, int h_dtype, void *workspace, size_t workspace_bytes,
                             void *stream);

/* Greedy sampling (transformer_glue.metal:407-494, temperature 0):
 * out[r] = index of the largest logits[r, :] (ties to the lowest index, NaN never taken). */
int kr_argmax(const float *logits, uint32_t rows, uint32_t n, uint32_t *out, void *stream);

/* The same greedy argmax (transformer_glue.metal:407-494, the same result bit for bit) with
 * each row spread over several blocks and a second, one-wave merge launch: for long rows
 * (a vocabulary of 151936 logits: one block per row reads at about 54 GB/s).  workspace:
 * kr_argmax_workspace_bytes(rows, n) bytes, 8-byte aligned, no initial contents; calls
 * sharing it must not overlap in time. */
size_t kr_argmax_workspace_bytes(uint32_t rows, uint32_t n);
int kr_argmax_ws(const float *logits, uint32_t rows, uint32_t n, uint32_t *out, void *workspace,
                 size_t workspace_bytes, void *stream);

#ifdef __cplusplus
}
#endif
#endif /* KRIYA_GLUE_H */
