/*
 * kr_oracle.h — CPU restatement of kriya-rt's Q4_G64 matmul path.
 *
 * TEST INFRASTRUCTURE ONLY.  This library is the checker that the HIP path is
 * compared against.  Only tests/, __graft_entry__.smoke() and bench.py's
 * cpu_baseline leg may load it; the product library (libkriya_q4.so) never
 * links, loads or calls it.
 *
 * Every function cites the reference file:line whose behaviour it restates.
 * Paths are relative to the kriya-rt source tree.
 *
 * Weight layout used by the matmul helpers is the planar "MLX" triplet:
 *   qw     u32 [n, k/8]   word w of row r holds elements 8w..8w+7, element
 *                         8w+j in bits 4j..4j+3 (low nibble first)
 *   scales bf16 [n, k/64]
 *   biases bf16 [n, k/64]
 * and w[r, c] = fma(q, scale, bias) (quantizer.rs:112-126).
 */
#ifndef KR_ORACLE_H
#define KR_ORACLE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ---- scalar conversions: crates/kriya-core/src/quantizer.rs:19-57 ---- */
uint16_t kro_f32_to_bf16(float v);
float kro_bf16_to_f32(uint16_t b);
float kro_f16_to_f32(uint16_t h);
/* safetensors_loader.rs:310-318 (parse_half_endian) */
uint16_t kro_half_to_bf16(uint16_t raw, int is_f16);

void kro_f32_to_bf16_n(const float *in, uint16_t *out, size_t n);
void kro_bf16_to_f32_n(const uint16_t *in, float *out, size_t n);
void kro_f16_to_f32_n(const uint16_t *in, float *out, size_t n);

/* ---- quantize / dequantize: quantizer.rs:61-126 ---- */
/* count % 64 != 0 -> returns -1 (TensorError::ShapeMismatch). */
int kro_quantize_q4_g64(const float *w, size_t count, uint8_t *blocks36);
void kro_dequant_blocks36(const uint8_t *blocks36, size_t nblocks, float *out);
void kro_dequant_planar(const uint32_t *qw, const uint16_t *sc, const uint16_t *bi,
                        uint32_t n, uint32_t k, float *out);

/* ---- layouts: tensor.rs:104-211, safetensors_loader.rs:221-273 ---- */
void kro_blocks36_to_planar(const uint8_t *blocks36, uint32_t n, uint32_t k,
                            uint32_t *qw, uint16_t *sc, uint16_t *bi);
void kro_planar_to_blocks36(const uint32_t *qw, const uint16_t *sc, const uint16_t *bi,
                            uint32_t n, uint32_t k, uint8_t *blocks36);
/* Returns number of blocks written, or -1 (bad weight length), -2 (scale/bias
 * length mismatch) exactly where the reference returns an error. */
long kro_mlx_pack_blocks36(const uint8_t *wbytes, size_t wlen,
                           const uint16_t *s_raw, size_t s_count, int s_is_f16,
                           const uint16_t *b_raw, size_t b_count, int b_is_f16,
                           uint8_t *out);
void kro_split_blocks36(const uint8_t *blocks36, size_t nblocks, uint8_t *qs32, uint16_t *sb);
void kro_join_blocks36(const uint8_t *qs32, const uint16_t *sb, size_t nblocks, uint8_t *blocks36);

/* ---- matmul: dequantize, then sequential f32 dot per (m, n)
 *      (test_shader_compile.rs:592-595, real_world_validation.rs:1625-1634) ---- */
void kro_q4_matmul(const uint32_t *qw, const uint16_t *sc, const uint16_t *bi,
                   uint32_t n, uint32_t k, const uint16_t *x_bf16, uint32_t m,
                   float *y, int nthreads);
/* Same products summed in double: the gold for error reporting. */
void kro_q4_matmul_f64(const uint32_t *qw, const uint16_t *sc, const uint16_t *bi,
                       uint32_t n, uint32_t k, const uint16_t *x_bf16, uint32_t m,
                       double *y, int nthreads);

/* Sequential f32 dot of pre-dequantised rows w f32 [n, k] with x f32 [m, k] (the CPU
 * baseline's upper bound: the reference test's dot without the per-call dequantisation). */
void kro_f32_matmul(const float *w, uint32_t n, uint32_t k, const float *x, uint32_t m, float *y, int nthreads);

/* ---- activation: q4_gemm_and_moe.metal:2064-2071, transformer_glue.metal:307-336 ---- */
float kro_activation(float g, int variant); /* 0 SwiGLU(silu), 1 GeGLU(tanh), 2 ReLU */

/* a[m, i] = act(gate_i . x_m) * (up_i . x_m), f32 (q4_gemm_and_moe.metal:2003-2091). */
void kro_q4_gate_up_act(const uint32_t *gqw, const uint16_t *gsc, const uint16_t *gbi,
                        const uint32_t *uqw, const uint16_t *usc, const uint16_t *ubi,
                        uint32_t inter, uint32_t k, const uint16_t *x_bf16, uint32_t m,
                        int variant, float *a, int nthreads);

/* Dense MLP (encoder.rs:2851-2906): y[m, h] = down . bf16(a[m, :]) with a from
 * kro_q4_gate_up_act.  bf16_intermediate = 1 rounds a to bf16 as the reference
 * kernels store it (q4_gemm_and_moe.metal:2076, 2087); 0 keeps it f32.
 * The residual add is left to the caller. */
void kro_q4_mlp(const uint32_t *gqw, const uint16_t *gsc, const uint16_t *gbi,
                const uint32_t *uqw, const uint16_t *usc, const uint16_t *ubi,
                const uint32_t *dqw, const uint16_t *dsc, const uint16_t *dbi,
                uint32_t hidden, uint32_t inter, const uint16_t *x_bf16, uint32_t m,
                int variant, int bf16_intermediate, float *y, int nthreads);

/* ---- MoE routing: q4_gemm_and_moe.metal:2495-2624, restated deterministically:
 * slot of an assignment inside its expert bucket = its rank among the
 * assignments of that expert in increasing assignment id (t*K + k).
 * Returns -1 if K == 0, K > E or K > 32. ---- */
int kro_moe_route(const float *logits, uint32_t T, uint32_t E, uint32_t K, int normalize,
                  uint32_t *experts, float *weights, uint32_t *counts,
                  uint32_t *offsets, uint32_t *sorted_assign);

/* Counts, exclusive offsets [E+1] and the expert-sorted assignment list for
 * given assignments (experts[a] < E).  Returns -1 on an expert id >= E. */
int kro_moe_scan_scatter(const uint32_t *experts, size_t num_assign, uint32_t E,
                         uint32_t *counts, uint32_t *offsets, uint32_t *sorted_assign);

/* MoE experts + combine (encoder.rs:5316-5445, transformer_glue.metal:373-401):
 * for assignment a = t*K + k with expert e: g,u = W_gate[e] x_t, W_up[e] x_t;
 * h = bf16(act(g)*u); d = W_down[e] h;  y[t] = sum_k fma(w[t,k], d, acc).
 * Stacked weights are expert-major: gate/up [E*inter, hidden/64 groups],
 * down [E*hidden, inter/64 groups]. */
void kro_moe_experts(const uint32_t *gqw, const uint16_t *gsc, const uint16_t *gbi,
                     const uint32_t *uqw, const uint16_t *usc, const uint16_t *ubi,
                     const uint32_t *dqw, const uint16_t *dsc, const uint16_t *dbi,
                     uint32_t E, uint32_t hidden, uint32_t inter,
                     const uint16_t *x_bf16, uint32_t T, uint32_t K,
                     const uint32_t *experts, const float *weights, int variant,
                     float *y, int nthreads);

#ifdef __cplusplus
}
#endif
#endif
