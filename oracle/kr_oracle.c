/*
 * kr_oracle.c — CPU restatement of kriya-rt's Q4_G64 matmul path.
 *
 * TEST INFRASTRUCTURE ONLY (see kr_oracle.h).  Built with -ffp-contract=off so
 * that "a * b + c" is two roundings, as in the reference's Rust code, and
 * fmaf() is used exactly where the reference calls mul_add / fma.
 *
 * Pinning (what checks each function beyond itself) is listed in the header
 * of tests/test_oracle.py.
 */
#include "kr_oracle.h"

#include <math.h>
#include <pthread.h>
#include <stdlib.h>
#include <string.h>

/* ------------------------------------------------------------------------ */
/* scalar conversions                                                        */
/* ------------------------------------------------------------------------ */

static inline uint32_t f2u(float f) { uint32_t u; memcpy(&u, &f, 4); return u; }
static inline float u2f(uint32_t u) { float f; memcpy(&f, &u, 4); return f; }

/* quantizer.rs:19-24: RNE with a wrapping u32 add; NaN is not special-cased. */
uint16_t kro_f32_to_bf16(float v) {
    uint32_t bits = f2u(v);
    uint32_t lsb = (bits >> 16) & 1u;
    return (uint16_t)((bits + (0x7FFFu + lsb)) >> 16);
}

/* quantizer.rs:26-29 */
float kro_bf16_to_f32(uint16_t b) { return u2f((uint32_t)b << 16); }

/* quantizer.rs:31-57 */
float kro_f16_to_f32(uint16_t h) {
    uint32_t sign = (h >> 15) & 1u;
    uint32_t exp = (h >> 10) & 0x1Fu;
    uint32_t mant = h & 0x03FFu;
    if (exp == 0) {
        if (mant == 0) return u2f(sign << 31);
        uint32_t m = mant;
        int32_t e = 127 - 14;
        while ((m & 0x0400u) == 0) { m <<= 1; e -= 1; }
        m &= 0x03FFu;
        return u2f((sign << 31) | ((uint32_t)e << 23) | (m << 13));
    }
    if (exp == 31) return u2f((sign << 31) | 0x7F800000u | (mant << 13));
    return u2f((sign << 31) | ((exp + (127 - 15)) << 23) | (mant << 13));
}

/* safetensors_loader.rs:310-318 */
uint16_t kro_half_to_bf16(uint16_t raw, int is_f16) {
    return is_f16 ? kro_f32_to_bf16(kro_f16_to_f32(raw)) : raw;
}

void kro_f32_to_bf16_n(const float *in, uint16_t *out, size_t n) {
    for (size_t i = 0; i < n; ++i) out[i] = kro_f32_to_bf16(in[i]);
}
void kro_bf16_to_f32_n(const uint16_t *in, float *out, size_t n) {
    for (size_t i = 0; i < n; ++i) out[i] = kro_bf16_to_f32(in[i]);
}
void kro_f16_to_f32_n(const uint16_t *in, float *out, size_t n) {
    for (size_t i = 0; i < n; ++i) out[i] = kro_f16_to_f32(in[i]);
}

/* ------------------------------------------------------------------------ */
/* quantize / dequantize                                                     */
/* ------------------------------------------------------------------------ */

/* Rust `f32 as u8`: saturating, NaN -> 0. */
static inline uint8_t sat_u8(float v) {
    if (isnan(v)) return 0;
    if (v <= 0.0f) return 0;
    if (v >= 255.0f) return 255;
    return (uint8_t)v;
}

/* Rust f32::clamp(lo, hi): NaN passes through. */
static inline float rclamp(float v, float lo, float hi) {
    if (v < lo) v = lo;
    if (v > hi) v = hi;
    return v;
}

static inline void put_u16(uint8_t *p, uint16_t v) { p[0] = (uint8_t)v; p[1] = (uint8_t)(v >> 8); }
static inline uint16_t get_u16(const uint8_t *p) { return (uint16_t)(p[0] | (p[1] << 8)); }

/* quantizer.rs:61-109.  Block bytes: {u16 scale_bf16, u16 bias_bf16, u8 qs[32]}
 * little endian, packed (tensor.rs:106-115). */
int kro_quantize_q4_g64(const float *w, size_t count, uint8_t *blocks36) {
    if (count % 64 != 0) return -1;
    size_t nblocks = count / 64;
    for (size_t b = 0; b < nblocks; ++b) {
        const float *chunk = w + b * 64;
        float mn = INFINITY, mx = -INFINITY;
        for (int i = 0; i < 64; ++i) { mn = fminf(mn, chunk[i]); mx = fmaxf(mx, chunk[i]); }
        float range = fmaxf(mx - mn, 1e-8f);
        float scale = range / 15.0f;
        float bias = mn;
        uint16_t scale_bf16 = kro_f32_to_bf16(scale);
        uint16_t bias_bf16 = kro_f32_to_bf16(bias);
        float eff_scale = fmaxf(kro_bf16_to_f32(scale_bf16), 1e-8f);
        float eff_bias = kro_bf16_to_f32(bias_bf16);
        uint8_t *blk = blocks36 + b * 36;
        put_u16(blk, scale_bf16);
        put_u16(blk + 2, bias_bf16);
        for (int i = 0; i < 32; ++i) {
            /* .round() rounds half away from zero, as C roundf does. */
            uint8_t q0 = sat_u8(rclamp(roundf((chunk[2 * i] - eff_bias) / eff_scale), 0.0f, 15.0f));
            uint8_t q1 = sat_u8(rclamp(roundf((chunk[2 * i + 1] - eff_bias) / eff_scale), 0.0f, 15.0f));
            blk[4 + i] = (uint8_t)((q0 & 0x0F) | ((q1 & 0x0F) << 4));
        }
    }
    return 0;
}

/* quantizer.rs:112-126: w = (q as f32).mul_add(scale, bias). */
void kro_dequant_blocks36(const uint8_t *blocks36, size_t nblocks, float *out) {
    for (size_t b = 0; b < nblocks; ++b) {
        const uint8_t *blk = blocks36 + b * 36;
        float s = kro_bf16_to_f32(get_u16(blk));
        float bi = kro_bf16_to_f32(get_u16(blk + 2));
        for (int i = 0; i < 32; ++i) {
            uint8_t p = blk[4 + i];
            out[b * 64 + 2 * i] = fmaf((float)(p & 0x0F), s, bi);
            out[b * 64 + 2 * i + 1] = fmaf((float)(p >> 4), s, bi);
        }
    }
}

/* Row r of a planar matrix, dequantized into out[0..k). */
static void dequant_row(const uint32_t *qw, const uint16_t *sc, const uint16_t *bi,
                        uint32_t k, size_t r, float *out) {
    const uint32_t G = k / 64;
    const uint32_t *words = qw + r * (size_t)(k / 8);
    for (uint32_t g = 0; g < G; ++g) {
        float s = kro_bf16_to_f32(sc[r * G + g]);
        float b = kro_bf16_to_f32(bi[r * G + g]);
        for (uint32_t w = 0; w < 8; ++w) {
            uint32_t word = words[g * 8 + w];
            for (uint32_t j = 0; j < 8; ++j)
                out[g * 64 + w * 8 + j] = fmaf((float)((word >> (4 * j)) & 0xF), s, b);
        }
    }
}

void kro_dequant_planar(const uint32_t *qw, const uint16_t *sc, const uint16_t *bi,
                        uint32_t n, uint32_t k, float *out) {
    for (size_t r = 0; r < n; ++r) dequant_row(qw, sc, bi, k, r, out + r * (size_t)k);
}

/* ------------------------------------------------------------------------ */
/* layouts                                                                   */
/* ------------------------------------------------------------------------ */

/* Block (r, g) sits at index r*G + g (q4_gemm_and_moe.metal:951).  Its 32 qs
 * bytes are the little-endian bytes of planar words 8g..8g+7 of row r: byte i
 * holds element 2i (low nibble) and 2i+1 (high nibble) in both layouts
 * (tensor.rs:113, safetensors_loader.rs:260-270). */
void kro_blocks36_to_planar(const uint8_t *blocks36, uint32_t n, uint32_t k,
                            uint32_t *qw, uint16_t *sc, uint16_t *bi) {
    const size_t G = k / 64;
    for (size_t r = 0; r < n; ++r)
        for (size_t g = 0; g < G; ++g) {
            const uint8_t *blk = blocks36 + (r * G + g) * 36;
            sc[r * G + g] = get_u16(blk);
            bi[r * G + g] = get_u16(blk + 2);
            memcpy((uint8_t *)(qw + r * (k / 8) + g * 8), blk + 4, 32);
        }
}

void kro_planar_to_blocks36(const uint32_t *qw, const uint16_t *sc, const uint16_t *bi,
                            uint32_t n, uint32_t k, uint8_t *blocks36) {
    const size_t G = k / 64;
    for (size_t r = 0; r < n; ++r)
        for (size_t g = 0; g < G; ++g) {
            uint8_t *blk = blocks36 + (r * G + g) * 36;
            put_u16(blk, sc[r * G + g]);
            put_u16(blk + 2, bi[r * G + g]);
            memcpy(blk + 4, (const uint8_t *)(qw + r * (k / 8) + g * 8), 32);
        }
}

/* safetensors_loader.rs:221-273 (method) with the length checks of :243-258. */
long kro_mlx_pack_blocks36(const uint8_t *wbytes, size_t wlen,
                           const uint16_t *s_raw, size_t s_count, int s_is_f16,
                           const uint16_t *b_raw, size_t b_count, int b_is_f16,
                           uint8_t *out) {
    if (wlen % 32 != 0) return -1;
    size_t nblocks = wlen / 32;
    if (s_count != nblocks || b_count != nblocks) return -2;
    for (size_t i = 0; i < nblocks; ++i) {
        uint8_t *blk = out + i * 36;
        put_u16(blk, kro_half_to_bf16(s_raw[i], s_is_f16));
        put_u16(blk + 2, kro_half_to_bf16(b_raw[i], b_is_f16));
        memcpy(blk + 4, wbytes + i * 32, 32);
    }
    return (long)nblocks;
}

/* tensor.rs:156-211: split into 32 B nibble planes and {scale, bias} pairs. */
void kro_split_blocks36(const uint8_t *blocks36, size_t nblocks, uint8_t *qs32, uint16_t *sb) {
    for (size_t i = 0; i < nblocks; ++i) {
        const uint8_t *blk = blocks36 + i * 36;
        sb[2 * i] = get_u16(blk);
        sb[2 * i + 1] = get_u16(blk + 2);
        memcpy(qs32 + i * 32, blk + 4, 32);
    }
}

void kro_join_blocks36(const uint8_t *qs32, const uint16_t *sb, size_t nblocks, uint8_t *blocks36) {
    for (size_t i = 0; i < nblocks; ++i) {
        uint8_t *blk = blocks36 + i * 36;
        put_u16(blk, sb[2 * i]);
        put_u16(blk + 2, sb[2 * i + 1]);
        memcpy(blk + 4, qs32 + i * 32, 32);
    }
}

/* ------------------------------------------------------------------------ */
/* threading                                                                 */
/* ------------------------------------------------------------------------ */

typedef void (*range_fn)(void *ctx, size_t begin, size_t end);
typedef struct { range_fn fn; void *ctx; size_t begin, end; } range_job;

static void *range_thunk(void *p) {
    range_job *j = (range_job *)p;
    j->fn(j->ctx, j->begin, j->end);
    return NULL;
}

static void parallel_for(size_t total, int nthreads, range_fn fn, void *ctx) {
    if (nthreads < 1) nthreads = 1;
    if ((size_t)nthreads > total) nthreads = total ? (int)total : 1;
    if (nthreads == 1) { fn(ctx, 0, total); return; }
    pthread_t th[256];
    range_job jobs[256];
    if (nthreads > 256) nthreads = 256;
    size_t per = (total + nthreads - 1) / nthreads;
    int launched = 0;
    for (int t = 0; t < nthreads; ++t) {
        size_t b = t * per, e = b + per < total ? b + per : total;
        if (b >= e) break;
        jobs[t] = (range_job){fn, ctx, b, e};
        if (pthread_create(&th[t], NULL, range_thunk, &jobs[t]) != 0) {
            fn(ctx, b, e); /* run inline if a thread cannot be created */
            jobs[t].fn = NULL;
        }
        launched = t + 1;
    }
    for (int t = 0; t < launched; ++t)
        if (jobs[t].fn) pthread_join(th[t], NULL);
}

/* ------------------------------------------------------------------------ */
/* matmul                                                                    */
/* ------------------------------------------------------------------------ */

typedef struct {
    const uint32_t *qw; const uint16_t *sc, *bi;
    uint32_t n, k, m;
    const float *x;  /* [m, k] f32 (already exact bf16 values) */
    float *y;        /* [m, n] */
    double *y64;     /* [m, n] or NULL */
} mm_ctx;

/* test_shader_compile.rs:592-595: `row.iter().zip(&input).map(|(w, x)| w * x).sum()`
 * is a left fold from 0.0 with one rounding for the product and one for the add. */
static void mm_range(void *p, size_t begin, size_t end) {
    mm_ctx *c = (mm_ctx *)p;
    float *row = (float *)malloc(sizeof(float) * c->k);
    for (size_t r = begin; r < end; ++r) {
        dequant_row(c->qw, c->sc, c->bi, c->k, r, row);
        for (size_t i = 0; i < c->m; ++i) {
            const float *x = c->x + i * c->k;
            if (c->y64) {
                double acc = 0.0;
                for (size_t j = 0; j < c->k; ++j) acc += (double)row[j] * (double)x[j];
                c->y64[i * c->n + r] = acc;
            } else {
                float acc = 0.0f;
                for (size_t j = 0; j < c->k; ++j) {
                    float prod = row[j] * x[j];
                    acc = acc + prod;
                }
                c->y[i * c->n + r] = acc;
            }
        }
    }
    free(row);
}

static void matmul_f32x(const uint32_t *qw, const uint16_t *sc, const uint16_t *bi,
                        uint32_t n, uint32_t k, const float *x, uint32_t m,
                        float *y, double *y64, int nthreads) {
    mm_ctx c = {qw, sc, bi, n, k, m, x, y, y64};
    parallel_for(n, nthreads, mm_range, &c);
}

/* The CPU baseline's upper bound: the same sequential f32 dot on weights that were
 * dequantised once beforehand (w f32 [n, k]), so only the dot products are timed. */
typedef struct { const float *w; uint32_t n, k, m; const float *x; float *y; } f32mm_ctx;

static void f32mm_range(void *p, size_t begin, size_t end) {
    f32mm_ctx *c = (f32mm_ctx *)p;
    for (size_t r = begin; r < end; ++r) {
        const float *row = c->w + r * c->k;
        for (size_t i = 0; i < c->m; ++i) {
            const float *x = c->x + i * c->k;
            float acc = 0.0f;
            for (size_t j = 0; j < c->k; ++j) {
                float prod = row[j] * x[j];
                acc = acc + prod;
            }
            c->y[i * c->n + r] = acc;
        }
    }
}

void kro_f32_matmul(const float *w, uint32_t n, uint32_t k, const float *x, uint32_t m, float *y, int nthreads) {
    f32mm_ctx c = {w, n, k, m, x, y};
    parallel_for(n, nthreads, f32mm_range, &c);
}

static float *bf16_rows_to_f32(const uint16_t *x, size_t count) {
    float *xf = (float *)malloc(sizeof(float) * (count ? count : 1));
    kro_bf16_to_f32_n(x, xf, count);
    return xf;
}

void kro_q4_matmul(const uint32_t *qw, const uint16_t *sc, const uint16_t *bi,
                   uint32_t n, uint32_t k, const uint16_t *x_bf16, uint32_t m,
                   float *y, int nthreads) {
    float *xf = bf16_rows_to_f32(x_bf16, (size_t)m * k);
    matmul_f32x(qw, sc, bi, n, k, xf, m, y, NULL, nthreads);
    free(xf);
}

void kro_q4_matmul_f64(const uint32_t *qw, const uint16_t *sc, const uint16_t *bi,
                       uint32_t n, uint32_t k, const uint16_t *x_bf16, uint32_t m,
                       double *y, int nthreads) {
    float *xf = bf16_rows_to_f32(x_bf16, (size_t)m * k);
    matmul_f32x(qw, sc, bi, n, k, xf, m, NULL, y, nthreads);
    free(xf);
}

/* ------------------------------------------------------------------------ */
/* activation, gate+up, MLP                                                  */
/* ------------------------------------------------------------------------ */

/* q4_gemm_and_moe.metal:2064-2071.  The GeGLU clamp to [-15, 15] of
 * transformer_glue.metal:326-328 does not change tanhf's result (tanhf is
 * +-1.0f beyond |x| ~ 9.01), so one form serves both kernels. */
float kro_activation(float g, int variant) {
    if (variant == 0) return g / (1.0f + expf(-g));
    if (variant == 1) {
        const float SQRT_2_OVER_PI = 0.7978845608f;
        float cubic = fmaf(0.044715f * g, g * g, g);
        return 0.5f * g * (1.0f + tanhf(SQRT_2_OVER_PI * cubic));
    }
    return fmaxf(g, 0.0f);
}

void kro_q4_gate_up_act(const uint32_t *gqw, const uint16_t *gsc, const uint16_t *gbi,
                        const uint32_t *uqw, const uint16_t *usc, const uint16_t *ubi,
                        uint32_t inter, uint32_t k, const uint16_t *x_bf16, uint32_t m,
                        int variant, float *a, int nthreads) {
    float *xf = bf16_rows_to_f32(x_bf16, (size_t)m * k);
    float *g = (float *)malloc(sizeof(float) * (size_t)m * inter);
    float *u = (float *)malloc(sizeof(float) * (size_t)m * inter);
    matmul_f32x(gqw, gsc, gbi, inter, k, xf, m, g, NULL, nthreads);
    matmul_f32x(uqw, usc, ubi, inter, k, xf, m, u, NULL, nthreads);
    for (size_t i = 0; i < (size_t)m * inter; ++i) a[i] = kro_activation(g[i], variant) * u[i];
    free(xf); free(g); free(u);
}

void kro_q4_mlp(const uint32_t *gqw, const uint16_t *gsc, const uint16_t *gbi,
                const uint32_t *uqw, const uint16_t *usc, const uint16_t *ubi,
                const uint32_t *dqw, const uint16_t *dsc, const uint16_t *dbi,
                uint32_t hidden, uint32_t inter, const uint16_t *x_bf16, uint32_t m,
                int variant, int bf16_intermediate, float *y, int nthreads) {
    float *a = (float *)malloc(sizeof(float) * (size_t)m * inter);
    kro_q4_gate_up_act(gqw, gsc, gbi, uqw, usc, ubi, inter, hidden, x_bf16, m, variant, a, nthreads);
    if (bf16_intermediate)
        for (size_t i = 0; i < (size_t)m * inter; ++i) a[i] = kro_bf16_to_f32(kro_f32_to_bf16(a[i]));
    matmul_f32x(dqw, dsc, dbi, hidden, inter, a, m, y, NULL, nthreads);
    free(a);
}

/* ------------------------------------------------------------------------ */
/* MoE                                                                       */
/* ------------------------------------------------------------------------ */

/* q4_gemm_and_moe.metal:2495-2572 (per-token softmax, insertion top-k with
 * strict '>' so ties keep the lower expert id first, renormalisation by
 * max(sum, 1e-8)) and :2578-2624 (exclusive scan, scatter). */
int kro_moe_route(const float *logits, uint32_t T, uint32_t E, uint32_t K, int normalize,
                  uint32_t *experts, float *weights, uint32_t *counts,
                  uint32_t *offsets, uint32_t *sorted_assign) {
    if (K == 0 || K > E || K > 32) return -1;
    for (uint32_t t = 0; t < T; ++t) {
        const float *l = logits + (size_t)t * E;
        float mx = -INFINITY;
        for (uint32_t e = 0; e < E; ++e) mx = fmaxf(mx, l[e]);
        float sum = 0.0f;
        for (uint32_t e = 0; e < E; ++e) sum += expf(l[e] - mx);
        uint32_t ti[32];
        float tv[32];
        for (uint32_t k = 0; k < K; ++k) { ti[k] = 0; tv[k] = -INFINITY; }
        for (uint32_t e = 0; e < E; ++e) {
            float prob = expf(l[e] - mx) / sum;
            if (prob > tv[K - 1]) {
                tv[K - 1] = prob;
                ti[K - 1] = e;
                for (int j = (int)K - 2; j >= 0; --j) {
                    if (tv[j + 1] > tv[j]) {
                        float fv = tv[j]; tv[j] = tv[j + 1]; tv[j + 1] = fv;
                        uint32_t iv = ti[j]; ti[j] = ti[j + 1]; ti[j + 1] = iv;
                    } else {
                        break;
                    }
                }
            }
        }
        float norm = 1.0f;
        if (normalize) {
            norm = 0.0f;
            for (uint32_t k = 0; k < K; ++k) norm += tv[k];
            norm = fmaxf(norm, 1e-8f);
        }
        for (uint32_t k = 0; k < K; ++k) {
            experts[(size_t)t * K + k] = ti[k];
            weights[(size_t)t * K + k] = tv[k] / norm;
        }
    }
    return kro_moe_scan_scatter(experts, (size_t)T * K, E, counts, offsets, sorted_assign);
}

/* q4_gemm_and_moe.metal:2578-2624 with the slots of the CPU expectation in
 * test_shader_compile.rs:3004-3033 (slot = order of the assignment id). */
int kro_moe_scan_scatter(const uint32_t *experts, size_t num_assign, uint32_t E,
                         uint32_t *counts, uint32_t *offsets, uint32_t *sorted_assign) {
    memset(counts, 0, sizeof(uint32_t) * E);
    for (size_t a = 0; a < num_assign; ++a) {
        if (experts[a] >= E) return -1;
        counts[experts[a]] += 1;
    }
    uint32_t run = 0;
    for (uint32_t e = 0; e < E; ++e) { offsets[e] = run; run += counts[e]; }
    offsets[E] = run;
    uint32_t *fill = (uint32_t *)calloc(E ? E : 1, sizeof(uint32_t));
    for (size_t a = 0; a < num_assign; ++a) {
        uint32_t e = experts[a];
        sorted_assign[offsets[e] + fill[e]] = (uint32_t)a;
        fill[e] += 1;
    }
    free(fill);
    return 0;
}

typedef struct {
    const uint32_t *gqw; const uint16_t *gsc, *gbi;
    const uint32_t *uqw; const uint16_t *usc, *ubi;
    const uint32_t *dqw; const uint16_t *dsc, *dbi;
    uint32_t hidden, inter, K;
    const float *xf;
    const uint32_t *experts;
    int variant;
    float *d; /* [T*K, hidden] */
} moe_ctx;

static float dot_seq(const float *w, const float *x, uint32_t k) {
    float acc = 0.0f;
    for (uint32_t j = 0; j < k; ++j) { float p = w[j] * x[j]; acc = acc + p; }
    return acc;
}

static void moe_range(void *p, size_t begin, size_t end) {
    moe_ctx *c = (moe_ctx *)p;
    float *row = (float *)malloc(sizeof(float) * (c->hidden > c->inter ? c->hidden : c->inter));
    float *h = (float *)malloc(sizeof(float) * c->inter);
    for (size_t a = begin; a < end; ++a) {
        size_t t = a / c->K;
        uint32_t e = c->experts[a];
        const float *x = c->xf + t * c->hidden;
        for (uint32_t i = 0; i < c->inter; ++i) {
            size_t r = (size_t)e * c->inter + i;
            dequant_row(c->gqw, c->gsc, c->gbi, c->hidden, r, row);
            float g = dot_seq(row, x, c->hidden);
            dequant_row(c->uqw, c->usc, c->ubi, c->hidden, r, row);
            float u = dot_seq(row, x, c->hidden);
            h[i] = kro_bf16_to_f32(kro_f32_to_bf16(kro_activation(g, c->variant) * u));
        }
        for (uint32_t o = 0; o < c->hidden; ++o) {
            dequant_row(c->dqw, c->dsc, c->dbi, c->inter, (size_t)e * c->hidden + o, row);
            c->d[a * c->hidden + o] = dot_seq(row, h, c->inter);
        }
    }
    free(row); free(h);
}

void kro_moe_experts(const uint32_t *gqw, const uint16_t *gsc, const uint16_t *gbi,
                     const uint32_t *uqw, const uint16_t *usc, const uint16_t *ubi,
                     const uint32_t *dqw, const uint16_t *dsc, const uint16_t *dbi,
                     uint32_t E, uint32_t hidden, uint32_t inter,
                     const uint16_t *x_bf16, uint32_t T, uint32_t K,
                     const uint32_t *experts, const float *weights, int variant,
                     float *y, int nthreads) {
    (void)E;
    float *xf = bf16_rows_to_f32(x_bf16, (size_t)T * hidden);
    float *d = (float *)malloc(sizeof(float) * ((size_t)T * K * hidden + 1));
    moe_ctx c = {gqw, gsc, gbi, uqw, usc, ubi, dqw, dsc, dbi, hidden, inter, K, xf, experts, variant, d};
    parallel_for((size_t)T * K, nthreads, moe_range, &c);
    /* transformer_glue.metal:385-392: acc = fma(w, e_k[d], acc) over k in order. */
    for (size_t t = 0; t < T; ++t)
        for (size_t o = 0; o < hidden; ++o) {
            float acc = 0.0f;
            for (size_t k = 0; k < K; ++k)
                acc = fmaf(weights[t * K + k], d[(t * K + k) * hidden + o], acc);
            y[t * hidden + o] = acc;
        }
    free(xf); free(d);
}
