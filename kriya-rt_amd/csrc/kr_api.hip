// kr_api.hip — the C ABI (include/kriya_q4.h): argument validation, dispatch
// policy and error reporting.  Mirrors the operator surface of
// crates/kriya-backend-metal/src/encoder.rs (encode_q4_linear :2361-2420,
// encode_q4_linear_accumulate :2497-2536, encode_fused_gate_up :2703-2848,
// encode_dense_mlp :2851-2906), with the shape checks the reference lacks.
#include <stdarg.h>
#include <stdio.h>

#include <algorithm>
#include <mutex>
#include <string>

#include "kriya_glue.h"
#include "kriya_q4.h"
#include "kr_internal.hpp"

namespace kr {

Tuning &tuning() {
    static Tuning t;
    return t;
}

namespace {

thread_local std::string g_err;

int fail(int code, const char *fmt, ...) {
    char buf[512];
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(buf, sizeof(buf), fmt, ap);
    va_end(ap);
    g_err = buf;
    return code;
}

int ok() {
    g_err.clear();
    return KR_OK;
}

int hip_status(hipError_t e, const char *what) {
    if (e != hipSuccess) return fail(KR_E_HIP, "%s: %s", what, hipGetErrorString(e));
    return ok();
}

bool aligned(const void *p, size_t a) { return ((uintptr_t)p % a) == 0; }

int check_matrix(const kr_q4_matrix *w, const char *name) {
    if (!w) return fail(KR_E_INVALID, "%s: matrix descriptor is NULL", name);
    if (!w->qw || !w->scales || !w->biases) return fail(KR_E_INVALID, "%s: qw/scales/biases must be non-NULL", name);
    if (w->k == 0 || w->k % 64 != 0) return fail(KR_E_SHAPE, "%s: k=%u is not a positive multiple of 64", name, w->k);
    if (w->n == 0) return fail(KR_E_SHAPE, "%s: n must be positive", name);
    if (!aligned(w->qw, 16)) return fail(KR_E_ALIGN, "%s: qw must be 16-byte aligned", name);
    if (!aligned(w->scales, 2) || !aligned(w->biases, 2))
        return fail(KR_E_ALIGN, "%s: scales/biases must be 2-byte aligned", name);
    if ((uint64_t)w->n * (w->k / 8) > (1ull << 40)) return fail(KR_E_SHAPE, "%s: matrix too large", name);
    if (w->k > kMaxGemvK) return fail(KR_E_SHAPE, "%s: k=%u exceeds the supported maximum %u", name, w->k, kMaxGemvK);
    return KR_OK;
}

Q4Mat to_mat(const kr_q4_matrix *w) { return Q4Mat{w->qw, w->scales, w->biases, w->n, w->k}; }

size_t dtype_size(int dt) { return dt == KR_DTYPE_F32 ? 4 : 2; }

bool valid_dtype(int dt) { return dt == KR_DTYPE_BF16 || dt == KR_DTYPE_F32; }
bool valid_act(int a) { return a == KR_ACT_SWIGLU || a == KR_ACT_GEGLU || a == KR_ACT_RELU; }

size_t round_up(size_t v, size_t a) { return (v + a - 1) / a * a; }

constexpr uint32_t kMaxSplitK = 8;

// M tile class of the matrix-core kernels: 32-row tiles for batched decode,
// 64 or 128 rows for prefill.
int bm_class(uint32_t m) { return m <= 16 ? 16 : (m <= 64 ? 64 : 128); }
int bn_of(int bm, bool gate_up) { return bm <= 16 ? 32 : (gate_up ? 64 : 64); }
int bm_rows(int bm) { return bm <= 16 ? 32 : bm; }

MfmaArgs mfma_args(const uint16_t *x, uint32_t m, uint32_t k, int out_dtype, int accumulate) {
    MfmaArgs a{};
    a.x = x;
    a.m = m;
    a.k = k;
    a.ldx = k;
    a.out_f32 = out_dtype == KR_DTYPE_F32;
    a.accumulate = accumulate;
    a.ksplit = 1;
    a.groups_per_split = k / 64;
    return a;
}

MfmaProblem problem(const Q4Mat &w, const Q4Mat *w2, void *out, const uint16_t *bias, uint32_t ldo) {
    MfmaProblem p{};
    p.w = w;
    if (w2) p.w2 = *w2;
    p.out = out;
    p.bias = bias;
    p.ldo = ldo;
    return p;
}

// Few-token matmul on the skinny kernel.  `partial` (f32 [ksplit, m, nw * n])
// is needed when the K split exceeds one block; without it the caller must use
// another path (returns hipErrorInvalidValue).  `tickets` (kSkinnyTickets zero
// words, left zero): the split is reduced inside the launch, else by a second one.
// More than one launch's rows (32, or 16 with KR_OPT_SKINNY_GROUPS = 1; up to kSkinnyChunkMaxM):
// chunks, one launch each, in row order; each reuses the partials and leaves the tickets at zero
// for the next.
hipError_t run_skinny(const Q4Mat &w, const Q4Mat *w2, const uint16_t *x, uint32_t m, void *out,
                      const uint16_t *bias, uint32_t ldo, int out_dtype, int accumulate, int act, float *partial,
                      hipStream_t s, const uint16_t *ln_w = nullptr, float eps = 0.0f,
                      uint32_t *tickets = nullptr) {
    if (const uint32_t chunk = skinny_chunk_rows(); m > chunk) {
        const size_t esz = dtype_size(out_dtype);
        for (uint32_t i0 = 0; i0 < m; i0 += chunk) {
            const uint32_t mc = std::min(chunk, m - i0);
            if (hipError_t e = run_skinny(w, w2, x + (size_t)i0 * w.k, mc, (char *)out + (size_t)i0 * ldo * esz, bias, ldo,
                                          out_dtype, accumulate, act, partial, s, ln_w, eps, tickets))
                return e;
        }
        return hipSuccess;
    }
    SkinnyArgs a{};
    a.ln_w = ln_w;
    a.eps = eps;
    a.w = w;
    if (w2) a.w2 = *w2;
    a.x = x;
    a.m = m;
    a.k = w.k;
    a.ldx = w.k;
    a.out = out;
    a.bias = bias;
    a.ldo = ldo;
    a.act = act;
    a.out_f32 = out_dtype == KR_DTYPE_F32;
    a.accumulate = accumulate;
    const uint32_t ks = skinny_ksplit(w.k);
    if (ks > 1) {
        if (!partial) return hipErrorInvalidValue;
        a.partial = partial;
        if (tickets && tuning().splitk_tickets && ks <= kSkinnyMaxTicketSplit) a.tickets = tickets;
    }
    hipError_t e = launch_skinny(a, s);
    if (e != hipSuccess || ks == 1 || a.tickets) return e;
    MfmaArgs r{};
    r.p[0].w = w;
    r.p[0].out = out;
    r.p[0].bias = bias;
    r.p[0].ldo = ldo;
    r.np = 1;
    r.m = m;
    r.act = act;
    r.out_f32 = a.out_f32;
    r.accumulate = accumulate;
    r.partial = partial;
    r.ksplit = ks;
    return launch_splitk_reduce(r, w2 ? 2 : 1, s);
}

// Q, K and V in one few-token launch (k within one slab), x optionally RMS-normalised while staged.
hipError_t run_skinny_qkv(const kr_q4_matrix *const *mats, const uint16_t *const *biases, void *const *outs,
                          const uint16_t *x, uint32_t m, int out_dtype, const uint16_t *ln_w, float eps,
                          hipStream_t s) {
    if (const uint32_t chunk = skinny_chunk_rows(); m > chunk) {  // chunks, as run_skinny
        const size_t esz = dtype_size(out_dtype);
        for (uint32_t i0 = 0; i0 < m; i0 += chunk) {
            void *o[3];
            for (int i = 0; i < 3; ++i) o[i] = (char *)outs[i] + (size_t)i0 * mats[i]->n * esz;
            if (hipError_t e = run_skinny_qkv(mats, biases, o, x + (size_t)i0 * mats[0]->k,
                                              std::min(chunk, m - i0), out_dtype, ln_w, eps, s))
                return e;
        }
        return hipSuccess;
    }
    SkinnyArgs a{};
    a.w = to_mat(mats[0]);
    a.x = x;
    a.m = m;
    a.k = mats[0]->k;
    a.ldx = mats[0]->k;
    a.out = outs[0];
    a.bias = biases[0];
    a.ldo = mats[0]->n;
    a.out_f32 = out_dtype == KR_DTYPE_F32;
    for (int i = 0; i < 2; ++i) a.more[i] = SkinnyArgs::More{to_mat(mats[i + 1]), outs[i + 1], biases[i + 1], mats[i + 1]->n};
    a.nmore = 2;
    a.ln_w = ln_w;
    a.eps = eps;
    return launch_skinny(a, s);
}

// The few-token kernel takes 2 <= m < 64 (above 16 rows in chunks): it is exact for any bf16 x,
// where the reference keeps f32 tiles (q4_gemm_and_moe.metal:2173-2486); the prefill kernel stages
// fp16, as the reference's M >= 64 kernels stage half.
bool skinny_fits(uint32_t m, const Q4Mat &w, bool have_partial) {
    return m >= 2 && m <= kSkinnyChunkMaxM && skinny_supported(w) && (have_partial || skinny_ksplit(w.k) == 1);
}

size_t partial_bytes(uint32_t m, uint32_t n, uint32_t k, int nw) {
    // the largest K split of any skinny launch shape (64-column lane groups, 4 waves), so that
    // a workspace sized once stays valid under every tuning option
    const uint32_t skinny_worst = ((k + 255) / 256 + 3) / 4;
    const uint32_t ks = std::max<uint32_t>(skinny_worst, kMaxSplitK);
    return round_up((size_t)ks * m * nw * n * 4, 256);
}

// Split K over the blocks when the tile grid alone would leave CUs idle.
void choose_split_k(MfmaArgs &a, int bm, float *partial) {
    const uint32_t groups = a.k / 64;
    const bool prefill = bm > 16 && tuning().prefill_kernel != 1 && prefill_supported(a);
    const uint32_t rows = prefill ? prefill_block_m(a.p[0].w2.qw != nullptr) : (uint32_t)bm_rows(bm);
    const uint32_t cols = prefill ? prefill_block_rows(a.p[0].w2.qw != nullptr) : (uint32_t)bn_of(bm, false);
    const uint32_t tiles = ((a.m + rows - 1) / rows) * ((a.p[0].w.n + cols - 1) / cols);
    // the prefill kernel's split tiles: about one block per CU (fewer partials to reduce); the
    // tiled kernel: two
    const uint32_t target = (prefill ? 1u : 2u) * (uint32_t)device_cus();
    uint32_t split = 1;
    while (split < kMaxSplitK && tiles * split < target && groups / (split * 2) >= 8) split *= 2;
    if (split > 1) {
        a.ksplit = split;
        a.groups_per_split = ((groups + split - 1) / split + 1) & ~1u;  // even: the prefill kernel's steps take two groups
        a.partial = partial;
    }
}

}  // namespace

int device_cus() {
    static thread_local int dev = -1, cus = 0;
    int d = 0;
    if (hipGetDevice(&d) != hipSuccess) d = 0;
    if (d != dev) {
        dev = d;
        if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, d) != hipSuccess || cus <= 0) cus = 256;
    }
    return cus;
}

// The message of kr_last_error() for the host-only parts of the library (csrc/safetensors.cpp).
int set_error(int code, const char *msg) {
    if (code == KR_OK) g_err.clear();
    else g_err = msg;
    return code;
}

}  // namespace kr

using namespace kr;

extern "C" {

int kr_abi_version(void) { return KR_ABI_VERSION; }

const char *kr_last_error(void) { return g_err.c_str(); }

int kr_set_option(int option, int value) {
    switch (option) {
        case KR_OPT_GEMV_ROWS_PER_WAVE:
            if (value != 1 && value != 2 && value != 4 && value != 8)
                return fail(KR_E_INVALID, "rows per wave must be 1, 2, 4 or 8");
            tuning().gemv_rows_per_wave = value;
            return ok();
        case KR_OPT_GEMV_MAX_BLOCKS:
            if (value < 0) return fail(KR_E_INVALID, "max blocks must be >= 0");
            tuning().gemv_max_blocks = value;
            return ok();
        case KR_OPT_GEMV_SPLIT_K_CHUNKS:
            if (value < 0) return fail(KR_E_INVALID, "split-k threshold must be >= 0");
            tuning().gemv_split_k_chunks = value;
            return ok();
        case KR_OPT_GEMV_BLOCK_ROWS:
            if (value != 1 && value != 2 && value != 4 && value != 8)
                return fail(KR_E_INVALID, "block rows must be 1, 2, 4 or 8");
            tuning().gemv_block_rows = value;
            return ok();
        case KR_OPT_GEMV_PERSISTENT_BLOCKS:
            if (value < 1) return fail(KR_E_INVALID, "persistent blocks must be >= 1");
            tuning().gemv_persistent_blocks = value;
            return ok();
        case KR_OPT_SKINNY_MAX_BLOCKS:
            if (value < 1) return fail(KR_E_INVALID, "skinny max blocks must be >= 1");
            tuning().skinny_max_blocks = value;
            return ok();
        case KR_OPT_GEMV_LONG_ROWS:
            if (value != 0 && value != 4 && value != 8 && value != 16)
                return fail(KR_E_INVALID, "long rows must be 0, 4, 8 or 16");
            tuning().gemv_long_rows = value;
            return ok();
        case KR_OPT_PREFILL_KERNEL:
            if (value < 0 || value > 2) return fail(KR_E_INVALID, "prefill kernel must be 0, 1 or 2");
            tuning().prefill_kernel = value;
            return ok();
        case KR_OPT_GEMV_TOKENS:
            if (value != 0 && value != 1) return fail(KR_E_INVALID, "gemv tokens must be 0 or 1");
            tuning().gemv_tokens = value;
            return ok();
        case KR_OPT_MOE_GEMV:
            if (value != 0 && value != 1) return fail(KR_E_INVALID, "moe gemv must be 0 or 1");
            tuning().moe_gemv = value;
            return ok();
        case KR_OPT_GEMV_LONG_GROUPS:
            if (value != 1 && value != 2) return fail(KR_E_INVALID, "long-row groups must be 1 or 2");
            tuning().gemv_long_groups = value;
            return ok();
        case KR_OPT_SPLITK_TICKETS:
            if (value != 0 && value != 1) return fail(KR_E_INVALID, "split-K tickets must be 0 or 1");
            tuning().splitk_tickets = value;
            return ok();
        case KR_OPT_ATTN_MERGE_WAVE:
            if (value != 0 && value != 1) return fail(KR_E_INVALID, "attention merge must be 0 or 1");
            tuning().attn_merge_wave = value;
            return ok();
        case KR_OPT_PREFILL_OPERANDS:
            if (value != 0 && value != 1) return fail(KR_E_INVALID, "prefill operands must be 0 or 1");
            tuning().prefill_operands = value;
            return ok();
        case KR_OPT_SKINNY_GROUPS:
            if (value != 1 && value != 2) return fail(KR_E_INVALID, "few-token row groups must be 1 or 2");
            tuning().skinny_groups = value;
            return ok();
        case KR_OPT_SKINNY_DEPTH:
            if (value != 0 && value != 2 && value != 3) return fail(KR_E_INVALID, "few-token depth must be 0, 2 or 3");
            tuning().skinny_depth = value;
            return ok();
        case KR_OPT_MOE_COMBINE:
            if (value != 0 && value != 1) return fail(KR_E_INVALID, "moe combine must be 0 or 1");
            tuning().moe_combine = value;
            return ok();
        case KR_OPT_MOE_ROUTE_FUSED:
            if (value != 0 && value != 1) return fail(KR_E_INVALID, "moe route fused must be 0 or 1");
            tuning().moe_route_fused = value;
            return ok();
        case KR_OPT_PREFILL_XCD_SPLIT:
            if (value != 0 && value != 1) return fail(KR_E_INVALID, "prefill xcd split must be 0 or 1");
            tuning().prefill_xcd_split = value;
            return ok();
        case KR_OPT_ATTN_MERGE_OPROJ:
            if (value != 0 && value != 1) return fail(KR_E_INVALID, "attention merge o_proj must be 0 or 1");
            tuning().attn_merge_oproj = value;
            return ok();
        case KR_OPT_ATTN_SLICE64:
            if (value < 0 || value > 2) return fail(KR_E_INVALID, "attention slice64 must be 0, 1 or 2");
            tuning().attn_slice64 = value;
            return ok();
        default: return fail(KR_E_INVALID, "unknown option %d", option);
    }
}

int kr_get_option(int option) {
    switch (option) {
        case KR_OPT_GEMV_ROWS_PER_WAVE: return tuning().gemv_rows_per_wave;
        case KR_OPT_GEMV_MAX_BLOCKS: return tuning().gemv_max_blocks;
        case KR_OPT_GEMV_SPLIT_K_CHUNKS: return tuning().gemv_split_k_chunks;
        case KR_OPT_GEMV_BLOCK_ROWS: return tuning().gemv_block_rows;
        case KR_OPT_GEMV_PERSISTENT_BLOCKS: return tuning().gemv_persistent_blocks;
        case KR_OPT_SKINNY_MAX_BLOCKS: return tuning().skinny_max_blocks;
        case KR_OPT_PREFILL_KERNEL: return tuning().prefill_kernel;
        case KR_OPT_GEMV_LONG_ROWS: return tuning().gemv_long_rows;
        case KR_OPT_GEMV_TOKENS: return tuning().gemv_tokens;
        case KR_OPT_MOE_GEMV: return tuning().moe_gemv;
        case KR_OPT_MOE_COMBINE: return tuning().moe_combine;
        case KR_OPT_MOE_ROUTE_FUSED: return tuning().moe_route_fused;
        case KR_OPT_PREFILL_XCD_SPLIT: return tuning().prefill_xcd_split;
        case KR_OPT_ATTN_SLICE64: return tuning().attn_slice64;
        case KR_OPT_ATTN_MERGE_OPROJ: return tuning().attn_merge_oproj;
        case KR_OPT_GEMV_LONG_GROUPS: return tuning().gemv_long_groups;
        case KR_OPT_SPLITK_TICKETS: return tuning().splitk_tickets;
        case KR_OPT_ATTN_MERGE_WAVE: return tuning().attn_merge_wave;
        case KR_OPT_PREFILL_OPERANDS: return tuning().prefill_operands;
        case KR_OPT_SKINNY_GROUPS: return tuning().skinny_groups;
        case KR_OPT_SKINNY_DEPTH: return tuning().skinny_depth;
        default: return fail(KR_E_INVALID, "unknown option %d", option);
    }
}

size_t kr_stream_read_pieces(size_t bytes) { return stream_read_pieces(bytes); }

int kr_stream_read(const void *buf, size_t bytes, uint32_t match, uint32_t *hits, void *stream) {
    if (!buf || !hits) return fail(KR_E_INVALID, "buf and hits must not be NULL");
    if (bytes == 0 || bytes % 16 != 0) return fail(KR_E_SHAPE, "bytes must be a positive multiple of 16");
    if (!aligned(buf, 16) || !aligned(hits, 4)) return fail(KR_E_ALIGN, "buf must be 16-byte aligned, hits 4-byte");
    if (bytes / 16 / 256 >= 0x7FFFFFFFu) return fail(KR_E_SHAPE, "bytes too large");
    return hip_status(launch_stream_read(buf, bytes, match, hits, (hipStream_t)stream), "kr_stream_read");
}

int kr_q4_dequant(const kr_q4_matrix *w, float *out, void *stream) {
    if (int rc = check_matrix(w, "w")) return rc;
    if (!out) return fail(KR_E_INVALID, "out is NULL");
    if (!aligned(out, 16)) return fail(KR_E_ALIGN, "out must be 16-byte aligned");
    return hip_status(launch_format_dequant(to_mat(w), out, (hipStream_t)stream), "kr_q4_dequant");
}

int kr_q4_from_blocks36(const void *blocks, uint32_t n, uint32_t k, uint32_t *qw, uint16_t *scales,
                        uint16_t *biases, void *stream) {
    if (!blocks || !qw || !scales || !biases) return fail(KR_E_INVALID, "NULL pointer");
    if (k == 0 || k % 64 != 0) return fail(KR_E_SHAPE, "k=%u is not a positive multiple of 64", k);
    if (!aligned(blocks, 4)) return fail(KR_E_ALIGN, "blocks must be 4-byte aligned");
    if (!aligned(qw, 16)) return fail(KR_E_ALIGN, "qw must be 16-byte aligned");
    if (!aligned(scales, 2) || !aligned(biases, 2)) return fail(KR_E_ALIGN, "scales/biases must be 2-byte aligned");
    return hip_status(launch_from_blocks36(blocks, n, k, qw, scales, biases, (hipStream_t)stream),
                      "kr_q4_from_blocks36");
}

int kr_q4_to_blocks36(const kr_q4_matrix *w, void *blocks, void *stream) {
    if (int rc = check_matrix(w, "w")) return rc;
    if (!blocks) return fail(KR_E_INVALID, "blocks is NULL");
    if (!aligned(blocks, 4)) return fail(KR_E_ALIGN, "blocks must be 4-byte aligned");
    return hip_status(launch_to_blocks36(to_mat(w), blocks, (hipStream_t)stream), "kr_q4_to_blocks36");
}

int kr_q4_from_split(const void *qs, const void *sb, uint32_t n, uint32_t k, uint32_t *qw, uint16_t *scales,
                     uint16_t *biases, void *stream) {
    if (!qs || !sb || !qw || !scales || !biases) return fail(KR_E_INVALID, "NULL pointer");
    if (k == 0 || k % 64 != 0) return fail(KR_E_SHAPE, "k=%u is not a positive multiple of 64", k);
    if (!aligned(qs, 16) || !aligned(qw, 16)) return fail(KR_E_ALIGN, "qs and qw must be 16-byte aligned");
    if (!aligned(sb, 4)) return fail(KR_E_ALIGN, "sb must be 4-byte aligned");
    if (!aligned(scales, 2) || !aligned(biases, 2)) return fail(KR_E_ALIGN, "scales/biases must be 2-byte aligned");
    return hip_status(launch_from_split(qs, sb, n, k, qw, scales, biases, (hipStream_t)stream), "kr_q4_from_split");
}

int kr_q4_to_split(const kr_q4_matrix *w, void *qs, void *sb, void *stream) {
    if (int rc = check_matrix(w, "w")) return rc;
    if (!qs || !sb) return fail(KR_E_INVALID, "qs and sb must not be NULL");
    if (!aligned(qs, 16)) return fail(KR_E_ALIGN, "qs must be 16-byte aligned");
    if (!aligned(sb, 4)) return fail(KR_E_ALIGN, "sb must be 4-byte aligned");
    return hip_status(launch_to_split(to_mat(w), qs, sb, (hipStream_t)stream), "kr_q4_to_split");
}

int kr_f16_to_bf16(const uint16_t *in, uint16_t *out, size_t count, void *stream) {
    if (count == 0) return ok();
    if (!in || !out) return fail(KR_E_INVALID, "NULL pointer");
    if (!aligned(in, 2) || !aligned(out, 2)) return fail(KR_E_ALIGN, "in/out must be 2-byte aligned");
    return hip_status(launch_f16_to_bf16(in, out, count, (hipStream_t)stream), "kr_f16_to_bf16");
}

int kr_q4_linear(const kr_q4_matrix *w, const uint16_t *x, uint32_t m, void *y, int y_dtype, int accumulate,
                 void *stream) {
    if (int rc = check_matrix(w, "w")) return rc;
    if (!valid_dtype(y_dtype)) return fail(KR_E_INVALID, "y_dtype %d is not KR_DTYPE_BF16/F32", y_dtype);
    if (accumulate != 0 && accumulate != 1) return fail(KR_E_INVALID, "accumulate must be 0 or 1");
    if (m == 0) return ok();
    if (!x || !y) return fail(KR_E_INVALID, "x/y must be non-NULL");
    if (!aligned(x, 16)) return fail(KR_E_ALIGN, "x must be 16-byte aligned");
    if (!aligned(y, dtype_size(y_dtype))) return fail(KR_E_ALIGN, "y is misaligned for its dtype");
    const Q4Mat a = to_mat(w);
    hipStream_t s = (hipStream_t)stream;
    if (m == 1) {
        const int epi = accumulate ? (y_dtype == KR_DTYPE_F32 ? kAccF32 : kAccBF16)
                                   : (y_dtype == KR_DTYPE_F32 ? kStoreF32 : kStoreBF16);
        return hip_status(launch_gemv(a, nullptr, x, y, epi, 0, nullptr, s), "kr_q4_linear");
    }
    if (tuning().gemv_tokens && gemv_tokens_supported(m, w->k, false)) {
        const int epi = accumulate ? (y_dtype == KR_DTYPE_F32 ? kAccF32 : kAccBF16)
                                   : (y_dtype == KR_DTYPE_F32 ? kStoreF32 : kStoreBF16);
        return hip_status(launch_gemv_tokens(a, nullptr, x, m, y, w->n, epi, 0, nullptr, s), "kr_q4_linear");
    }
    if (skinny_fits(m, to_mat(w), false))
        return hip_status(run_skinny(a, nullptr, x, m, y, nullptr, w->n, y_dtype, accumulate, 0, nullptr, s),
                          "kr_q4_linear");
    if (m <= 16 && tuning().gemv_tokens && gemv_tokens_supported(kGemvMaxTokens, w->k, false)) {
        // A few tokens over a K the few-token kernel needs a split-K workspace for (none here): the
        // token GEMV in chunks of up to kGemvMaxTokens tokens, every weight row read once per chunk
        // (m = 16, K = 11008: 36 us against 145 us for the unsplit tiled kernel).  Each token's row is
        // the one a call with that token alone gives.
        const int epi = accumulate ? (y_dtype == KR_DTYPE_F32 ? kAccF32 : kAccBF16)
                                   : (y_dtype == KR_DTYPE_F32 ? kStoreF32 : kStoreBF16);
        const size_t ysz = dtype_size(y_dtype);
        for (uint32_t t0 = 0; t0 < m; t0 += kGemvMaxTokens) {
            const uint32_t mc = std::min<uint32_t>(kGemvMaxTokens, m - t0);
            const uint16_t *xc = x + (size_t)t0 * w->k;
            void *yc = static_cast<char *>(y) + (size_t)t0 * w->n * ysz;
            const hipError_t e = mc == 1 ? launch_gemv(a, nullptr, xc, yc, epi, 0, nullptr, s)
                                         : launch_gemv_tokens(a, nullptr, xc, mc, yc, w->n, epi, 0, nullptr, s);
            if (int rc = hip_status(e, "kr_q4_linear")) return rc;
        }
        return ok();
    }
    MfmaArgs args = mfma_args(x, m, w->k, y_dtype, accumulate);
    args.p[0] = problem(a, nullptr, y, nullptr, w->n);
    args.np = 1;
    return hip_status(launch_mfma(args, bm_class(m), s), "kr_q4_linear");
}

// Gate/up at 2 <= m <= 4 on the token GEMV kernel, except at m = 4 where the few-token matrix-core
// kernel is faster when it fits (cfg1 shape: 9.7 against 11.3 us; m = 3: 9.7 both, m = 2: 8.4
// against 9.7).  The down projection keeps the token GEMV at m <= 4 (cfg1 m = 4: 9.0 against 10.8).
static bool gate_up_on_tokens(uint32_t m, const Q4Mat &g, const Q4Mat &u) {
    if (!(tuning().gemv_tokens && gemv_tokens_supported(m, g.k, true))) return false;
    return m <= 3 || !(skinny_fits(m, g, false) && skinny_supported(u));
}

int kr_q4_gate_up_act(const kr_q4_matrix *gate, const kr_q4_matrix *up, const uint16_t *x, uint32_t m,
                      void *act_out, int act_dtype, int activation, void *stream) {
    if (int rc = check_matrix(gate, "gate")) return rc;
    if (int rc = check_matrix(up, "up")) return rc;
    if (gate->n != up->n || gate->k != up->k)
        return fail(KR_E_SHAPE, "gate [%u,%u] and up [%u,%u] differ", gate->n, gate->k, up->n, up->k);
    if (!valid_dtype(act_dtype)) return fail(KR_E_INVALID, "act_dtype %d invalid", act_dtype);
    if (!valid_act(activation)) return fail(KR_E_INVALID, "activation %d invalid", activation);
    if (m == 0) return ok();
    if (!x || !act_out) return fail(KR_E_INVALID, "x/act_out must be non-NULL");
    if (!aligned(x, 16)) return fail(KR_E_ALIGN, "x must be 16-byte aligned");
    if (!aligned(act_out, dtype_size(act_dtype))) return fail(KR_E_ALIGN, "act_out misaligned");
    const Q4Mat g = to_mat(gate), u = to_mat(up);
    hipStream_t s = (hipStream_t)stream;
    if (m == 1) {
        const int epi = act_dtype == KR_DTYPE_F32 ? kGateUpF32 : kGateUpBF16;
        return hip_status(launch_gemv(g, &u, x, act_out, epi, activation, nullptr, s), "kr_q4_gate_up_act");
    }
    if (gate_up_on_tokens(m, g, u)) {
        const int epi = act_dtype == KR_DTYPE_F32 ? kGateUpF32 : kGateUpBF16;
        return hip_status(launch_gemv_tokens(g, &u, x, m, act_out, gate->n, epi, activation, nullptr, s),
                          "kr_q4_gate_up_act");
    }
    if (skinny_fits(m, to_mat(gate), false) && skinny_supported(to_mat(up)))
        return hip_status(run_skinny(g, &u, x, m, act_out, nullptr, gate->n, act_dtype, 0, activation, nullptr, s),
                          "kr_q4_gate_up_act");
    MfmaArgs args = mfma_args(x, m, gate->k, act_dtype, 0);
    args.act = activation;
    args.p[0] = problem(g, &u, act_out, nullptr, gate->n);
    args.np = 1;
    return hip_status(launch_mfma(args, bm_class(m), s), "kr_q4_gate_up_act");
}

int kr_q4_qkv(const kr_q4_matrix *q, const kr_q4_matrix *k, const kr_q4_matrix *v, const uint16_t *q_bias,
              const uint16_t *k_bias, const uint16_t *v_bias, const uint16_t *x, uint32_t m, void *q_out,
              void *k_out, void *v_out, int out_dtype, void *stream) {
    if (int rc = check_matrix(q, "q")) return rc;
    if (int rc = check_matrix(k, "k")) return rc;
    if (int rc = check_matrix(v, "v")) return rc;
    if (q->k != k->k || q->k != v->k) return fail(KR_E_SHAPE, "q, k, v must share k");
    if (!valid_dtype(out_dtype)) return fail(KR_E_INVALID, "out_dtype %d invalid", out_dtype);
    if (m == 0) return ok();
    if (!x || !q_out || !k_out || !v_out) return fail(KR_E_INVALID, "x and the outputs must be non-NULL");
    if (!aligned(x, 16)) return fail(KR_E_ALIGN, "x must be 16-byte aligned");
    const size_t osz = dtype_size(out_dtype);
    if (!aligned(q_out, osz) || !aligned(k_out, osz) || !aligned(v_out, osz)) return fail(KR_E_ALIGN, "output misaligned");
    if ((q_bias && !aligned(q_bias, 2)) || (k_bias && !aligned(k_bias, 2)) || (v_bias && !aligned(v_bias, 2)))
        return fail(KR_E_ALIGN, "bias misaligned");
    hipStream_t s = (hipStream_t)stream;
    const kr_q4_matrix *mats[3] = {q, k, v};
    const uint16_t *biases[3] = {q_bias, k_bias, v_bias};
    void *outs[3] = {q_out, k_out, v_out};
    if (m == 1) {
        const int epi = out_dtype == KR_DTYPE_F32 ? kStoreF32 : kStoreBF16;
        if (gemv_batch_supported(q->k)) {  // the three projections in one launch
            const Q4Mat ms[3] = {to_mat(q), to_mat(k), to_mat(v)};
            return hip_status(launch_gemv_batch(ms, nullptr, x, outs, biases, 3, epi, 0, nullptr, 0.0f, s),
                              "kr_q4_qkv");
        }
        for (int i = 0; i < 3; ++i) {
            const hipError_t e = launch_gemv(to_mat(mats[i]), nullptr, x, outs[i], epi, 0, biases[i], s);
            if (e != hipSuccess) return hip_status(e, "kr_q4_qkv");
        }
        return ok();
    }
    if (skinny_fits(m, to_mat(q), false) && skinny_supported(to_mat(k)) && skinny_supported(to_mat(v)))
        return hip_status(run_skinny_qkv(mats, biases, outs, x, m, out_dtype, nullptr, 0.0f, s), "kr_q4_qkv");
    MfmaArgs args = mfma_args(x, m, q->k, out_dtype, 0);
    for (int i = 0; i < 3; ++i) args.p[i] = problem(to_mat(mats[i]), nullptr, outs[i], biases[i], mats[i]->n);
    args.np = 3;
    return hip_status(launch_mfma(args, bm_class(m), s), "kr_q4_qkv");
}

// MLP workspace layout: the tickets of the in-launch split-K reduction first, at the same place for
// every m (zero between calls, so a workspace can serve several m), then the bf16 activation
// [m, inter], then (m > 1) the f32 split-K partials of the down projection, then (m on the prefill
// kernel) x and the activation converted to the prefill kernel's fp16 operand order.
constexpr size_t kMlpTicketBytes = ((size_t)kSkinnyTickets * 4 + 255) / 256 * 256;
static uint32_t *mlp_ws_tickets(void *ws) { return (uint32_t *)ws; }
static uint16_t *mlp_ws_act(void *ws) { return (uint16_t *)((char *)ws + kMlpTicketBytes); }
static float *mlp_ws_partial(void *ws, uint32_t m, uint32_t inter) {
    return (float *)((char *)ws + kMlpTicketBytes + round_up((size_t)m * inter * 2, 256));
}
static bool mlp_prefill_operands(uint32_t m) { return m > kSkinnyChunkMaxM; }
static uint16_t *mlp_ws_xh(void *ws, uint32_t m, uint32_t hidden, uint32_t inter) {
    return (uint16_t *)((char *)mlp_ws_partial(ws, m, inter) + partial_bytes(m, hidden, inter, 1));
}
static uint16_t *mlp_ws_acth(void *ws, uint32_t m, uint32_t hidden, uint32_t inter) {
    return (uint16_t *)((char *)mlp_ws_xh(ws, m, hidden, inter) + round_up((size_t)m * hidden * 2, 256));
}

size_t kr_q4_mlp_workspace_bytes(uint32_t m, uint32_t hidden, uint32_t intermediate) {
    size_t bytes = kMlpTicketBytes + round_up((size_t)m * intermediate * 2, 256);
    if (m > 1) bytes += partial_bytes(m, hidden, intermediate, 1);  // split-K partials of the down projection
    if (mlp_prefill_operands(m))  // fp16 operands of the prefill kernel
        bytes += round_up((size_t)m * hidden * 2, 256) + round_up((size_t)m * intermediate * 2, 256);
    return bytes;
}

// The MLP's down projection, accumulated into h, after the activation `act` (bf16 [m, inter]) was
// written to the workspace (layout above).
static int mlp_down(const kr_q4_matrix *gate, const kr_q4_matrix *down, const uint16_t *act, void *h, int h_dtype,
                    uint32_t m, void *workspace, void *stream) {
    if (m == 1 || (tuning().gemv_tokens && gemv_tokens_supported(m, gate->k, true) &&
                   gemv_tokens_supported(m, down->k, false)))
        return kr_q4_linear(down, act, m, h, h_dtype, 1, stream);
    // down projection: few N tiles at small m, so K is split over blocks; partials (and the
    // tickets of the in-launch reduction) live in the workspace
    float *partial = mlp_ws_partial(workspace, m, gate->n);
    uint32_t *tickets = mlp_ws_tickets(workspace);
    if (skinny_fits(m, to_mat(down), true))
        return hip_status(run_skinny(to_mat(down), nullptr, act, m, h, nullptr, down->n, h_dtype, 1, 0, partial,
                                     (hipStream_t)stream, nullptr, 0.0f, tickets),
                          "kr_q4_mlp (down)");
    MfmaArgs args = mfma_args(act, m, down->k, h_dtype, 1);
    args.p[0] = problem(to_mat(down), nullptr, h, nullptr, down->n);
    args.np = 1;
    const int bm = bm_class(m);
    choose_split_k(args, bm, partial);
    return hip_status(launch_mfma(args, bm, (hipStream_t)stream), "kr_q4_mlp (down)");
}

// kr_q4_linear with a workspace: [ticket words][split-K partials], the layout of the MLP's down
// projection (its tickets first, at the same place for every m).
size_t kr_q4_linear_workspace_bytes(uint32_t m, uint32_t n, uint32_t k) {
    if (m <= 1) return 0;
    return kMlpTicketBytes + partial_bytes(m, n, k, 1);
}

int kr_q4_linear_ws(const kr_q4_matrix *w, const uint16_t *x, uint32_t m, void *y, int y_dtype, int accumulate,
                    void *workspace, size_t workspace_bytes, void *stream) {
    if (int rc = check_matrix(w, "w")) return rc;
    if (!valid_dtype(y_dtype)) return fail(KR_E_INVALID, "y_dtype %d is not KR_DTYPE_BF16/F32", y_dtype);
    if (accumulate != 0 && accumulate != 1) return fail(KR_E_INVALID, "accumulate must be 0 or 1");
    if (m == 0) return ok();
    if (!x || !y) return fail(KR_E_INVALID, "x/y must be non-NULL");
    const size_t need = kr_q4_linear_workspace_bytes(m, w->n, w->k);
    if (need && (!workspace || workspace_bytes < need))
        return fail(KR_E_WORKSPACE, "workspace of %zu bytes required, %zu given", need, workspace_bytes);
    if (need && !aligned(workspace, 16)) return fail(KR_E_ALIGN, "workspace must be 16-byte aligned");
    const Q4Mat a = to_mat(w);
    // the shapes that split nothing: as kr_q4_linear (one token, the token GEMV, one K slab)
    if (m == 1 || (tuning().gemv_tokens && gemv_tokens_supported(m, w->k, false)) || skinny_fits(m, a, false))
        return kr_q4_linear(w, x, m, y, y_dtype, accumulate, stream);
    if (!aligned(x, 16)) return fail(KR_E_ALIGN, "x must be 16-byte aligned");
    if (!aligned(y, dtype_size(y_dtype))) return fail(KR_E_ALIGN, "y is misaligned for its dtype");
    hipStream_t s = (hipStream_t)stream;
    float *partial = (float *)((char *)workspace + kMlpTicketBytes);
    if (skinny_fits(m, a, true))  // 5 <= m <= 63 over more than one K slab
        return hip_status(run_skinny(a, nullptr, x, m, y, nullptr, w->n, y_dtype, accumulate, 0, partial, s, nullptr,
                                     0.0f, (uint32_t *)workspace),
                          "kr_q4_linear_ws");
    MfmaArgs args = mfma_args(x, m, w->k, y_dtype, accumulate);
    args.p[0] = problem(a, nullptr, y, nullptr, w->n);
    args.np = 1;
    const int bm = bm_class(m);
    choose_split_k(args, bm, partial);
    return hip_status(launch_mfma(args, bm, s), "kr_q4_linear_ws");
}

int kr_q4_mlp(const kr_q4_matrix *gate, const kr_q4_matrix *up, const kr_q4_matrix *down, const uint16_t *x,
              void *h, int h_dtype, uint32_t m, int activation, void *workspace, size_t workspace_bytes,
              void *stream) {
    if (int rc = check_matrix(gate, "gate")) return rc;
    if (int rc = check_matrix(up, "up")) return rc;
    if (int rc = check_matrix(down, "down")) return rc;
    if (gate->n != up->n || gate->k != up->k) return fail(KR_E_SHAPE, "gate and up shapes differ");
    if (down->k != gate->n || down->n != gate->k)
        return fail(KR_E_SHAPE, "down [%u,%u] does not match gate/up [%u,%u]", down->n, down->k, gate->n, gate->k);
    if (!valid_dtype(h_dtype)) return fail(KR_E_INVALID, "h_dtype %d invalid", h_dtype);
    if (!valid_act(activation)) return fail(KR_E_INVALID, "activation %d invalid", activation);
    if (m == 0) return ok();
    if (!h) return fail(KR_E_INVALID, "h is NULL");
    if (!x) {
        if (h_dtype != KR_DTYPE_BF16) return fail(KR_E_INVALID, "x is required when h is f32");
        x = (const uint16_t *)h;
    }
    if (!aligned(x, 16)) return fail(KR_E_ALIGN, "x must be 16-byte aligned");
    if (!aligned(h, dtype_size(h_dtype))) return fail(KR_E_ALIGN, "h misaligned");
    const size_t need = kr_q4_mlp_workspace_bytes(m, gate->k, gate->n);
    if (!workspace || workspace_bytes < need)
        return fail(KR_E_WORKSPACE, "workspace of %zu bytes required, %zu given", need, workspace_bytes);
    if (!aligned(workspace, 16)) return fail(KR_E_ALIGN, "workspace must be 16-byte aligned");
    uint16_t *act = mlp_ws_act(workspace);
    if (mlp_prefill_operands(m) && tuning().prefill_kernel != 1 && tuning().prefill_operands) {
        // Prefill kernel for both: x converted to its fp16 operand order once (not once per block),
        // and the gate/up epilogue writes the activation in that form too for the down projection
        // (the bf16 activation stays the exact operand of the kernel's overflow fallback).
        const Q4Mat g = to_mat(gate), u = to_mat(up);
        hipStream_t s = (hipStream_t)stream;
        MfmaArgs gu = mfma_args(x, m, gate->k, KR_DTYPE_BF16, 0);
        gu.act = activation;
        gu.p[0] = problem(g, &u, act, nullptr, gate->n);
        gu.np = 1;
        MfmaArgs dn = mfma_args(act, m, down->k, h_dtype, 1);
        dn.p[0] = problem(to_mat(down), nullptr, h, nullptr, down->n);
        dn.np = 1;
        if (prefill_supported(gu) && prefill_supported(dn)) {
            uint16_t *xh = mlp_ws_xh(workspace, m, gate->k, gate->n);
            uint16_t *acth = mlp_ws_acth(workspace, m, gate->k, gate->n);
            if (int rc = hip_status(launch_x_to_f16(x, m, gate->k, xh, s), "kr_q4_mlp (x to fp16)")) return rc;
            gu.xh = xh;
            gu.out_h = acth;
            if (int rc = hip_status(launch_prefill(gu, s), "kr_q4_mlp (gate/up)")) return rc;
            dn.xh = acth;
            choose_split_k(dn, bm_class(m), mlp_ws_partial(workspace, m, gate->n));
            return hip_status(launch_prefill(dn, s), "kr_q4_mlp (down)");
        }
    }
    if (int rc = kr_q4_gate_up_act(gate, up, x, m, act, KR_DTYPE_BF16, activation, stream)) return rc;
    return mlp_down(gate, down, act, h, h_dtype, m, workspace, stream);
}

int kr_moe_route(const float *logits, uint32_t tokens, uint32_t experts, uint32_t topk, int normalize,
                 uint32_t *selected, float *weights, uint32_t *counts, uint32_t *offsets, uint32_t *sorted_assign,
                 void *stream) {
    if (experts == 0 || experts > kMaxExperts) return fail(KR_E_INVALID, "experts=%u must be in 1..%u", experts, kMaxExperts);
    if (topk == 0 || topk > experts || topk > kRouteMaxTopK)
        return fail(KR_E_INVALID, "topk=%u must be in 1..min(experts, %u)", topk, kRouteMaxTopK);
    if ((uint64_t)tokens * topk > kRouteMaxAssign)
        return fail(KR_E_SHAPE, "tokens * topk = %llu exceeds %u", (unsigned long long)tokens * topk, kRouteMaxAssign);
    if (!counts || !offsets) return fail(KR_E_INVALID, "counts/offsets must be non-NULL");
    if (tokens > 0 && (!logits || !selected || !weights || !sorted_assign))
        return fail(KR_E_INVALID, "logits/selected/weights/sorted_assign must be non-NULL");
    if (!aligned(logits, 4) || !aligned(selected, 4) || !aligned(weights, 4) || !aligned(counts, 4) ||
        !aligned(offsets, 4) || !aligned(sorted_assign, 4))
        return fail(KR_E_ALIGN, "routing arrays must be 4-byte aligned");
    return hip_status(launch_moe_route(tokens ? logits : nullptr, tokens, experts, topk, normalize, selected, weights,
                                       counts, offsets, sorted_assign, (hipStream_t)stream),
                      "kr_moe_route");
}

int kr_moe_scan_scatter(const uint32_t *selected, uint32_t num_assign, uint32_t experts, uint32_t *counts,
                        uint32_t *offsets, uint32_t *sorted_assign, void *stream) {
    if (experts == 0 || experts > kMaxExperts) return fail(KR_E_INVALID, "experts=%u must be in 1..%u", experts, kMaxExperts);
    if (num_assign > kRouteMaxAssign) return fail(KR_E_SHAPE, "num_assign=%u exceeds %u", num_assign, kRouteMaxAssign);
    if (!counts || !offsets) return fail(KR_E_INVALID, "counts/offsets must be non-NULL");
    if (num_assign > 0 && (!selected || !sorted_assign))
        return fail(KR_E_INVALID, "selected/sorted_assign must be non-NULL");
    if (!aligned(selected, 4) || !aligned(counts, 4) || !aligned(offsets, 4) || !aligned(sorted_assign, 4))
        return fail(KR_E_ALIGN, "routing arrays must be 4-byte aligned");
    // the kernel's given-assignment mode: T = num_assign rows of one slot each
    return hip_status(launch_moe_route(nullptr, num_assign, experts, 1, 0, const_cast<uint32_t *>(selected), nullptr,
                                       counts, offsets, sorted_assign, (hipStream_t)stream),
                      "kr_moe_scan_scatter");
}

size_t kr_q4_moe_workspace_bytes(uint32_t tokens, uint32_t topk, uint32_t hidden, uint32_t inter) {
    const size_t assign = (size_t)tokens * topk;
    return round_up(assign * inter * 2, 256) + round_up(assign * hidden * 4, 256);
}

namespace {
// Routing computed inside the experts' first launch (kr_q4_moe_route_experts, one token).
struct FusedRoute {
    const float *logits;
    int normalize;
    uint32_t *selected, *counts;
};

// The routed GEMV path: few assignments, rows of <= 2048 columns.
bool moe_gemv_path(uint32_t tokens, uint32_t topk, uint32_t hidden, uint32_t inter) {
    return tuning().moe_gemv && (uint64_t)tokens * topk <= kMoeGemvMaxAssign && moe_gemv_fits(hidden) &&
           moe_gemv_fits(inter);
}

// kr_q4_moe_experts' argument checks; hidden and inter on success.  tokens == 0 passes without the
// pointer checks (the call then does nothing).
int check_moe_experts(const kr_q4_matrix *gate, const kr_q4_matrix *up, const kr_q4_matrix *down, uint32_t experts,
                      const uint16_t *x, uint32_t tokens, uint32_t topk, const float *weights,
                      const uint32_t *offsets, const uint32_t *sorted_assign, int activation, void *y, int y_dtype,
                      int accumulate, void *workspace, size_t workspace_bytes, uint32_t &hidden, uint32_t &inter) {
    if (int rc = check_matrix(gate, "gate")) return rc;
    if (int rc = check_matrix(up, "up")) return rc;
    if (int rc = check_matrix(down, "down")) return rc;
    if (experts == 0 || experts > kMaxExperts) return fail(KR_E_INVALID, "experts=%u must be in 1..%u", experts, kMaxExperts);
    if (gate->n != up->n || gate->k != up->k) return fail(KR_E_SHAPE, "gate and up shapes differ");
    if (gate->n % experts != 0) return fail(KR_E_SHAPE, "gate rows %u are not a multiple of experts=%u", gate->n, experts);
    hidden = gate->k;
    inter = gate->n / experts;
    if (down->k != inter || down->n != experts * hidden)
        return fail(KR_E_SHAPE, "down [%u,%u] does not stack %u experts of [%u,%u]", down->n, down->k, experts, hidden,
                    inter);
    if (!skinny_grouped_fits(hidden) || !skinny_grouped_fits(inter))
        return fail(KR_E_UNSUPPORTED, "hidden=%u / inter=%u: need multiples of 128 up to 2048", hidden, inter);
    if (!skinny_supported(to_mat(gate)) || !skinny_supported(to_mat(up)) || !skinny_supported(to_mat(down)))
        return fail(KR_E_ALIGN, "expert scales/biases must be 4-byte aligned");
    if (topk == 0 || topk > experts) return fail(KR_E_INVALID, "topk=%u must be in 1..experts", topk);
    if (!valid_dtype(y_dtype)) return fail(KR_E_INVALID, "y_dtype %d invalid", y_dtype);
    if (!valid_act(activation)) return fail(KR_E_INVALID, "activation %d invalid", activation);
    if (accumulate != 0 && accumulate != 1) return fail(KR_E_INVALID, "accumulate must be 0 or 1");
    if (tokens == 0) return KR_OK;
    if ((uint64_t)tokens * topk > 0xFFFFFFFFull / 2) return fail(KR_E_SHAPE, "too many assignments");
    if (!x || !weights || !offsets || !sorted_assign || !y) return fail(KR_E_INVALID, "NULL pointer");
    if (!aligned(x, 16)) return fail(KR_E_ALIGN, "x must be 16-byte aligned");
    if (!aligned(y, dtype_size(y_dtype) * 4)) return fail(KR_E_ALIGN, "y must be aligned to 4 elements");
    if (!aligned(weights, 4) || !aligned(offsets, 4) || !aligned(sorted_assign, 4))
        return fail(KR_E_ALIGN, "routing arrays must be 4-byte aligned");
    const size_t need = kr_q4_moe_workspace_bytes(tokens, topk, hidden, inter);
    if (!workspace || workspace_bytes < need)
        return fail(KR_E_WORKSPACE, "workspace of %zu bytes required, %zu given", need, workspace_bytes);
    if (!aligned(workspace, 16)) return fail(KR_E_ALIGN, "workspace must be 16-byte aligned");
    return KR_OK;
}

// The experts after the checks: gate/up + activation, down, combine.  fr != nullptr (one token,
// routed GEMV path): the gate/up launch routes the token and writes the routing arrays itself.
int run_moe_experts(const kr_q4_matrix *gate, const kr_q4_matrix *up, const kr_q4_matrix *down, uint32_t experts,
                    const uint16_t *x, uint32_t tokens, uint32_t topk, const float *weights,
                    const uint32_t *offsets, const uint32_t *sorted_assign, int activation, void *y, int y_dtype,
                    int accumulate, void *workspace, uint32_t hidden, uint32_t inter, void *stream,
                    const FusedRoute *fr) {
    hipStream_t s = (hipStream_t)stream;
    const uint32_t assign = tokens * topk;
    uint16_t *h = (uint16_t *)workspace;                                              // [assign, inter] bf16, sorted order
    float *d = (float *)((char *)workspace + round_up((size_t)assign * inter * 2, 256));  // [assign, hidden] f32

    if (moe_gemv_path(tokens, topk, hidden, inter)) {
        // few assignments: one m = 1 GEMV per (expert, token) pair, every expert row read once per assignment
        MoeGemvArgs g{};
        g.w = to_mat(gate);
        g.w2 = to_mat(up);
        g.rows = inter;
        g.x = x;
        g.x_div = topk;  // X row of an assignment = its token
        g.offsets = offsets;
        g.sorted = sorted_assign;
        g.experts = experts;
        g.assign = assign;
        g.out = h;
        g.ldo = inter;
        g.act = activation;
        if (fr) {  // one token: the launch routes it and writes selected, weights, counts, offsets, sorted
            g.logits = fr->logits;
            g.normalize = fr->normalize;
            g.topk = topk;
            g.r_selected = fr->selected;
            g.r_counts = fr->counts;
            g.r_weights = const_cast<float *>(weights);
        }
        if (hipError_t e = launch_moe_gemv(g, kGateUpBF16, s)) return hip_status(e, "kr_q4_moe_experts (gate/up)");
        MoeGemvArgs dn{};
        dn.w = dn.w2 = to_mat(down);
        dn.rows = hidden;
        dn.x = h;
        dn.offsets = offsets;
        dn.sorted = sorted_assign;
        dn.experts = experts;
        dn.assign = assign;
        dn.out = d;
        dn.ldo = hidden;
        if (tuning().moe_combine && moe_down_combine_fits(inter, topk)) {
            // the down projection sums the slots of each token itself: no d rows, no combine launch
            MoeDownArgs dc{};
            dc.w = to_mat(down);
            dc.rows = hidden;
            dc.h = h;
            dc.offsets = offsets;
            dc.sorted = sorted_assign;
            dc.weights = weights;
            dc.experts = experts;
            dc.tokens = tokens;
            dc.topk = topk;
            dc.y = y;
            dc.y_f32 = y_dtype == KR_DTYPE_F32;
            dc.accumulate = accumulate;
            return hip_status(launch_moe_down_combine(dc, s), "kr_q4_moe_experts (down + combine)");
        }
        dn.out_scatter = 1;  // result rows back in assignment order
        if (hipError_t e = launch_moe_gemv(dn, kStoreF32, s)) return hip_status(e, "kr_q4_moe_experts (down)");
        return hip_status(launch_moe_combine(d, weights, tokens, topk, hidden, y, y_dtype == KR_DTYPE_F32, accumulate, s),
                          "kr_q4_moe_experts (combine)");
    }

    SkinnyArgs g{};
    g.w = to_mat(gate);
    g.w2 = to_mat(up);
    g.x = x;
    g.k = hidden;
    g.ldx = hidden;
    g.out = h;
    g.ldo = inter;
    g.act = activation;
    g.offsets = offsets;
    g.sorted = sorted_assign;
    g.experts = experts;
    g.expert_rows = inter;
    g.x_div = topk;  // X row of an assignment = its token
    g.max_active = std::min(experts, assign);
    if (hipError_t e = launch_skinny(g, s)) return hip_status(e, "kr_q4_moe_experts (gate/up)");

    SkinnyArgs dn{};
    dn.w = to_mat(down);
    dn.x = h;
    dn.k = inter;
    dn.ldx = inter;
    dn.out = d;
    dn.ldo = hidden;
    dn.out_f32 = 1;
    dn.offsets = offsets;
    dn.sorted = sorted_assign;
    dn.experts = experts;
    dn.expert_rows = hidden;
    dn.out_scatter = 1;  // result rows back in assignment order
    dn.max_active = g.max_active;
    if (hipError_t e = launch_skinny(dn, s)) return hip_status(e, "kr_q4_moe_experts (down)");

    return hip_status(launch_moe_combine(d, weights, tokens, topk, hidden, y, y_dtype == KR_DTYPE_F32, accumulate, s),
                      "kr_q4_moe_experts (combine)");
}
}  // namespace

int kr_q4_moe_experts(const kr_q4_matrix *gate, const kr_q4_matrix *up, const kr_q4_matrix *down, uint32_t experts,
                      const uint16_t *x, uint32_t tokens, uint32_t topk, const float *weights, const uint32_t *offsets,
                      const uint32_t *sorted_assign, int activation, void *y, int y_dtype, int accumulate,
                      void *workspace, size_t workspace_bytes, void *stream) {
    uint32_t hidden = 0, inter = 0;
    if (int rc = check_moe_experts(gate, up, down, experts, x, tokens, topk, weights, offsets, sorted_assign,
                                   activation, y, y_dtype, accumulate, workspace, workspace_bytes, hidden, inter))
        return rc;
    if (tokens == 0) return ok();
    return run_moe_experts(gate, up, down, experts, x, tokens, topk, weights, offsets, sorted_assign, activation, y,
                           y_dtype, accumulate, workspace, hidden, inter, stream, nullptr);
}

int kr_q4_moe_route_experts(const kr_q4_matrix *gate, const kr_q4_matrix *up, const kr_q4_matrix *down,
                            uint32_t experts, const uint16_t *x, uint32_t tokens, uint32_t topk, const float *logits,
                            int normalize, uint32_t *selected, float *weights, uint32_t *counts, uint32_t *offsets,
                            uint32_t *sorted_assign, int activation, void *y, int y_dtype, int accumulate,
                            void *workspace, size_t workspace_bytes, void *stream) {
    // every check of both stages before the first launch: a failing call enqueues nothing
    if (experts == 0 || experts > kMaxExperts) return fail(KR_E_INVALID, "experts=%u must be in 1..%u", experts, kMaxExperts);
    if (topk == 0 || topk > experts || topk > kRouteMaxTopK)
        return fail(KR_E_INVALID, "topk=%u must be in 1..min(experts, %u)", topk, kRouteMaxTopK);
    if ((uint64_t)tokens * topk > kRouteMaxAssign)
        return fail(KR_E_SHAPE, "tokens * topk = %llu exceeds %u", (unsigned long long)tokens * topk, kRouteMaxAssign);
    if (!counts || !offsets) return fail(KR_E_INVALID, "counts/offsets must be non-NULL");
    if (tokens > 0 && (!logits || !selected || !weights || !sorted_assign))
        return fail(KR_E_INVALID, "logits/selected/weights/sorted_assign must be non-NULL");
    if (!aligned(logits, 4) || !aligned(selected, 4) || !aligned(weights, 4) || !aligned(counts, 4) ||
        !aligned(offsets, 4) || !aligned(sorted_assign, 4))
        return fail(KR_E_ALIGN, "routing arrays must be 4-byte aligned");
    uint32_t hidden = 0, inter = 0;
    if (int rc = check_moe_experts(gate, up, down, experts, x, tokens, topk, weights, offsets, sorted_assign,
                                   activation, y, y_dtype, accumulate, workspace, workspace_bytes, hidden, inter))
        return rc;
    if (tuning().moe_route_fused && tokens == 1 && moe_gemv_path(tokens, topk, hidden, inter) &&
        moe_gemv_route_fits(experts, topk)) {
        const FusedRoute fr{logits, normalize, selected, counts};
        return run_moe_experts(gate, up, down, experts, x, tokens, topk, weights, offsets, sorted_assign, activation,
                               y, y_dtype, accumulate, workspace, hidden, inter, stream, &fr);
    }
    if (int rc = kr_moe_route(logits, tokens, experts, topk, normalize, selected, weights, counts, offsets,
                              sorted_assign, stream))
        return rc;
    if (tokens == 0) return ok();
    return run_moe_experts(gate, up, down, experts, x, tokens, topk, weights, offsets, sorted_assign, activation, y,
                           y_dtype, accumulate, workspace, hidden, inter, stream, nullptr);
}

// kr_q4_moe_block workspace: router logits f32 [T, E], selected u32 [T*K], weights f32 [T*K],
// counts u32 [E], offsets u32 [E+1], sorted u32 [T*K], then the experts' workspace.
namespace {
struct MoeBlockLayout {
    size_t logits, selected, weights, counts, offsets, sorted, experts, total;
};
MoeBlockLayout moe_block_layout(uint32_t tokens, uint32_t experts, uint32_t topk, uint32_t hidden, uint32_t inter) {
    const size_t assign = (size_t)tokens * topk;
    MoeBlockLayout L{};
    size_t o = 0;
    L.logits = o;   o += round_up((size_t)tokens * experts * 4, 256);
    L.selected = o; o += round_up(std::max<size_t>(assign, 1) * 4, 256);
    L.weights = o;  o += round_up(std::max<size_t>(assign, 1) * 4, 256);
    L.counts = o;   o += round_up((size_t)experts * 4, 256);
    L.offsets = o;  o += round_up(((size_t)experts + 1) * 4, 256);
    L.sorted = o;   o += round_up(std::max<size_t>(assign, 1) * 4, 256);
    L.experts = o;  o += kr_q4_moe_workspace_bytes(tokens, topk, hidden, inter);
    L.total = o;
    return L;
}
}  // namespace

size_t kr_q4_moe_block_workspace_bytes(uint32_t tokens, uint32_t experts, uint32_t topk, uint32_t hidden,
                                       uint32_t inter) {
    return moe_block_layout(tokens, experts, topk, hidden, inter).total;
}

int kr_q4_moe_block(const kr_q4_matrix *router, const kr_q4_matrix *gate, const kr_q4_matrix *up,
                    const kr_q4_matrix *down, uint32_t experts, const uint16_t *x, uint32_t tokens, uint32_t topk,
                    int normalize, int activation, void *y, int y_dtype, int accumulate, void *workspace,
                    size_t workspace_bytes, void *stream) {
    if (int rc = check_matrix(router, "router")) return rc;
    if (int rc = check_matrix(gate, "gate")) return rc;
    if (experts == 0 || experts > kMaxExperts) return fail(KR_E_INVALID, "experts=%u must be in 1..%u", experts, kMaxExperts);
    if (router->n != experts || router->k != gate->k)
        return fail(KR_E_SHAPE, "router [%u,%u] must be [experts=%u, hidden=%u]", router->n, router->k, experts, gate->k);
    if (gate->n % experts != 0) return fail(KR_E_SHAPE, "gate rows %u are not a multiple of experts=%u", gate->n, experts);
    // every check of the three stages before the first launch: a failing call enqueues nothing
    if (int rc = check_matrix(up, "up")) return rc;
    if (int rc = check_matrix(down, "down")) return rc;
    const uint32_t hidden = gate->k, inter = gate->n / experts;
    if (up->n != gate->n || up->k != hidden) return fail(KR_E_SHAPE, "gate and up shapes differ");
    if (down->k != inter || down->n != experts * hidden)
        return fail(KR_E_SHAPE, "down [%u,%u] does not stack %u experts of [%u,%u]", down->n, down->k, experts, hidden,
                    inter);
    if (!skinny_grouped_fits(hidden) || !skinny_grouped_fits(inter))
        return fail(KR_E_UNSUPPORTED, "hidden=%u / inter=%u: need multiples of 128 up to 2048", hidden, inter);
    if (!skinny_supported(to_mat(gate)) || !skinny_supported(to_mat(up)) || !skinny_supported(to_mat(down)))
        return fail(KR_E_ALIGN, "expert scales/biases must be 4-byte aligned");
    if (topk == 0 || topk > experts || topk > kRouteMaxTopK)
        return fail(KR_E_INVALID, "topk=%u must be in 1..min(experts, %u)", topk, kRouteMaxTopK);
    if (!valid_dtype(y_dtype)) return fail(KR_E_INVALID, "y_dtype %d invalid", y_dtype);
    if (!valid_act(activation)) return fail(KR_E_INVALID, "activation %d invalid", activation);
    if (accumulate != 0 && accumulate != 1) return fail(KR_E_INVALID, "accumulate must be 0 or 1");
    if (tokens == 0) return ok();
    if ((uint64_t)tokens * topk > kRouteMaxAssign)
        return fail(KR_E_SHAPE, "tokens * topk = %llu exceeds %u", (unsigned long long)tokens * topk, kRouteMaxAssign);
    if (!x || !y) return fail(KR_E_INVALID, "x/y must be non-NULL");
    if (!aligned(x, 16)) return fail(KR_E_ALIGN, "x must be 16-byte aligned");
    if (!aligned(y, dtype_size(y_dtype) * 4)) return fail(KR_E_ALIGN, "y must be aligned to 4 elements");
    const MoeBlockLayout L = moe_block_layout(tokens, experts, topk, hidden, inter);
    if (!workspace || workspace_bytes < L.total)
        return fail(KR_E_WORKSPACE, "workspace of %zu bytes required, %zu given", L.total, workspace_bytes);
    if (!aligned(workspace, 16)) return fail(KR_E_ALIGN, "workspace must be 16-byte aligned");
    char *ws = (char *)workspace;
    float *logits = (float *)(ws + L.logits);
    uint32_t *selected = (uint32_t *)(ws + L.selected);
    float *weights = (float *)(ws + L.weights);
    uint32_t *counts = (uint32_t *)(ws + L.counts), *offsets = (uint32_t *)(ws + L.offsets);
    uint32_t *sorted = (uint32_t *)(ws + L.sorted);
    // 1. router logits in f32 (the reference stores them as bf16 and reads them as f32)
    if (int rc = kr_q4_linear(router, x, tokens, logits, KR_DTYPE_F32, 0, stream)) return rc;
    // 2. softmax, top-k, renormalisation, deterministic buckets; 3. experts (gate/up + activation,
    // down) and the weighted combine into y
    return kr_q4_moe_route_experts(gate, up, down, experts, x, tokens, topk, logits, normalize, selected, weights,
                                   counts, offsets, sorted, activation, y, y_dtype, accumulate, ws + L.experts,
                                   L.total - L.experts, stream);
}

int kr_q4_embedding(const kr_q4_matrix *w, const uint32_t *tokens, uint32_t count, uint16_t *out, void *stream) {
    if (int rc = check_matrix(w, "w")) return rc;
    if (count == 0) return ok();
    if (!tokens || !out) return fail(KR_E_INVALID, "tokens/out must be non-NULL");
    if (!aligned(tokens, 4) || !aligned(out, 2)) return fail(KR_E_ALIGN, "tokens/out misaligned");
    if (count > 65535) return fail(KR_E_SHAPE, "count=%u exceeds 65535", count);
    return hip_status(launch_q4_embedding(to_mat(w), tokens, count, out, (hipStream_t)stream), "kr_q4_embedding");
}

int kr_rmsnorm(const uint16_t *x, const uint16_t *weight, uint32_t rows, uint32_t dim, float eps, uint16_t *out,
               void *stream) {
    if (rows == 0) return ok();
    if (!x || !weight || !out) return fail(KR_E_INVALID, "NULL pointer");
    if (dim == 0) return fail(KR_E_SHAPE, "dim must be positive");
    if (!aligned(x, 2) || !aligned(weight, 2) || !aligned(out, 2)) return fail(KR_E_ALIGN, "bf16 arrays misaligned");
    if (!(eps >= 0.0f)) return fail(KR_E_INVALID, "eps must be >= 0");
    return hip_status(launch_rmsnorm(x, weight, rows, dim, eps, out, (hipStream_t)stream), "kr_rmsnorm");
}

static int check_heads(uint32_t q_heads, uint32_t kv_heads, uint32_t head_dim, uint32_t max_ctx) {
    if (q_heads == 0 || kv_heads == 0 || q_heads % kv_heads != 0)
        return fail(KR_E_SHAPE, "q_heads=%u must be a positive multiple of kv_heads=%u", q_heads, kv_heads);
    if (head_dim == 0 || head_dim % 8 != 0 || head_dim > kGlueMaxHeadDim)
        return fail(KR_E_SHAPE, "head_dim=%u must be a multiple of 8 and <= %u", head_dim, kGlueMaxHeadDim);
    if (max_ctx == 0 || max_ctx > kGlueMaxCtx) return fail(KR_E_SHAPE, "max_ctx=%u must be in 1..%u", max_ctx, kGlueMaxCtx);
    return KR_OK;
}

int kr_rope_kv_append(uint16_t *q, const uint16_t *k, const uint16_t *v, const float *cos_sin,
                      const uint32_t *positions, uint32_t batch, uint32_t q_heads, uint32_t kv_heads,
                      uint32_t head_dim, uint16_t *k_cache, uint16_t *v_cache, uint32_t max_ctx, void *stream) {
    if (int rc = check_heads(q_heads, kv_heads, head_dim, max_ctx)) return rc;
    if (batch == 0) return ok();
    if (!q || !k || !v || !cos_sin || !positions || !k_cache || !v_cache) return fail(KR_E_INVALID, "NULL pointer");
    if (batch > 65535) return fail(KR_E_SHAPE, "batch=%u exceeds 65535", batch);
    return hip_status(launch_rope_kv_append(q, k, v, cos_sin, positions, batch, q_heads, kv_heads, head_dim, k_cache,
                                            v_cache, max_ctx, (hipStream_t)stream),
                      "kr_rope_kv_append");
}

int kr_attention_decode(const uint16_t *q, const uint16_t *k_cache, const uint16_t *v_cache,
                        const uint32_t *positions, uint32_t batch, uint32_t q_heads, uint32_t kv_heads,
                        uint32_t head_dim, uint32_t max_ctx, uint16_t *out, void *stream) {
    if (int rc = check_heads(q_heads, kv_heads, head_dim, max_ctx)) return rc;
    if (batch == 0) return ok();
    if (!q || !k_cache || !v_cache || !positions || !out) return fail(KR_E_INVALID, "NULL pointer");
    if (!aligned(q, 16) || !aligned(k_cache, 16) || !aligned(v_cache, 16))
        return fail(KR_E_ALIGN, "q, k_cache and v_cache must be 16-byte aligned");
    if (batch > 65535) return fail(KR_E_SHAPE, "batch=%u exceeds 65535", batch);
    return hip_status(launch_attention_decode(q, k_cache, v_cache, positions, batch, q_heads, kv_heads, head_dim,
                                              max_ctx, out, (hipStream_t)stream),
                      "kr_attention_decode");
}

int kr_rmsnorm_q4_qkv(const uint16_t *h, const uint16_t *ln_weight, float eps, const kr_q4_matrix *q,
                      const kr_q4_matrix *k, const kr_q4_matrix *v, const uint16_t *q_bias, const uint16_t *k_bias,
                      const uint16_t *v_bias, uint32_t m, void *q_out, void *k_out, void *v_out, int out_dtype,
                      uint16_t *xnorm, void *stream) {
    if (int rc = check_matrix(q, "q")) return rc;
    if (int rc = check_matrix(k, "k")) return rc;
    if (int rc = check_matrix(v, "v")) return rc;
    if (q->k != k->k || q->k != v->k) return fail(KR_E_SHAPE, "q, k, v must share k");
    if (!valid_dtype(out_dtype)) return fail(KR_E_INVALID, "out_dtype %d invalid", out_dtype);
    if (m == 0) return ok();
    if (!h || !ln_weight || !q_out || !k_out || !v_out) return fail(KR_E_INVALID, "NULL pointer");
    if (!aligned(h, 16) || !aligned(ln_weight, 16)) return fail(KR_E_ALIGN, "h and ln_weight must be 16-byte aligned");
    const size_t osz = dtype_size(out_dtype);
    if (!aligned(q_out, osz) || !aligned(k_out, osz) || !aligned(v_out, osz)) return fail(KR_E_ALIGN, "output misaligned");
    hipStream_t s = (hipStream_t)stream;
    if (m == 1 && gemv_batch_supported(q->k)) {
        const Q4Mat ms[3] = {to_mat(q), to_mat(k), to_mat(v)};
        void *outs[3] = {q_out, k_out, v_out};
        const uint16_t *biases[3] = {q_bias, k_bias, v_bias};
        const int epi = out_dtype == KR_DTYPE_F32 ? kStoreF32 : kStoreBF16;
        return hip_status(launch_gemv_batch(ms, nullptr, h, outs, biases, 3, epi, 0, ln_weight, eps, s),
                          "kr_rmsnorm_q4_qkv");
    }
    if (skinny_fits(m, to_mat(q), false) && skinny_supported(to_mat(k)) && skinny_supported(to_mat(v))) {
        // few tokens: the norm is applied while the few-token kernel stages x (xnorm is not written)
        const kr_q4_matrix *mats[3] = {q, k, v};
        const uint16_t *biases[3] = {q_bias, k_bias, v_bias};
        void *outs[3] = {q_out, k_out, v_out};
        return hip_status(run_skinny_qkv(mats, biases, outs, h, m, out_dtype, ln_weight, eps, s), "kr_rmsnorm_q4_qkv");
    }
    if (!xnorm || !aligned(xnorm, 16)) return fail(KR_E_INVALID, "xnorm (16-byte aligned) is required for m > 1");
    if (int rc = hip_status(launch_rmsnorm(h, ln_weight, m, q->k, eps, xnorm, s), "kr_rmsnorm_q4_qkv")) return rc;
    return kr_q4_qkv(q, k, v, q_bias, k_bias, v_bias, xnorm, m, q_out, k_out, v_out, out_dtype, stream);
}

size_t kr_rmsnorm_q4_mlp_workspace_bytes(uint32_t m, uint32_t hidden, uint32_t intermediate) {
    return kr_q4_mlp_workspace_bytes(m, hidden, intermediate) + round_up((size_t)m * hidden * 2, 256);
}

int kr_rmsnorm_q4_mlp(const kr_q4_matrix *gate, const kr_q4_matrix *up, const kr_q4_matrix *down, uint16_t *h,
                      const uint16_t *ln_weight, float eps, uint32_t m, int activation, void *workspace,
                      size_t workspace_bytes, void *stream) {
    if (int rc = check_matrix(gate, "gate")) return rc;
    if (int rc = check_matrix(up, "up")) return rc;
    if (int rc = check_matrix(down, "down")) return rc;
    if (gate->n != up->n || gate->k != up->k) return fail(KR_E_SHAPE, "gate and up shapes differ");
    if (down->k != gate->n || down->n != gate->k)
        return fail(KR_E_SHAPE, "down [%u,%u] does not match gate/up [%u,%u]", down->n, down->k, gate->n, gate->k);
    if (!valid_act(activation)) return fail(KR_E_INVALID, "activation %d invalid", activation);
    if (m == 0) return ok();
    if (!h || !ln_weight) return fail(KR_E_INVALID, "NULL pointer");
    if (!aligned(h, 16) || !aligned(ln_weight, 16)) return fail(KR_E_ALIGN, "h and ln_weight must be 16-byte aligned");
    const size_t need = kr_rmsnorm_q4_mlp_workspace_bytes(m, gate->k, gate->n);
    if (!workspace || workspace_bytes < need)
        return fail(KR_E_WORKSPACE, "workspace of %zu bytes required, %zu given", need, workspace_bytes);
    if (!aligned(workspace, 16)) return fail(KR_E_ALIGN, "workspace must be 16-byte aligned");
    hipStream_t s = (hipStream_t)stream;
    const size_t mlp_bytes = kr_q4_mlp_workspace_bytes(m, gate->k, gate->n);
    if (m == 1 && gemv_batch_supported(gate->k)) {
        // gate/up with the norm fused into the x load, then the accumulating down projection
        uint16_t *act = mlp_ws_act(workspace);
        const Q4Mat g = to_mat(gate), u = to_mat(up);
        void *outs[1] = {act};
        const uint16_t *biases[1] = {nullptr};
        if (int rc = hip_status(launch_gemv_batch(&g, &u, h, outs, biases, 1, kGateUpBF16, activation, ln_weight, eps, s),
                                "kr_rmsnorm_q4_mlp"))
            return rc;
        return kr_q4_linear(down, act, 1, h, KR_DTYPE_BF16, 1, stream);
    }
    const bool tokens = gate_up_on_tokens(m, to_mat(gate), to_mat(up));
    if (!tokens && skinny_fits(m, to_mat(gate), false) && skinny_supported(to_mat(up))) {
        // few tokens on the matrix cores: the norm is applied while gate/up stages x
        uint16_t *act = mlp_ws_act(workspace);
        const Q4Mat g = to_mat(gate), u = to_mat(up);
        if (int rc = hip_status(run_skinny(g, &u, h, m, act, nullptr, gate->n, KR_DTYPE_BF16, 0, activation, nullptr, s,
                                           ln_weight, eps),
                                "kr_rmsnorm_q4_mlp"))
            return rc;
        return mlp_down(gate, down, act, h, KR_DTYPE_BF16, m, workspace, stream);
    }
    uint16_t *xnorm = (uint16_t *)((char *)workspace + mlp_bytes);
    if (int rc = hip_status(launch_rmsnorm(h, ln_weight, m, gate->k, eps, xnorm, s), "kr_rmsnorm_q4_mlp")) return rc;
    return kr_q4_mlp(gate, up, down, xnorm, h, KR_DTYPE_BF16, m, activation, workspace, mlp_bytes, stream);
}

size_t kr_attention_workspace_bytes(uint32_t batch, uint32_t q_heads, uint32_t head_dim, uint32_t max_ctx) {
    return attention_workspace_bytes(batch, q_heads, head_dim, max_ctx);
}

int kr_rope_attention_decode(const uint16_t *q, const uint16_t *k, const uint16_t *v, const float *cos_sin,
                             const uint32_t *positions, uint32_t batch, uint32_t q_heads, uint32_t kv_heads,
                             uint32_t head_dim, uint16_t *k_cache, uint16_t *v_cache, uint32_t max_ctx,
                             uint16_t *out, void *workspace, size_t workspace_bytes, void *stream) {
    if (int rc = check_heads(q_heads, kv_heads, head_dim, max_ctx)) return rc;
    if (q_heads / kv_heads > kGlueMaxGroup)
        return fail(KR_E_SHAPE, "q_heads / kv_heads = %u exceeds %u", q_heads / kv_heads, kGlueMaxGroup);
    if (batch == 0) return ok();
    if (!q || !k || !v || !cos_sin || !positions || !k_cache || !v_cache || !out)
        return fail(KR_E_INVALID, "NULL pointer");
    if (!aligned(k_cache, 16) || !aligned(v_cache, 16)) return fail(KR_E_ALIGN, "k_cache and v_cache must be 16-byte aligned");
    if (!aligned(cos_sin, 8)) return fail(KR_E_ALIGN, "cos_sin must be 8-byte aligned");
    if (batch > 65535) return fail(KR_E_SHAPE, "batch=%u exceeds 65535", batch);
    const size_t need = attention_workspace_bytes(batch, q_heads, head_dim, max_ctx);
    if (!workspace || workspace_bytes < need)
        return fail(KR_E_WORKSPACE, "workspace of %zu bytes required, %zu given", need, workspace_bytes);
    if (!aligned(workspace, 16)) return fail(KR_E_ALIGN, "workspace must be 16-byte aligned");
    return hip_status(launch_rope_attention(q, k, v, cos_sin, positions, batch, q_heads, kv_heads, head_dim, k_cache,
                                            v_cache, max_ctx, out, (float *)workspace, (hipStream_t)stream),
                      "kr_rope_attention_decode");
}

size_t kr_attention_q4_out_workspace_bytes(uint32_t batch, uint32_t q_heads, uint32_t head_dim, uint32_t max_ctx) {
    // the slices' partials, then the attention output [batch, q_heads * head_dim] bf16 (unfused path)
    return round_up(attention_workspace_bytes(batch, q_heads, head_dim, max_ctx), 256) +
           round_up((size_t)batch * q_heads * head_dim * 2, 256);
}

int kr_rope_attention_q4_out(const uint16_t *q, const uint16_t *k, const uint16_t *v, const float *cos_sin,
                             const uint32_t *positions, uint32_t batch, uint32_t q_heads, uint32_t kv_heads,
                             uint32_t head_dim, uint16_t *k_cache, uint16_t *v_cache, uint32_t max_ctx,
                             const kr_q4_matrix *o_proj, void *h, int h_dtype, void *workspace, size_t workspace_bytes,
                             void *stream) {
    // every check of both stages first: a failing call enqueues nothing
    if (int rc = check_heads(q_heads, kv_heads, head_dim, max_ctx)) return rc;
    if (q_heads / kv_heads > kGlueMaxGroup)
        return fail(KR_E_SHAPE, "q_heads / kv_heads = %u exceeds %u", q_heads / kv_heads, kGlueMaxGroup);
    if (int rc = check_matrix(o_proj, "o_proj")) return rc;
    if (o_proj->k != q_heads * head_dim)
        return fail(KR_E_SHAPE, "o_proj k=%u must be q_heads * head_dim = %u", o_proj->k, q_heads * head_dim);
    if (!valid_dtype(h_dtype)) return fail(KR_E_INVALID, "h_dtype %d invalid", h_dtype);
    if (batch == 0) return ok();
    if (!q || !k || !v || !cos_sin || !positions || !k_cache || !v_cache || !h) return fail(KR_E_INVALID, "NULL pointer");
    if (!aligned(k_cache, 16) || !aligned(v_cache, 16)) return fail(KR_E_ALIGN, "k_cache and v_cache must be 16-byte aligned");
    if (!aligned(cos_sin, 8)) return fail(KR_E_ALIGN, "cos_sin must be 8-byte aligned");
    if (!aligned(h, dtype_size(h_dtype))) return fail(KR_E_ALIGN, "h misaligned");
    if (batch > 65535) return fail(KR_E_SHAPE, "batch=%u exceeds 65535", batch);
    const size_t need = kr_attention_q4_out_workspace_bytes(batch, q_heads, head_dim, max_ctx);
    if (!workspace || workspace_bytes < need)
        return fail(KR_E_WORKSPACE, "workspace of %zu bytes required, %zu given", need, workspace_bytes);
    if (!aligned(workspace, 16)) return fail(KR_E_ALIGN, "workspace must be 16-byte aligned");
    hipStream_t s = (hipStream_t)stream;
    float *part = (float *)workspace;
    const uint32_t slices = attention_slices64(max_ctx);
    if (tuning().attn_merge_oproj && batch == 1 && head_dim == 128 && q_heads <= 16 && o_proj->k <= 2048 &&
        slices <= kMergeOprojMaxSlices && (uint64_t)slices * q_heads * (head_dim + 2) * 4 <= need) {
        if (hipError_t e = launch_rope_attention_partials64(q, k, v, cos_sin, positions, batch, q_heads, kv_heads,
                                                            k_cache, v_cache, max_ctx, part, s))
            return hip_status(e, "kr_rope_attention_q4_out (attention)");
        return hip_status(launch_attention_merge_oproj(part, q_heads, kv_heads, slices, to_mat(o_proj), h,
                                                       h_dtype == KR_DTYPE_F32, s),
                          "kr_rope_attention_q4_out (merge + o_proj)");
    }
    uint16_t *attn = (uint16_t *)((char *)workspace + round_up(attention_workspace_bytes(batch, q_heads, head_dim, max_ctx), 256));
    if (int rc = kr_rope_attention_decode(q, k, v, cos_sin, positions, batch, q_heads, kv_heads, head_dim, k_cache,
                                          v_cache, max_ctx, attn, workspace, need, stream))
        return rc;
    return kr_q4_linear(o_proj, attn, batch, h, h_dtype, 1, stream);
}

int kr_argmax(const float *logits, uint32_t rows, uint32_t n, uint32_t *out, void *stream) {
    if (rows == 0) return ok();
    if (!logits || !out) return fail(KR_E_INVALID, "NULL pointer");
    if (n == 0) return fail(KR_E_SHAPE, "n must be positive");
    if (!aligned(logits, 4) || !aligned(out, 4)) return fail(KR_E_ALIGN, "logits/out misaligned");
    return hip_status(launch_argmax(logits, rows, n, out, (hipStream_t)stream), "kr_argmax");
}

size_t kr_argmax_workspace_bytes(uint32_t rows, uint32_t n) {
    return rows == 0 || n == 0 ? 0 : round_up(argmax_workspace_bytes(rows, n), 256);
}

int kr_argmax_ws(const float *logits, uint32_t rows, uint32_t n, uint32_t *out, void *workspace,
                 size_t workspace_bytes, void *stream) {
    if (rows == 0) return ok();
    if (!logits || !out) return fail(KR_E_INVALID, "NULL pointer");
    if (n == 0) return fail(KR_E_SHAPE, "n must be positive");
    if (!aligned(logits, 4) || !aligned(out, 4)) return fail(KR_E_ALIGN, "logits/out misaligned");
    const size_t need = kr_argmax_workspace_bytes(rows, n);
    if (!workspace || workspace_bytes < need)
        return fail(KR_E_WORKSPACE, "workspace of %zu bytes required, %zu given", need, workspace_bytes);
    if (!aligned(workspace, 8)) return fail(KR_E_ALIGN, "workspace must be 8-byte aligned");
    return hip_status(launch_argmax_split(logits, rows, n, out, workspace, (hipStream_t)stream), "kr_argmax_ws");
}


}  // extern "C"

// ---------------------------------------------------------------- kr_q4_mlp_noalloc
// kr_q4_mlp for callers that cannot allocate device memory (code under HIP graph
// capture, serving loops, harnesses that forbid hipMalloc): the workspace is the file-scope
// device array `scratch`, one copy per GPU, held until the process ends.  Its device address
// is taken once per device with hipGetSymbolAddress; the host never passes the array's own
// name to a kernel or a copy.  The kernels are kr_q4_mlp's.

namespace {

constexpr size_t kMlpScratchBytes = (size_t)4 << 20;  // 4 MiB per GPU
__device__ __align__(256) unsigned char scratch[kMlpScratchBytes];

constexpr int kScratchMaxDevices = 64;
std::mutex g_scratch_mu;
void *g_scratch_ptr[kScratchMaxDevices];  // device address of `scratch` on each device, once set up

__global__ void zero_words_kernel(uint32_t *p, uint32_t n) {
    const uint32_t i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i < n) p[i] = 0u;
}

// The scratch address on the current device.  The first call on a device takes the address and
// enqueues a fill kernel on `s` that zeroes the split-K tickets (every call leaves them zero
// after that); a kernel, not hipMemsetAsync, so that a first call under graph capture records a
// plain kernel node.
int scratch_on_current_device(hipStream_t s, void **out) {
    int dev = 0;
    if (hipError_t e = hipGetDevice(&dev)) return hip_status(e, "kr_q4_mlp_noalloc: hipGetDevice");
    if (dev < 0 || dev >= kScratchMaxDevices) return fail(KR_E_UNSUPPORTED, "kr_q4_mlp_noalloc: device %d", dev);
    std::lock_guard<std::mutex> lock(g_scratch_mu);
    if (!g_scratch_ptr[dev]) {
        void *p = nullptr;
        if (hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch)))
            return hip_status(e, "kr_q4_mlp_noalloc: hipGetSymbolAddress(scratch)");
        const uint32_t words = (uint32_t)(kMlpTicketBytes / 4);
        hipLaunchKernelGGL(zero_words_kernel, dim3((words + 255) / 256), dim3(256), 0, s, (uint32_t *)p, words);
        if (hipError_t e = hipGetLastError()) return hip_status(e, "kr_q4_mlp_noalloc: clearing the tickets");
        g_scratch_ptr[dev] = p;
    }
    *out = g_scratch_ptr[dev];
    return KR_OK;
}

}  // namespace

extern "C" {

size_t kr_q4_mlp_noalloc_max_bytes(void) { return kMlpScratchBytes; }

int kr_q4_mlp_noalloc(const kr_q4_matrix *gate, const kr_q4_matrix *up, const kr_q4_matrix *down, const uint16_t *x,
                      void *h, int h_dtype, uint32_t m, int activation, void *stream) {
    if (int rc = check_matrix(gate, "gate")) return rc;
    const size_t need = kr_q4_mlp_workspace_bytes(m, gate->k, gate->n);
    if (need > kMlpScratchBytes)
        return fail(KR_E_WORKSPACE,
                    "kr_q4_mlp_noalloc: m=%u hidden=%u intermediate=%u needs %zu bytes of scratch, more than the "
                    "%zu the library holds per GPU; call kr_q4_mlp with a workspace",
                    m, gate->k, gate->n, need, kMlpScratchBytes);
    if (m == 0) return kr_q4_mlp(gate, up, down, x, h, h_dtype, m, activation, nullptr, 0, stream);
    void *ws = nullptr;
    if (int rc = scratch_on_current_device((hipStream_t)stream, &ws)) return rc;
    return kr_q4_mlp(gate, up, down, x, h, h_dtype, m, activation, ws, kMlpScratchBytes, stream);
}

}  // extern "C"
