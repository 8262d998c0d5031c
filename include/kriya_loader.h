/*
 * kriya_loader.h — on-disk checkpoint formats feeding the Q4_G64 path: safetensors
 * archives (one file or a sharded directory), memory-mapped, and the binding of
 * their Q4 weights into the planar device layout of kr_q4_matrix.
 *
 * Replaces kriya-core's safetensors reader and kriya-backend-metal's bind step:
 *   open_safetensors_file                  crates/kriya-core/src/safetensors_loader.rs:67-119
 *   ShardedCheckpointLoader::open / get    safetensors_loader.rs:122-208
 *   MappedWeightArchive::open (bounds)     crates/kriya-core/src/tensor.rs:373-405
 *   TensorDescriptor::validate             tensor.rs:266-275
 *   pack_mlx_affine_q4_group64 (+ f16)     safetensors_loader.rs:221-273, 310-318
 *   bind_q4_buffer Path A / Path B         crates/kriya-backend-metal/src/encoder.rs:651-703
 *   validate_production_checkpoint         encoder.rs:452-591 (require_q4_weight :332-418,
 *                                          require_norm_tensor :306-328)
 *
 * Conventions as in kriya_q4.h: 0 or a negative KR_E* code, the message in
 * kr_last_error().  Archive functions run on the host (no GPU work) except
 * kr_archive_load_*, which copy to device memory the caller owns and return
 * when the data is there (loading is not a hot path).  Every check fails
 * closed: a malformed header, an unknown dtype, a size that does not match the
 * shape, or a tensor past the end of its file is an error, never a guess.
 */
#ifndef KRIYA_LOADER_H
#define KRIYA_LOADER_H

#include <stddef.h>
#include <stdint.h>

#include "kriya_q4.h"

#ifdef __cplusplus
extern "C" {
#endif

#define KR_E_IO (-7)     /* a file could not be opened, read or mapped            */
#define KR_E_FORMAT (-8) /* malformed or inconsistent archive contents            */
#define KR_E_MISSING (-9) /* a tensor the call needs is not in the archive        */

/* safetensors dtype strings accepted (DType::from_safetensors_str,
 * safetensors_loader.rs:36-55) and their storage (tensor.rs:62-101). */
#define KR_ST_F32 0
#define KR_ST_F16 1
#define KR_ST_BF16 2
#define KR_ST_F8_E4M3 3
#define KR_ST_Q4_G64 4  /* 36-byte BlockQ4Group64 per 64 elements */
#define KR_ST_Q2_G128 5 /* 36 bytes per 128 elements              */
#define KR_ST_Q3_G64 6  /* 28 bytes per 64 elements               */
#define KR_ST_U32 7
#define KR_ST_U8 8
#define KR_ST_I32 9
#define KR_ST_I8 10

#define KR_MAX_DIMS 8

typedef struct kr_archive kr_archive; /* opaque */

typedef struct kr_tensor_info {
    int dtype;                    /* KR_ST_*                                   */
    uint32_t ndim;
    uint64_t shape[KR_MAX_DIMS];
    uint64_t byte_len;
    const void *data;             /* host address inside the mapping           */
    const char *shard;            /* file name of the shard holding it         */
} kr_tensor_info;

/* Opens `path`: a .safetensors file, or a directory holding
 * model.safetensors.index.json (sharded: every shard its weight_map names) or
 * model.safetensors (ShardedCheckpointLoader::open).  Files are mapped
 * read-only; headers larger than 100 MB or of length 0 are rejected. */
int kr_archive_open(const char *path, kr_archive **out);
void kr_archive_close(kr_archive *a);
/* Number of tensors, and the name of the i-th in a fixed (sorted) order. */
size_t kr_archive_tensor_count(const kr_archive *a);
const char *kr_archive_tensor_name(const kr_archive *a, size_t i);
/* KR_E_MISSING when absent. */
int kr_archive_tensor(const kr_archive *a, const char *name, kr_tensor_info *info);

/* A Q4 projection `prefix` of shape [n, k] (require_q4_weight, encoder.rs:332-418):
 *   Path A: `prefix.weight` (or `prefix`) of dtype Q4_G64 and shape [n, k]
 *           (36-byte blocks, block (r, g) at r * k/64 + g);
 *   Path B: `prefix.weight` (or `prefix`) with `prefix.scales` and `prefix.biases`:
 *           the MLX affine triplet, weight n * k/64 * 32 bytes (U32 [n, k/8]),
 *           scales/biases BF16 or F16 with n * k/64 elements.
 * F32 scales or biases are rejected: the reference's validation admits them
 * (encoder.rs:366-374) but its repack fails on them (safetensors_loader.rs:253-258).
 * Returns the path taken (1 = A, 2 = B) in *path_out (may be NULL). */
int kr_archive_check_q4(const kr_archive *a, const char *prefix, uint32_t n, uint32_t k, int *path_out);

/* Device bytes of staging that kr_archive_load_q4 needs for `prefix`
 * (Path A: the 36-byte blocks; Path B: 0). */
int kr_archive_q4_staging_bytes(const kr_archive *a, const char *prefix, uint32_t n, uint32_t k, size_t *bytes);

/* Loads `prefix` into the planar triplet qw [n, k/8] (16-byte aligned), scales
 * and biases [n, k/64] (bf16 bits) on the device.  Path B copies the MLX planes
 * as they are (they are the planar layout) and converts F16 scale/bias planes
 * to bf16 on the device (kr_f16_to_bf16: bf16_rne(f16_to_f32), as
 * parse_half_endian); Path A copies the blocks to `staging` and splits them
 * with kr_q4_from_blocks36.  Synchronises `stream` before returning. */
int kr_archive_load_q4(const kr_archive *a, const char *prefix, uint32_t n, uint32_t k, uint32_t *qw,
                       uint16_t *scales, uint16_t *biases, void *staging, size_t staging_bytes, void *stream);

/* A floating-point vector `name` of `len` elements (norm weights, biases;
 * require_norm_tensor, encoder.rs:306-328) -> bf16 bits on the device: BF16
 * as is, F16 and F32 rounded to nearest even (tensor_view_to_bf16_bytes). */
int kr_archive_load_bf16(const kr_archive *a, const char *name, uint64_t len, uint16_t *out, void *stream);

/* A dense decoder with grouped-query attention and a SwiGLU-family MLP
 * (Qwen2 / Llama / Mistral layout). */
typedef struct kr_dense_model_desc {
    uint32_t hidden, intermediate, layers, vocab;
    uint32_t q_heads, kv_heads, head_dim;
    int qkv_bias;             /* Qwen2: q/k/v projections carry biases          */
    int tie_word_embeddings;  /* no separate lm_head                            */
} kr_dense_model_desc;

/* validate_production_checkpoint (encoder.rs:452-591) for that architecture:
 * every tensor a decode step binds is present, of a usable dtype and of the
 * shape the descriptor implies (Q4 projections through kr_archive_check_q4,
 * including a dry run of the MLX repack).  Names follow the Hugging Face /
 * MLX convention model.embed_tokens, model.layers.{i}.self_attn.{q,k,v,o}_proj,
 * model.layers.{i}.mlp.{gate,up,down}_proj, *_layernorm.weight, model.norm.weight,
 * lm_head.  The first failure is reported. */
int kr_checkpoint_validate_dense(const kr_archive *a, const kr_dense_model_desc *desc);

#ifdef __cplusplus
}
#endif
#endif /* KRIYA_LOADER_H */
