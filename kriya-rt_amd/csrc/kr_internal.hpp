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
};
Tuning &tuning();

// Largest k of the m == 1 kernels (three 16-byte chunks per thread of a 256-thread block).
constexpr uint32_t kMaxGemvK = 3 * 256 * 32;

hipError_t launch_format_dequant(const Q4Mat &w, float *out, hipStream_t s);
hipError_t launch_from_blocks36(const void *blocks, uint32_t n, uint32_t k, uint32_t *qw, uint16_t *sc,
                                uint16_t *bi, hipStream_t s);
hipError_t launch_to_blocks36(const Q4Mat &w, void *blocks, hipStream_t s);
hipError_t launch_f16_to_bf16(const uint16_t *in, uint16_t *out, size_t count, hipStream_t s);

// y = W x for one token; `b` is the up matrix for the gate/up epilogues.
hipError_t launch_gemv(const Q4Mat &a, const Q4Mat *b, const uint16_t *x, void *out, int epilogue,
                       int activation, hipStream_t s);

}  // namespace kr
