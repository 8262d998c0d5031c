// q4_mlp_fused.hip — the single-token (m == 1) dense MLP in one launch:
//   h += down . bf16(act(gate . x) * (up . x))
// Replaces the reference's decode pair q4_g64_decode_gate_up_swiglu_gemv +
// q4_g64_decode_gemv_accumulate (kernels/metal/q4_gemm_and_moe.metal:1850-2158,
// 1081-1157) as encoded by encode_dense_mlp (crates/kriya-backend-metal/src/
// encoder.rs:2851-2906).  The activations are bitwise those of the two-launch
// path (same GEMV code); the down sums have their own fixed reduction order
// (one chunk per thread, butterfly, then the waves of a row group in order), so
// results are reproducible and differ from the two-launch path only in f32
// summation order.
//
// Why one launch: at decode the MLP is a pure weight stream (3 x 12.7 MB at the
// Qwen2.5-3B shape).  Two launches each pay a ramp and a tail, and the down
// projection cannot start streaming before the gate/up launch has drained.
// Here every block owns `rpb` rows of the down matrix and starts copying them
// into its LDS (direct-to-LDS buffer loads) before it takes part in the
// gate/up GEMV, so the down weights stream from HBM concurrently with gate/up.
// After a grid barrier, each block reads the activation vector (L2) into LDS
// and finishes its down rows from LDS.
//
// Grid: one block of 1024 threads per CU.  The grid barrier needs every block
// resident at once; the grid never exceeds the CU count and a block fits a CU
// (<= 128 VGPRs, LDS checked by the launcher).  A barrier wait gives up after
// a bounded number of polls (the kernel then exits with a flag set instead of
// waiting for a block that cannot arrive).
#include "q4_dot2.hpp"

namespace kr {

namespace {

using rsrc_t = __amdgpu_buffer_rsrc_t;

constexpr int kThreads = 1024;
constexpr int kWaves = kThreads / kWave;
constexpr uint32_t kSpinLimit = 1u << 22;  // polls of a barrier wait (each with s_sleep) before giving up

// Barrier state: arrivals of the open barrier (0 at rest) and its generation.
__device__ uint32_t g_bar_count;
__device__ uint32_t g_bar_gen;
__device__ uint32_t g_bar_timeouts;  // incremented when a wait gave up

__device__ __forceinline__ rsrc_t make_rsrc(const void *p, uint32_t bytes) {
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<void *>(p), (short)0, (int)bytes, 0x00020000);
}

// lane l copies `size` bytes from the buffer at voffset to lds[size * l]; `lds` is wave-uniform.
__device__ __forceinline__ void dma16(rsrc_t r, char *lds, uint32_t voffset) {
    __builtin_amdgcn_raw_ptr_buffer_load_lds(r, (__attribute__((address_space(3))) void *)lds, 16, voffset, 0, 0, 0);
}
__device__ __forceinline__ void dma4(rsrc_t r, char *lds, uint32_t voffset) {
    __builtin_amdgcn_raw_ptr_buffer_load_lds(r, (__attribute__((address_space(3))) void *)lds, 4, voffset, 0, 0, 0);
}

// All blocks of the grid reach this point before any continues.  Thread 0 of
// each block arrives with a device-scope atomic after a release fence; the
// last arrival resets the count and publishes a new generation, which the
// others poll for (acquire).  Returns false when the wait gave up.
__device__ bool grid_barrier(uint32_t nblocks) {
    // every wave's stores have reached its L2 before thread 0's release fence writes that L2 back
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    __syncthreads();
    __shared__ int ok;
    if (threadIdx.x == 0) {
        ok = 1;
        const uint32_t gen = __hip_atomic_load(&g_bar_gen, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        const uint32_t arrived =
            __hip_atomic_fetch_add(&g_bar_count, 1u, __ATOMIC_ACQ_REL, __HIP_MEMORY_SCOPE_AGENT);
        if (arrived == nblocks - 1) {
            __hip_atomic_store(&g_bar_count, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            __hip_atomic_store(&g_bar_gen, gen + 1, __ATOMIC_RELEASE, __HIP_MEMORY_SCOPE_AGENT);
        } else {
            // relaxed polls (an acquire per poll would invalidate the L2 each time), one acquire after
            uint32_t polls = 0;
            while (__hip_atomic_load(&g_bar_gen, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) == gen) {
                if (++polls >= kSpinLimit) {
                    __hip_atomic_fetch_add(&g_bar_timeouts, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                    ok = 0;
                    break;
                }
                __builtin_amdgcn_s_sleep(1);
            }
            __atomic_thread_fence(__ATOMIC_ACQUIRE);
        }
    }
    __syncthreads();
    return ok != 0;
}

}  // namespace

// LDS layout of a block (byte offsets): `rpb` consecutive rows of a matrix with
// k columns (nibbles, then scales, then biases, each region padded to whole DMA
// instructions) and the x vector (k bf16).
struct RowsLayout {
    uint32_t rowbytes, groups;
    uint32_t sc, bi, x, total;
    __host__ __device__ RowsLayout(uint32_t rpb, uint32_t k) {
        rowbytes = k / 2;
        groups = k / 64;
        const uint32_t qw_units = rpb * rowbytes / 16, sb_dwords = rpb * groups / 2;
        sc = (qw_units + 63) / 64 * 1024;
        bi = sc + (sb_dwords + 63) / 64 * 256;
        x = bi + (sb_dwords + 63) / 64 * 256;
        total = x + (k * 2 + 1023) / 1024 * 1024;
    }
};

// Rows [r0, r0 + rows) of A -> LDS (asynchronous).  Wave w of `nwaves` issues
// the DMA instructions w, w + nwaves, ...; pad lanes of a last instruction
// re-read the region's last unit and land in the region's padding.
__device__ __forceinline__ void dma_rows(const Q4Mat &A, uint32_t r0, uint32_t rows, const RowsLayout &L, char *lds,
                                         uint32_t wave, uint32_t lane, uint32_t nwaves) {
    const rsrc_t rq = make_rsrc(A.qw, A.n * L.rowbytes);
    const rsrc_t rs = make_rsrc(A.sc, A.n * L.groups * 2);
    const rsrc_t rb = make_rsrc(A.bi, A.n * L.groups * 2);
    const uint32_t units = rows * L.rowbytes / 16, dwords = rows * L.groups / 2;
    const uint32_t nq = (units + 63) / 64, ns = (dwords + 63) / 64;
    for (uint32_t j = wave; j < nq; j += nwaves) {
        const uint32_t u = min(j * 64 + lane, units - 1);
        dma16(rq, lds + j * 1024, r0 * L.rowbytes + u * 16);
    }
    for (uint32_t j = wave; j < ns; j += nwaves) {
        const uint32_t d = min(j * 64 + lane, dwords - 1);
        dma4(rs, lds + L.sc + j * 256, r0 * L.groups * 2 + d * 4);
        dma4(rb, lds + L.bi + j * 256, r0 * L.groups * 2 + d * 4);
    }
}

// x (k bf16, 16-byte aligned) -> LDS (asynchronous).
__device__ __forceinline__ void dma_x(const uint16_t *x, uint32_t k, const RowsLayout &L, char *lds, uint32_t wave,
                                      uint32_t lane, uint32_t nwaves) {
    const rsrc_t r = make_rsrc(x, k * 2);
    const uint32_t units = k / 8, n = (units + 63) / 64;
    for (uint32_t j = wave; j < n; j += nwaves) {
        const uint32_t u = min(j * 64 + lane, units - 1);
        dma16(r, lds + L.x + j * 1024, u * 16);
    }
}

// The rows staged in LDS times the staged x, reduced in a fixed order: thread
// (group g = wave / 8, chunk c = 64 (wave mod 8) + lane) takes chunk c of rows
// g, g + 2, ... (<= 16 rows, <= 512 chunks); butterfly within the wave, then
// the 8 waves of the group in order.  Every thread calls it; thread t < rows
// gets the sum of row t.
__device__ __forceinline__ float lds_rows_dot(const char *lds, const RowsLayout &L, uint32_t rows, uint32_t k,
                                              uint32_t wave, uint32_t lane) {
    const uint32_t kMask = sgpr_const(0x000F000Fu);
    const uint32_t kMagic = vgpr_const(0x43004300u);
    const uint32_t kSelLo = sgpr_const(0x05040100u);
    const uint32_t kSelHi = sgpr_const(0x07060302u);
    const uint32_t grp = wave >> 3;
    const uint32_t c = (wave & 7) * kWave + lane;
    float acc[8];
#pragma unroll
    for (int i = 0; i < 8; ++i) acc[i] = 0.0f;
    if (c < (k >> 5)) {
        XChunk xc;
        load_xchunk(xc, reinterpret_cast<const uint16_t *>(lds + L.x), c, kSelLo, kSelHi);
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            const uint32_t row = grp + 2 * i;
            if (row < rows) {
                const u32x4 wv = *reinterpret_cast<const u32x4 *>(lds + row * L.rowbytes + c * 16);
                const uint32_t sb = (row * L.groups + (c >> 1)) * 2;
                const uint32_t sv = *reinterpret_cast<const uint16_t *>(lds + L.sc + sb);
                const uint32_t bv = *reinterpret_cast<const uint16_t *>(lds + L.bi + sb);
                acc[i] = chunk_dot(wv, sv, bv, xc, 0.0f, kMask, kMagic);
            }
        }
    }
    const float tot = wave_reduce_rows<8>(acc, lane);
    __shared__ float red[2][8][8];  // [group][wave of group][row slot]
    if ((lane & 7) == 0) red[grp][wave & 7][lane >> 3] = tot;
    __syncthreads();
    float s = 0.0f;
    if (threadIdx.x < rows) {
        const uint32_t g = threadIdx.x & 1, slot = threadIdx.x >> 1;
#pragma unroll
        for (int w = 0; w < 8; ++w) s += red[g][w][slot];
    }
    return s;
}

template <int EPI>
__device__ __forceinline__ float epilogue_operand(const GemvOut &o, uint32_t row) {
    if (EPI == kAccF32) return reinterpret_cast<const float *>(o.out)[row];
    if (EPI == kAccBF16) return bf16_to_f32(reinterpret_cast<const uint16_t *>(o.out)[row]);
    if ((EPI == kStoreF32 || EPI == kStoreBF16) && o.bias) return bf16_to_f32(o.bias[row]);
    return 0.0f;
}

template <int C>
__global__ __launch_bounds__(kThreads) void q4_mlp_fused_kernel(FusedMlp a) {
    extern __shared__ __align__(16) char lds[];
    const int tid = threadIdx.x;
    const uint32_t lane = tid & (kWave - 1);
    const uint32_t wave = __builtin_amdgcn_readfirstlane(tid / kWave);
    const uint32_t hidden = a.down.n, inter = a.down.k;
    const RowsLayout L(a.rpb, inter);
    const uint32_t r0 = blockIdx.x * a.rpb;
    const uint32_t rows = r0 < hidden ? min(a.rpb, hidden - r0) : 0;

    // ---- 1. this block's down rows -> LDS (asynchronous; waited for before step 4)
    if (rows > 0) dma_rows(a.down, r0, rows, L, lds, wave, lane, kWaves);

    // ---- 2. gate/up GEMV: persistent waves over (gate row, up row) tiles -> act (bf16, global)
    const GemvOut go{a.act, nullptr, a.activation};
    gemv_wave_loop<2, C, kGateUpBF16>(a.gate, a.up, a.x, go, inter, blockIdx.x * kWaves + wave, gridDim.x * kWaves);

    // ---- 3. every act value is written
    if (!grid_barrier(gridDim.x)) return;

    // ---- 4. act -> LDS; own DMA done; publish both to the block
    dma_x(a.act, inter, L, lds, wave, lane, kWaves);
    const GemvOut ho{a.h, nullptr, 0};
    const float pre = (uint32_t)tid < rows ? (a.h_f32 ? epilogue_operand<kAccF32>(ho, r0 + tid)
                                                      : epilogue_operand<kAccBF16>(ho, r0 + tid))
                                           : 0.0f;
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    __syncthreads();
    if (rows == 0) return;

    // ---- 5. down rows from LDS, accumulated into h
    const float sum = lds_rows_dot(lds, L, rows, inter, wave, lane);
    if ((uint32_t)tid < rows) {
        if (a.h_f32)
            store_row<kAccF32>(ho, r0 + tid, sum, pre);
        else
            store_row<kAccBF16>(ho, r0 + tid, sum, pre);
    }
}

static uint32_t fused_rpb(uint32_t hidden, uint32_t nblocks) { return (hidden + nblocks - 1) / nblocks; }

bool mlp_fused_supported(const Q4Mat &gate, const Q4Mat &down, uint32_t nblocks) {
    const uint32_t hidden = down.n, inter = down.k;
    if (nblocks == 0 || gate.k > 2 * 64 * 32 || inter % 128 != 0 || inter / 32 > 512) return false;
    const uint32_t rpb = fused_rpb(hidden, nblocks);
    if (rpb > 16) return false;
    if ((uint64_t)hidden * (inter / 2) >= (1ull << 31)) return false;
    return RowsLayout(rpb, inter).total <= 160u * 1024u;
}

uint32_t mlp_fused_timeouts() {
    uint32_t v = 0;
    if (hipMemcpyFromSymbol(&v, HIP_SYMBOL(g_bar_timeouts), sizeof(v), 0, hipMemcpyDeviceToHost) != hipSuccess)
        return 0xFFFFFFFFu;
    return v;
}

hipError_t launch_mlp_fused(FusedMlp a, uint32_t nblocks, hipStream_t s) {
    a.rpb = fused_rpb(a.down.n, nblocks);
    const uint32_t bytes = RowsLayout(a.rpb, a.down.k).total;
    auto kernel = a.gate.k <= 64 * 32 ? q4_mlp_fused_kernel<1> : q4_mlp_fused_kernel<2>;
    hipError_t e = hipFuncSetAttribute(reinterpret_cast<const void *>(kernel),
                                       hipFuncAttributeMaxDynamicSharedMemorySize, (int)bytes);
    if (e != hipSuccess) return e;
    hipLaunchKernelGGL(kernel, dim3(nblocks), dim3(kThreads), bytes, s, a);
    return hipGetLastError();
}

}  // namespace kr
