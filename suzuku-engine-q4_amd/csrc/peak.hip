// MFMA throughput probe: measures the dense matrix-core rate of the GPU it
// runs on, so that the prefill MMQ's fraction of peak can be quoted against
// a measured figure as well as the datasheet's.
//
// Every wave runs four independent accumulator chains of one MFMA shape
// (enough to cover the instruction's latency), two 256-thread blocks per CU.
// The operands depend on the thread index, and every accumulator is reduced
// into a store, so nothing can be folded away.
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "q4mi_internal.h"

// Built into the measurement library (libq4mi_meas.so, -DQ4MI_MEASURE) only.
#ifdef Q4MI_MEASURE

namespace q4mi {

typedef int pk_v4i __attribute__((ext_vector_type(4)));
typedef int pk_v16i __attribute__((ext_vector_type(16)));
typedef float pk_v16f __attribute__((ext_vector_type(16)));
typedef _Float16 pk_h8 __attribute__((ext_vector_type(8)));

constexpr int kChains = 4;

// KIND 0: v_mfma_i32_32x32x32_i8 (65536 ops), 1: v_mfma_f32_32x32x16_f16
// (32768 flops).
template <int KIND>
__global__ __launch_bounds__(256) void mfma_peak_k(uint32_t iters, float *__restrict__ sink) {
    const uint32_t t = threadIdx.x + blockIdx.x * 256u;
    float keep = 0.f;
    if constexpr (KIND == 0) {
        const pk_v4i a = {(int)t, (int)(t * 3u), (int)(t ^ 0x5a5a5a5au), (int)(t + 7u)};
        const pk_v4i b = {(int)(t * 5u), (int)(t + 1u), (int)(t ^ 0x33u), (int)(t * 9u)};
        pk_v16i c[kChains] = {};
        for (uint32_t i = 0; i < iters; i++) {
#pragma unroll
            for (int k = 0; k < kChains; k++)
                c[k] = __builtin_amdgcn_mfma_i32_32x32x32_i8(a, b, c[k], 0, 0, 0);
        }
#pragma unroll
        for (int k = 0; k < kChains; k++)
#pragma unroll
            for (int j = 0; j < 16; j++) keep += (float)c[k][j];
    } else {
        pk_h8 a, b;
#pragma unroll
        for (int j = 0; j < 8; j++) {
            a[j] = (_Float16)(float)((t + j) & 7u);
            b[j] = (_Float16)(float)((t * 3u + j) & 7u);
        }
        pk_v16f c[kChains] = {};
        for (uint32_t i = 0; i < iters; i++) {
#pragma unroll
            for (int k = 0; k < kChains; k++)
                c[k] = __builtin_amdgcn_mfma_f32_32x32x16_f16(a, b, c[k], 0, 0, 0);
        }
#pragma unroll
        for (int k = 0; k < kChains; k++)
#pragma unroll
            for (int j = 0; j < 16; j++) keep += c[k][j];
    }
    sink[t] = keep;
}

static float *g_sink = nullptr;
static uint32_t g_sink_n = 0;

// Floor probes of the decode kernels' structure (one 1024-thread block per
// CU, as moe_gu_k / moe_dn_k): `waves` producer waves of each block copy the
// block's `per_block` bytes (contiguous, at src + block * per_block) into LDS
// with 1 KB global_load_lds_dwordx4 operations, then wait for them; the
// other waves exit.  per_block = 0: an empty kernel of the same shape.
__global__ __launch_bounds__(1024) void stream_probe_k(const uint8_t *__restrict__ src,
                                                       uint32_t per_block, uint32_t waves) {
    extern __shared__ __align__(16) uint8_t sm[];
    const uint32_t w = threadIdx.x >> 6, lane = threadIdx.x & 63u;
    if (w >= waves || !per_block) return;
    const uint8_t *s = src + (size_t)blockIdx.x * per_block;
    const uint32_t nops = per_block / 1024, base = (uint32_t)(uintptr_t)sm;
    for (uint32_t j = w; j < nops; j += waves) {
        const uint32_t lds = __builtin_amdgcn_readfirstlane(base + (j % 150u) * 1024u);
        asm volatile("s_mov_b32 m0, %1\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %0, off"
                     :: "v"(s + (size_t)j * 1024 + lane * 16), "s"(lds) : "memory", "m0");
    }
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
}

// Floor probe of the chip itself (not of the decode kernels' structure):
// a plain register-load streaming kernel.  Many 256-thread blocks; thread t
// of block b loads U 16-byte units at src + 16 (b*256*U + u*256 + t), u < U
// (one coalesced 4 KB wave-group access per u), all issued before any is
// used.  The loaded words are folded into one value that is stored only if
// it equals a key the data never produces, so no load can be dropped and
// nothing is written.
template <int U>
__global__ __launch_bounds__(256) void plain_stream_k(const uint4 *__restrict__ src, uint32_t key,
                                                      uint32_t *__restrict__ sink) {
    const uint4 *s = src + (size_t)blockIdx.x * 256u * U + threadIdx.x;
    uint4 v[U];
#pragma unroll
    for (int u = 0; u < U; u++) v[u] = s[256 * u];
    uint32_t f = 0;
#pragma unroll
    for (int u = 0; u < U; u++) f ^= v[u].x ^ v[u].y ^ v[u].z ^ v[u].w;
    if (f == key) sink[threadIdx.x] = f;
}

}  // namespace q4mi

using namespace q4mi;

extern "C" {

/* Measurement hook (no reference counterpart): one launch of the MFMA
 * throughput probe on the library stream; kind 0 = int8 32x32x32, 1 = fp16
 * 32x32x16.  *ops receives the launch's integer ops / flops, so that the
 * caller's timing of the launch gives the rate. */
/* Measurement hook: one launch of the stream floor probe (one 1024-thread
 * block per CU, `waves` producer waves copying per_block bytes each into LDS;
 * per_block = 0: empty kernel).  src must hold cu_count() * per_block bytes;
 * *bytes = the launch's total. */
bool q4mi_stream_probe(const void *src, uint32_t per_block, uint32_t waves, uint64_t *bytes) {
    if ((per_block && !src) || per_block % 1024 || per_block > 150u * 1024 || !waves ||
        waves > 16 || !bytes) {
        set_error("q4mi_stream_probe: bad arguments");
        return false;
    }
    static bool attr = false;
    if (!attr) {
        if (hipFuncSetAttribute((const void *)stream_probe_k,
                                hipFuncAttributeMaxDynamicSharedMemorySize,
                                150 * 1024) != hipSuccess) {
            set_error("q4mi_stream_probe: LDS limit");
            return false;
        }
        attr = true;
    }
    const uint32_t blocks = (uint32_t)cu_count();
    *bytes = (uint64_t)blocks * per_block;
    stream_probe_k<<<dim3(blocks), dim3(1024), 150 * 1024, stream()>>>((const uint8_t *)src,
                                                                       per_block, waves);
    return launch_ok("stream_probe_k");
}

/* Measurement hook: one launch of the plain streaming probe, reading
 * `bytes` (a multiple of 4096 * unroll) from src with `unroll` (1, 4 or 8)
 * 16-byte loads per thread in 256-thread blocks.  The probe writes nothing
 * unless the data XOR-folds to 0x9e3779b9 in some thread (the caller's fill
 * must avoid that; a uniform byte fill folds to 0). */
bool q4mi_plain_stream_probe(const void *src, uint64_t bytes, uint32_t unroll) {
    const uint64_t per = 4096ull * unroll;
    if (!src || ((uintptr_t)src & 15) || (unroll != 1 && unroll != 4 && unroll != 8) ||
        !bytes || bytes % per || bytes / per > 0x7fffffffull) {
        set_error("q4mi_plain_stream_probe: bad arguments");
        return false;
    }
    if (!g_sink) {
        if (hipMalloc(&g_sink, 1024 * sizeof(float)) != hipSuccess) {
            set_error("q4mi_plain_stream_probe: sink allocation failed");
            return false;
        }
        g_sink_n = 1024;
    }
    const dim3 grid((uint32_t)(bytes / per));
    uint32_t *sk = (uint32_t *)g_sink;
    const uint4 *s = (const uint4 *)src;
    if (unroll == 1) plain_stream_k<1><<<grid, dim3(256), 0, stream()>>>(s, 0x9e3779b9u, sk);
    else if (unroll == 4) plain_stream_k<4><<<grid, dim3(256), 0, stream()>>>(s, 0x9e3779b9u, sk);
    else plain_stream_k<8><<<grid, dim3(256), 0, stream()>>>(s, 0x9e3779b9u, sk);
    return launch_ok("plain_stream_k");
}

bool q4mi_mfma_probe(int kind, uint32_t iters, uint64_t *ops) {
    if ((kind != 0 && kind != 1) || !iters || !ops) {
        set_error("q4mi_mfma_probe: bad arguments");
        return false;
    }
    const uint32_t blocks = 2u * (uint32_t)cu_count();
    const uint32_t n = blocks * 256u;
    if (g_sink_n < n) {
        if (g_sink) (void)hipFree(g_sink);
        g_sink = nullptr;
        g_sink_n = 0;
        if (hipMalloc(&g_sink, (size_t)n * sizeof(float)) != hipSuccess) {
            set_error("q4mi_mfma_probe: sink allocation failed");
            return false;
        }
        g_sink_n = n;
    }
    const uint64_t waves = (uint64_t)blocks * 4u;
    const uint64_t per = kind == 0 ? 32ull * 32 * 32 * 2 : 32ull * 32 * 16 * 2;
    *ops = waves * iters * kChains * per;
    if (kind == 0)
        mfma_peak_k<0><<<dim3(blocks), dim3(256), 0, stream()>>>(iters, g_sink);
    else
        mfma_peak_k<1><<<dim3(blocks), dim3(256), 0, stream()>>>(iters, g_sink);
    return launch_ok("mfma_peak_k");
}

}  // extern "C"

#endif  // Q4MI_MEASURE
