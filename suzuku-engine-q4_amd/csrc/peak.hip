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

}  // namespace q4mi

using namespace q4mi;

extern "C" {

/* Measurement hook (no reference counterpart): one launch of the MFMA
 * throughput probe on the library stream; kind 0 = int8 32x32x32, 1 = fp16
 * 32x32x16.  *ops receives the launch's integer ops / flops, so that the
 * caller's timing of the launch gives the rate. */
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
