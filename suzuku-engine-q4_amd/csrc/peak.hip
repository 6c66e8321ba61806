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
typedef float f32x16_t __attribute__((ext_vector_type(16)));

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

// A/B of the prefill MMQ's inner product loop: exact-integer fp16 MFMA
// (this library's design) against int8 MFMA, on the same work -- one wave
// owns 32 IQ3_S weight rows x 128 tokens (four 32-token sub-tiles) and walks
// K one 32-value q8 group at a time, operands from LDS, no global traffic.
//   KIND 0 (fp16): the lane decodes its row's 16 values of the group (grid
//     magnitudes and sign masks from LDS tables, times the (2s+1) multiplier,
//     as fp16), then per sub-tile two v_mfma_f32_32x32x16_f16 give the exact
//     group sums S and 16 FMAs add S * d_x;
//   KIND 1 (int8): the lane decodes its 16 values as signed int8 (one lookup
//     per 4 values in the 8192-entry signed table; the multiplier cannot be
//     folded: |w (2s+1)| reaches 465), then per sub-tile one
//     v_mfma_i32_32x32x32_i8 gives S, and each of the lane's 16 outputs (16
//     rows, each with its own multiplier) takes S * (2s+1), a conversion and
//     an FMA with d_x.
// Both flush inner * d_w into acc every 8 groups (a superblock).  The raw
// bytes, activations and scales are synthetic; the sink keeps every result
// live.
typedef int ab_v16i __attribute__((ext_vector_type(16)));
typedef _Float16 ab_h8 __attribute__((ext_vector_type(8)));
typedef _Float16 ab_h2 __attribute__((ext_vector_type(2)));

template <int KIND>
__global__ __launch_bounds__(256, 2) void mmq_ab_k(uint32_t groups, float *__restrict__ sink) {
    // LDS: raw rows (4 waves x 32 rows x 29 dwords, one superblock), the
    // activation stage (128 tokens x 32 values: fp16 or int8), scales, tables
    __shared__ uint32_t raw[4 * 32 * 29];
    __shared__ __align__(16) uint32_t act[128 * 16];
    __shared__ float dxs[128];
    __shared__ uint2 g16[512];
    __shared__ uint2 sm16[16];
    __shared__ uint32_t stab[KIND == 1 ? 8192 : 1];
    __shared__ __align__(16) int32_t mrow[4][32][8];   // (2s+1) of row r, group j
    const uint32_t tid = threadIdx.x, lane = tid & 63u, kh = lane >> 5, wv = tid >> 6;
    uint32_t seed = tid * 2654435761u + blockIdx.x * 40503u;
    auto rnd = [&]() { seed = seed * 1664525u + 1013904223u; return seed; };
    for (uint32_t i = tid; i < 4 * 32 * 29; i += 256) raw[i] = rnd();
    for (uint32_t i = tid; i < 128 * 16; i += 256) act[i] = KIND == 0 ? 0x3c003c00u ^ (rnd() & 0x80008000u) : rnd() & 0x7f7f7f7fu;
    if (tid < 128) dxs[tid] = 1.f / (1.f + tid);
    for (uint32_t i = tid; i < 512; i += 256) g16[i] = make_uint2(0x3c003c00u, 0x42004200u);
    if (tid < 16) sm16[tid] = make_uint2((tid & 1u) << 15 | (tid & 2u) << 30, (tid & 4u) << 13 | (tid & 8u) << 28);
    if (KIND == 1)
        for (uint32_t i = tid; i < 8192; i += 256) stab[i] = (i * 0x01030507u) & 0x0f0f0f0fu;
    for (uint32_t i = tid; i < 4 * 32 * 8; i += 256) (&mrow[0][0][0])[i] = 2 * (int)(rnd() & 15u) + 1;
    __syncthreads();
    const uint32_t row = lane & 31u;
    const uint8_t *R = (const uint8_t *)&raw[(wv * 32 + row) * 29];
    f32x16_t acc[4], inner[4];
#pragma unroll
    for (int t = 0; t < 4; t++) acc[t] = inner[t] = f32x16_t{};
    for (uint32_t g = 0; g < groups; g++) {
        const uint32_t j = g & 7u;
        if constexpr (KIND == 0) {
            const uint32_t qa = *(const uint16_t *)(R + 2 + 8 * j + 2 * kh);
            const uint32_t qb = *(const uint16_t *)(R + 6 + 8 * j + 2 * kh);
            const uint32_t qh = R[66 + j], sa = R[74 + 4 * j + kh], sb = R[76 + 4 * j + kh];
            const uint32_t sc = R[106 + (j >> 1)];
            const float m = (float)(2u * ((j & 1u) ? (sc >> 4) : (sc & 15u)) + 1u);
            const ab_h2 mm = {(_Float16)m, (_Float16)m};
            uint32_t o[8];
#pragma unroll
            for (int q = 0; q < 4; q++) {
                const uint32_t e = (q < 2 ? 2 * kh : 4 + 2 * kh) + (q & 1);
                const uint32_t qs8 = ((q < 2 ? qa : qb) >> (8 * (q & 1))) & 0xffu;
                const uint32_t idx = qs8 | (((qh >> e) & 1u) << 8);
                const uint32_t nib = ((q < 2 ? sa : sb) >> (4 * (q & 1))) & 15u;
                const uint2 gg = g16[idx], ss = sm16[nib];
                o[2 * q] = __builtin_bit_cast(uint32_t, __builtin_bit_cast(ab_h2, gg.x ^ ss.x) * mm);
                o[2 * q + 1] = __builtin_bit_cast(uint32_t, __builtin_bit_cast(ab_h2, gg.y ^ ss.y) * mm);
            }
            const ab_h8 A0 = __builtin_bit_cast(ab_h8, make_uint4(o[0], o[1], o[2], o[3]));
            const ab_h8 A1 = __builtin_bit_cast(ab_h8, make_uint4(o[4], o[5], o[6], o[7]));
#pragma unroll
            for (int t = 0; t < 4; t++) {
                const uint32_t tok = 32 * t + row;
                const ab_h8 B0 = *(const ab_h8 *)&act[tok * 16 + 4 * kh];
                const ab_h8 B1 = *(const ab_h8 *)&act[tok * 16 + 8 + 4 * kh];
                const float dx = dxs[tok];
                f32x16_t S = __builtin_amdgcn_mfma_f32_32x32x16_f16(A0, B0, f32x16_t{}, 0, 0, 0);
                S = __builtin_amdgcn_mfma_f32_32x32x16_f16(A1, B1, S, 0, 0, 0);
#pragma unroll
                for (int i = 0; i < 16; i++) inner[t][i] = fmaf(S[i], dx, inner[t][i]);
            }
        } else {
            // lane half kh: values 16kh..16kh+15 = grid entries 4kh..4kh+3
            const uint32_t qo = 2 + 8 * j + 4 * kh;
            const uint32_t q4 = *(const uint16_t *)(R + qo) | ((uint32_t)*(const uint16_t *)(R + qo + 2) << 16);
            const uint32_t qh = (uint32_t)R[66 + j] >> (4 * kh);
            const uint32_t sg = *(const uint16_t *)(R + 74 + 4 * j + 2 * kh);
            // byte k: (sign nibble k) << 1 | qh bit k -> index bits 8..12
            const uint32_t nb = (sg & 0x0Fu) | ((sg & 0xF0u) << 4) | ((sg & 0xF00u) << 8) | ((sg & 0xF000u) << 12);
            const uint32_t hv = (nb << 1) | (__umul24(qh & 15u, 0x00204081u) & 0x01010101u);
            int32_t w[4];
#pragma unroll
            for (int q = 0; q < 4; q++) {
                const uint32_t idx = __builtin_amdgcn_perm(hv, q4, 0x0C0C0400u | (uint32_t)q | ((uint32_t)q << 8));
                w[q] = (int32_t)stab[idx & 8191u];
            }
            const pk_v4i A = {w[0], w[1], w[2], w[3]};
            // the lane's 16 output rows' multipliers for this group
            int32_t m[16];
#pragma unroll
            for (int b = 0; b < 4; b++) {
                const int4 v = *(const int4 *)&mrow[wv][8 * b + 4 * kh][j & 3u];
                m[4 * b] = v.x; m[4 * b + 1] = v.y; m[4 * b + 2] = v.z; m[4 * b + 3] = v.w;
            }
#pragma unroll
            for (int t = 0; t < 4; t++) {
                const uint32_t tok = 32 * t + row;
                const int4 bb = *(const int4 *)&act[tok * 8 + 4 * kh];
                const pk_v4i B = {bb.x, bb.y, bb.z, bb.w};
                const float dx = dxs[tok];
                const ab_v16i S = __builtin_amdgcn_mfma_i32_32x32x32_i8(A, B, ab_v16i{}, 0, 0, 0);
#pragma unroll
                for (int i = 0; i < 16; i++)
                    inner[t][i] = fmaf((float)__mul24(S[i], m[i]), dx, inner[t][i]);
            }
        }
        if (j == 7u) {   // superblock flush: acc += inner * d_w
            const float dw = 1.f + (float)R[0] * (1.f / 256.f);
#pragma unroll
            for (int t = 0; t < 4; t++)
#pragma unroll
                for (int i = 0; i < 16; i++) {
                    acc[t][i] = fmaf(inner[t][i], dw, acc[t][i]);
                    inner[t][i] = 0.f;
                }
        }
    }
    float z = 0.f;
#pragma unroll
    for (int t = 0; t < 4; t++)
#pragma unroll
        for (int i = 0; i < 16; i++) z += acc[t][i] + inner[t][i];
    sink[blockIdx.x * 256 + tid] = z;
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

/* Measurement hook: one launch of the prefill MMQ inner-loop A/B (kind 0 =
 * exact-integer fp16 MFMA, 1 = int8 MFMA), two 256-thread blocks per CU,
 * each wave 32 x 128 outputs over `groups` 32-value groups.  *ops = the
 * launch's integer ops (2 per multiply-add), for a caller-timed rate. */
bool q4mi_mmq_ab_probe(int kind, uint32_t groups, uint64_t *ops) {
    if ((kind != 0 && kind != 1) || !groups || groups % 8 || !ops) {
        set_error("q4mi_mmq_ab_probe: bad arguments");
        return false;
    }
    const uint32_t blocks = 2u * (uint32_t)cu_count();
    const uint32_t n = blocks * 256u;
    if (g_sink_n < n) {
        if (g_sink) (void)hipFree(g_sink);
        g_sink = nullptr;
        g_sink_n = 0;
        if (hipMalloc(&g_sink, (size_t)n * sizeof(float)) != hipSuccess) {
            set_error("q4mi_mmq_ab_probe: sink allocation failed");
            return false;
        }
        g_sink_n = n;
    }
    *ops = (uint64_t)blocks * 4u * groups * 32ull * 128ull * 32ull * 2ull;
    if (kind == 0)
        mmq_ab_k<0><<<dim3(blocks), dim3(256), 0, stream()>>>(groups, g_sink);
    else
        mmq_ab_k<1><<<dim3(blocks), dim3(256), 0, stream()>>>(groups, g_sink);
    return launch_ok("mmq_ab_k");
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
