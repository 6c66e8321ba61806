// MoE router front: the router GEMV (expert logits from the hidden state)
// and the shared-expert gate, then softmax + top-k into the per-token device
// lists the decode / verify-window entry points read.
//
// Reference:
//   router GEMV + shared expert + sgate dot      q4_moe_gpu_a, src/q4_moe.c:1360-1440
//   device top-k into per-token lists           route_dev_n_k, src/q4_rocm.cu:5930-6060
//   sgate: sigmoid(w . x), then y += sg * shared  src/q4_moe.c:297-306,
//                                               sgate_axpy_k src/q4_rocm.cu:15775-15790
//
// Dot order (fixed, so the logits are reproducible bit for bit): for row e
// and token t, lane l of a wave accumulates, for i = 0 .. K/256 - 1, the
// four products of its float4 at element 4(64i + l) in component order with
// fmaf; the 64 lane sums are then joined by an xor butterfly over lane
// distances 32, 16, 8, 4, 2, 1 (a + b, the same value on every lane).
#include "q4mi_common.h"
#include "q4mi_internal.h"

namespace q4mi {

constexpr uint32_t kRtF32 = 0, kRtF16 = 1, kRtBF16 = 30;   // ggml type ids

__device__ inline float bf16f(uint32_t b) { return __uint_as_float(b << 16); }
__device__ inline float f16f(uint32_t h) { return (float)__builtin_bit_cast(_Float16, (uint16_t)h); }

// Four consecutive weights of a router row as fp32.
template <uint32_t WT>
__device__ inline float4 load_w4(const uint8_t *row, uint32_t e4) {
    if constexpr (WT == kRtF32) {
        return ((const float4 *)row)[e4];
    } else {
        const uint2 v = ((const uint2 *)row)[e4];
        if constexpr (WT == kRtF16)
            return make_float4(f16f(v.x & 0xffffu), f16f(v.x >> 16), f16f(v.y & 0xffffu),
                               f16f(v.y >> 16));
        else
            return make_float4(bf16f(v.x & 0xffffu), bf16f(v.x >> 16), bf16f(v.y & 0xffffu),
                               bf16f(v.y >> 16));
    }
}

__device__ inline float xor_sum64(float v) {
#pragma unroll
    for (int o = 32; o >= 1; o >>= 1) v += __shfl_xor(v, o, 64);
    return v;
}

constexpr uint32_t kRtMaxK = 16384;   // x tile: TT * K fp32 <= 64 KB
constexpr uint32_t kRtMaxNI = 16;     // float4 per lane per row: K <= 16384

// Block (bx, by): tokens [TT*by, TT*by + TT) with their x in LDS; wave w
// takes rows bx*4 + w, then + 4*gridDim.x, ...  Rows 0..n_exp-1 are the
// router's (logits[t][e]); row n_exp, when sgw is given, is the shared
// expert's gate vector (sg[t] = sigmoid of its dot).
template <uint32_t WT>
__global__ __launch_bounds__(256) void router_gemv_k(const uint8_t *__restrict__ w,
                                                     const float *__restrict__ sgw,
                                                     const float *__restrict__ x,
                                                     uint32_t n_tok, uint32_t K, uint32_t n_exp,
                                                     uint32_t TT, float *__restrict__ logits,
                                                     float *__restrict__ sg) {
    extern __shared__ __align__(16) float xs[];
    const uint32_t lane = threadIdx.x & 63u;
    const uint32_t wave = threadIdx.x >> 6;
    const uint32_t t0 = blockIdx.y * TT, nt = min(TT, n_tok - t0);
    const uint32_t q4 = K / 4;
    const uint32_t rows = n_exp + (sgw ? 1u : 0u);
    const uint32_t ni = K / 256;
    const size_t rb = (size_t)K * (WT == kRtF32 ? 4 : 2);
    // this wave's first row is loaded before the block stages x, so the two
    // memory round trips overlap
    float4 wv[kRtMaxNI];
    auto load_row = [&](uint32_t r) __attribute__((always_inline)) {
        const bool gate = r == n_exp;
#pragma unroll
        for (uint32_t i = 0; i < kRtMaxNI; i++) {
            if (i < ni)
                wv[i] = gate ? ((const float4 *)sgw)[64 * i + lane]
                             : load_w4<WT>(w + (size_t)r * rb, 64 * i + lane);
        }
    };
    const uint32_t r0 = blockIdx.x * 4 + wave;
    if (r0 < rows) load_row(r0);
    for (uint32_t i = threadIdx.x; i < nt * q4; i += 256)
        ((float4 *)xs)[i] = ((const float4 *)(x + (size_t)t0 * K))[i];
    __syncthreads();
    for (uint32_t r = r0; r < rows; r += gridDim.x * 4) {
        const bool gate = r == n_exp;
        if (r != r0) load_row(r);
        for (uint32_t t = 0; t < nt; t++) {
            const float4 *xt = (const float4 *)(xs + (size_t)t * K);
            float acc = 0.f;
#pragma unroll
            for (uint32_t i = 0; i < kRtMaxNI; i++) {
                if (i < ni) {
                    const float4 xv = xt[64 * i + lane];
                    acc = fmaf(wv[i].x, xv.x, acc);
                    acc = fmaf(wv[i].y, xv.y, acc);
                    acc = fmaf(wv[i].z, xv.z, acc);
                    acc = fmaf(wv[i].w, xv.w, acc);
                }
            }
            acc = xor_sum64(acc);
            if (lane == 0) {
                if (gate)
                    sg[t0 + t] = 1.f / (1.f + expf(-acc));
                else
                    logits[(size_t)(t0 + t) * n_exp + r] = acc;
            }
        }
    }
}

// One wave's dot of w and x in the router's fixed order; every lane returns
// the total.  With both vectors 16-byte aligned the first K - K % 256
// elements go by float4 as above; the rest (or all of K when either vector
// is not 16-byte aligned) are taken lane-strided -- lane l adds elements
// b + l, b + l + 64, ... in order -- before the butterfly.
__device__ inline float wave_dot(const float *__restrict__ w, const float *__restrict__ x,
                                 uint32_t K, uint32_t lane) {
    float acc = 0.f;
    const bool vec = (((uintptr_t)w | (uintptr_t)x) & 15u) == 0;
    const uint32_t kv = vec ? K / 256 * 256 : 0u;
    for (uint32_t i = 0; i < kv / 256; i++) {
        const float4 a = ((const float4 *)w)[64 * i + lane];
        const float4 b = ((const float4 *)x)[64 * i + lane];
        acc = fmaf(a.x, b.x, acc);
        acc = fmaf(a.y, b.y, acc);
        acc = fmaf(a.z, b.z, acc);
        acc = fmaf(a.w, b.w, acc);
    }
    for (uint32_t i = kv + lane; i < K; i += 64) acc = fmaf(w[i], x[i], acc);
    return xor_sum64(acc);
}

// dy[t][i] += sigmoid(w . x[t]) * sh[t][i]: block (bx, t) recomputes its
// token's gate with its first wave (the same bits in every block) and adds
// its 256-value slice.
__global__ __launch_bounds__(256) void sgate_axpy_k(float *__restrict__ dy,
                                                    const float *__restrict__ sh,
                                                    const float *__restrict__ w,
                                                    const float *__restrict__ x, uint32_t n) {
    __shared__ float s_sg;
    const uint32_t t = blockIdx.y;
    if (threadIdx.x < 64) {
        const float d = wave_dot(w, x + (size_t)t * n, n, threadIdx.x);
        if (threadIdx.x == 0) s_sg = 1.f / (1.f + expf(-d));
    }
    __syncthreads();
    const uint32_t i = blockIdx.x * 256 + threadIdx.x;
    if (i < n) dy[(size_t)t * n + i] = fmaf(s_sg, sh[(size_t)t * n + i], dy[(size_t)t * n + i]);
}

__global__ void dot_sigmoid_k(const float *__restrict__ a, const float *__restrict__ b,
                              float *__restrict__ out, uint32_t n) {
    const float d = wave_dot(a, b, n, threadIdx.x);
    if (threadIdx.x == 0) *out = 1.f / (1.f + expf(-d));
}

// The router GEMV of q4mi_moe_route (logits [n_tok][n_exp] and, with a gate
// vector, sg[t] = sigmoid(w_sg . x_t)); launch = false only checks the
// arguments (the error text says which is wrong).
bool router_front(const void *d_wr, uint32_t wr_type, const float *d_sgw, const float *d_x,
                  uint32_t n_tok, uint32_t n_embd, uint32_t n_exp, uint32_t topk,
                  float *d_logits, uint32_t ostride, int32_t shared_slot, float *d_sg,
                  bool launch) {
    if (!d_wr || !d_x || !d_logits || !n_tok || !n_exp || n_exp > 512u ||
        !topk || topk > 64u) {
        set_error("q4mi_moe_route: bad arguments");
        return false;
    }
    if (wr_type != kRtF32 && wr_type != kRtF16 && wr_type != kRtBF16) {
        set_error("q4mi_moe_route: router type %u not covered (F32, F16, BF16)", wr_type);
        return false;
    }
    if (!n_embd || n_embd % 256 || n_embd > kRtMaxK) {
        set_error("q4mi_moe_route: n_embd %u not covered (a multiple of 256, <= %u)", n_embd,
                  kRtMaxK);
        return false;
    }
    if (d_sgw && !d_sg) {
        set_error("q4mi_moe_route: a gate vector needs d_sg");
        return false;
    }
    const uint32_t need = topk + (shared_slot >= 0 ? 1u : 0u);
    if (ostride < need) {
        set_error("q4mi_moe_route: ostride %u < %u entries per token", ostride, need);
        return false;
    }
    const uintptr_t al = (uintptr_t)d_x | (uintptr_t)d_wr | (uintptr_t)d_sgw;
    if (al & 15u) {
        set_error("q4mi_moe_route: x, router and gate rows must be 16-byte aligned");
        return false;
    }
    if (!launch) return true;
    const uint32_t TT = std::min<uint32_t>(std::min<uint32_t>(8u, 16384u / n_embd), n_tok);
    const uint32_t gy = (n_tok + TT - 1) / TT;
    const uint32_t rows = n_exp + (d_sgw ? 1u : 0u);
    const uint32_t gx = std::max<uint32_t>(1u, std::min<uint32_t>((rows + 3) / 4,
                                                                  std::max<uint32_t>(8u, 4096u / gy)));
    const size_t lds = (size_t)TT * n_embd * 4;
    const uint8_t *w = (const uint8_t *)d_wr;
    const dim3 grid(gx, gy);
    if (wr_type == kRtF32)
        router_gemv_k<kRtF32><<<grid, 256, lds, stream()>>>(w, d_sgw, d_x, n_tok, n_embd, n_exp,
                                                            TT, d_logits, d_sg);
    else if (wr_type == kRtF16)
        router_gemv_k<kRtF16><<<grid, 256, lds, stream()>>>(w, d_sgw, d_x, n_tok, n_embd, n_exp,
                                                            TT, d_logits, d_sg);
    else
        router_gemv_k<kRtBF16><<<grid, 256, lds, stream()>>>(w, d_sgw, d_x, n_tok, n_embd, n_exp,
                                                             TT, d_logits, d_sg);
    return launch_ok("router_gemv_k");
}

}  // namespace q4mi

using namespace q4mi;

extern "C" {

/* Router front of a MoE layer (see include/q4mi.h). */
bool q4mi_moe_route(const void *d_wr, uint32_t wr_type, const float *d_sgw, const float *d_x,
                    uint32_t n_tok, uint32_t n_embd, uint32_t n_exp, uint32_t topk,
                    float *d_logits, int32_t *d_ids, float *d_wts, int32_t *d_nh,
                    uint32_t ostride, int32_t shared_slot, float *d_sg) {
    if (!d_ids || !d_wts) {
        set_error("q4mi_moe_route: bad arguments");
        return false;
    }
    if (!router_front(d_wr, wr_type, d_sgw, d_x, n_tok, n_embd, n_exp, topk, d_logits, ostride,
                      shared_slot, d_sg, false) ||
        !router_front(d_wr, wr_type, d_sgw, d_x, n_tok, n_embd, n_exp, topk, d_logits, ostride,
                      shared_slot, d_sg, true))
        return false;
    return route_list_launch(d_logits, d_ids, d_wts, d_nh, n_tok, n_exp, topk, ostride,
                             shared_slot, d_sgw ? d_sg : nullptr);
}

/* d_y[t] += sigmoid(d_w . d_x[t]) * d_sh[t] for t < n_tok, in one launch
 * (see include/q4mi.h). */
bool q4_hip_sgate_axpy(float *d_y, const float *d_sh, const float *d_w, const float *d_x,
                       uint32_t n, uint32_t n_tok) {
    if (!d_y || !d_sh || !d_w || !d_x || !n || !n_tok) {
        set_error("q4_hip_sgate_axpy: bad arguments");
        return false;
    }
    sgate_axpy_k<<<dim3((n + 255) / 256, n_tok), dim3(256), 0, stream()>>>(d_y, d_sh, d_w, d_x,
                                                                          n);
    return launch_ok("sgate_axpy_k");
}

/* *out = sigmoid(a . b), one launch (see include/q4mi.h). */
bool q4_hip_dot_sigmoid(const float *a, const float *b, float *out, uint32_t n) {
    if (!a || !b || !out || !n) {
        set_error("q4_hip_dot_sigmoid: bad arguments");
        return false;
    }
    dot_sigmoid_k<<<dim3(1), dim3(64), 0, stream()>>>(a, b, out, n);
    return launch_ok("dot_sigmoid_k");
}

}  // extern "C"
