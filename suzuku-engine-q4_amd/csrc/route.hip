// Routing (softmax + top-k + renormalisation), the expert pack (a stable
// counting sort of the (token, pick) pairs by expert) and the weighted
// scatter-back of expert outputs.
//
// Semantics follow the reference host path:
//   q4_softmax + q4_topk(renorm)        src/q4_quant.c:715-755
//   host pack (ebase, a_tok, rsrc, rw, stg)  src/q4_moe.c:3404-3451
//   MMQ bounds                           src/q4_moe.c:3558-3571
//   reduce_expert_k                      src/q4_rocm.cu:15739-15750
// The reference's own GPU pack orders rows inside an expert by atomic
// arrival; this one reproduces the host's stable (t, k) order exactly.
#include "q4mi_common.h"
#include "q4mi_internal.h"

namespace q4mi {

// float -> uint key with the same order (negatives included)
__device__ inline uint32_t f2key(float f) {
    const uint32_t b = __float_as_uint(f);
    return (b & 0x80000000u) ? ~b : (b | 0x80000000u);
}

// One wave per token; up to 512 experts (8 per lane), k <= 64.
// Ranking uses (logit desc, index asc): softmax is monotonic, so this is the
// host's (probability desc, index asc) order except where two different
// logits round to the same probability.  Weights: p_i = e_i * (1/sum e),
// then p_i * (1/sum of the k picked p, in rank order).
__global__ __launch_bounds__(256) void route_k(const float *__restrict__ logits, uint32_t n_tok,
                                               uint32_t n_exp, uint32_t topk,
                                               int32_t *__restrict__ ids,
                                               float *__restrict__ wts) {
    __shared__ int32_t s_id[4][64];
    __shared__ float s_p[4][64];
    const uint32_t w = threadIdx.x >> 6, lane = threadIdx.x & 63u;
    const uint32_t t = blockIdx.x * 4 + w;
    if (t >= n_tok) return;
    const float *lg = logits + (size_t)t * n_exp;
    float v[8];
    float mx = -INFINITY;
#pragma unroll
    for (int j = 0; j < 8; j++) {
        const uint32_t i = lane + 64u * j;
        v[j] = i < n_exp ? lg[i] : -INFINITY;
        mx = fmaxf(mx, v[j]);
    }
#pragma unroll
    for (int o = 32; o; o >>= 1) mx = fmaxf(mx, __shfl_xor(mx, o));
    float e[8], s = 0.f;
#pragma unroll
    for (int j = 0; j < 8; j++) {
        e[j] = (lane + 64u * j) < n_exp ? expf(v[j] - mx) : 0.f;
        s += e[j];
    }
#pragma unroll
    for (int o = 32; o; o >>= 1) s += __shfl_xor(s, o);
    const float inv = s > 0.f ? __fdiv_rn(1.f, s) : 0.f;
    uint32_t alive = 0;
#pragma unroll
    for (int j = 0; j < 8; j++)
        if ((lane + 64u * j) < n_exp) alive |= 1u << j;
    const uint32_t tk = topk < n_exp ? topk : n_exp;
    for (uint32_t k = 0; k < tk; k++) {
        uint64_t best = 0;
#pragma unroll
        for (int j = 0; j < 8; j++) {
            const uint32_t i = lane + 64u * j;
            if (alive & (1u << j)) {
                const uint64_t key = ((uint64_t)f2key(v[j]) << 32) | (uint32_t)(~i);
                best = key > best ? key : best;
            }
        }
#pragma unroll
        for (int o = 32; o; o >>= 1) {
            const uint64_t b2 = __shfl_xor(best, o);
            best = b2 > best ? b2 : best;
        }
        const uint32_t wi = ~(uint32_t)(best & 0xffffffffu);
        if ((wi & 63u) == lane) {
            const uint32_t j = wi >> 6;
            alive &= ~(1u << j);
            float pe = 0.f;
#pragma unroll
            for (int jj = 0; jj < 8; jj++)
                if ((uint32_t)jj == j) pe = e[jj];
            s_id[w][k] = (int32_t)wi;
            s_p[w][k] = pe * inv;
        }
    }
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQ_REL, "wavefront");
    float sk = 0.f;
    for (uint32_t k = 0; k < tk; k++) sk += s_p[w][k];
    const float inv2 = sk > 0.f ? __fdiv_rn(1.f, sk) : 0.f;
    for (uint32_t k = lane; k < topk; k += 64) {
        ids[(size_t)t * topk + k] = k < tk ? s_id[w][k] : -1;
        wts[(size_t)t * topk + k] = k < tk ? (sk > 0.f ? s_p[w][k] * inv2 : s_p[w][k]) : 0.f;
    }
}

// Stable pack of one token group per block (1024 threads = 16 waves).
// Rounds of 1024 consecutive (t, k) entries: inside a wave, entries with
// the same expert are found with 10 ballots (ids < 1024); a wave's offset
// for expert e adds the counts of the earlier waves of the round and the
// expert's running cursor, so positions follow scan order exactly.
__global__ __launch_bounds__(1024) void assign_k(
    const int32_t *__restrict__ ids, const float *__restrict__ wts, int32_t *__restrict__ a_tok,
    int32_t *__restrict__ rsrc, float *__restrict__ rw, int32_t *__restrict__ stg,
    uint32_t *__restrict__ stgn, uint32_t *__restrict__ ek, int32_t *__restrict__ bounds,
    uint32_t gsz, uint32_t topk, uint32_t n_exp, uint32_t n_tok) {
    __shared__ uint32_t s_cnt[512];
    __shared__ uint32_t s_cur[512];
    __shared__ uint16_t s_wc[16][512];
    const uint32_t g = blockIdx.x, tid = threadIdx.x;
    const uint32_t wv = tid >> 6, lane = tid & 63u;
    const uint32_t t0 = g * gsz;
    const uint32_t t1 = min(t0 + gsz, n_tok);
    const uint32_t rows = (t1 - t0) * topk;
    const size_t seg = (size_t)g * gsz * topk;
    const int32_t *gid = ids + (size_t)t0 * topk;
    for (uint32_t i = tid; i < 512; i += 1024) s_cnt[i] = 0;
    for (uint32_t i = tid; i < 16 * 512; i += 1024) (&s_wc[0][0])[i] = 0;
    __syncthreads();
    for (uint32_t i = tid; i < rows; i += 1024) {
        const int32_t e = gid[i];
        if (e >= 0 && (uint32_t)e < n_exp) atomicAdd(&s_cnt[e], 1u);
    }
    __syncthreads();
    if (tid == 0) {
        uint32_t b = 0, ns = 0;
        for (uint32_t e = 0; e < n_exp; e++) {
            const uint32_t c = s_cnt[e];
            s_cur[e] = b;
            if (bounds) bounds[(size_t)g * (n_exp + 1) + e] = (int32_t)b;
            if (c) stg[(size_t)g * 512 + ns++] = (int32_t)e;
            b += c;
        }
        if (bounds) bounds[(size_t)g * (n_exp + 1) + n_exp] = (int32_t)b;
        stgn[g] = ns;
    }
    for (uint32_t i = tid; i < 512; i += 1024) ek[(size_t)g * 512 + i] = i < n_exp ? s_cnt[i] : 0;
    __syncthreads();
    const uint64_t lt = (1ull << lane) - 1ull;
    for (uint32_t base = 0; base < rows; base += 1024) {
        const uint32_t i = base + tid;
        const bool in = i < rows;
        const int32_t e = in ? gid[i] : -1;
        const bool valid = in && e >= 0 && (uint32_t)e < n_exp;
        uint64_t same = __ballot(valid);
#pragma unroll
        for (int b = 0; b < 10; b++) {
            const bool bit = valid && ((e >> b) & 1);
            const uint64_t m = __ballot(bit);
            same &= bit ? m : ~m;
        }
        if (!valid) same = 0;
        const uint32_t rank = (uint32_t)__popcll(same & lt);
        const bool leader = valid && rank == 0;
        if (leader) s_wc[wv][e] = (uint16_t)__popcll(same);
        __syncthreads();
        if (valid) {
            uint32_t p = s_cur[e] + rank;
            for (uint32_t w2 = 0; w2 < wv; w2++) p += s_wc[w2][e];
            const uint32_t t = t0 + i / topk;
            a_tok[seg + p] = (int32_t)t;
            rsrc[(size_t)t0 * topk + i] = (int32_t)p;
            rw[(size_t)t0 * topk + i] = wts[(size_t)t0 * topk + i];
        } else if (in) {
            rsrc[(size_t)t0 * topk + i] = -1;
            rw[(size_t)t0 * topk + i] = 0.f;
        }
        __syncthreads();
        if (leader) {
            atomicAdd(&s_cur[e], (uint32_t)s_wc[wv][e]);
            s_wc[wv][e] = 0;
        }
        __syncthreads();
    }
}

// dy[t][i] += sum_k rw[t*topk+k] * pd[rsrc[t*topk+k]][i], k in order.
__global__ __launch_bounds__(256) void reduce_k(float *__restrict__ dy,
                                                const float *__restrict__ pd,
                                                const int32_t *__restrict__ rsrc,
                                                const float *__restrict__ rw, uint32_t topk,
                                                uint32_t n_embd) {
    const uint32_t t = blockIdx.y;
    const uint32_t i = (blockIdx.x * 256 + threadIdx.x) * 4;
    if (i >= n_embd) return;
    float4 acc = make_float4(0.f, 0.f, 0.f, 0.f);
    for (uint32_t k = 0; k < topk; k++) {
        const int32_t src = rsrc[(size_t)t * topk + k];
        if (src < 0) continue;
        const float w = rw[(size_t)t * topk + k];
        const float4 v = *(const float4 *)(pd + (size_t)src * n_embd + i);
        acc.x += w * v.x;
        acc.y += w * v.y;
        acc.z += w * v.z;
        acc.w += w * v.w;
    }
    float4 *o = (float4 *)(dy + (size_t)t * n_embd + i);
    float4 c = *o;
    c.x += acc.x;
    c.y += acc.y;
    c.z += acc.z;
    c.w += acc.w;
    *o = c;
}

bool route_launch(const float *lg, int32_t *ids, float *wts, uint32_t n_tok, uint32_t n_exp,
                  uint32_t topk) {
    route_k<<<dim3((n_tok + 3) / 4), dim3(256), 0, stream()>>>(lg, n_tok, n_exp, topk, ids,
                                                              wts);
    return launch_ok("route_k");
}

bool assign_launch(const int32_t *ids, const float *wts, int32_t *a_tok, int32_t *rsrc,
                   float *rw, int32_t *stg, uint32_t *stgn, uint32_t *ek, int32_t *bounds,
                   uint32_t gsz, uint32_t topk, uint32_t n_exp, uint32_t n_tok) {
    const uint32_t n_g = (n_tok + gsz - 1) / gsz;
    assign_k<<<dim3(n_g), dim3(1024), 0, stream()>>>(ids, wts, a_tok, rsrc, rw, stg, stgn, ek,
                                                    bounds, gsz, topk, n_exp, n_tok);
    return launch_ok("assign_k");
}

bool reduce_launch(float *dy, const float *pd, const int32_t *rsrc, const float *rw,
                   uint32_t n_tok, uint32_t topk, uint32_t n_embd) {
    const dim3 grid((n_embd / 4 + 255) / 256, n_tok);
    reduce_k<<<grid, dim3(256), 0, stream()>>>(dy, pd, rsrc, rw, topk, n_embd);
    return launch_ok("reduce_k");
}

}  // namespace q4mi

using namespace q4mi;

extern "C" {

/* Per-token softmax + top-k (renormalised) over n_exp <= 512 logits,
 * topk 1..64: ids/wts [n_tok][topk] (device). */
bool q4_hip_route_pf(const float *d_rlog, int32_t *d_ids, float *d_wts, uint32_t n_tok,
                     uint32_t n_exp, uint32_t topk) {
    if (!d_rlog || !d_ids || !d_wts || !n_tok || !n_exp || n_exp > 512u || !topk ||
        topk > 64u) {
        set_error("q4_hip_route_pf: bad arguments");
        return false;
    }
    return route_launch(d_rlog, d_ids, d_wts, n_tok, n_exp, topk);
}

/* Single token, caller-owned device ids/weights.  n <= 512, k <= 64. */
bool q4_hip_softmax_topk_launch(const float *d_logits, uint32_t n, uint32_t k, int32_t *d_ids,
                                float *d_wts) {
    return q4_hip_route_pf(d_logits, d_ids, d_wts, 1, n, k);
}

/* Single token with the result copied to host arrays (synchronises). */
bool q4_hip_softmax_topk(const float *d_logits, uint32_t n, uint32_t k, int32_t *h_ids,
                         float *h_wts) {
    if (!h_ids || !h_wts || !k || k > 64) return false;
    static int32_t *d_ids = nullptr;
    static float *d_w = nullptr;
    if (!d_ids) {
        if (hipMalloc(&d_ids, 64 * sizeof(int32_t)) != hipSuccess ||
            hipMalloc(&d_w, 64 * sizeof(float)) != hipSuccess) {
            set_error("q4_hip_softmax_topk: hipMalloc failed");
            return false;
        }
    }
    if (!q4_hip_route_pf(d_logits, d_ids, d_w, 1, n, k)) return false;
    return hipMemcpyAsync(h_ids, d_ids, k * sizeof(int32_t), hipMemcpyDeviceToHost, stream()) ==
               hipSuccess &&
           hipMemcpyAsync(h_wts, d_w, k * sizeof(float), hipMemcpyDeviceToHost, stream()) ==
               hipSuccess &&
           hipStreamSynchronize(stream()) == hipSuccess;
}

/* Stable pack, per group of gsz tokens (one block each).  Same outputs as
 * the reference's q4_hip_assign_pf; rows inside an expert follow (t, k)
 * scan order.  d_bounds (optional, [n_g][n_exp+1]) = MMQ expert bounds. */
bool q4mi_assign(const int32_t *d_ids, const float *d_wts, int32_t *d_atok, int32_t *d_rsrc,
                 float *d_rw, int32_t *d_stg, uint32_t *d_stgn, uint32_t *d_ek,
                 int32_t *d_bounds, uint32_t gsz, uint32_t topk, uint32_t n_exp,
                 uint32_t n_tok) {
    if (!d_ids || !d_wts || !d_atok || !d_rsrc || !d_rw || !d_stg || !d_stgn || !d_ek ||
        !n_tok || !gsz || !topk || topk > 64u || !n_exp || n_exp > 512u) {
        set_error("q4mi_assign: bad arguments");
        return false;
    }
    return assign_launch(d_ids, d_wts, d_atok, d_rsrc, d_rw, d_stg, d_stgn, d_ek, d_bounds, gsz,
                         topk, n_exp, n_tok);
}

bool q4_hip_assign_pf(const int32_t *d_ids, const float *d_wts, int32_t *d_atok,
                      int32_t *d_rsrc, float *d_rw, int32_t *d_stg, uint32_t *d_stgn,
                      uint32_t *d_ek, uint32_t gsz, uint32_t topk, uint32_t n_exp,
                      uint32_t n_tok) {
    return q4mi_assign(d_ids, d_wts, d_atok, d_rsrc, d_rw, d_stg, d_stgn, d_ek, nullptr, gsz,
                       topk, n_exp, n_tok);
}

/* dy[tok] += sum_k rw * pd[rsrc] (deterministic; rsrc < 0 skipped). */
bool q4_hip_expert_reduce(float *d_y, const float *d_pd, const int32_t *d_rsrc,
                          const float *d_rw, uint32_t n_tok, uint32_t topk, uint32_t n_embd) {
    if (!d_y || !d_pd || !d_rsrc || !d_rw || !n_tok || !topk || (n_embd % 4) ||
        ((uintptr_t)d_y & 15) || ((uintptr_t)d_pd & 15)) {
        set_error("q4_hip_expert_reduce: bad arguments");
        return false;
    }
    return reduce_launch(d_y, d_pd, d_rsrc, d_rw, n_tok, topk, n_embd);
}

}  // extern "C"
