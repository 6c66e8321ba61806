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
#include <stddef.h>

#include "q4mi_common.h"
#include "q4mi_internal.h"
#include "route_wave.h"

namespace q4mi {

// One wave per token; up to 512 experts (8 per lane), k <= 64.
// Ranking uses the rounded probabilities p_i = e_i * (1/sum e) with the
// lower index winning ties, as q4_topk does (src/q4_quant.c:728-750): two
// different logits whose probabilities round to the same value (near-equal
// logits, or probabilities that underflow to 0) go to the lower index.
// Weights: p_i * (1/sum of the k picked p, in rank order).
// Output row t of ids/wts starts at t * ostride (ostride >= topk).  With
// shared >= 0 one more entry follows the topk picks: expert `shared` with
// weight sg[t] (or 1 when sg is null), and nh[t] (when given) = topk + 1
// (else topk): the per-token device lists of q4_hip_moe_exec_win /
// q4_hip_moe_exec_dev.
__global__ __launch_bounds__(256) void route_k(const float *__restrict__ logits, uint32_t n_tok,
                                               uint32_t n_exp, uint32_t topk,
                                               int32_t *__restrict__ ids,
                                               float *__restrict__ wts, uint32_t ostride,
                                               int32_t shared, const float *__restrict__ sg,
                                               int32_t *__restrict__ nh) {
    __shared__ int32_t s_id[4][64];
    __shared__ float s_p[4][64];
    const uint32_t w = threadIdx.x >> 6, lane = threadIdx.x & 63u;
    const uint32_t t = blockIdx.x * 4 + w;
    if (t >= n_tok) return;
    const uint32_t tk = route_wave<8>(logits + (size_t)t * n_exp, n_exp, topk, lane, s_id[w], s_p[w]);
    float sk = 0.f;
    for (uint32_t k = 0; k < tk; k++) sk += s_p[w][k];
    const float inv2 = sk > 0.f ? __fdiv_rn(1.f, sk) : 0.f;
    for (uint32_t k = lane; k < topk; k += 64) {
        ids[(size_t)t * ostride + k] = k < tk ? s_id[w][k] : -1;
        wts[(size_t)t * ostride + k] = k < tk ? (sk > 0.f ? s_p[w][k] * inv2 : s_p[w][k]) : 0.f;
    }
    if (lane == 0) {
        if (shared >= 0) {
            ids[(size_t)t * ostride + topk] = shared;
            wts[(size_t)t * ostride + topk] = sg ? sg[t] : 1.f;
        }
        if (nh) nh[t] = (int32_t)(topk + (shared >= 0 ? 1u : 0u));
    }
}

// ------------------------------------------------- device routing, verify
// The reference's device-side decode routing (q4_hip_route_dev_n,
// src/q4_rocm.cu:6106-6283): per token the softmax top-k of route_wave, the
// picks mapped through devtab (expert -> arena slot, < 0 = not resident),
// hits compacted into the token's device list (slots at t * 64, count in
// nh[t]), misses published through the engine's mailbox in token order.
// The mailbox layout is the reference's q4_mail_t prefix (its host mirror is
// moe_mail_t, src/q4_moe.c:368-386); seq is the last field and is bumped
// last.
struct RouteMail {
    int32_t ids[64];      // misses, token-major
    float wts[64];
    uint32_t n;           // miss count
    uint32_t ntok;
    uint32_t tn[8];       // misses of token t
    int32_t hs[8 * 16];   // token t's hit slots
    uint32_t hn[8];       // hits of token t
    uint8_t rk[64];       // each miss's rank in its token's top-k
    int32_t routed[16];   // token 0's top-k (profile channel)
    unsigned long long rseq;
    unsigned long long seq;
};
static_assert(offsetof(RouteMail, n) == 512 && offsetof(RouteMail, hs) == 552 &&
                  offsetof(RouteMail, rk) == 1096 && offsetof(RouteMail, routed) == 1160 &&
                  offsetof(RouteMail, rseq) == 1224 && offsetof(RouteMail, seq) == 1232,
              "mailbox layout of the reference engine");

template <int NJ>
__global__ __launch_bounds__(512) void route_dev_n_k(
    const float *__restrict__ rlog, const int32_t *__restrict__ devtab, int32_t *__restrict__ es,
    float *__restrict__ ew, int32_t *__restrict__ nh, RouteMail *__restrict__ mail,
    unsigned long long *seq, unsigned long long *rseq, unsigned long long *prof,
    uint32_t n_exp, uint32_t topk, uint32_t n_tok) {
    __shared__ int32_t s_id[8][64];
    __shared__ float s_p[8][64];
    __shared__ int32_t s_mid[8][16];
    __shared__ float s_mwt[8][16];
    __shared__ uint32_t s_mrk[8][16];
    __shared__ uint32_t s_tn[8];
    const unsigned long long t0 = wall_clock64();
    const uint32_t t = threadIdx.x >> 6, lane = threadIdx.x & 63u;
    if (t < n_tok) {
        const uint32_t tk = route_wave<NJ>(rlog + (size_t)t * n_exp, n_exp, topk, lane, s_id[t], s_p[t]);
        const float inv = route_inv_sum(s_p[t], tk);
        const bool pick = lane < tk;
        const int32_t id = pick ? s_id[t][lane] : -1;
        const float wq = pick ? s_p[t][lane] * inv : 0.f;
        const int32_t slot = id >= 0 ? devtab[id] : -1;
        const uint64_t hitm = __ballot(pick && slot >= 0), missm = __ballot(pick && slot < 0);
        const uint64_t below = (1ull << lane) - 1ull;
        const uint32_t hr = (uint32_t)__popcll(hitm & below), mr = (uint32_t)__popcll(missm & below);
        if (pick && slot >= 0) {
            es[(size_t)t * 64 + hr] = slot;
            ew[(size_t)t * 64 + hr] = wq;
            mail->hs[t * 16 + hr] = slot;
        } else if (pick) {
            s_mid[t][mr] = id;
            s_mwt[t][mr] = wq;
            s_mrk[t][mr] = lane;
        }
        if (t == 0 && rseq && lane < 16) mail->routed[lane] = pick ? id : 0;
        if (lane == 0) {
            nh[t] = (int32_t)__popcll(hitm);
            s_tn[t] = (uint32_t)__popcll(missm);
            mail->hn[t] = (uint32_t)__popcll(hitm);
        }
    }
    __syncthreads();
    if (t != 0) return;
    uint32_t nm = 0;
    for (uint32_t u = 0; u < n_tok; u++) {
        const uint32_t c = s_tn[u];
        if (lane < c) {
            mail->ids[nm + lane] = s_mid[u][lane];
            mail->wts[nm + lane] = s_mwt[u][lane];
            mail->rk[nm + lane] = (uint8_t)s_mrk[u][lane];
        }
        nm += c;
    }
    if (lane < 8) {
        mail->tn[lane] = lane < n_tok ? s_tn[lane] : 0u;
        if (lane >= n_tok) mail->hn[lane] = 0u;
    }
    if (lane == 0) {
        mail->ntok = n_tok;
        mail->n = nm;
        if (rseq) mail->rseq = ++(*rseq);
        // the engine reads the mailbox through a copy ordered after this
        // kernel on the stream, so the kernel's end makes every field
        // visible before seq is seen
        mail->seq = ++(*seq);
        if (prof) {
            prof[0] += wall_clock64() - t0;
            prof[1] += 1;
        }
    }
}

// ----------------------------------------------------------------- pack
// Stable counting sort of a token group's (token, pick) rows by expert, in
// two launches over 512-row chunks so that every chunk has its own block:
//   pack_hist_k   per chunk: rows per expert -> hist[g][chunk][e]
//   pack_place_k  per chunk: the expert's first position (its exclusive
//                 prefix over experts + the counts of earlier chunks), then
//                 each row's rank among the chunk's earlier rows of the same
//                 expert (wave ballots on the expert id bits, then the
//                 counts of earlier waves).  Rows keep their (t, k) order
//                 inside an expert: the host pack's order, bit for bit.
constexpr uint32_t kPackCh = 512;

__global__ __launch_bounds__(512) void pack_hist_k(const int32_t *__restrict__ ids,
                                                   uint32_t *__restrict__ hist, uint32_t gsz,
                                                   uint32_t topk, uint32_t n_exp, uint32_t n_tok,
                                                   uint32_t nch) {
    __shared__ uint32_t h[512];
    const uint32_t c = blockIdx.x, g = blockIdx.y, tid = threadIdx.x;
    h[tid] = 0;
    __syncthreads();
    const uint32_t t0 = g * gsz, t1 = min(t0 + gsz, n_tok);
    const uint32_t rows = (t1 - t0) * topk;
    const uint32_t i = c * kPackCh + tid;
    if (i < rows) {
        const int32_t e = ids[(size_t)t0 * topk + i];
        if (e >= 0 && (uint32_t)e < n_exp) atomicAdd(&h[e], 1u);
    }
    __syncthreads();
    hist[((size_t)g * nch + c) * 512 + tid] = h[tid];
}

// Inclusive sum over the block's 512 threads (one value each).
__device__ inline uint32_t scan512(uint32_t v, uint32_t *tmp, uint32_t tid) {
    tmp[tid] = v;
    __syncthreads();
    for (uint32_t o = 1; o < 512; o <<= 1) {
        const uint32_t u = tid >= o ? tmp[tid - o] : 0u;
        __syncthreads();
        tmp[tid] += u;
        __syncthreads();
    }
    const uint32_t r = tmp[tid];
    __syncthreads();
    return r;
}

__global__ __launch_bounds__(512) void pack_place_k(
    const int32_t *__restrict__ ids, const float *__restrict__ wts, int32_t *__restrict__ a_tok,
    int32_t *__restrict__ rsrc, float *__restrict__ rw, int32_t *__restrict__ stg,
    uint32_t *__restrict__ stgn, uint32_t *__restrict__ ek, int32_t *__restrict__ bounds,
    const uint32_t *__restrict__ hist, uint32_t gsz, uint32_t topk, uint32_t n_exp,
    uint32_t n_tok, uint32_t nch) {
    __shared__ uint32_t s_base[512];
    __shared__ uint32_t s_tmp[512];
    __shared__ uint16_t s_wc[8][512];
    const uint32_t c = blockIdx.x, g = blockIdx.y, tid = threadIdx.x;
    const uint32_t wv = tid >> 6, lane = tid & 63u;
    const uint32_t t0 = g * gsz, t1 = min(t0 + gsz, n_tok);
    const uint32_t rows = (t1 - t0) * topk;
    const size_t seg = (size_t)g * gsz * topk;
    // expert tid: rows in the whole group and in the chunks before this one
    uint32_t tot = 0, before = 0;
    const uint32_t *hg = hist + (size_t)g * nch * 512 + tid;
    for (uint32_t c0 = 0; c0 < nch; c0 += 8) {   // eight loads in flight at a time
        uint32_t v[8];
#pragma unroll
        for (uint32_t k = 0; k < 8; k++) v[k] = c0 + k < nch ? hg[(size_t)(c0 + k) * 512] : 0u;
#pragma unroll
        for (uint32_t k = 0; k < 8; k++) {
            tot += v[k];
            before += c0 + k < c ? v[k] : 0u;
        }
    }
    for (uint32_t k = tid; k < 8 * 512; k += 512) (&s_wc[0][0])[k] = 0;
    const uint32_t incl = scan512(tot, s_tmp, tid);
    const uint32_t ebase = incl - tot;
    s_base[tid] = ebase + before;
    if (c == 0) {   // group-level outputs, once
        if (bounds) {
            if (tid < n_exp) bounds[(size_t)g * (n_exp + 1) + tid] = (int32_t)ebase;
            if (tid == n_exp - 1) bounds[(size_t)g * (n_exp + 1) + n_exp] = (int32_t)incl;
        }
        ek[(size_t)g * 512 + tid] = tid < n_exp ? tot : 0u;
    }
    // used experts in ascending order
    const uint32_t used = (tid < n_exp && tot) ? 1u : 0u;
    const uint32_t uincl = scan512(used, s_tmp, tid);
    if (c == 0) {
        if (used) stg[(size_t)g * 512 + uincl - 1] = (int32_t)tid;
        if (tid == 511) stgn[g] = uincl;
    }
    // this chunk's rows, one per thread
    const uint32_t i = c * kPackCh + tid;
    const bool in = i < rows;
    const int32_t e = in ? ids[(size_t)t0 * topk + i] : -1;
    const bool valid = in && e >= 0 && (uint32_t)e < n_exp;
    uint64_t same = __ballot(valid);
#pragma unroll
    for (int b = 0; b < 9; b++) {
        const bool bit = valid && ((e >> b) & 1);
        const uint64_t m = __ballot(bit);
        same &= bit ? m : ~m;
    }
    if (!valid) same = 0;
    const uint32_t rank = (uint32_t)__popcll(same & ((1ull << lane) - 1ull));
    if (valid && rank == 0) s_wc[wv][e] = (uint16_t)__popcll(same);
    __syncthreads();
    if (valid) {
        uint32_t p = s_base[e] + rank;
        for (uint32_t w2 = 0; w2 < wv; w2++) p += s_wc[w2][e];
        const uint32_t t = t0 + i / topk;
        a_tok[seg + p] = (int32_t)t;
        rsrc[(size_t)t0 * topk + i] = (int32_t)p;
        rw[(size_t)t0 * topk + i] = wts[(size_t)t0 * topk + i];
    } else if (in) {
        rsrc[(size_t)t0 * topk + i] = -1;
        rw[(size_t)t0 * topk + i] = 0.f;
    }
}

// dy[t][i] += sum_k rw[t*topk+k] * pd[rsrc[t*topk+k]][i], k in order.
__global__ __launch_bounds__(256) void reduce_k(float *__restrict__ dy,
                                                const float *__restrict__ pd,
                                                const int32_t *__restrict__ rsrc,
                                                const float *__restrict__ rw, uint32_t topk,
                                                uint32_t n_embd, int64_t x_row0,
                                                const float *__restrict__ xw) {
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
    if (x_row0 >= 0) {   // one more expert row per token: pd[x_row0 + t], weight xw[t] or 1
        const float w = xw ? xw[t] : 1.f;
        const float4 v = *(const float4 *)(pd + (size_t)(x_row0 + t) * n_embd + i);
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
                                                              wts, topk, -1, nullptr, nullptr);
    return launch_ok("route_k");
}

bool route_dev_n_launch(const float *rlog, const int32_t *devtab, int32_t *es, float *ew,
                        int32_t *nh, void *mail, unsigned long long *seq, unsigned long long *rseq,
                        unsigned long long *prof, uint32_t n_exp, uint32_t topk, uint32_t n_tok) {
    RouteMail *m = (RouteMail *)mail;
    if (n_exp <= 512)
        route_dev_n_k<8><<<dim3(1), dim3(64 * n_tok), 0, stream()>>>(rlog, devtab, es, ew, nh, m,
                                                                  seq, rseq, prof, n_exp, topk,
                                                                  n_tok);
    else
        route_dev_n_k<16><<<dim3(1), dim3(64 * n_tok), 0, stream()>>>(rlog, devtab, es, ew, nh, m,
                                                                   seq, rseq, prof, n_exp, topk,
                                                                   n_tok);
    return launch_ok("route_dev_n_k");
}

bool route_list_launch(const float *lg, int32_t *ids, float *wts, int32_t *nh, uint32_t n_tok,
                       uint32_t n_exp, uint32_t topk, uint32_t ostride, int32_t shared,
                       const float *sg) {
    route_k<<<dim3((n_tok + 3) / 4), dim3(256), 0, stream()>>>(lg, n_tok, n_exp, topk, ids,
                                                              wts, ostride, shared, sg, nh);
    return launch_ok("route_k");
}

// per-chunk expert histograms of the pack (library scratch; grown on demand,
// so a caller that captures graphs runs one pack of its largest size first)
static uint32_t *g_hist = nullptr;
static size_t g_hist_words = 0;

bool assign_launch(const int32_t *ids, const float *wts, int32_t *a_tok, int32_t *rsrc,
                   float *rw, int32_t *stg, uint32_t *stgn, uint32_t *ek, int32_t *bounds,
                   uint32_t gsz, uint32_t topk, uint32_t n_exp, uint32_t n_tok) {
    const uint32_t n_g = (n_tok + gsz - 1) / gsz;
    const uint32_t nch = (gsz * topk + kPackCh - 1) / kPackCh;
    const size_t words = (size_t)n_g * nch * 512;
    if (g_hist_words < words) {
        if (!scratch_grow((void **)&g_hist, words * 4, "pack histograms")) return false;
        g_hist_words = words;
    }
    pack_hist_k<<<dim3(nch, n_g), dim3(512), 0, stream()>>>(ids, g_hist, gsz, topk, n_exp, n_tok,
                                                           nch);
    if (!launch_ok("pack_hist_k")) return false;
    pack_place_k<<<dim3(nch, n_g), dim3(512), 0, stream()>>>(ids, wts, a_tok, rsrc, rw, stg, stgn,
                                                            ek, bounds, g_hist, gsz, topk, n_exp,
                                                            n_tok, nch);
    return launch_ok("pack_place_k");
}

bool reduce_launch(float *dy, const float *pd, const int32_t *rsrc, const float *rw,
                   uint32_t n_tok, uint32_t topk, uint32_t n_embd, int64_t x_row0 = -1,
                   const float *xw = nullptr) {
    const dim3 grid((n_embd / 4 + 255) / 256, n_tok);
    reduce_k<<<grid, dim3(256), 0, stream()>>>(dy, pd, rsrc, rw, topk, n_embd, x_row0, xw);
    return launch_ok("reduce_k");
}

}  // namespace q4mi

using namespace q4mi;

extern "C" {

/* Per-token softmax + top-k (renormalised) over n_exp <= 512 logits,
 * topk 1..64: ids/wts [n_tok][topk] (device). */
/* Device routing of a decode or verify batch (reference signature,
 * src/q4.h:1289-1294): per token the softmax top-k of d_rlog[t][n_exp]
 * (bit-exact with q4_hip_route_pf), picks mapped through devtab; hits go to
 * d_es/d_ew at t*64 (count d_nh[t]), misses to the mailbox, whose seq (and
 * rseq when d_rseq is given) is bumped from the device counters.  All
 * experts resident (devtab[e] >= 0 for every e) leaves the miss list empty.
 * false (nothing launched): a null argument, n_exp > 1024, n_tok outside
 * 1..8, topk outside 1..16 or n_tok * topk > 64. */
bool q4_hip_route_dev_n(const float *d_rlog, const int32_t *devtab, int32_t *d_es, float *d_ew,
                        int32_t *d_nh, void *mail, unsigned long long *d_seq,
                        unsigned long long *d_rseq, unsigned long long *d_prof,
                        uint32_t n_exp, uint32_t topk, uint32_t n_tok) {
    if (!d_rlog || !devtab || !d_es || !d_ew || !d_nh || !mail || !d_seq || !n_exp ||
        n_exp > 1024 || !n_tok || n_tok > 8 || !topk || topk > 16 || n_tok * topk > 64) {
        set_error("q4_hip_route_dev_n: bad arguments");
        return false;
    }
    return route_dev_n_launch(d_rlog, devtab, d_es, d_ew, d_nh, mail, d_seq, d_rseq, d_prof,
                              n_exp, topk, n_tok);
}

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
        if (!lib_malloc((void **)&d_ids, 64 * sizeof(int32_t)) ||
            !lib_malloc((void **)&d_w, 64 * sizeof(float))) {
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

/* q4_hip_expert_reduce plus one more expert row per token:
 * dy[t] += sum_k rw * pd[rsrc] + xw[t] * pd[x_row0 + t] (xw NULL: weight 1).
 * The extra rows are a shared expert's outputs appended after the routed
 * rows (the _x MMQ entry points). */
bool q4mi_expert_reduce_x(float *d_y, const float *d_pd, const int32_t *d_rsrc,
                          const float *d_rw, uint32_t n_tok, uint32_t topk, uint32_t n_embd,
                          uint64_t x_row0, const float *d_xw) {
    if (!d_y || !d_pd || !d_rsrc || !d_rw || !n_tok || !topk || (n_embd % 4) ||
        ((uintptr_t)d_y & 15) || ((uintptr_t)d_pd & 15) || x_row0 > (1ull << 40)) {
        set_error("q4mi_expert_reduce_x: bad arguments");
        return false;
    }
    return reduce_launch(d_y, d_pd, d_rsrc, d_rw, n_tok, topk, n_embd, (int64_t)x_row0, d_xw);
}

}  // extern "C"
