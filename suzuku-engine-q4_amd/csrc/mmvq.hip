// Dense decode MMVQ: y[t][r] = scale * (W_r . q8(x_t)) for 1..8 tokens over
// IQ3_S, Q8_0, IQ4_NL, Q2_0, IQ2_S or Q6_K weight rows.  C ABI: q4_mmvq_n and friends (reference
// src/q4_mmvq.cu:266-349, src/q4.h:914-927) plus q4mi_mmvq, which takes
// already-quantized activations and can export the per-group int32 sums.
#include <stdlib.h>

#include "mmvq_engine.h"
#include "q4mi_internal.h"

namespace q4mi {

// Optional build (-DQ4MI_GTRACE): thread 0 of each of the first 1024 blocks
// records wall-clock phase timestamps (10 ns ticks) of the last call.
#ifdef Q4MI_GTRACE
static __device__ unsigned long long g_gtr[1024 * 8];
#define Q4MI_GTR(k) do { if (threadIdx.x == 0 && blockIdx.x < 1024) g_gtr[blockIdx.x * 8 + (k)] = wall_clock64(); } while (0)
#else
#define Q4MI_GTR(k) do { } while (0)
#endif

bool quant8_launch(const float *x, const int32_t *ids, uint64_t rows, uint32_t cols,
                   int8_t *q, float *d, int32_t *bs);

// XF: fp32 activations xf [nt][K], quantized by every block into LDS
// behind its weight tile (the q8 codes and scales of q8_quant_k, bit for
// bit), so a call needs no separate quantize launch; else xq / xd hold them.
// (Two instantiations: the in-block quantizer's batched loads take 32
// registers, which the pre-quantized kernel does not pay for.)
template <class F, int NT, int TPR, int GPT, bool XF, int NTHR>
__global__ __launch_bounds__(NTHR) void mmvq_k(const uint8_t *__restrict__ W, uint32_t rows,
                                              uint32_t K, uint32_t rb, uint32_t R,
                                              const float *__restrict__ xf,
                                              const int8_t *__restrict__ xq,
                                              const float *__restrict__ xd, uint32_t nt,
                                              float *__restrict__ y, float scale,
                                              int32_t *__restrict__ sums) {
    extern __shared__ __align__(16) uint8_t smem[];
    void *tab = smem;
    uint8_t *tile = smem + F::kTabBytes;
    const uint32_t tid = threadIdx.x;
    const uint32_t r0 = blockIdx.x * R;
    const uint32_t nr = min(R, rows - r0);
    const uint32_t G = K / 32;
    // Tables first, then the tile's copies, then the x loads: a wave's VMEM
    // operations complete in issue order, so loads issued behind the copies
    // return when the copies have landed (measured: copies first, or copies
    // from fewer waves while the others build the table and quantize, are
    // slower for configs[0]).
    Q4MI_GTR(0);
    F::init(tab, tid, NTHR);
    Q4MI_GTR(1);
    stage_tile_issue(tile, W + (size_t)r0 * rb, nr * rb, tid, NTHR);
    Q4MI_GTR(2);
    const uint32_t hid = tid, nh = NTHR;
    const uint32_t gi = tid % TPR;
    XRegs<NT, GPT> x;
    // pre-quantized codes: loaded while the tile copy is in flight
    if constexpr (!XF) load_xregs<NT, GPT, TPR>(x, xq, xd, K, nt, gi);
    if constexpr (XF) {
        // 8 lanes per 32-value group, nh / 8 groups per pass; the loads of
        // kB passes are issued before any is used (a load issued behind the
        // tile copies returns only when they have landed, so one wait must
        // cover all of them)
        int8_t *lq = (int8_t *)(tile + ((R * rb + 15u) & ~15u));
        float *ld = (float *)(lq + (size_t)NT * K);
        // kB passes per round: one round covers a short x at any block size
        // (a larger kB is start-up code that such a call skips)
        constexpr int kB = NTHR >= 1024 ? 2 : NTHR >= 512 ? 4 : 8;
        const uint32_t ng = nt * G, step = nh / 8, sub = hid & 7u;
        for (uint32_t g0 = hid >> 3; g0 < ng; g0 += kB * step) {
            float4 v[kB];
#pragma unroll
            for (int k = 0; k < kB; k++) {
                const uint32_t gid = g0 + k * step;
                if (gid < ng) {
                    const uint32_t t = gid / G, g = gid % G;
                    v[k] = *(const float4 *)(xf + (size_t)t * K + 32u * g + 4u * sub);
                }
            }
#pragma unroll
            for (int k = 0; k < kB; k++) {
                const uint32_t gid = g0 + k * step;
                if (gid < ng) {   // uniform per 8-lane team
                    const uint32_t t = gid / G, g = gid % G;
                    float dd;
                    int bsum;
                    const uint32_t packed = q4mi_quant_team8(v[k], &dd, &bsum);
                    *(uint32_t *)(lq + (size_t)t * K + 32u * g + 4u * sub) = packed;
                    if (sub == 0) ld[gid] = dd;
                }
            }
        }
    }
    if constexpr (XF) {
        xq = (const int8_t *)(tile + ((R * rb + 15u) & ~15u));
        xd = (const float *)(xq + (size_t)NT * K);
    }
    Q4MI_GTR(3);
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    Q4MI_GTR(4);
    __syncthreads();
    Q4MI_GTR(5);
    if constexpr (XF) load_xregs<NT, GPT, TPR>(x, xq, xd, K, nt, gi);
    for (uint32_t rr = tid / TPR; rr < nr; rr += NTHR / TPR) {
        float acc[NT];
#pragma unroll
        for (int t = 0; t < NT; t++) acc[t] = 0.f;
        int32_t *srow = sums ? sums + (size_t)(r0 + rr) * G : nullptr;
        row_dot<F, NT, GPT, TPR>(tab, tile, (const uint32_t *)tile, rr * rb, gi, x, acc, srow,
                                 (size_t)rows * G);
        reduce_acc<TPR, NT>(acc);
        if (gi == TPR - 1) {
#pragma unroll
            for (int t = 0; t < NT; t++)
                if ((uint32_t)t < nt) y[(size_t)t * rows + r0 + rr] = scale * acc[t];
        }
    }
    Q4MI_GTR(6);
}

// weight bytes per row tile
static uint32_t tile_target(uint32_t ty) {
    return ty == Q4MI_T_Q8_0 || ty == Q4MI_T_Q6_K ? 24576u : 14336u;
}

template <class F, int NT>
static bool mmvq_launch_nt(const uint8_t *W, uint32_t rows, uint32_t K, const float *xf,
                           const int8_t *xq, const float *xd, uint32_t nt, float *y,
                           float scale, int32_t *sums) {
    const uint32_t G = K / 32;
    const RowLayout L = layout_for(G);
    const uint32_t rb = (uint32_t)q4mi_row_bytes(F::kType, K);
    const size_t xlds = xf ? (size_t)NT * K + (size_t)NT * (K / 32) * 4 : 0;
    auto lds_of = [&](uint32_t r) {
        return F::kTabBytes + (((size_t)r * rb + 15) & ~(size_t)15) + xlds + 64;
    };
    uint32_t nthr = 256;
    uint32_t R = L.tpr ? tile_rows(rb, L.tpr, tile_target(F::kType)) : 1;
    // fp32 x (the short matrices): a 1024-thread block per 1024 / tpr rows
    // (one row per wave) while that still fills the CUs, else 512 threads
    // per 512 / tpr rows.  The compute after a tile lands is then a quarter
    // (a half) of a 256-thread block's, whose waves take four rows each
    // (configs[0]: 256 blocks of 16 rows, 6.2 against 7.1 us).  Several
    // tokens' x registers fit 1024-thread blocks (128 VGPRs) only at one
    // token, 512-thread blocks up to two.
    if (xf && L.tpr) {
        const uint32_t cus = (uint32_t)cu_count();
        for (uint32_t n = 1024; n >= 512; n /= 2) {
            const uint32_t r = n / (uint32_t)L.tpr;
            if ((n == 1024 ? NT == 1 : NT <= 2) && (rows + r - 1) / r >= cus && lds_of(r) <= 65536) {
                nthr = n;
                R = r;
                break;
            }
        }
    }
    // pre-quantized x at one token (the tall matrices, many tiles per CU):
    // 512-thread blocks of one row per wave (configs[4] n=1: 59.8 against
    // 61.2 us, 8-row tiles either way)
    if (!xf && NT == 1 && L.tpr) {
        const uint32_t r = 512u / (uint32_t)L.tpr;
        if ((rows + r - 1) / r >= 4u * (uint32_t)cu_count() && lds_of(r) <= 65536) {
            nthr = 512;
            R = r;
        }
    }
#ifdef Q4MI_KNOBS
    if (getenv("Q4MI_GEMV_NTHR") && L.tpr && NT == 1 && xf) {
        nthr = (uint32_t)atoi(getenv("Q4MI_GEMV_NTHR"));
        R = tile_rows(rb, L.tpr, getenv("Q4MI_GEMV_TILE") ? (uint32_t)atoi(getenv("Q4MI_GEMV_TILE"))
                                                          : tile_target(F::kType), nthr);
    }
#endif
    const size_t lds = lds_of(R);
    const dim3 grid((rows + R - 1) / R), blk(nthr);
#define Q4MI_L(T, P)                                                                     \
    if (L.tpr == T && L.gpt == P) {                                                      \
        const auto args = [&](auto kern) {                                               \
            kern<<<grid, blk, lds, stream()>>>(W, rows, K, rb, R, xf, xq, xd, nt, y, scale, sums); \
        };                                                                               \
        if constexpr (NT == 1) {                                                         \
            if (xf && nthr == 1024) args(mmvq_k<F, NT, T, P, true, 1024>);              \
            else if (xf && nthr == 512) args(mmvq_k<F, NT, T, P, true, 512>);           \
            else if (xf) args(mmvq_k<F, NT, T, P, true, 256>);                          \
            else if (nthr == 512) args(mmvq_k<F, NT, T, P, false, 512>);                 \
            else args(mmvq_k<F, NT, T, P, false, 256>);                                 \
        } else if constexpr (NT == 2) {                                                  \
            if (xf && nthr == 512) args(mmvq_k<F, NT, T, P, true, 512>);                \
            else if (xf) args(mmvq_k<F, NT, T, P, true, 256>);                          \
            else args(mmvq_k<F, NT, T, P, false, 256>);                                 \
        } else {                                                                         \
            if (xf) args(mmvq_k<F, NT, T, P, true, 256>);                               \
            else args(mmvq_k<F, NT, T, P, false, 256>);                                 \
        }                                                                                \
        return launch_ok("mmvq_k");                                                      \
    }
    Q4MI_L(8, 1) Q4MI_L(16, 1) Q4MI_L(32, 1) Q4MI_L(64, 1) Q4MI_L(64, 2) Q4MI_L(64, 4)
    Q4MI_L(16, 5) Q4MI_L(4, 5)
#undef Q4MI_L
    set_error("mmvq: K=%u not covered", K);
    return false;
}

template <class F>
static bool mmvq_launch(const uint8_t *W, uint32_t rows, uint32_t K, const float *xf,
                        const int8_t *xq, const float *xd, uint32_t nt, float *y, float scale,
                        int32_t *sums) {
    if (nt == 1) return mmvq_launch_nt<F, 1>(W, rows, K, xf, xq, xd, nt, y, scale, sums);
    if (nt == 2) return mmvq_launch_nt<F, 2>(W, rows, K, xf, xq, xd, nt, y, scale, sums);
    if (nt <= 4) return mmvq_launch_nt<F, 4>(W, rows, K, xf, xq, xd, nt, y, scale, sums);
    return mmvq_launch_nt<F, 8>(W, rows, K, xf, xq, xd, nt, y, scale, sums);
}

// IQ3_S, Q8_0, IQ4_NL, Q2_0, IQ2_S, Q6_K with 8..256 groups per row (a
// whole number of blocks).
bool mmvq_covered(uint32_t ty, uint64_t K) {
    switch (ty) {
    case Q4MI_T_IQ3_S: case Q4MI_T_Q8_0: case Q4MI_T_IQ4_NL: case Q4MI_T_Q2_0:
    case Q4MI_T_IQ2_S: case Q4MI_T_Q6_K: break;
    default: return false;
    }
    if (!q4mi_row_bytes(ty, K) || K > 8192) return false;
    return layout_for((uint32_t)(K / 32)).tpr != 0;
}

// one launch for the type: pre-quantized (xq, xd) or fp32 x (xf)
static bool mmvq_any(uint32_t ty, const uint8_t *W, uint64_t rows, uint64_t K, const float *xf,
                     const int8_t *xq, const float *xd, uint32_t nt, float *y, float scale,
                     int32_t *sums) {
    const uint32_t r = (uint32_t)rows, k = (uint32_t)K;
    switch (ty) {
    case Q4MI_T_IQ3_S: return mmvq_launch<FmtIQ3S>(W, r, k, xf, xq, xd, nt, y, scale, sums);
    case Q4MI_T_Q8_0: return mmvq_launch<FmtQ80>(W, r, k, xf, xq, xd, nt, y, scale, sums);
    case Q4MI_T_IQ4_NL: return mmvq_launch<FmtIQ4NL>(W, r, k, xf, xq, xd, nt, y, scale, sums);
    case Q4MI_T_Q2_0: return mmvq_launch<FmtQ20>(W, r, k, xf, xq, xd, nt, y, scale, sums);
    case Q4MI_T_IQ2_S: return mmvq_launch<FmtIQ2S>(W, r, k, xf, xq, xd, nt, y, scale, sums);
    case Q4MI_T_Q6_K: return mmvq_launch<FmtQ6K>(W, r, k, xf, xq, xd, nt, y, scale, sums);
    }
    set_error("mmvq: type %u not covered", ty);
    return false;
}

bool mmvq_q8(uint32_t ty, const uint8_t *W, uint64_t rows, uint64_t K, const int8_t *xq,
             const float *xd, uint32_t nt, float *y, float scale, int32_t *sums) {
    return mmvq_any(ty, W, rows, K, nullptr, xq, xd, nt, y, scale, sums);
}

// Activations quantized inside the GEMV blocks: used while the codes of the
// padded token count fit 16 KB of LDS beside the tile and the call has at
// most 1024 row tiles.  Every block re-reads and re-quantizes all of x, so
// a tall matrix (config 4: 18992 tiles) is faster with one quantize launch
// (measured: 56.5 against 70.8 us at 1 token), a short one (config 0: 512
// tiles) without it (7.97 against 7.32 us).
static bool mmvq_fused_fits(uint32_t ty, uint64_t rows, uint64_t K, uint32_t nt) {
    const uint32_t ntp = nt == 1 ? 1 : nt == 2 ? 2 : nt <= 4 ? 4 : 8;
    if ((uint64_t)ntp * K > 16384) return false;
    const RowLayout L = layout_for((uint32_t)(K / 32));
    const uint32_t rb = (uint32_t)q4mi_row_bytes(ty, K);
    const uint32_t R = tile_rows(rb, L.tpr, tile_target(ty));
    return (rows + R - 1) / R <= 1024;
}

static bool mmvq_f32(uint32_t ty, const uint8_t *W, uint64_t rows, uint64_t K, const float *x,
                     uint32_t nt, float *y, float scale) {
    return mmvq_any(ty, W, rows, K, x, nullptr, nullptr, nt, y, scale, nullptr);
}

static int g_on = -1;
static const float *g_hold = nullptr;
static const float *g_cur_x = nullptr;
static uint64_t g_cur_k = 0;
static uint32_t g_cur_n = 0;

}  // namespace q4mi

using namespace q4mi;

extern "C" {

/* Q4_MMVQ=0 turns the int8 GEMV off (callers keep another path); any
 * other value or unset: on. */
int q4_mmvq_on(void) {
    if (g_on < 0) {
        const char *e = getenv("Q4_MMVQ");
        g_on = (e && e[0] == '0') ? 0 : 1;
    }
    return g_on;
}
void q4_mmvq_set(int v) { g_on = v; }
/* Kept for ABI shape: this library has no verify-only policy. */
void q4_mmvq_verify(int on) { (void)on; }

/* Allocate the activation buffers (call outside any stream capture). */
void q4_mmvq_warm(void) { (void)ensure_xq((size_t)8 * 8192); }

void q4_mmvq_hold(const float *d_x) {
    g_hold = d_x;
    g_cur_x = nullptr;
}
void q4_mmvq_release(void) {
    g_hold = nullptr;
    g_cur_x = nullptr;
}

/* y[t*nrows + r] = scale * dot(W row r, q8(x[t])), t < n (1..8).  Types:
 * IQ3_S, Q8_0; ncols a multiple of 256 (IQ3_S) / 32 (Q8_0) with
 * ncols/32 in {8,16,32,64,128,256}.  false = not covered; nothing launched. */
bool q4_mmvq_n(uint32_t ty, const uint8_t *d_w, uint64_t nrows, uint64_t ncols,
               const float *d_x, float *d_y, float scale, uint32_t n) {
    if (!q4_mmvq_on() || n < 1 || n > 8 || !d_w || !d_x || !d_y || !nrows ||
        nrows > 0x7fffffffu || !mmvq_covered(ty, ncols)) {
        set_error("q4_mmvq_n: not covered");
        return false;
    }
    if ((uintptr_t)d_x % 16 == 0 && mmvq_fused_fits(ty, nrows, ncols, n)) {
        // every block quantizes x itself: no quantize launch, no held codes
        g_cur_x = nullptr;
        return mmvq_f32(ty, d_w, nrows, ncols, d_x, n, d_y, scale);
    }
    if (!ensure_xq((size_t)8 * 8192)) return false;
    Scratch &s = lib_scratch();
    const bool reuse = g_hold && g_hold == d_x && g_cur_x == d_x && g_cur_k == ncols &&
                       g_cur_n >= n;
    if (!reuse) {
        if (!quant8_launch(d_x, nullptr, n, (uint32_t)ncols, s.xq, s.xd, nullptr))
            return false;
        g_cur_x = d_x;
        g_cur_k = ncols;
        g_cur_n = n;
    }
    return mmvq_q8(ty, d_w, nrows, ncols, s.xq, s.xd, n, d_y, scale, nullptr);
}

/* Pre-quantized variant: xq [n][ncols] int8, xd [n][ncols/32] fp32 (the
 * q4mi_quant8 layout).  d_sums (optional) receives the exact int32 group
 * sums, d_sums[(t*nrows + r)*(ncols/32) + g] = (2s+1) * sum w*q. */
bool q4mi_mmvq(uint32_t ty, const uint8_t *d_w, uint64_t nrows, uint64_t ncols,
               const int8_t *d_xq, const float *d_xd, uint32_t n, float *d_y, float scale,
               int32_t *d_sums) {
    if (n < 1 || n > 8 || !d_w || !d_xq || !d_xd || !d_y || !nrows || nrows > 0x7fffffffu ||
        !mmvq_covered(ty, ncols) || ((uintptr_t)d_xq & 15)) {
        set_error("q4mi_mmvq: not covered");
        return false;
    }
    return mmvq_q8(ty, d_w, nrows, ncols, d_xq, d_xd, n, d_y, scale, d_sums);
}

}  // extern "C"

#ifdef Q4MI_GTRACE
/* GEMV trace build only: the phase timestamps [1024 blocks][8] of the last
 * call. */
extern "C" bool q4mi_gtrace_read(unsigned long long *dst) {
    if (hipDeviceSynchronize() != hipSuccess) return false;
    return hipMemcpyFromSymbol(dst, HIP_SYMBOL(q4mi::g_gtr), sizeof(q4mi::g_gtr)) == hipSuccess;
}
#endif
