// Routed-expert decode (1 token) and verify window (2..8 tokens) over
// IQ3_S / Q8_0 experts resident at base + slot*stride.
//
// Two launches per layer:
//   moe_gu_k   block = (row tile, unique expert u): q8(x_t) in LDS, gate and
//              up rows of the tile, h[u][t][r] = silu(g)*up for every token.
//   moe_dn_k   block = (row tile, u): q8(h[u][t]) in LDS, down rows, weighted
//              partials pd[u][t][r]; the last block of each row tile (an
//              agent-scope ticket) adds sum_u pd[u][t][r] into y[t][r] in
//              unique-expert order, so y is deterministic run to run.
// Each unique expert's rows are read once per launch and dotted with every
// token that selected it (the verify window's reuse; reference
// q4_hip_moe_exec_win src/q4_rocm.cu:7444-7531, CPU twin
// q4_cpuex_dispatch_win src/q4_cpuexp.c:2618-2753).
//
// The unique-expert plan (first-appearance order over (token, pick), token
// bitmask, per-token weights) is rebuilt by wave 0 of every block from the
// caller's lists, which may live in device memory (graph-capturable).
#include <stdlib.h>

#include "mmvq_engine.h"
#include "q4mi_internal.h"

namespace q4mi {

constexpr uint32_t kMaxU = 64;   // unique experts per call (reference bound n<=64)
constexpr uint32_t kMaxT = 8;    // tokens per call

struct HostList {
    int32_t id[kMaxU];
    float w[kMaxU];
};

struct ListSrc {
    const int32_t *es;   // device ids (null: use the HostList argument)
    const float *ew;     // device weights
    const int32_t *nh;   // device per-token counts (null: n_fixed)
    uint32_t stride;     // entries between tokens in es/ew
    uint32_t n_tok;
    uint32_t n_fixed;    // count per token when nh is null / host list length
};

struct __align__(16) Plan {
    uint32_t nu;
    int32_t uid[kMaxU];
    uint32_t sel[kMaxU];
    float w[kMaxU][kMaxT];
};

// Wave 0 builds the plan; callers sync afterwards.
__device__ void build_plan(Plan *P, const ListSrc &s, const HostList &hl, uint32_t lane) {
    // flatten (t, i) entries in token order into lanes 0..E-1
    uint32_t cnt[kMaxT];
    uint32_t E = 0;
    for (uint32_t t = 0; t < s.n_tok; t++) {
        int c = s.nh ? s.nh[t] : (int)s.n_fixed;
        if (c < 0) c = 0;
        if ((uint32_t)c > s.stride) c = (int)s.stride;
        cnt[t] = (uint32_t)c;
        E += (uint32_t)c;
    }
    if (E > kMaxU) E = kMaxU;
    int32_t id = -1;
    float w = 0.f;
    uint32_t tok = 0;
    if (lane < E) {
        uint32_t rem = lane, t = 0;
        while (rem >= cnt[t]) rem -= cnt[t++];
        tok = t;
        if (s.es) {
            id = s.es[(size_t)t * s.stride + rem];
            w = s.ew[(size_t)t * s.stride + rem];
        } else {
            id = hl.id[rem];
            w = hl.w[rem];
        }
    }
    const bool valid = lane < E && id >= 0;
    // first occurrence of each id among valid entries
    uint32_t first_j = lane;
    for (uint32_t j = 0; j < E; j++) {
        const int32_t idj = __shfl(id, j);
        const bool vj = __shfl((int)valid, j) != 0;
        if (vj && idj == id && j < first_j) first_j = j;
    }
    const bool first = valid && first_j == lane;
    const uint64_t fm = __ballot(first);
    const uint32_t u = (uint32_t)__popcll(fm & ((1ull << first_j) - 1ull));
    // clear, then fill
    for (uint32_t i = lane; i < kMaxU; i += 64) {
        P->sel[i] = 0;
#pragma unroll
        for (uint32_t t = 0; t < kMaxT; t++) P->w[i][t] = 0.f;
    }
    if (lane == 0) P->nu = (uint32_t)__popcll(fm);
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup");
    if (first) P->uid[u] = id;
    if (valid) {
        atomicOr(&P->sel[u], 1u << tok);
        P->w[u][tok] = w;
    }
}

// q8 of nt rows of K floats (global) into LDS q[nt][K], d[nt][K/32];
// rows nt..NT-1 untouched.  All 256 threads take part.
__device__ inline void quant_rows_lds(const float *src, size_t src_stride, uint32_t nt,
                                      uint32_t K, int8_t *q, float *d, uint32_t tid) {
    const uint32_t quads = nt * (K / 4);
    for (uint32_t i = tid; i < quads; i += 256) {
        const uint32_t t = i / (K / 4), c = (i % (K / 4)) * 4;
        const float4 v = *(const float4 *)(src + (size_t)t * src_stride + c);
        float dd;
        int bs;
        const uint32_t p = q4mi_quant_team8(v, &dd, &bs);
        *(uint32_t *)(q + (size_t)t * K + c) = p;
        if ((i & 7u) == 0) d[(size_t)t * (K / 32) + c / 32] = dd;
    }
}

struct MoeArgs {
    const uint8_t *base;
    uint64_t stride, og, ou, od;
    uint32_t K;      // in_dim (gate/up columns)
    uint32_t n_ff;
    uint32_t n_embd;
    uint32_t rb_gu, rb_dn;
    uint32_t R;      // rows per block tile
    const float *x;  // [n_tok][K]
    float *h;        // [kMaxU][kMaxT][n_ff]
    float *pd;       // [kMaxU][kMaxT][n_embd]
    float *y;        // [n_tok][n_embd], accumulated
    uint32_t *tickets;
    ListSrc src;
};

__device__ inline float silu_f(float v) { return v / (1.f + expf(-v)); }

template <class F, int NT, int TPR, int GPT>
__global__ __launch_bounds__(256) void moe_gu_k(MoeArgs a, HostList hl) {
    extern __shared__ __align__(16) uint8_t smem[];
    Iq3sLds *tab = (Iq3sLds *)smem;
    Plan *P = (Plan *)(smem + sizeof(Iq3sLds));
    int8_t *xq = (int8_t *)(smem + sizeof(Iq3sLds) + sizeof(Plan));
    float *xd = (float *)(xq + NT * a.K);
    uint8_t *tile = (uint8_t *)(xd + NT * (a.K / 32));
    const uint32_t tid = threadIdx.x, u = blockIdx.y;
    if (tid < 64) build_plan(P, a.src, hl, tid);
    __syncthreads();
    if (u >= P->nu) return;
    const uint32_t r0 = blockIdx.x * a.R;
    const uint32_t nr = min(a.R, a.n_ff - r0);
    const uint8_t *pe = a.base + (uint64_t)P->uid[u] * a.stride;
    if (F::kTables) q4mi_iq3s_tables_init(tab, tid, 256);
    stage_tile(tile, pe + a.og + (size_t)r0 * a.rb_gu, nr * a.rb_gu, tid, 256);
    stage_tile(tile + a.R * a.rb_gu, pe + a.ou + (size_t)r0 * a.rb_gu, nr * a.rb_gu, tid, 256);
    const uint32_t nt = a.src.n_tok;
    quant_rows_lds(a.x, a.K, nt, a.K, xq, xd, tid);
    __syncthreads();
    const uint32_t gi = tid % TPR;
    XRegs<NT, GPT> x;
    load_xregs<NT, GPT, TPR>(x, xq, xd, a.K, nt, gi);
    const uint32_t *tw = (const uint32_t *)tile;
    for (uint32_t rr = tid / TPR; rr < nr; rr += 256 / TPR) {
        float ag[NT], au[NT];
#pragma unroll
        for (int t = 0; t < NT; t++) ag[t] = au[t] = 0.f;
        row_dot<F, NT, GPT, TPR>(tab, tile, tw, rr * a.rb_gu, gi, x, ag, nullptr, 0);
        row_dot<F, NT, GPT, TPR>(tab, tile, tw, (a.R + rr) * a.rb_gu, gi, x, au, nullptr, 0);
        reduce_acc<TPR, NT>(ag);
        reduce_acc<TPR, NT>(au);
        if (gi == 0) {
#pragma unroll
            for (int t = 0; t < NT; t++)
                if ((uint32_t)t < nt)
                    a.h[((size_t)u * kMaxT + t) * a.n_ff + r0 + rr] = silu_f(ag[t]) * au[t];
        }
    }
}

template <class F, int NT, int TPR, int GPT>
__global__ __launch_bounds__(256) void moe_dn_k(MoeArgs a, HostList hl) {
    extern __shared__ __align__(16) uint8_t smem[];
    Iq3sLds *tab = (Iq3sLds *)smem;
    Plan *P = (Plan *)(smem + sizeof(Iq3sLds));
    int8_t *hq = (int8_t *)(smem + sizeof(Iq3sLds) + sizeof(Plan));
    float *hd = (float *)(hq + NT * a.n_ff);
    uint8_t *tile = (uint8_t *)(hd + NT * (a.n_ff / 32));
    __shared__ uint32_t s_last;
    const uint32_t tid = threadIdx.x, u = blockIdx.y;
    if (tid < 64) build_plan(P, a.src, hl, tid);
    __syncthreads();
    const uint32_t nu = P->nu;
    if (u >= nu) return;
    const uint32_t r0 = blockIdx.x * a.R;
    const uint32_t nr = min(a.R, a.n_embd - r0);
    const uint8_t *pe = a.base + (uint64_t)P->uid[u] * a.stride;
    if (F::kTables) q4mi_iq3s_tables_init(tab, tid, 256);
    stage_tile(tile, pe + a.od + (size_t)r0 * a.rb_dn, nr * a.rb_dn, tid, 256);
    const uint32_t nt = a.src.n_tok;
    quant_rows_lds(a.h + (size_t)u * kMaxT * a.n_ff, a.n_ff, nt, a.n_ff, hq, hd, tid);
    __syncthreads();
    const uint32_t gi = tid % TPR;
    XRegs<NT, GPT> x;
    load_xregs<NT, GPT, TPR>(x, hq, hd, a.n_ff, nt, gi);
    const uint32_t sel = P->sel[u];
    for (uint32_t rr = tid / TPR; rr < nr; rr += 256 / TPR) {
        float acc[NT];
#pragma unroll
        for (int t = 0; t < NT; t++) acc[t] = 0.f;
        row_dot<F, NT, GPT, TPR>(tab, tile, (const uint32_t *)tile, rr * a.rb_dn, gi, x, acc,
                                 nullptr, 0);
        reduce_acc<TPR, NT>(acc);
        if (gi == 0) {
#pragma unroll
            for (int t = 0; t < NT; t++)
                if ((uint32_t)t < nt)
                    a.pd[((size_t)u * kMaxT + t) * a.n_embd + r0 + rr] =
                        ((sel >> t) & 1u) ? P->w[u][t] * acc[t] : 0.f;
        }
    }
    // ticket: the last of the nu blocks of this row tile reduces it
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "agent");
    __syncthreads();
    if (tid == 0) {
        const uint32_t old = __hip_atomic_fetch_add(&a.tickets[blockIdx.x], 1u,
                                                    __ATOMIC_ACQ_REL, __HIP_MEMORY_SCOPE_AGENT);
        s_last = (old == nu - 1) ? 1u : 0u;
    }
    __syncthreads();
    if (!s_last) return;
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "agent");
    for (uint32_t i = tid; i < nr * nt; i += 256) {
        const uint32_t t = i / nr, r = r0 + i % nr;
        float s = 0.f;
        for (uint32_t uu = 0; uu < nu; uu++)
            s += a.pd[((size_t)uu * kMaxT + t) * a.n_embd + r];
        a.y[(size_t)t * a.n_embd + r] += s;
    }
    if (tid == 0)
        __hip_atomic_store(&a.tickets[blockIdx.x], 0u, __ATOMIC_RELAXED,
                           __HIP_MEMORY_SCOPE_AGENT);
}

template <class F, int NT, int TPR, int GPT>
static bool launch_gu(const MoeArgs &a, const HostList &hl, uint32_t grid_u) {
    const size_t lds = sizeof(Iq3sLds) + sizeof(Plan) + (size_t)NT * a.K +
                       (size_t)NT * (a.K / 32) * 4 + 2ull * a.R * a.rb_gu + 64;
    if (lds > 65536) {
        set_error("moe_gu_k: %zu bytes of LDS exceeds 64 KiB", lds);
        return false;
    }
    const dim3 grid((a.n_ff + a.R - 1) / a.R, grid_u);
    moe_gu_k<F, NT, TPR, GPT><<<grid, dim3(256), lds, stream()>>>(a, hl);
    return launch_ok("moe_gu_k");
}

template <class F, int NT, int TPR, int GPT>
static bool launch_dn(const MoeArgs &a, const HostList &hl, uint32_t grid_u) {
    const size_t lds = sizeof(Iq3sLds) + sizeof(Plan) + (size_t)NT * a.n_ff +
                       (size_t)NT * (a.n_ff / 32) * 4 + (size_t)a.R * a.rb_dn + 64;
    if (lds > 65536) {
        set_error("moe_dn_k: %zu bytes of LDS exceeds 64 KiB", lds);
        return false;
    }
    const dim3 grid((a.n_embd + a.R - 1) / a.R, grid_u);
    moe_dn_k<F, NT, TPR, GPT><<<grid, dim3(256), lds, stream()>>>(a, hl);
    return launch_ok("moe_dn_k");
}

template <class F, int NT>
static bool gu_dispatch(MoeArgs a, const HostList &hl, uint32_t grid_u) {
    const RowLayout L = layout_for(a.K / 32);
    a.R = tile_rows(a.rb_gu, L.tpr, 7168u);
#define Q4MI_L(T, P) \
    if (L.tpr == T && L.gpt == P) return launch_gu<F, NT, T, P>(a, hl, grid_u);
    Q4MI_L(8, 1) Q4MI_L(16, 1) Q4MI_L(32, 1) Q4MI_L(64, 1) Q4MI_L(64, 2) Q4MI_L(64, 4)
#undef Q4MI_L
    return false;
}

template <class F, int NT>
static bool dn_dispatch(MoeArgs a, const HostList &hl, uint32_t grid_u) {
    const RowLayout L = layout_for(a.n_ff / 32);
    a.R = tile_rows(a.rb_dn, L.tpr, 14336u);
#define Q4MI_L(T, P) \
    if (L.tpr == T && L.gpt == P) return launch_dn<F, NT, T, P>(a, hl, grid_u);
    Q4MI_L(8, 1) Q4MI_L(16, 1) Q4MI_L(32, 1) Q4MI_L(64, 1) Q4MI_L(64, 2) Q4MI_L(64, 4)
#undef Q4MI_L
    return false;
}

// Measurement hook: bit 0 runs the gate/up launch, bit 1 the down launch
// (default both).  Lets a benchmark time each kernel of the pair alone.
static int g_phases = 3;

template <int NT>
static bool run_nt(uint32_t ty_gu, uint32_t ty_dn, MoeArgs a, const HostList &hl,
                   uint32_t grid_u) {
    if (g_phases & 1) {
        const bool ok = ty_gu == Q4MI_T_IQ3_S ? gu_dispatch<FmtIQ3S, NT>(a, hl, grid_u)
                                              : gu_dispatch<FmtQ80, NT>(a, hl, grid_u);
        if (!ok) return false;
    }
    if (!(g_phases & 2)) return true;
    return ty_dn == Q4MI_T_IQ3_S ? dn_dispatch<FmtIQ3S, NT>(a, hl, grid_u)
                                 : dn_dispatch<FmtQ80, NT>(a, hl, grid_u);
}

static bool type_ok(uint32_t ty, uint32_t K) {
    if (ty != Q4MI_T_IQ3_S && ty != Q4MI_T_Q8_0) return false;
    if (!q4mi_row_bytes(ty, K) || K > 8192) return false;
    return layout_for(K / 32).tpr != 0;
}

static bool shape_ok(uint32_t gt, uint32_t ut, uint32_t dt, uint32_t in_dim, uint32_t n_ff,
                     uint32_t n_embd) {
    return gt == ut && type_ok(gt, in_dim) && type_ok(dt, n_ff) && n_embd == in_dim;
}

bool moe_warm(uint32_t n_ff, uint32_t n_embd) {
    if (!ensure_pd((size_t)kMaxU * kMaxT * ((size_t)n_ff + n_embd))) return false;
    return ensure_tickets(n_embd);  // >= row tiles of any layout
}

// Common driver.  All checks happen before the first launch so that a false
// return never leaves half of the work queued.
static bool moe_run(const uint8_t *base, uint64_t stride, const ListSrc &src,
                    const HostList &hl, uint32_t grid_u, uint32_t gt, uint64_t og, uint32_t ut,
                    uint64_t ou, uint32_t dt, uint64_t od, const float *d_x, float *d_y,
                    uint32_t n_ff, uint32_t in_dim, uint32_t n_embd) {
    if (!base || !d_x || !d_y || !grid_u || src.n_tok < 1 || src.n_tok > kMaxT) {
        set_error("moe: bad arguments");
        return false;
    }
    if (!shape_ok(gt, ut, dt, in_dim, n_ff, n_embd)) {
        set_error("moe: types/shape not covered (gt=%u ut=%u dt=%u in=%u ff=%u)", gt, ut, dt,
                  in_dim, n_ff);
        return false;
    }
    if (((uintptr_t)d_x & 15) || (in_dim % 4)) {
        set_error("moe: x must be 16-byte aligned");
        return false;
    }
    if (!moe_warm(n_ff, n_embd)) return false;
    Scratch &s = scratch();
    MoeArgs a;
    a.base = base;
    a.stride = stride;
    a.og = og;
    a.ou = ou;
    a.od = od;
    a.K = in_dim;
    a.n_ff = n_ff;
    a.n_embd = n_embd;
    a.rb_gu = (uint32_t)q4mi_row_bytes(gt, in_dim);
    a.rb_dn = (uint32_t)q4mi_row_bytes(dt, n_ff);
    a.R = 0;
    a.x = d_x;
    a.h = s.pd;
    a.pd = s.pd + (size_t)kMaxU * kMaxT * n_ff;
    a.y = d_y;
    a.tickets = s.tickets;
    a.src = src;
    const uint32_t nt = src.n_tok;
    if (nt == 1) return run_nt<1>(gt, dt, a, hl, grid_u);
    if (nt == 2) return run_nt<2>(gt, dt, a, hl, grid_u);
    if (nt <= 4) return run_nt<4>(gt, dt, a, hl, grid_u);
    return run_nt<8>(gt, dt, a, hl, grid_u);
}

}  // namespace q4mi

using namespace q4mi;

extern "C" void q4_mmvq_warm(void);

extern "C" {

/* Benchmark hook: 1 = gate/up launch only, 2 = down only, 3 = both. */
void q4mi_moe_phases(int mask) { g_phases = mask & 3; }

/* Allocate the decode scratch (call before any stream capture). */
void q4_hip_moe_scratch_warm(void) {
    (void)moe_warm(2048, 8192);
    q4_mmvq_warm();
}

/* One token, n (<=64) experts given as HOST arrays: slot ids (expert index
 * into the arena) and routing weights.  d_y += sum_e wts[e] * FFN_e(x).
 * d_h, d_h2, d_down are accepted for ABI compatibility with the reference
 * (src/q4.h:951-956) and not used: intermediates live in library scratch. */
bool q4_hip_moe_exec(const uint8_t *base, uint64_t stride, const int32_t *slots,
                     const float *wts, uint32_t n, uint32_t gt, uint64_t og, uint32_t ut,
                     uint64_t ou, uint32_t dt, uint64_t od, const float *d_x, float *d_h,
                     float *d_h2, float *d_down, float *d_y, uint32_t n_ff, uint32_t in_dim,
                     uint32_t n_embd) {
    (void)d_h;
    (void)d_h2;
    (void)d_down;
    if (!slots || !wts || !n || n > kMaxU) {
        set_error("q4_hip_moe_exec: bad expert list");
        return false;
    }
    HostList hl;
    for (uint32_t i = 0; i < kMaxU; i++) {
        hl.id[i] = i < n ? slots[i] : -1;
        hl.w[i] = i < n ? wts[i] : 0.f;
    }
    uint32_t nu = 0;  // grid height = unique ids (the plan dedupes the same way)
    for (uint32_t i = 0; i < n; i++) {
        bool dup = slots[i] < 0;
        for (uint32_t j = 0; j < i && !dup; j++) dup = slots[j] == slots[i];
        nu += dup ? 0 : 1;
    }
    if (!nu) return true;
    ListSrc src = {nullptr, nullptr, nullptr, kMaxU, 1, n};
    return moe_run(base, stride, src, hl, nu, gt, og, ut, ou, dt, od, d_x, d_y, n_ff, in_dim,
                   n_embd);
}

/* Same, with slots/weights/count in device memory (count d_nhit[0]). */
bool q4_hip_moe_exec_dev(const uint8_t *base, uint64_t stride, const int32_t *d_es,
                         const float *d_ew, const int32_t *d_nhit, uint32_t gt, uint64_t og,
                         uint32_t ut, uint64_t ou, uint32_t dt, uint64_t od, const float *d_x,
                         float *d_h, float *d_h2, float *d_down, float *d_y, uint32_t n_ff,
                         uint32_t in_dim, uint32_t n_embd) {
    (void)d_h;
    (void)d_h2;
    (void)d_down;
    if (!d_es || !d_ew || !d_nhit) {
        set_error("q4_hip_moe_exec_dev: null list");
        return false;
    }
    HostList hl = {};
    ListSrc src = {d_es, d_ew, d_nhit, kMaxU, 1, 0};
    return moe_run(base, stride, src, hl, kMaxU, gt, og, ut, ou, dt, od, d_x, d_y, n_ff,
                   in_dim, n_embd);
}

/* Window coverage: 2..8 tokens, gate type == up type, IQ3_S or Q8_0 with a
 * covered K (the reference additionally limited the down type; here every
 * covered type runs the window). */
bool q4_hip_moe_win_ok(uint32_t gt, uint32_t ut, uint32_t dt, uint32_t in_dim, uint32_t n_ff,
                       uint32_t n_tok) {
    return n_tok >= 2 && n_tok <= kMaxT && gt == ut && type_ok(gt, in_dim) &&
           type_ok(dt, n_ff);
}

/* 2..8 tokens; token t's picks are d_es/d_ew[t*64 .. t*64 + d_nh[t]) (the
 * device route layout).  Experts picked by several tokens are read once.
 * x and y are token-major [n_tok][n_embd]; y is accumulated. */
bool q4_hip_moe_exec_win(const uint8_t *base, uint64_t stride, const int32_t *d_es,
                         const float *d_ew, const int32_t *d_nh, uint32_t n_tok, uint32_t gt,
                         uint64_t og, uint32_t ut, uint64_t ou, uint32_t dt, uint64_t od,
                         const float *d_x, float *d_h, float *d_y, uint32_t n_ff,
                         uint32_t in_dim, uint32_t n_embd) {
    (void)d_h;
    if (!q4_hip_moe_win_ok(gt, ut, dt, in_dim, n_ff, n_tok) || !d_es || !d_ew || !d_nh) {
        set_error("q4_hip_moe_exec_win: not covered");
        return false;
    }
    HostList hl = {};
    ListSrc src = {d_es, d_ew, d_nh, kMaxU, n_tok, 0};
    return moe_run(base, stride, src, hl, kMaxU, gt, og, ut, ou, dt, od, d_x, d_y, n_ff,
                   in_dim, n_embd);
}

}  // extern "C"
