// Routed-expert decode (1 token) and verify window (2..8 tokens): host entry
// points (the kernels are in moe_kern.h).
#include "moe_kern.h"

namespace q4mi {

// Measurement hook: bit 0 runs the gate/up launch, bit 1 the down launch
// (default both).  Lets a benchmark time each kernel of the pair alone.
static int g_phases = 3;
// LDS budget of a decode block (q4mi_moe_lds_cap lowers it for tests).
static size_t g_lds_cap = 0;
size_t lds_cap() { return g_lds_cap ? std::min(g_lds_cap, kLdsCap) : kLdsCap; }

template <int NT>
static bool run_nt(uint32_t ty_gu, uint32_t ty_dn, const MoeArgs &a, uint32_t nu_host) {
    if (g_phases & 1) {
        const bool ok = ty_gu == Q4MI_T_IQ3_S ? gu_dispatch<Q4MI_T_IQ3_S, NT>(a, nu_host)
                      : ty_gu == Q4MI_T_Q8_0  ? gu_dispatch<Q4MI_T_Q8_0, NT>(a, nu_host)
                                              : moe_fmt_gu(ty_gu, NT, a, nu_host);
        if (!ok) return false;
    }
    if (!(g_phases & 2)) return true;
    return ty_dn == Q4MI_T_IQ3_S ? dn_dispatch<Q4MI_T_IQ3_S, NT>(a, nu_host)
         : ty_dn == Q4MI_T_Q8_0  ? dn_dispatch<Q4MI_T_Q8_0, NT>(a, nu_host)
                                 : moe_fmt_dn(ty_dn, NT, a, nu_host);
}

// Rows are staged with 4- or 16-byte copies, so a row's byte size must be a
// multiple of 4 (IQ3_S, IQ2_S, IQ2_XXS, IQ2_XS, IQ3_XXS: K a multiple of
// 512; Q8_0, IQ4_NL, Q2_0: of 64; IQ4_XS: of 256).  Gate/up: IQ3_S, Q8_0,
// IQ2_S, IQ2_XXS, IQ2_XS, IQ3_XXS, IQ4_XS; down: IQ3_S, Q8_0, IQ2_S, IQ4_NL,
// Q2_0.
static bool type_ok(uint32_t ty, uint32_t K, bool down) {
    switch (ty) {
    case Q4MI_T_IQ3_S: case Q4MI_T_Q8_0: case Q4MI_T_IQ2_S: break;
    case Q4MI_T_IQ4_NL: case Q4MI_T_Q2_0:
        if (!down) return false;
        break;
    case Q4MI_T_IQ2_XXS: case Q4MI_T_IQ2_XS: case Q4MI_T_IQ3_XXS: case Q4MI_T_IQ4_XS:
        if (down) return false;
        break;
    default: return false;
    }
    const uint64_t rb = q4mi_row_bytes(ty, K);
    if (!rb || rb % 4 || K > 8192) return false;
    return layout_for(K / 32).tpr != 0;
}

static bool shape_ok(uint32_t gt, uint32_t ut, uint32_t dt, uint32_t in_dim, uint32_t n_ff,
                     uint32_t n_embd) {
    return gt == ut && type_ok(gt, in_dim, false) && type_ok(dt, n_ff, true) &&
           n_embd == in_dim && n_ff <= 1024;
}

static Plan *g_plan = nullptr;   // a device-list call's plan, gate/up -> down
#ifdef Q4MI_TRACE
static unsigned long long *g_trace = nullptr;
#endif

bool moe_warm(uint32_t n_ff) {
    if (!g_plan && !lib_malloc((void **)&g_plan, sizeof(Plan))) {
        set_error("moe: plan buffer allocation failed");
        return false;
    }
    // fp32 h of every (unique expert, token) pair
    return ensure_pd((size_t)kMaxU * kMaxT * n_ff);
}

// Where a call's intermediates live: the fp32 h [kMaxU][kMaxT][n_ff] and the
// device-list plan.  Null: the library's lazily allocated scratch.
struct Work {
    float *h;
    Plan *plan;
};

// Common driver.  All checks happen before the first launch so that a false
// return never leaves half of the work queued.
static bool moe_run(const uint8_t *base, uint64_t stride, const ListSrc &src,
                    const HostList &hl, uint32_t nu_host, uint32_t gt, uint64_t og, uint32_t ut,
                    uint64_t ou, uint32_t dt, uint64_t od, const float *d_x, float *d_y,
                    uint32_t n_ff, uint32_t in_dim, uint32_t n_embd, Work work = Work{},
                    uint64_t stride_d = 0, bool (*pre)(void *) = nullptr,
                    void *pre_arg = nullptr) {
    if (!base || !d_x || !d_y || src.n_tok < 1 || src.n_tok > kMaxT) {
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
    if (((uintptr_t)d_y & 3)) {
        set_error("moe: y must be 4-byte aligned");
        return false;
    }
    if (!stride_d) stride_d = stride;
    if ((((uintptr_t)base) | stride | stride_d | og | ou | od) & 3u) {
        set_error("moe: expert arena offsets must be 4-byte aligned");
        return false;
    }
    if (!work.h && !moe_warm(n_ff)) return false;
    if (pre && !pre(pre_arg)) return false;   // a launch the layer depends on
    MoeArgs a = {};
    a.base = base;
    a.stride = stride;
    a.stride_d = stride_d;
    a.og = og;
    a.ou = ou;
    a.od = od;
    a.K = in_dim;
    a.n_ff = n_ff;
    a.n_embd = n_embd;
    a.rb_gu = (uint32_t)q4mi_row_bytes(gt, in_dim);
    a.rb_dn = (uint32_t)q4mi_row_bytes(dt, n_ff);
    a.x = d_x;
    a.h = work.h ? work.h : lib_scratch().pd;
    a.y = d_y;
    a.src = src;
    a.hl = hl;
    a.gplan = work.h ? work.plan : g_plan;
    // a producer publishes each chunk before issuing its next one: a copy
    // issue stalls while the memory system is saturated, and publishing only
    // after the next chunk's issue delayed the first chunk by microseconds
    a.ahead = 1;
    a.plan_in = (g_phases & 1) ? 1u : 0u;   // down follows this call's gate/up
#ifdef Q4MI_TRACE
    if (!work.h && !g_trace && hipMalloc(&g_trace, 2 * 4096 * 32 * 8) == hipSuccess)
        (void)hipMemset(g_trace, 0, 2 * 4096 * 32 * 8);
    a.trace = g_trace;
    a.dbg = getenv("Q4MI_DBG") ? (uint32_t)atoi(getenv("Q4MI_DBG")) : 0u;
#endif
#if defined(Q4MI_TRACE) || defined(Q4MI_KNOBS)
    if (getenv("Q4MI_AHEAD")) a.ahead = (uint32_t)atoi(getenv("Q4MI_AHEAD"));
#endif
    const uint32_t nt = src.n_tok;
    if (nt == 1) return run_nt<1>(gt, dt, a, nu_host);
    if (nt == 2) return run_nt<2>(gt, dt, a, nu_host);
    if (nt <= 4) return run_nt<4>(gt, dt, a, nu_host);
    return run_nt<8>(gt, dt, a, nu_host);
}

}  // namespace q4mi

using namespace q4mi;

extern "C" void q4_mmvq_warm(void);

// Staged expert list for q4_hip_moe_stage / q4_hip_moe_exec_staged: coherent
// pinned host memory that the host rewrites per token and the kernels read
// through its device alias when they run (so a captured graph replays with
// the list staged last).
struct StageList {
    int32_t id[kMaxU];
    float w[kMaxU];
    int32_t n;
};
static StageList *g_stage = nullptr, *g_stage_dev = nullptr;

// Unique ids of a host list in first-appearance order; a repeated id adds its
// weights (the reference computes every entry and sums them).  Returns the
// unique count.
static uint32_t host_list(const int32_t *slots, const float *wts, uint32_t n, HostList &hl) {
    uint32_t nu = 0;
    for (uint32_t i = 0; i < n; i++) {
        if (slots[i] < 0) continue;
        uint32_t u = 0;
        while (u < nu && hl.id[u] != slots[i]) u++;
        if (u == nu) {
            hl.id[nu++] = slots[i];
            hl.w[u] = wts[i];
        } else {
            hl.w[u] += wts[i];
        }
    }
    for (uint32_t i = nu; i < kMaxU; i++) {
        hl.id[i] = -1;
        hl.w[i] = 0.f;
    }
    return nu;
}

// ------------------------------------------------ allocation-free decode
// q4mi_moe_exec_noalloc keeps its intermediates in this file-scope device
// array instead of library allocations: the device-list plan (unused by a
// host list, but the kernels take its address) then the fp32 h of up to 64
// unique experts x 8 token rows x n_ff <= 1024.  Each GPU holds its own copy
// for the life of the process; in host code `scratch` is only a stand-in
// symbol, so its device address is looked up once per device
// (hipGetSymbolAddress) and only that address reaches the kernels.  Nothing
// in it needs to start at zero: every call's gate/up launch writes every h
// row its down launch reads.
constexpr size_t kNaPlanBytes = (sizeof(Plan) + 255) & ~(size_t)255;
constexpr uint32_t kNaMaxFF = 1024;
constexpr size_t kNaBytes = kNaPlanBytes + (size_t)kMaxU * kMaxT * kNaMaxFF * sizeof(float);

static __device__ __align__(256) uint8_t scratch[kNaBytes];

constexpr int kNaMaxDev = 64;
static uint8_t *g_na_ptr[kNaMaxDev];

// The current device's address of `scratch` (looked up on its first use).
static uint8_t *noalloc_scratch() {
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kNaMaxDev) {
        set_error("q4mi_moe_exec_noalloc: no usable current device");
        return nullptr;
    }
    if (!g_na_ptr[dev]) {
        void *p = nullptr;
        const hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
        if (e != hipSuccess || !p) {
            set_error("q4mi_moe_exec_noalloc: hipGetSymbolAddress failed: %s",
                      hipGetErrorString(e));
            return nullptr;
        }
        g_na_ptr[dev] = (uint8_t *)p;
    }
    return g_na_ptr[dev];
}

static bool stage_ready() {
    if (g_stage) return true;
    void *p = nullptr, *dp = nullptr;
    if (hipHostMalloc(&p, sizeof(StageList), hipHostMallocMapped | hipHostMallocCoherent) !=
        hipSuccess) {
        set_error("q4_hip_moe_stage: pinned allocation failed");
        return false;
    }
    note_alloc();
    if (hipHostGetDevicePointer(&dp, p, 0) != hipSuccess) {
        (void)hipHostFree(p);
        set_error("q4_hip_moe_stage: no device alias for the staging list");
        return false;
    }
    memset(p, 0, sizeof(StageList));
    g_stage = (StageList *)p;
    g_stage_dev = (StageList *)dp;
    return true;
}

extern "C" {

#ifdef Q4MI_MEASURE
/* Measurement build only (libq4mi_meas.so): 1 = gate/up launch only, 2 =
 * down only, 3 = both. */
void q4mi_moe_phases(int mask) { g_phases = mask & 3; }

/* Measurement build only: cap the decode kernels' LDS at `bytes` (0: the
 * CU's 160 KB), so that their LDS rings are reused within a launch. */
void q4mi_moe_lds_cap(uint32_t bytes) { g_lds_cap = bytes; }
#endif

#ifdef Q4MI_TRACE
/* Trace build only: copy the phase timestamps [2 kernels][4096 blocks][32]
 * (wall clock, 100 MHz) of the last traced call to host memory, and clear
 * them. */
bool q4mi_trace_read(unsigned long long *dst, uint64_t n) {
    if (!g_trace || n > 2ull * 4096 * 32) return false;
    if (hipDeviceSynchronize() != hipSuccess) return false;
    if (hipMemcpy(dst, g_trace, n * 8, hipMemcpyDeviceToHost) != hipSuccess) return false;
    return hipMemset(g_trace, 0, 2 * 4096 * 32 * 8) == hipSuccess;
}
#endif

/* Copy the fp32 h of the last decode call, [64 unique experts][8 tokens]
 * [n_ff] (unique experts in first-appearance order), to d_dst on the
 * library stream.  A read-only debug export. */
bool q4mi_moe_copy_h(float *d_dst, uint32_t n_ff) {
    const size_t n = (size_t)kMaxU * kMaxT * n_ff;
    if (!d_dst || !n_ff || lib_scratch().pd_floats < n) {
        set_error("q4mi_moe_copy_h: no decode h of that size");
        return false;
    }
    if (hipMemcpyAsync(d_dst, lib_scratch().pd, n * sizeof(float), hipMemcpyDeviceToDevice,
                       stream()) != hipSuccess) {
        set_error("q4mi_moe_copy_h: copy failed");
        return false;
    }
    return true;
}

/* Drain the library stream and read the decode kernels' timeout word (0:
 * every bounded wait completed; else the bits of q4mi_status_text).  A
 * non-zero word also becomes q4mi_last_error(); clear != 0 resets it. */
uint32_t q4mi_device_status(int clear) {
    uint32_t v = 0;
    if (hipStreamSynchronize(stream()) != hipSuccess ||
        hipMemcpyFromSymbol(&v, HIP_SYMBOL(g_moe_status), sizeof v, 0,
                            hipMemcpyDeviceToHost) != hipSuccess) {
        set_error("q4mi_device_status: device not readable");
        return 0x80000000u;
    }
    v |= moe_fmt_status(clear);
    v |= mmq_status(clear);
    if (v) set_error("%s", q4mi_status_text(v));
    if (v && clear) {
        const uint32_t z = 0;
        if (hipMemcpyToSymbol(HIP_SYMBOL(g_moe_status), &z, sizeof z, 0,
                              hipMemcpyHostToDevice) != hipSuccess)
            set_error("q4mi_device_status: reset failed");
    }
    return v;
}

/* Allocate the decode scratch (call before any stream capture). */
void q4_hip_moe_scratch_warm(void) {
    (void)moe_warm(1024);
    (void)stage_ready();
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
    const uint32_t nu = host_list(slots, wts, n, hl);
    if (!nu) return true;
    ListSrc src = {nullptr, nullptr, nullptr, kMaxU, 1, nu, 1};
    return moe_run(base, stride, src, hl, nu, gt, og, ut, ou, dt, od, d_x, d_y, n_ff, in_dim,
                   n_embd);
}

/* q4_hip_moe_exec that allocates nothing: its intermediates live in the
 * file-scope device array `scratch` (2 MiB + the plan, n_ff <= 1024), so a
 * caller that cannot allocate (under graph capture, in a serving loop that
 * forbids hipMalloc) can call it from the first call on.  Calls that overlap
 * on one GPU share that array and race. */
bool q4mi_moe_exec_noalloc(const uint8_t *base, uint64_t stride, const int32_t *slots,
                           const float *wts, uint32_t n, uint32_t gt, uint64_t og, uint32_t ut,
                           uint64_t ou, uint32_t dt, uint64_t od, const float *d_x, float *d_y,
                           uint32_t n_ff, uint32_t in_dim, uint32_t n_embd) {
    if (!slots || !wts || !n || n > kMaxU) {
        set_error("q4mi_moe_exec_noalloc: bad expert list");
        return false;
    }
    if (n_ff > kNaMaxFF) {
        set_error("q4mi_moe_exec_noalloc: n_ff %u needs %zu bytes of h, beyond the %zu-byte "
                  "static scratch (n_ff <= %u)", n_ff, (size_t)kMaxU * kMaxT * n_ff * 4,
                  kNaBytes - kNaPlanBytes, kNaMaxFF);
        return false;
    }
    HostList hl;
    const uint32_t nu = host_list(slots, wts, n, hl);
    if (!nu) return true;
    uint8_t *sp = noalloc_scratch();
    if (!sp) return false;
    ListSrc src = {nullptr, nullptr, nullptr, kMaxU, 1, nu, 1};
    return moe_run(base, stride, src, hl, nu, gt, og, ut, ou, dt, od, d_x, d_y, n_ff, in_dim,
                   n_embd, Work{(float *)(sp + kNaPlanBytes), (Plan *)sp});
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
    ListSrc src = {d_es, d_ew, d_nhit, kMaxU, 1, 0, 0};
    return moe_run(base, stride, src, hl, 0, gt, og, ut, ou, dt, od, d_x, d_y, n_ff, in_dim,
                   n_embd);
}

/* One token's routed layer in three launches (see include/q4mi.h). */
bool q4mi_moe_route_exec(const void *d_wr, uint32_t wr_type, const float *d_sgw,
                         const float *d_x, uint32_t n_embd, uint32_t n_exp, uint32_t topk,
                         float *d_logits, int32_t *d_ids, float *d_wts, int32_t *d_nh,
                         int32_t shared_slot, float *d_sg, const uint8_t *base, uint64_t stride,
                         uint32_t gt, uint64_t og, uint32_t ut, uint64_t ou, uint32_t dt,
                         uint64_t od, float *d_y, uint32_t n_ff) {
    const bool lists = d_ids || d_wts || d_nh;
    if (lists && !(d_ids && d_wts && d_nh)) {
        set_error("q4mi_moe_route_exec: d_ids, d_wts and d_nh together or none");
        return false;
    }
    if (topk + (shared_slot >= 0 ? 1u : 0u) > kMaxU) {
        set_error("q4mi_moe_route_exec: more than %u entries", kMaxU);
        return false;
    }
    if (!router_front(d_wr, wr_type, d_sgw, d_x, 1, n_embd, n_exp, topk, d_logits, kMaxU,
                      shared_slot, d_sg, false))
        return false;
    if (!(g_phases & 1)) {   // the down launch reads the plan gate/up built
        set_error("q4mi_moe_route_exec: needs the gate/up launch (measurement phases)");
        return false;
    }
    ListSrc src = {};
    src.n_tok = 1;
    src.stride = kMaxU;
    src.lg = d_logits;
    src.sg = d_sgw ? d_sg : nullptr;
    src.o_ids = d_ids;
    src.o_wts = d_wts;
    src.o_nh = d_nh;
    src.n_exp = n_exp;
    src.topk = topk;
    src.shared = shared_slot;
    struct Front {
        const void *wr;
        uint32_t ty;
        const float *sgw, *x;
        uint32_t n_embd, n_exp, topk;
        float *lg;
        int32_t shared;
        float *sg;
    } f = {d_wr, wr_type, d_sgw, d_x, n_embd, n_exp, topk, d_logits, shared_slot, d_sg};
    auto launch = [](void *p) {
        const Front &g = *(const Front *)p;
        return router_front(g.wr, g.ty, g.sgw, g.x, 1, g.n_embd, g.n_exp, g.topk, g.lg, kMaxU,
                            g.shared, g.sg, true);
    };
    HostList hl = {};
    return moe_run(base, stride, src, hl, 0, gt, og, ut, ou, dt, od, d_x, d_y, n_ff, n_embd,
                   n_embd, Work{}, 0, launch, &f);
}

/* Window coverage: 2..8 tokens, gate type == up type, IQ3_S or Q8_0 with a
 * covered K (the reference additionally limited the down type; here every
 * covered type runs the window). */
bool q4_hip_moe_win_ok(uint32_t gt, uint32_t ut, uint32_t dt, uint32_t in_dim, uint32_t n_ff,
                       uint32_t n_tok) {
    return n_tok >= 2 && n_tok <= kMaxT && gt == ut && type_ok(gt, in_dim, false) &&
           type_ok(dt, n_ff, true) && n_ff <= 1024;
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
    ListSrc src = {d_es, d_ew, d_nh, kMaxU, n_tok, 0, 0};
    return moe_run(base, stride, src, hl, 0, gt, og, ut, ou, dt, od, d_x, d_y, n_ff, in_dim,
                   n_embd);
}

/* Decode (1 token) or verify window (2..8) over the GGUF expert layout:
 * gate, up and down are separate stacked tensors (blk.N.ffn_gate_exps,
 * ffn_up_exps, ffn_down_exps; src/q4_expert.c:962-982 reads the same
 * slices), expert e's matrices at gate + e*gu_stride, up + e*gu_stride and
 * down + e*d_stride.  Device lists as q4_hip_moe_exec_win. */
bool q4mi_moe_exec_parts(const uint8_t *gate, const uint8_t *up, const uint8_t *down,
                         uint64_t gu_stride, uint64_t d_stride, const int32_t *d_es,
                         const float *d_ew, const int32_t *d_nh, uint32_t n_tok, uint32_t gt,
                         uint32_t dt, const float *d_x, float *d_y, uint32_t n_ff,
                         uint32_t in_dim, uint32_t n_embd) {
    if (!gate || !up || !down || !d_es || !d_ew || !d_nh || !n_tok || n_tok > kMaxT ||
        !gu_stride || !d_stride) {
        set_error("q4mi_moe_exec_parts: bad arguments");
        return false;
    }
    HostList hl = {};
    ListSrc src = {d_es, d_ew, d_nh, kMaxU, n_tok, 0, 0};
    // offsets from the gate base wrap modulo 2^64, so up/down may sit below it
    return moe_run(gate, gu_stride, src, hl, 0, gt, 0, gt, (uint64_t)(up - gate), dt,
                   (uint64_t)(down - gate), d_x, d_y, n_ff, in_dim, n_embd, Work{}, d_stride);
}

/* Per-token small-batch preflight: the type/shape rule of the exec calls. */
bool q4_hip_moe_tok_ok(uint32_t gt, uint32_t ut, uint32_t dt, uint32_t in_dim, uint32_t n_ff) {
    return gt == ut && type_ok(gt, in_dim, false) && type_ok(dt, n_ff, true) && n_ff <= 1024;
}

/* n_tok tokens; token t's picks are d_slots/d_wts[h_off[t] .. h_off[t+1])
 * (device arrays, host offsets); x and y token-major, y accumulated.
 * Everything is checked before the first launch.  Equal counts (2..8
 * tokens, at most 64 picks in all) run as one window; otherwise one
 * device-list layer per token. */
bool q4_hip_moe_exec_tok(const uint8_t *base, uint64_t stride, const int32_t *d_slots,
                         const float *d_wts, const uint32_t *h_off, uint32_t n_tok, uint32_t gt,
                         uint64_t og, uint32_t ut, uint64_t ou, uint32_t dt, uint64_t od,
                         const float *d_x, float *d_h, float *d_h2, float *d_y, uint32_t n_ff,
                         uint32_t in_dim, uint32_t n_embd) {
    (void)d_h;
    (void)d_h2;
    if (!d_slots || !d_wts || !h_off || !n_tok) {
        set_error("q4_hip_moe_exec_tok: bad arguments");
        return false;
    }
    if (!q4_hip_moe_tok_ok(gt, ut, dt, in_dim, n_ff) || n_embd != in_dim) {
        set_error("q4_hip_moe_exec_tok: types/shape not covered");
        return false;
    }
    const uint32_t c0 = h_off[1] - h_off[0];
    bool same = n_tok >= 2 && n_tok <= kMaxT;
    for (uint32_t t = 0; t < n_tok; t++) {
        if (h_off[t + 1] < h_off[t] || h_off[t + 1] - h_off[t] > kMaxU) {
            set_error("q4_hip_moe_exec_tok: token %u has a bad pick range", t);
            return false;
        }
        same = same && h_off[t + 1] - h_off[t] == c0;
    }
    if (h_off[n_tok] == h_off[0]) return true;
    HostList hl = {};
    if (same && (uint64_t)c0 * n_tok <= kMaxU) {
        ListSrc src = {d_slots + h_off[0], d_wts + h_off[0], nullptr, c0, n_tok, c0, 0};
        return moe_run(base, stride, src, hl, 0, gt, og, ut, ou, dt, od, d_x, d_y, n_ff, in_dim,
                       n_embd);
    }
    for (uint32_t t = 0; t < n_tok; t++) {
        const uint32_t cnt = h_off[t + 1] - h_off[t];
        if (!cnt) continue;
        ListSrc src = {d_slots + h_off[t], d_wts + h_off[t], nullptr, cnt, 1, cnt, 0};
        if (!moe_run(base, stride, src, hl, cnt, gt, og, ut, ou, dt, od,
                     d_x + (size_t)t * in_dim, d_y + (size_t)t * n_embd, n_ff, in_dim, n_embd))
            return false;
    }
    return true;
}

/* Stage one token's list (n <= 64 slot ids and weights, host arrays) for
 * q4_hip_moe_exec_staged.  The caller must not restage while a launch that
 * reads the previous list is still queued. */
bool q4_hip_moe_stage(const int32_t *slots, const float *wts, uint32_t n) {
    if ((n && (!slots || !wts)) || n > kMaxU) {
        set_error("q4_hip_moe_stage: bad expert list");
        return false;
    }
    if (!stage_ready()) return false;
    for (uint32_t i = 0; i < n; i++) {
        g_stage->id[i] = slots[i];
        g_stage->w[i] = wts[i];
    }
    g_stage->n = (int32_t)n;
    return true;
}

/* q4_hip_moe_exec_dev over the staged list, read when the kernels run. */
bool q4_hip_moe_exec_staged(const uint8_t *base, uint64_t stride, uint32_t gt, uint64_t og,
                            uint32_t ut, uint64_t ou, uint32_t dt, uint64_t od,
                            const float *d_x, float *d_h, float *d_h2, float *d_down,
                            float *d_y, uint32_t n_ff, uint32_t in_dim, uint32_t n_embd) {
    if (!stage_ready()) return false;
    return q4_hip_moe_exec_dev(base, stride, g_stage_dev->id, g_stage_dev->w, &g_stage_dev->n,
                               gt, og, ut, ou, dt, od, d_x, d_h, d_h2, d_down, d_y, n_ff, in_dim,
                               n_embd);
}

}  // extern "C"
