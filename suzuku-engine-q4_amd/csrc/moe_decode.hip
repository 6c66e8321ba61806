// Routed-expert decode (1 token) and verify window (2..8 tokens) over
// IQ3_S / Q8_0 experts resident at base + slot*stride.
//
// Two persistent launches per layer, one 512-thread block per CU:
//   moe_gu_k  the (unique expert u, intermediate row r) pairs are split into
//             one contiguous share per block; the share's gate and up rows
//             stream HBM -> LDS (global_load_lds) in double-buffered chunks,
//             the next chunk in flight while the current one is computed, and
//             h[u][t][r] = silu(gate_r . q8(x_t)) * (up_r . q8(x_t)).
//   moe_dn_k  each block owns 8 output rows: it quantizes every selected
//             h[u][t] into LDS, dots its rows of every expert's down matrix,
//             and adds sum_u w[u][t] * pd[u][t][r] into y[t][r] in
//             unique-expert order -- deterministic, no atomics.
// Each unique expert's rows are read once per launch and dotted with every
// token that selected it (the verify window's reuse; reference
// q4_hip_moe_exec_win src/q4_rocm.cu:7444-7531, CPU twin
// q4_cpuex_dispatch_win src/q4_cpuexp.c:2618-2753).
//
// IQ3_S decode: one LDS lookup per 4 values into an 8192-entry table of
// signed int8 quads indexed by (sign nibble, qh bit, qs byte), one
// v_dot4_i32_i8 per quad per token, the (2s+1) multiplier on the exact int32
// group sum, then float(S) * (d_w * d_x).
#include <stdlib.h>

#include "mmvq_engine.h"
#include "q4mi_internal.h"

namespace q4mi {

constexpr uint32_t kMaxU = 64;    // unique experts per call (reference bound n<=64)
constexpr uint32_t kMaxT = 8;     // tokens per call
constexpr uint32_t kThreads = 1024;
constexpr uint32_t kDnRows = 8;   // output rows per down block

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
    uint32_t unique;     // host list already deduplicated (one token)
};

struct __align__(16) Plan {
    uint32_t nu;
    uint32_t nsel;                  // selected (u, t) pairs
    int32_t uid[kMaxU];
    uint32_t sel[kMaxU];            // token bitmask per unique expert
    uint32_t pslot[kMaxU];          // first pair slot of u (slots in (u, t) order)
    float w[kMaxU][kMaxT];
};

// Wave 0 builds the plan (first-appearance order over (token, pick));
// callers sync afterwards.
__device__ void build_plan(Plan *P, const ListSrc &s, const HostList &hl, uint32_t lane) {
    if (s.unique) {   // deduplicated on the host: the plan is the list itself
        const uint32_t nu = s.n_fixed;
        // uniform loop: the kernel-argument list is read with scalar loads
        for (uint32_t u = 0; u < nu; u++) {
            const int32_t id = hl.id[u];
            const float w = hl.w[u];
            if (lane == 0) {
                P->uid[u] = id;
                P->w[u][0] = w;
            }
        }
        if (lane < kMaxU) {
            P->sel[lane] = lane < nu ? 1u : 0u;
            P->pslot[lane] = lane;
#pragma unroll
            for (uint32_t t = 1; t < kMaxT; t++) P->w[lane][t] = 0.f;
            if (lane >= nu) {
                P->uid[lane] = -1;
                P->w[lane][0] = 0.f;
            }
        }
        if (lane == 0) {
            P->nu = nu;
            P->nsel = nu;
        }
        return;
    }
    // lane -> (token, pick) of the flattened lists, token-major
    uint32_t E = 0, tok = 0, rem = 0;
    bool found = false;
    for (uint32_t t = 0; t < s.n_tok; t++) {
        int c = s.nh ? s.nh[t] : (int)s.n_fixed;
        if (c < 0) c = 0;
        if ((uint32_t)c > s.stride) c = (int)s.stride;
        if (!found && lane < E + (uint32_t)c) {
            found = true;
            tok = t;
            rem = lane - E;
        }
        E += (uint32_t)c;
    }
    if (E > kMaxU) E = kMaxU;
    int32_t id = -1;
    float w = 0.f;
    if (lane < E) {
        if (s.es) {
            id = s.es[(size_t)tok * s.stride + rem];
            w = s.ew[(size_t)tok * s.stride + rem];
        } else {
            id = hl.id[rem];
            w = hl.w[rem];
        }
    }
    const bool valid = lane < E && id >= 0;
    uint32_t first_j = lane;
    for (uint32_t j = 0; j < E; j++) {
        const int32_t idj = __shfl(id, j);
        const bool vj = __shfl((int)valid, j) != 0;
        if (vj && idj == id && j < first_j) first_j = j;
    }
    const bool first = valid && first_j == lane;
    const uint64_t fm = __ballot(first);
    const uint32_t u = (uint32_t)__popcll(fm & ((1ull << first_j) - 1ull));
    for (uint32_t i = lane; i < kMaxU; i += 64) {
        P->sel[i] = 0;
#pragma unroll
        for (uint32_t t = 0; t < kMaxT; t++) P->w[i][t] = 0.f;
    }
    const uint32_t nu = (uint32_t)__popcll(fm);
    if (lane == 0) P->nu = nu;
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup");
    if (first) P->uid[u] = id;
    if (valid) {
        atomicOr(&P->sel[u], 1u << tok);
        P->w[u][tok] = w;
    }
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQ_REL, "workgroup");
    // pair slots: exclusive prefix of popcount(sel) over u (lane u)
    const uint32_t c = lane < nu ? (uint32_t)__popc(P->sel[lane]) : 0u;
    uint32_t incl = c;
#pragma unroll
    for (int o = 1; o < 64; o <<= 1) {
        const uint32_t v = __shfl_up(incl, o);
        if (lane >= (uint32_t)o) incl += v;
    }
    if (lane < nu) P->pslot[lane] = incl - c;
    if (lane == 63) P->nsel = incl;
}

// DPP reduction over aligned groups of W lanes (W = 8, 16, 32, 64); the
// group's total lands in its last lane (lane % W == W-1).
template <int W>
__device__ inline float rsum(float v) {
    v += __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), 0x111, 0xF, 0xF, true));
    v += __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), 0x112, 0xF, 0xF, true));
    v += __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), 0x114, 0xF, 0xF, true));
    if (W >= 16)
        v += __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), 0x118, 0xF, 0xF, true));
    if (W >= 32)
        v += __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), 0x142, 0xA, 0xF, true));
    if (W >= 64)
        v += __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), 0x143, 0xC, 0xF, true));
    return v;
}

// Signed int8 quads of IQ3_S group g of the row at LDS offset `row`.
__device__ inline void iq3s_group(const uint32_t *stab, const uint8_t *lb, const uint32_t *lw,
                                  uint32_t row, uint32_t g, int32_t (&w)[8], int &mult,
                                  float &d) {
    const uint32_t B = row + (g >> 3) * IQ3S_BYTES;
    const uint32_t j = g & 7u;
    d = q4mi_h2f(lds_u16_at(lb, B));
    const uint32_t qo = B + 2u + 8u * j;
    const uint32_t i0 = qo >> 2, sh = qo & 3u;
    const uint32_t w0 = lw[i0], w1 = lw[i0 + 1], w2 = lw[i0 + 2];
    const uint32_t q0 = __builtin_amdgcn_alignbyte(w1, w0, sh);
    const uint32_t q1 = __builtin_amdgcn_alignbyte(w2, w1, sh);
    const uint32_t qh = lb[B + 66u + j];
    const uint32_t sg = lds_u32_at(lw, B + 74u + 4u * j);
    const uint32_t sc = lb[B + 106u + (j >> 1)];
    mult = 2 * (int)((j & 1u) ? (sc >> 4) : (sc & 15u)) + 1;
#pragma unroll
    for (int k = 0; k < 8; k++) {
        const uint32_t qb = __builtin_amdgcn_ubfe(k < 4 ? q0 : q1, 8 * (k & 3), 8);
        const uint32_t hs = (__builtin_amdgcn_ubfe(sg, 4 * k, 4) << 1) | __builtin_amdgcn_ubfe(qh, k, 1);
        w[k] = (int32_t)stab[qb | (hs << 8)];
    }
}

__device__ inline void q80_group(const uint8_t *lb, const uint32_t *lw, uint32_t row, uint32_t g,
                                 int32_t (&w)[8], int &mult, float &d) {
    const uint32_t B = row + g * Q80_BYTES;
    d = q4mi_h2f(lds_u16_at(lb, B));
    mult = 1;
    const uint32_t i0 = (B + 2u) >> 2, sh = (B + 2u) & 3u;
    uint32_t prev = lw[i0];
#pragma unroll
    for (int k = 0; k < 8; k++) {
        const uint32_t nx = lw[i0 + 1 + k];
        w[k] = (int32_t)__builtin_amdgcn_alignbyte(nx, prev, sh);
        prev = nx;
    }
}

template <uint32_t TY>
__device__ inline void group_w(const uint32_t *stab, const uint8_t *lb, const uint32_t *lw,
                               uint32_t row, uint32_t g, int32_t (&w)[8], int &mult, float &d) {
    if (TY == Q4MI_T_IQ3_S)
        iq3s_group(stab, lb, lw, row, g, w, mult, d);
    else
        q80_group(lb, lw, row, g, w, mult, d);
}

struct MoeArgs {
    const uint8_t *base;
    uint64_t stride, og, ou, od;
    uint32_t K;       // in_dim (gate/up columns)
    uint32_t n_ff;
    uint32_t n_embd;
    uint32_t rb_gu, rb_dn;
    uint32_t chunk;   // gate/up: pairs per chunk; down: experts per chunk
    const float *x;   // [n_tok][K]
    int8_t *hq;       // [kMaxU][kMaxT][n_ff] q8 codes of h
    float *hd;        // [kMaxU][kMaxT][n_ff/32] their scales
    float *y;         // [n_tok][n_embd], accumulated
    const uint32_t *stab;   // signed IQ3_S table (device)
    ListSrc src;
    uint32_t dbg;     // Q4MI_DBG phase-skip mask (measurement only; 0 = normal)
};

__device__ inline float silu_f(float v) { return v / (1.f + expf(-v)); }

// Asynchronous row staging, global -> LDS without registers (gfx950
// global_load_lds): wave w copies rows w, w+8, ... of `nrows` rows of `rb`
// bytes (row i from src(i)) to dst + i*rb, in UNIT-byte lanes (16 when
// every row start and rb are 16-aligned, else 4).  The caller waits with
// wait_stage() and a barrier before reading.
template <uint32_t UNIT, class SrcFn>
__device__ inline void stage_rows(uint8_t *dst, SrcFn src, uint32_t nrows, uint32_t rb,
                                  uint32_t wave, uint32_t lane) {
    const uint32_t units = rb / UNIT;
    for (uint32_t r = wave; r < nrows; r += kThreads / 64) {
        const uint8_t *sp = src(r);
        uint8_t *dp = dst + (size_t)r * rb;
        for (uint32_t u0 = 0; u0 < units; u0 += 64) {
            if (u0 + lane < units) {
                const void *g = (const void *)(sp + (size_t)(u0 + lane) * UNIT);
                auto *l = (__attribute__((address_space(3))) void *)(dp + (size_t)u0 * UNIT);
                if constexpr (UNIT == 16)
                    __builtin_amdgcn_global_load_lds(g, l, 16, 0, 0);
                else
                    __builtin_amdgcn_global_load_lds(g, l, 4, 0, 0);
            }
        }
    }
}

__device__ inline void wait_stage() { asm volatile("s_waitcnt vmcnt(0)" ::: "memory"); }

// Asynchronous contiguous copy of `bytes` (multiple of 1024) global -> LDS.
__device__ inline void dma_copy(uint8_t *dst, const uint8_t *src, uint32_t bytes, uint32_t wave,
                                uint32_t lane) {
    for (uint32_t o = wave * 1024; o < bytes; o += (kThreads / 64) * 1024)
        __builtin_amdgcn_global_load_lds((const void *)(src + o + lane * 16),
                                         (__attribute__((address_space(3))) void *)(dst + o), 16,
                                         0, 0);
}

// ------------------------------------------------------------- gate / up
template <uint32_t TY, int NT, int TPR, int GPT, uint32_t UNIT>
__global__ __launch_bounds__(kThreads) void moe_gu_k(MoeArgs a, HostList hl) {
    extern __shared__ __align__(16) uint8_t smem[];
    uint32_t *stab = (uint32_t *)smem;                              // 32 KB (IQ3_S)
    Plan *P = (Plan *)(smem + (TY == Q4MI_T_IQ3_S ? 32768 : 0));
    int8_t *xq = (int8_t *)(P + 1);
    float *xd = (float *)(xq + NT * a.K);
    float *hbuf = xd + NT * (a.K / 32);               // [32][NT] h of the current unit
    uint8_t *tile0 = (uint8_t *)(hbuf + 32 * NT);
    uint8_t *tile1 = tile0 + (size_t)2 * a.chunk * a.rb_gu;
    const uint32_t tid = threadIdx.x, wave = tid >> 6, lane = tid & 63u;
    if (a.dbg & 256) {
        if (tid < kMaxU) {
            P->uid[tid] = tid;
            P->sel[tid] = 1;
            P->pslot[tid] = tid;
            P->w[tid][0] = 0.1f;
        }
        if (tid == 0) P->nu = P->nsel = 11;
    } else if (tid < 64) {
        build_plan(P, a.src, hl, tid);
    }
    __syncthreads();
    if (a.dbg & 512) return;
    const uint32_t nt = a.src.n_tok;
    const uint32_t nu = P->nu;
    // shares are whole 32-row units (one q8 group of h per token)
    const uint32_t U = nu * a.n_ff / 32;
    const uint32_t p0 = 32u * (uint32_t)(((uint64_t)U * blockIdx.x) / gridDim.x);
    const uint32_t p1 = 32u * (uint32_t)(((uint64_t)U * (blockIdx.x + 1)) / gridDim.x);
    const uint32_t rb = a.rb_gu;
    const uint32_t n_ff = a.n_ff;
    const uint8_t *base = a.base;
    const uint64_t stride = a.stride, og = a.og, ou = a.ou;
    const int32_t *uid = P->uid;
    auto src_of = [=](uint32_t pc0) {
        return [=](uint32_t i) -> const uint8_t * {
            const uint32_t p = pc0 + (i >> 1), u = p / n_ff, r = p % n_ff;
            return base + (uint64_t)uid[u] * stride + ((i & 1) ? ou : og) + (uint64_t)r * rb;
        };
    };
    // Weights and the decode table are fetched asynchronously into LDS
    // first; x is loaded after them.  VMEM results return in issue order, so
    // quantizing x waits for the whole fetch -- which compute needs anyway --
    // and adds only the quantization itself to the critical path.
    uint32_t pc = p0;
    uint32_t n = min(a.chunk, p1 - pc);
    if (n && !(a.dbg & 4)) stage_rows<UNIT>(tile0, src_of(pc), 2 * n, rb, wave, lane);
    if (TY == Q4MI_T_IQ3_S && !(a.dbg & 1))
        dma_copy((uint8_t *)stab, (const uint8_t *)a.stab, 32768, wave, lane);
    if (!(a.dbg & 2)) {
        const uint32_t quads = nt * (a.K / 4);
        for (uint32_t i = tid; i < quads; i += kThreads) {
            const float4 v = *(const float4 *)(a.x + (size_t)i * 4);
            float dd;
            int bs;
            const uint32_t q = q4mi_quant_team8(v, &dd, &bs);
            *(uint32_t *)(xq + (size_t)i * 4) = q;
            if ((i & 7u) == 0) xd[i / 8] = dd;
        }
    }
    wait_stage();
    __syncthreads();
    const uint32_t gi = tid % TPR, slot = tid / TPR;
    constexpr uint32_t kSlots = kThreads / TPR;
    XRegs<NT, GPT> xr;
    load_xregs<NT, GPT, TPR>(xr, xq, xd, a.K, nt, gi);
    uint32_t buf = 0;
    while (n) {
        wait_stage();
        __syncthreads();                      // chunk landed in tile[buf]
        uint8_t *tile = buf ? tile1 : tile0;
        const uint32_t pn = pc + n;
        const uint32_t nn = min(a.chunk, p1 - pn);
        if (nn && !(a.dbg & 4)) stage_rows<UNIT>(buf ? tile0 : tile1, src_of(pn), 2 * nn, rb, wave, lane);
        const uint32_t *tw = (const uint32_t *)tile;
        for (uint32_t i = slot; i < n && !(a.dbg & 8); i += kSlots) {
            const uint32_t p = pc + i, u = p / n_ff, r = p % n_ff;
            const uint32_t sel = P->sel[u];
            float ag[NT], au[NT];
#pragma unroll
            for (int t = 0; t < NT; t++) ag[t] = au[t] = 0.f;
#pragma unroll
            for (int m = 0; m < GPT; m++) {
                const uint32_t g = gi + TPR * m;
#pragma unroll
                for (int which = 0; which < 2; which++) {
                    int32_t w[8];
                    int mult;
                    float d;
                    group_w<TY>(stab, tile, tw, (2 * i + which) * rb, g, w, mult, d);
#pragma unroll
                    for (int t = 0; t < NT; t++) {
                        if (!((sel >> t) & 1u)) continue;
                        int s = 0;
#pragma unroll
                        for (int k = 0; k < 8; k++) s = q4mi_sdot4(w[k], xr.q[m][t][k], s);
                        const float f = (float)(s * mult) * (d * xr.d[m][t]);
                        if (which == 0) ag[t] += f;
                        else au[t] += f;
                    }
                }
            }
#pragma unroll
            for (int t = 0; t < NT; t++) {
                if (!((sel >> t) & 1u)) continue;
                const float gs = rsum<TPR>(ag[t]), us = rsum<TPR>(au[t]);
                if (gi == TPR - 1) hbuf[(p & 31u) * NT + t] = silu_f(gs) * us;
            }
        }
        __syncthreads();                      // tile[buf] free; hbuf complete
        if ((pn & 31u) == 0) {
            // a 32-row unit is complete: q8 of h for every selected token
            const uint32_t pu = pn - 32, u = pu / n_ff, r = pu % n_ff;
            const uint32_t sel = P->sel[u];
            if (tid < 8u * nt) {
                const uint32_t t = tid >> 3, sub = tid & 7u;
                if ((sel >> t) & 1u) {
                    const float4 v = make_float4(hbuf[(4 * sub) * NT + t], hbuf[(4 * sub + 1) * NT + t],
                                                 hbuf[(4 * sub + 2) * NT + t], hbuf[(4 * sub + 3) * NT + t]);
                    float dd;
                    int bs;
                    const uint32_t q = q4mi_quant_team8(v, &dd, &bs);
                    *(uint32_t *)(a.hq + ((size_t)u * kMaxT + t) * n_ff + r + 4 * sub) = q;
                    if (sub == 0) a.hd[((size_t)u * kMaxT + t) * (n_ff / 32) + r / 32] = dd;
                }
            }
        }
        pc = pn;
        n = nn;
        buf ^= 1u;
    }
}

// ---------------------------------------------------------------- down
template <uint32_t TY, int NT, int TPR, int GPT, uint32_t UNIT>
__global__ __launch_bounds__(kThreads) void moe_dn_k(MoeArgs a, HostList hl) {
    extern __shared__ __align__(16) uint8_t smem[];
    uint32_t *stab = (uint32_t *)smem;
    Plan *P = (Plan *)(smem + (TY == Q4MI_T_IQ3_S ? 32768 : 0));
    float *part = (float *)(P + 1);                           // [kMaxU][kMaxT][kDnRows]
    int8_t *hq = (int8_t *)(part + kMaxU * kMaxT * kDnRows);  // [nsel][n_ff]
    float *hd = (float *)(hq + kMaxU * a.n_ff);               // [nsel][n_ff/32]
    uint8_t *tile0 = (uint8_t *)(hd + kMaxU * (a.n_ff / 32));
    uint8_t *tile1 = tile0 + (size_t)a.chunk * kDnRows * a.rb_dn;
    const uint32_t tid = threadIdx.x, wave = tid >> 6, lane = tid & 63u;
    if (tid < 64) build_plan(P, a.src, hl, tid);
    __syncthreads();
    const uint32_t nu = P->nu;
    const uint32_t nt = a.src.n_tok;
    const uint32_t r0 = blockIdx.x * kDnRows;
    const uint32_t nr = min(kDnRows, a.n_embd - r0);
    const uint32_t rb = a.rb_dn;
    const uint8_t *base = a.base;
    const uint64_t stride = a.stride, od = a.od;
    const int32_t *uid = P->uid;
    auto src_of = [=](uint32_t u0) {
        return [=](uint32_t i) -> const uint8_t * {
            const uint32_t u = u0 + i / nr, r = r0 + i % nr;
            return base + (uint64_t)uid[u] * stride + od + (uint64_t)r * rb;
        };
    };
    // y of this block's rows, needed at the very end: load it first
    float yv = 0.f;
    if (tid < nt * nr) yv = a.y[(size_t)(tid / nr) * a.n_embd + r0 + tid % nr];
    // weights, table and the q8 of h, all asynchronously into LDS
    uint32_t uc = 0;
    uint32_t n = min(a.chunk, nu);
    if (n && !(a.dbg & 64)) stage_rows<UNIT>(tile0, src_of(0), n * nr, rb, wave, lane);
    if (TY == Q4MI_T_IQ3_S && !(a.dbg & 16))
        dma_copy((uint8_t *)stab, (const uint8_t *)a.stab, 32768, wave, lane);
    if (!(a.dbg & 32)) {
        const uint32_t n_ff = a.n_ff;
        const Plan *PP = P;
        const int8_t *ghq = a.hq;
        const float *ghd = a.hd;
        // pair slot -> (u, t): the slots of u are its selected tokens in order
        auto pair_ut = [=](uint32_t slot, uint32_t &u, uint32_t &t) {
            u = 0;
            while (u + 1 < nu && PP->pslot[u + 1] <= slot) u++;
            uint32_t sel = PP->sel[u], kk = slot - PP->pslot[u];
            t = 0;
            for (;; t++)
                if ((sel >> t) & 1u) {
                    if (!kk) break;
                    kk--;
                }
        };
        stage_rows<16>((uint8_t *)hq, [=](uint32_t i) -> const uint8_t * {
            uint32_t u, t;
            pair_ut(i, u, t);
            return (const uint8_t *)(ghq + ((size_t)u * kMaxT + t) * n_ff);
        }, P->nsel, n_ff, wave, lane);
        stage_rows<4>((uint8_t *)hd, [=](uint32_t i) -> const uint8_t * {
            uint32_t u, t;
            pair_ut(i, u, t);
            return (const uint8_t *)(ghd + ((size_t)u * kMaxT + t) * (n_ff / 32));
        }, P->nsel, n_ff / 8, wave, lane);
    }
    const uint32_t gi = tid % TPR, slot = tid / TPR;
    constexpr uint32_t kSlots = kThreads / TPR;
    uint32_t buf = 0;
    while (n) {
        wait_stage();
        __syncthreads();
        uint8_t *tile = buf ? tile1 : tile0;
        const uint32_t un = uc + n;
        const uint32_t nn = min(a.chunk, nu - un);
        if (nn) stage_rows<UNIT>(buf ? tile0 : tile1, src_of(un), nn * nr, rb, wave, lane);
        const uint32_t *tw = (const uint32_t *)tile;
        for (uint32_t it = slot; it < n * nr && !(a.dbg & 128); it += kSlots) {
            const uint32_t u = uc + it / nr, rr = it % nr;
            const uint32_t sel = P->sel[u];
            const uint32_t ps = P->pslot[u];
            float acc[NT];
#pragma unroll
            for (int t = 0; t < NT; t++) acc[t] = 0.f;
#pragma unroll
            for (int m = 0; m < GPT; m++) {
                const uint32_t g = gi + TPR * m;
                int32_t w[8];
                int mult;
                float d;
                group_w<TY>(stab, tile, tw, it * rb, g, w, mult, d);
                uint32_t s2 = ps;
#pragma unroll
                for (int t = 0; t < NT; t++) {
                    if (!((sel >> t) & 1u)) continue;
                    const int4 qa = *(const int4 *)(hq + (size_t)s2 * a.n_ff + 32 * g);
                    const int4 qb = *(const int4 *)(hq + (size_t)s2 * a.n_ff + 32 * g + 16);
                    int s = 0;
                    s = q4mi_sdot4(w[0], qa.x, s);
                    s = q4mi_sdot4(w[1], qa.y, s);
                    s = q4mi_sdot4(w[2], qa.z, s);
                    s = q4mi_sdot4(w[3], qa.w, s);
                    s = q4mi_sdot4(w[4], qb.x, s);
                    s = q4mi_sdot4(w[5], qb.y, s);
                    s = q4mi_sdot4(w[6], qb.z, s);
                    s = q4mi_sdot4(w[7], qb.w, s);
                    acc[t] = fmaf((float)(s * mult), d * hd[(size_t)s2 * (a.n_ff / 32) + g], acc[t]);
                    s2++;
                }
            }
#pragma unroll
            for (int t = 0; t < NT; t++) {
                const float v = ((sel >> t) & 1u) ? rsum<TPR>(acc[t]) : 0.f;
                if (gi == TPR - 1) part[((size_t)u * kMaxT + t) * kDnRows + rr] = v;
            }
        }
        __syncthreads();
        uc = un;
        n = nn;
        buf ^= 1u;
    }
    __syncthreads();
    // y[t][r] += sum_u w[u][t] * pd[u][t][r], u in plan order
    for (uint32_t i = tid; i < nt * nr; i += kThreads) {   // nt * nr <= kThreads
        const uint32_t t = i / nr, rr = i % nr;
        float s = 0.f;
        for (uint32_t u = 0; u < nu; u++)
            if ((P->sel[u] >> t) & 1u) s += P->w[u][t] * part[((size_t)u * kMaxT + t) * kDnRows + rr];
        a.y[(size_t)t * a.n_embd + r0 + rr] = yv + s;
    }
}

template <uint32_t TY, int NT, int TPR, int GPT>
static bool launch_gu(MoeArgs a, const HostList &hl, uint32_t nu_host) {
    const size_t fixed = (TY == Q4MI_T_IQ3_S ? 32768 : 0) + sizeof(Plan) + (size_t)NT * a.K +
                         (size_t)NT * (a.K / 32) * 4 + 32 * NT * 4;
    // pairs per chunk (two rows each; a divisor of the 32-row unit), two
    // chunk buffers in LDS
    uint32_t ch = 16;
    const size_t lds_cap = 150 * 1024;
    while (ch > 1 && fixed + 4ull * ch * a.rb_gu + 64 > lds_cap) ch /= 2;
    a.chunk = ch;
    const size_t lds = fixed + 4ull * ch * a.rb_gu + 64;
    const bool wide = ((((uintptr_t)a.base) | a.stride | a.og | a.ou | a.rb_gu) & 15u) == 0;
    const void *fn = wide ? (const void *)moe_gu_k<TY, NT, TPR, GPT, 16>
                          : (const void *)moe_gu_k<TY, NT, TPR, GPT, 4>;
    if (!ch || lds > lds_cap ||
        hipFuncSetAttribute(fn, hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds) !=
            hipSuccess) {
        set_error("moe_gu_k: LDS limit");
        return false;
    }
    // one block per CU, fewer when there is little work
    const uint32_t pairs = (nu_host ? nu_host : kMaxU) * a.n_ff;
    uint32_t grid = (uint32_t)cu_count();
    if (grid > pairs / 4) grid = pairs / 4 > 0 ? pairs / 4 : 1;
    if (wide)
        moe_gu_k<TY, NT, TPR, GPT, 16><<<dim3(grid), dim3(kThreads), lds, stream()>>>(a, hl);
    else
        moe_gu_k<TY, NT, TPR, GPT, 4><<<dim3(grid), dim3(kThreads), lds, stream()>>>(a, hl);
    return launch_ok("moe_gu_k");
}

template <uint32_t TY, int NT, int TPR, int GPT>
static bool launch_dn(MoeArgs a, const HostList &hl) {
    const size_t fixed = (TY == Q4MI_T_IQ3_S ? 32768 : 0) + sizeof(Plan) +
                         (size_t)kMaxU * kMaxT * kDnRows * 4 + (size_t)kMaxU * a.n_ff +
                         (size_t)kMaxU * (a.n_ff / 32) * 4;
    static_assert(kMaxT * kDnRows <= kThreads, "final reduce assumes one pass");
    uint32_t ch = 16;   // experts per chunk, two chunk buffers in LDS
    const size_t lds_cap = 150 * 1024;
    while (ch > 1 && fixed + 2ull * ch * kDnRows * a.rb_dn + 64 > lds_cap) ch--;
    a.chunk = ch;
    const size_t lds = fixed + 2ull * ch * kDnRows * a.rb_dn + 64;
    const bool wide = ((((uintptr_t)a.base) | a.stride | a.od | a.rb_dn) & 15u) == 0 &&
                      a.n_embd % kDnRows == 0;
    const void *fn = wide ? (const void *)moe_dn_k<TY, NT, TPR, GPT, 16>
                          : (const void *)moe_dn_k<TY, NT, TPR, GPT, 4>;
    if (!ch || lds > lds_cap ||
        hipFuncSetAttribute(fn, hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds) !=
            hipSuccess) {
        set_error("moe_dn_k: LDS limit");
        return false;
    }
    const uint32_t grid = (a.n_embd + kDnRows - 1) / kDnRows;
    if (wide)
        moe_dn_k<TY, NT, TPR, GPT, 16><<<dim3(grid), dim3(kThreads), lds, stream()>>>(a, hl);
    else
        moe_dn_k<TY, NT, TPR, GPT, 4><<<dim3(grid), dim3(kThreads), lds, stream()>>>(a, hl);
    return launch_ok("moe_dn_k");
}

template <uint32_t TY, int NT>
static bool gu_dispatch(const MoeArgs &a, const HostList &hl, uint32_t nu_host) {
    const RowLayout L = layout_for(a.K / 32);
#define Q4MI_L(T, P) \
    if (L.tpr == T && L.gpt == P) return launch_gu<TY, NT, T, P>(a, hl, nu_host);
    Q4MI_L(8, 1) Q4MI_L(16, 1) Q4MI_L(32, 1) Q4MI_L(64, 1) Q4MI_L(64, 2) Q4MI_L(64, 4)
#undef Q4MI_L
    return false;
}

template <uint32_t TY, int NT>
static bool dn_dispatch(const MoeArgs &a, const HostList &hl) {
    const RowLayout L = layout_for(a.n_ff / 32);
#define Q4MI_L(T, P) \
    if (L.tpr == T && L.gpt == P) return launch_dn<TY, NT, T, P>(a, hl);
    Q4MI_L(8, 1) Q4MI_L(16, 1) Q4MI_L(32, 1) Q4MI_L(64, 1) Q4MI_L(64, 2) Q4MI_L(64, 4)
#undef Q4MI_L
    return false;
}

// Measurement hook: bit 0 runs the gate/up launch, bit 1 the down launch
// (default both).  Lets a benchmark time each kernel of the pair alone.
static int g_phases = 3;

template <int NT>
static bool run_nt(uint32_t ty_gu, uint32_t ty_dn, const MoeArgs &a, const HostList &hl,
                   uint32_t nu_host) {
    if (g_phases & 1) {
        const bool ok = ty_gu == Q4MI_T_IQ3_S ? gu_dispatch<Q4MI_T_IQ3_S, NT>(a, hl, nu_host)
                                              : gu_dispatch<Q4MI_T_Q8_0, NT>(a, hl, nu_host);
        if (!ok) return false;
    }
    if (!(g_phases & 2)) return true;
    return ty_dn == Q4MI_T_IQ3_S ? dn_dispatch<Q4MI_T_IQ3_S, NT>(a, hl)
                                 : dn_dispatch<Q4MI_T_Q8_0, NT>(a, hl);
}

// Rows are staged with 4- or 16-byte copies, so a row's byte size must be a
// multiple of 4 (IQ3_S: K a multiple of 512; Q8_0: of 64).
static bool type_ok(uint32_t ty, uint32_t K) {
    if (ty != Q4MI_T_IQ3_S && ty != Q4MI_T_Q8_0) return false;
    const uint64_t rb = q4mi_row_bytes(ty, K);
    if (!rb || rb % 4 || K > 8192) return false;
    return layout_for(K / 32).tpr != 0;
}

static bool shape_ok(uint32_t gt, uint32_t ut, uint32_t dt, uint32_t in_dim, uint32_t n_ff,
                     uint32_t n_embd) {
    return gt == ut && type_ok(gt, in_dim) && type_ok(dt, n_ff) && n_embd == in_dim &&
           n_ff <= 1024;
}

bool moe_warm(uint32_t n_ff) {
    // q8 of h: kMaxU * kMaxT * n_ff codes + their fp32 scales
    if (!ensure_pd((size_t)kMaxU * kMaxT * n_ff / 4 + (size_t)kMaxU * kMaxT * n_ff / 32 + 64))
        return false;
    return iq3s_signed_table() != nullptr;
}

// Common driver.  All checks happen before the first launch so that a false
// return never leaves half of the work queued.
static bool moe_run(const uint8_t *base, uint64_t stride, const ListSrc &src,
                    const HostList &hl, uint32_t nu_host, uint32_t gt, uint64_t og, uint32_t ut,
                    uint64_t ou, uint32_t dt, uint64_t od, const float *d_x, float *d_y,
                    uint32_t n_ff, uint32_t in_dim, uint32_t n_embd) {
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
    if ((((uintptr_t)base) | stride | og | ou | od) & 3u) {
        set_error("moe: expert arena offsets must be 4-byte aligned");
        return false;
    }
    if (!moe_warm(n_ff)) return false;
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
    a.chunk = 0;
    a.x = d_x;
    a.hq = (int8_t *)scratch().pd;
    a.hd = (float *)((int8_t *)scratch().pd + (size_t)kMaxU * kMaxT * n_ff);
    a.y = d_y;
    a.stab = iq3s_signed_table();
    a.src = src;
    {
        static int dbg = -1;
        if (dbg < 0) {
            const char *e = getenv("Q4MI_DBG");
            dbg = e ? atoi(e) : 0;
        }
        a.dbg = (uint32_t)dbg;
    }
    const uint32_t nt = src.n_tok;
    if (nt == 1) return run_nt<1>(gt, dt, a, hl, nu_host);
    if (nt == 2) return run_nt<2>(gt, dt, a, hl, nu_host);
    if (nt <= 4) return run_nt<4>(gt, dt, a, hl, nu_host);
    return run_nt<8>(gt, dt, a, hl, nu_host);
}

}  // namespace q4mi

using namespace q4mi;

extern "C" void q4_mmvq_warm(void);

extern "C" {

/* Benchmark hook: 1 = gate/up launch only, 2 = down only, 3 = both. */
void q4mi_moe_phases(int mask) { g_phases = mask & 3; }

/* Allocate the decode scratch and tables (call before any stream capture). */
void q4_hip_moe_scratch_warm(void) {
    (void)moe_warm(1024);
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
    // unique ids in first-appearance order; a repeated id keeps the weight
    // of its last occurrence (the device plan's rule for device lists)
    HostList hl;
    uint32_t nu = 0;
    for (uint32_t i = 0; i < n; i++) {
        if (slots[i] < 0) continue;
        uint32_t u = 0;
        while (u < nu && hl.id[u] != slots[i]) u++;
        if (u == nu) hl.id[nu++] = slots[i];
        hl.w[u] = wts[i];
    }
    for (uint32_t i = nu; i < kMaxU; i++) {
        hl.id[i] = -1;
        hl.w[i] = 0.f;
    }
    if (!nu) return true;
    ListSrc src = {nullptr, nullptr, nullptr, kMaxU, 1, nu, 1};
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
    ListSrc src = {d_es, d_ew, d_nhit, kMaxU, 1, 0, 0};
    return moe_run(base, stride, src, hl, 0, gt, og, ut, ou, dt, od, d_x, d_y, n_ff, in_dim,
                   n_embd);
}

/* Window coverage: 2..8 tokens, gate type == up type, IQ3_S or Q8_0 with a
 * covered K (the reference additionally limited the down type; here every
 * covered type runs the window). */
bool q4_hip_moe_win_ok(uint32_t gt, uint32_t ut, uint32_t dt, uint32_t in_dim, uint32_t n_ff,
                       uint32_t n_tok) {
    return n_tok >= 2 && n_tok <= kMaxT && gt == ut && type_ok(gt, in_dim) &&
           type_ok(dt, n_ff) && n_ff <= 1024;
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

}  // extern "C"
