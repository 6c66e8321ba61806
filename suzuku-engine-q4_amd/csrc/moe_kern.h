// Routed-expert decode / verify-window kernels and their launch templates,
// shared by the translation units that instantiate them per weight type
// (moe_decode.hip: IQ3_S and Q8_0, plus the host entry points;
// moe_fmt_gu.hip / moe_fmt_dn.hip: the other formats of formats.h).
// Routed-expert decode (1 token) and verify window (2..8 tokens) over
// experts resident at base + slot*stride (gate/up IQ3_S, Q8_0, IQ2_S; down
// IQ3_S, Q8_0, IQ4_NL, Q2_0, IQ2_S).
//
// Two launches per layer, one 1024-thread block per CU:
//   moe_gu_k  the (unique expert u, intermediate row r) pairs are split into
//             one contiguous share per block; h[u][t][r] =
//             silu(gate_r . q8(x_t)) * (up_r . q8(x_t)) goes out as fp32.
//   moe_dn_k  each block owns 8 output rows: it quantizes every selected
//             h[u][t] (q8, 32-value groups) into LDS, dots its rows of every
//             expert's down matrix and writes y[t][r] += sum_u w[u][t] *
//             part[u][t][r] in unique-expert order -- deterministic, no atomics.
// Each unique expert's rows are read once per launch and dotted with every
// token that selected it (the verify window's reuse; reference
// q4_hip_moe_exec_win src/q4_rocm.cu:7444-7531, CPU twin
// q4_cpuex_dispatch_win src/q4_cpuexp.c:2618-2753).
//
// Memory pipeline (both kernels), after the block's single barrier:
//   producers (waves 0..kProd-1) issue the block's weight rows as chunks
//     into an LDS ring with gfx950 global_load_lds (no registers) and
//     publish each chunk (landed[] in LDS) once its own copies are complete,
//     waiting with s_waitcnt vmcnt(#copies issued after it): VMEM loads of a
//     wave complete in issue order, so no wait covers more than it needs;
//     a slot is refilled only after its previous chunk was consumed;
//   consumers (the other waves) load the codebook and x (or h) through
//     registers in the prologue, build the signed table and the q8
//     activations in LDS, then compute each (expert, row) item as soon as
//     its chunk is published and count it consumed (cons[] in LDS).
//
// IQ3_S decode: one LDS lookup per 4 values into an 8192-entry table of
// signed int8 quads (index = sign nibble << 9 | qh bit << 8 | qs byte), built
// in LDS from the 512-entry codebook at kernel start.  The index of quad k
// is one v_perm_b32 of the qs bytes with a per-group byte vector of
// (sign nibble << 1 | qh bit); then v_dot4_i32_i8 per quad and token, the
// (2s+1) multiplier on the exact int32 group sum, and float(S) * (d_w * d_x).
#pragma once
#include <stddef.h>
#include <stdlib.h>
#include <string.h>

#include <algorithm>

#include "formats.h"
#include "mmvq_engine.h"
#include "route_wave.h"
#include "q4mi_internal.h"

namespace q4mi {

constexpr uint32_t kMaxU = 64;    // unique experts per call (reference bound n<=64)
constexpr uint32_t kMaxT = 8;     // tokens per call
#ifndef Q4MI_THREADS
#define Q4MI_THREADS 1024
#endif
constexpr uint32_t kT = Q4MI_THREADS;   // threads per block
#ifndef Q4MI_PROD
#define Q4MI_PROD 4
#endif
constexpr uint32_t kProd = Q4MI_PROD;   // producer waves (issue the LDS copies)
constexpr uint32_t kCons = kT - kProd * 64;   // consumer threads
constexpr uint32_t kConsW = kCons / 64;       // consumer waves
constexpr uint32_t kDnRows = 8;       // output rows per down block (a call may take more)
constexpr uint32_t kDnRowsMax = 16;   // ... up to this many, so the grid fits the CUs
constexpr uint32_t kMaxS = 32;    // LDS ring slots
constexpr int kSrcDev = 0, kSrcHost = 1, kSrcLogits = 2;   // list source of a launch
// x quads per consumer thread loaded before the block barrier: all of a
// window's, and a decode token's with the least prologue code (the prologue
// runs with a cold instruction cache, on the critical path)
template <int NT> constexpr uint32_t kXPre = NT == 1 ? 1u : 4u;
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
    // One token's router logits in place of the lists (lg non-null): the
    // plan's entries are route_k's top-k of lg [n_exp] plus, with shared >= 0,
    // expert `shared` at weight sg[0] (or 1); gate/up block 0 writes them to
    // o_ids / o_wts / o_nh (row 0, topk + 1 entries) as route_k would.
    const float *lg;
    const float *sg;
    int32_t *o_ids;
    float *o_wts;
    int32_t *o_nh;
    uint32_t n_exp, topk;
    int32_t shared;
};

struct __align__(16) Plan {
    uint32_t nu;
    uint32_t nsel;                  // selected (u, t) pairs
    int32_t uid[kMaxU];
    uint32_t sel[kMaxU];            // token bitmask per unique expert
    uint32_t pslot[kMaxU];          // first pair slot of u (slots in (u, t) order)
    uint32_t prow[kMaxU];           // pair slot -> h row u * kMaxT + t
    float w[kMaxT][kMaxU];          // routing weight of (token, unique expert)
    uint32_t ends[kProd][kMaxS];    // per producer: copies issued up to the end of a ring chunk
};

// Device lists: wave 0 builds the plan (first-appearance order over
// (token, pick)); callers sync afterwards.
// LG: the source holds one token's router logits (ListSrc::lg) instead of
// the lists; a separate instantiation, so that the other kernels do not
// carry the top-k code (their start-up runs with a cold instruction cache).
template <bool LG>
__device__ void build_plan(Plan *P, const ListSrc &s, uint32_t lane, uint32_t *ht) {
    uint32_t E = 0, tok = 0;
    int32_t id = -1;
    float w = 0.f;
    if constexpr (LG) {
        // one token's router logits: route_k's top-k (same code, same
        // picks and weights) and the shared entry after them; gate/up block
        // 0 also writes them out as route_k's lists
        int32_t *s_id = (int32_t *)(ht + 1024);
        float *s_p = (float *)(ht + 1024 + 64);
        const uint32_t tk = route_wave<8>(s.lg, s.n_exp, s.topk, lane, s_id, s_p);
        float sk = 0.f;
        for (uint32_t k = 0; k < tk; k++) sk += s_p[k];
        const float inv2 = sk > 0.f ? __fdiv_rn(1.f, sk) : 0.f;
        const uint32_t nsh = s.shared >= 0 ? 1u : 0u;
        E = s.topk + nsh;
        if (lane < s.topk) {
            id = lane < tk ? s_id[lane] : -1;
            w = lane < tk ? (sk > 0.f ? s_p[lane] * inv2 : s_p[lane]) : 0.f;
        } else if (lane == s.topk && nsh) {
            id = s.shared;
            w = s.sg ? s.sg[0] : 1.f;
        }
        if (s.o_ids && blockIdx.x == 0) {
            if (lane < E) {
                s.o_ids[lane] = id;
                s.o_wts[lane] = w;
            }
            if (lane == 0 && s.o_nh) s.o_nh[0] = (int32_t)E;
        }
    } else {
        // lane -> (token, pick) of the flattened lists, token-major
        // every token's count in one load (lane t holds token t's), then
        // read back lane by lane: one memory round trip, not one per token
        const int cnt_l = lane < s.n_tok ? (s.nh ? s.nh[lane] : (int)s.n_fixed) : 0;
        // the entries are loaded in the same round trip as the counts, assuming
        // each token has at most CAP = 64 / (n_tok rounded up to a power of two)
        // of them (lane l: token l / CAP, entry l % CAP; within the lists' rows);
        // a longer list loads them again once the counts are known
        const uint32_t cap_sh = s.n_tok <= 1 ? 6u : s.n_tok == 2 ? 5u : s.n_tok <= 4 ? 4u : 3u;
        const uint32_t st = lane >> cap_sh, sr = lane & ((1u << cap_sh) - 1u);
        int32_t sid = -1;
        float sw = 0.f;
        if (st < s.n_tok && sr < s.stride) {
            sid = s.es[(size_t)st * s.stride + sr];
            sw = s.ew[(size_t)st * s.stride + sr];
        }
        uint32_t rem = 0;
        bool found = false;
        for (uint32_t t = 0; t < s.n_tok; t++) {
            int c = __builtin_amdgcn_readlane(cnt_l, t);
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
        if (__ballot(lane < E && rem >= (1u << cap_sh)) == 0) {
            const int src = (int)((tok << cap_sh) + rem);
            const int32_t gid = __shfl(sid, src);
            const float gw = __shfl(sw, src);
            if (lane < E) {
                id = gid;
                w = gw;
            }
        } else if (lane < E) {
            id = s.es[(size_t)tok * s.stride + rem];
            w = s.ew[(size_t)tok * s.stride + rem];
        }
    }
    const bool valid = lane < E && id >= 0;
    // First occurrence of each id, through a 1024-bucket table in LDS (ht,
    // 4 KB of the not-yet-used ring): every valid lane takes the minimum
    // lane of its bucket; that lane holds the first occurrence of the id
    // unless it holds another id of the same bucket (ids 1024 apart), which
    // only the exact pass over the lanes (v_readlane per lane) settles.
    const uint64_t vmask = __ballot(valid);
    const uint32_t hb = (uint32_t)id & 1023u;
    if (valid) ht[hb] = 0xFFFFFFFFu;
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQ_REL, "workgroup");
    if (valid) atomicMin(&ht[hb], lane);
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQ_REL, "workgroup");
    const uint32_t mlane = valid ? ht[hb] : lane;
    const bool clash = valid && __shfl(id, (int)mlane) != id;
    uint32_t first_j = (valid && !clash) ? mlane : lane;
    if (__builtin_expect(__ballot(clash) != 0, 0)) {
        first_j = lane;
        for (uint32_t j = 0; j < E; j++) {
            if (!((vmask >> j) & 1ull)) continue;
            const int32_t idj = __builtin_amdgcn_readlane(id, j);
            if (idj == id && j < first_j) first_j = j;
        }
    }
    const bool first = valid && first_j == lane;
    const uint64_t fm = __ballot(first);
    const uint32_t u = (uint32_t)__popcll(fm & ((1ull << first_j) - 1ull));
    for (uint32_t i = lane; i < kMaxU; i += 64) {
        P->sel[i] = 0;
        P->uid[i] = -1;
#pragma unroll
        for (uint32_t t = 0; t < kMaxT; t++) P->w[t][i] = 0.f;
    }
    const uint32_t nu = (uint32_t)__popcll(fm);
    if (lane == 0) P->nu = nu;
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup");
    if (first) P->uid[u] = id;
    if (valid) {   // a token's repeated id adds its weights
        atomicOr(&P->sel[u], 1u << tok);
        atomicAdd(&P->w[tok][u], w);
    }
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQ_REL, "workgroup");
    // pair slots: pslot[u] = sum over v < u of popcount(sel[v]), counted
    // per token bit with a ballot and mbcnt (no cross-lane round trips)
    const uint32_t sl = lane < nu ? P->sel[lane] : 0u;
    uint32_t below = 0, nsel = 0;
#pragma unroll
    for (uint32_t t = 0; t < kMaxT; t++) {
        const uint64_t b = __ballot((sl >> t) & 1u);
        below += __builtin_amdgcn_mbcnt_hi((uint32_t)(b >> 32),
                                           __builtin_amdgcn_mbcnt_lo((uint32_t)b, 0u));
        nsel += (uint32_t)__popcll(b);
    }
    if (lane < nu) {
        P->pslot[lane] = below;
        uint32_t k = below;
        for (uint32_t t = 0; t < kMaxT; t++)
            if ((sl >> t) & 1u) P->prow[k++] = lane * kMaxT + t;
    }
    if (lane == 0) P->nsel = nsel;
}

// ------------------------------------------------------------ LDS pipeline
// Workgroup barrier without the compiler's fence: LDS ops of this wave are
// complete (lgkmcnt) but outstanding VMEM copies are left in flight.
__device__ inline void bar() { asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory"); }

// One global -> LDS wave copy (gfx950 global_load_lds): lane i's UNIT bytes
// at g land at LDS byte address m0 + i*UNIT.  Written as inline asm so that
// the compiler does not track it: its own tracking of LDS copies waits for
// all of them (vmcnt(0)) before any later LDS read, which would serialize
// the pipeline.  Completion is this library's business: wait_vm + bar.
template <uint32_t UNIT>
__device__ inline void lds_copy(const void *g, uint32_t lds_addr) {
    lds_addr = __builtin_amdgcn_readfirstlane(lds_addr);
    if constexpr (UNIT == 16)
        asm volatile("s_mov_b32 m0, %1\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %0, off"
                     :: "v"(g), "s"(lds_addr) : "memory", "m0");
    else
        asm volatile("s_mov_b32 m0, %1\n\ts_nop 0\n\tglobal_load_lds_dword %0, off"
                     :: "v"(g), "s"(lds_addr) : "memory", "m0");
}

// LDS address of a generic pointer into LDS: the low half of a flat address
// in the LDS aperture (an address-space cast would add a null check)
__device__ inline uint32_t lds_addr_of(const void *p) { return (uint32_t)(uintptr_t)p; }

// Asynchronous copy of `bytes` (a multiple of UNIT, both ends UNIT-aligned)
// global -> LDS by the calling wave, in operations of 64*UNIT bytes.
// Returns the number of operations issued.
template <uint32_t UNIT>
__device__ inline uint32_t dma1(uint8_t *dst, const uint8_t *src, uint32_t bytes, uint32_t lane) {
    constexpr uint32_t OPB = 64 * UNIT;
    const uint32_t nops = (bytes + OPB - 1) / OPB;
    const uint32_t l0 = lds_addr_of(dst);
    for (uint32_t j = 0; j < nops; j++) {
        const uint32_t off = j * OPB + lane * UNIT;
        if (off < bytes) lds_copy<UNIT>(src + off, l0 + j * OPB);
    }
    return nops;
}

// Signed IQ3_S table in LDS, built by the consumer threads from the
// 512-entry codebook.  Thread ct owns entries ct, ct + kCons, ... (the first
// one's code `c` loaded by the caller).
__device__ inline void build_stab(uint32_t *stab, uint32_t c, uint32_t ct) {
    for (uint32_t i = ct; i < 512; i += kCons) {
        if (i != ct) c = q4mi_iq3s_code_dev[i];
        uint32_t g = 0;
#pragma unroll
        for (int j = 0; j < 4; j++) g |= (2u * ((c >> (3 * j)) & 7u) + 1u) << (8 * j);
#pragma unroll
        for (uint32_t s4 = 0; s4 < 16; s4++)
            stab[(s4 << 9) | i] = (uint32_t)q4mi_sign4(g, q4mi_expand4(s4));
    }
}

// q8 of quad i (values 4i..4i+3) of a run of 32-value groups: the 8 lanes
// holding quads 8g..8g+7 quantize group g together (all 8 must be active).
__device__ inline void quant_quad(float4 v, uint32_t i, int8_t *q, float *d) {
    float dd;
    int bs;
    const uint32_t c = q4mi_quant_team8(v, &dd, &bs);
    ((uint32_t *)q)[i] = c;
    if ((i & 7u) == 0) d[i / 8] = dd;
}


// Signed int8 quads of one IQ3_S group from its raw bytes: q0, q1 = the 8
// qs bytes, qh = its high-bit byte, sg = its 4 sign bytes.
__device__ inline void iq3s_quads(const uint32_t *stab, uint32_t q0, uint32_t q1, uint32_t qh,
                                  uint32_t sg, int32_t (&w)[8]) {
    // byte k of hlo / hhi: (sign nibble << 1 | qh bit) of quad k / k+4
    const uint32_t ne = sg & 0x0F0F0F0Fu, no = (sg >> 4) & 0x0F0F0F0Fu;
    const uint32_t slo = __builtin_amdgcn_perm(no, ne, 0x05010400u);
    const uint32_t shi = __builtin_amdgcn_perm(no, ne, 0x07030602u);
    const uint32_t blo = __umul24(qh & 15u, 0x00204081u) & 0x01010101u;
    const uint32_t bhi = __umul24((qh >> 4) & 15u, 0x00204081u) & 0x01010101u;
    const uint32_t hlo = (slo << 1) | blo, hhi = (shi << 1) | bhi;
#pragma unroll
    for (int k = 0; k < 8; k++) {
        const uint32_t sel = 0x0C0C0000u | ((4u + (k & 3)) << 8) | (uint32_t)(k & 3);
        const uint32_t idx = __builtin_amdgcn_perm(k < 4 ? hlo : hhi, k < 4 ? q0 : q1, sel);
        w[k] = (int32_t)stab[idx];
    }
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
    iq3s_quads(stab, q0, q1, qh, sg, w);
}

// Groups g and g + 1 (g even: one superblock, one scale byte) with their
// shared reads done once: d, the scale byte, both qh bytes in one 16-bit
// read (B is even), the 16 qs bytes from five dwords.
__device__ inline void iq3s_group2(const uint32_t *stab, const uint8_t *lb, const uint32_t *lw,
                                   uint32_t row, uint32_t g, int32_t (&wa)[8], int32_t (&wb)[8],
                                   int &ma, int &mb, float &d) {
    const uint32_t B = row + (g >> 3) * IQ3S_BYTES;
    const uint32_t j = g & 7u;
    d = q4mi_h2f(lds_u16_at(lb, B));
    const uint32_t qo = B + 2u + 8u * j;
    const uint32_t i0 = qo >> 2, sh = qo & 3u;
    const uint32_t w0 = lw[i0], w1 = lw[i0 + 1], w2 = lw[i0 + 2], w3 = lw[i0 + 3],
                   w4 = lw[i0 + 4];
    const uint32_t qh2 = lds_u16_at(lb, B + 66u + j);
    const uint32_t sga = lds_u32_at(lw, B + 74u + 4u * j);
    const uint32_t sgb = lds_u32_at(lw, B + 78u + 4u * j);
    const uint32_t sc = lb[B + 106u + (j >> 1)];
    ma = 2 * (int)(sc & 15u) + 1;
    mb = 2 * (int)(sc >> 4) + 1;
    iq3s_quads(stab, __builtin_amdgcn_alignbyte(w1, w0, sh), __builtin_amdgcn_alignbyte(w2, w1, sh),
               qh2 & 0xffu, sga, wa);
    iq3s_quads(stab, __builtin_amdgcn_alignbyte(w3, w2, sh), __builtin_amdgcn_alignbyte(w4, w3, sh),
               qh2 >> 8, sgb, wb);
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

// LDS table bytes of a format's decoder (at the start of the kernel's LDS).
template <uint32_t TY>
__host__ __device__ constexpr uint32_t tab_bytes() {
    if constexpr (TY == Q4MI_T_IQ3_S) return 32768u;
    else if constexpr (TY == Q4MI_T_Q8_0) return 0u;
    else return (uint32_t)FmtOf<TY>::F::kTabBytes;
}
template <uint32_t TY>
__host__ __device__ constexpr bool two_mult() {
    return TY == Q4MI_T_IQ2_S || TY == Q4MI_T_IQ2_XS;
}

// One 32-value group: signed quads, the multipliers of quads 0-3 / 4-7 and
// the block scale (formats.h for the types beside IQ3_S / Q8_0).
template <uint32_t TY>
__device__ inline void group_w(const uint32_t *stab, const uint8_t *lb, const uint32_t *lw,
                               uint32_t row, uint32_t g, int32_t (&w)[8], int &mult, int &mult2,
                               float &d) {
    if constexpr (TY == Q4MI_T_IQ3_S) {
        iq3s_group(stab, lb, lw, row, g, w, mult, d);
        mult2 = mult;
    } else if constexpr (TY == Q4MI_T_Q8_0) {
        q80_group(lb, lw, row, g, w, mult, d);
        mult2 = mult;
    } else {
        WGroup o;
        FmtOf<TY>::F::decode(stab, lb, lw, row, g, o);
#pragma unroll
        for (int k = 0; k < 8; k++) w[k] = o.w[k];
        mult = o.m1;
        mult2 = o.m2;
        d = o.d;
    }
}

// Exact group sum of one token: m1 * quads 0-3 + m2 * quads 4-7 (24-bit
// multiplies, full rate: |sums| < 2^20, |multipliers| <= 2^7).
template <uint32_t TY>
__device__ inline int tsum(const int32_t (&w)[8], const int32_t (&q)[8], int m1, int m2) {
    if constexpr (two_mult<TY>()) {
        int a = 0, b = 0;
#pragma unroll
        for (int k = 0; k < 4; k++) a = q4mi_sdot4(w[k], q[k], a);
#pragma unroll
        for (int k = 4; k < 8; k++) b = q4mi_sdot4(w[k], q[k], b);
        return __mul24(a, m1) + __mul24(b, m2);
    } else {
        int s = 0;
#pragma unroll
        for (int k = 0; k < 8; k++) s = q4mi_sdot4(w[k], q[k], s);
        return __mul24(s, m1);
    }
}

// The decoder's LDS tables, built by the consumer threads (ct of kCons).
template <uint32_t TY>
__device__ inline void build_tables(uint8_t *smem, uint32_t code, uint32_t ct);

struct MoeArgs {
    const uint8_t *base;
    uint64_t stride, og, ou, od;
    uint64_t stride_d;  // bytes between experts' down matrices (= stride when packed)
    uint32_t K;       // in_dim (gate/up columns)
    uint32_t n_ff;
    uint32_t n_embd;
    uint32_t rb_gu, rb_dn;
    uint32_t chunk;   // gate/up: pairs per chunk; down: experts per chunk
    uint32_t ahead;   // chunks a producer may have issued and not yet published (<= kMaxS)
    uint32_t slots;   // LDS ring slots (<= kMaxS)
    uint32_t nsel_cap;  // down: q8(h) rows the LDS holds
    uint32_t dn_rows;   // down: output rows per block (kDnRows .. kDnRowsMax)
    const float *x;   // [n_tok][K]
    float *h;         // [kMaxU][kMaxT][n_ff] fp32 h
    float *y;         // [n_tok][n_embd], accumulated
    ListSrc src;
#ifdef Q4MI_TRACE
    unsigned long long *trace;   // [2 kernels][4096 blocks][32] phase timestamps
    uint32_t dbg;                // trace build experiments (Q4MI_DBG)
#endif
    Plan *gplan;      // device list: the plan gate/up block 0 publishes for down
    uint32_t plan_in; // down: load gplan instead of building the plan
    HostList hl;      // host list (src.unique), read in place from the kernel arguments
};

// Optional build (-DQ4MI_TRACE): the first producer and the first consumer
// thread of every block record wall-clock phase timestamps (10 ns ticks).
#ifdef Q4MI_TRACE
#define Q4MI_TR_DECL(b) unsigned long long *const q4tr = a.trace; const uint32_t q4bid = (b)
#define Q4MI_TR(k, kern, who) do { if (q4tr && (who)) q4tr[((size_t)(kern) * 4096 + q4bid) * 32 + (k)] = wall_clock64(); } while (0)
#else
#define Q4MI_TR_DECL(b) do { } while (0)
#define Q4MI_TR(k, kern, who) do { } while (0)
#endif

// The kernel's own argument block (kernel parameters start at offset 0 of
// the kernarg segment).  Uniform reads through it are scalar loads, and the
// host list can be copied from it into LDS like any other global bytes.
typedef const __attribute__((address_space(4))) MoeArgs *KArgs;
__device__ inline KArgs kargs() { return (KArgs)__builtin_amdgcn_kernarg_segment_ptr(); }

// The host list's ids, one per lane (lane u holds id u), gathered with
// constant-offset scalar loads (a vector load of the kernel arguments costs
// a full memory round trip at kernel start).
typedef const __attribute__((address_space(4))) int32_t *KWords;

template <int K>
__device__ inline int32_t put_lane(int32_t v, int32_t s) {
    asm("v_writelane_b32 %0, %1, %2" : "+v"(v) : "s"(s), "i"(K));
    return v;
}
// Words [16B, 16B + 16) of w into lanes 16B.. of v: sixteen constant-offset
// scalar loads (merged into wide loads) and sixteen v_writelane.
template <int B>
__device__ inline int32_t put16(int32_t v, KWords w) {
    int32_t s[16];
#pragma unroll
    for (int k = 0; k < 16; k++) s[k] = w[16 * B + k];
    v = put_lane<16 * B + 0>(v, s[0]);   v = put_lane<16 * B + 1>(v, s[1]);
    v = put_lane<16 * B + 2>(v, s[2]);   v = put_lane<16 * B + 3>(v, s[3]);
    v = put_lane<16 * B + 4>(v, s[4]);   v = put_lane<16 * B + 5>(v, s[5]);
    v = put_lane<16 * B + 6>(v, s[6]);   v = put_lane<16 * B + 7>(v, s[7]);
    v = put_lane<16 * B + 8>(v, s[8]);   v = put_lane<16 * B + 9>(v, s[9]);
    v = put_lane<16 * B + 10>(v, s[10]); v = put_lane<16 * B + 11>(v, s[11]);
    v = put_lane<16 * B + 12>(v, s[12]); v = put_lane<16 * B + 13>(v, s[13]);
    v = put_lane<16 * B + 14>(v, s[14]); v = put_lane<16 * B + 15>(v, s[15]);
    return v;
}
// The first n words of w, word k in lane k (entries beyond n keep `fill`).
__device__ inline int32_t host_words(KWords w, uint32_t n, int32_t fill) {
    int32_t v = fill;
    v = put16<0>(v, w);
    if (n > 16) v = put16<1>(v, w);
    if (n > 32) v = put16<2>(v, w);
    if (n > 48) v = put16<3>(v, w);
    return v;
}
__device__ inline int32_t host_ids(KArgs ka, uint32_t n) { return host_words(ka->hl.id, n, -1); }
__device__ inline float host_weights(KArgs ka, uint32_t n) {
    return __builtin_bit_cast(float, host_words((KWords)ka->hl.w, n, 0));
}


__host__ __device__ inline size_t al16(size_t v) { return (v + 15) & ~(size_t)15; }

__device__ inline float silu_f(float v) { return v / (1.f + expf(-v)); }


// ------------------------------------------------------------- pipeline sync
// Producer waves never take part in a barrier (a copy issue stalls while
// the memory system is saturated, and a stalled producer must not hold the
// consumers back).  All hand-offs go through LDS counters instead:
//   Sync::landed[p]  chunks of producer p that have landed (chunk c belongs
//                    to producer c % kProd, landed in order)
//   Sync::cons[s]    items finished in the chunk held by ring slot s
//   Sync::owner[s]   that chunk's index
//   Sync::ready      consumer waves done with the shared prologue work
//   Sync::fin        consumer waves done with every item
struct Sync {
    uint32_t ready;
    uint32_t fin;
    uint32_t landed[kProd];
    uint32_t cons[kMaxS];
    uint32_t owner[kMaxS];   // chunk last issued into ring slot s
};

__device__ inline uint32_t lds_ld(const uint32_t *p) { return *(const volatile uint32_t *)p; }
__device__ inline void lds_st(uint32_t *p, uint32_t v) {
    asm volatile("" ::: "memory");
    *(volatile uint32_t *)p = v;
}
// Every wait is bounded: a block that would wait longer than about 0.1 s
// gives up and runs on, so a protocol error can never hang the device.  Its
// results are then wrong, and the block records that in g_moe_status (bit
// kStConsumer / kStProducer), which q4mi_device_status() reads back after
// the stream drained and reports through q4mi_last_error().
constexpr uint32_t kSpinMax = 1u << 22;
constexpr uint32_t kStConsumer = 1u;   // a consumer wait timed out
constexpr uint32_t kStProducer = 2u;   // a producer's slot wait timed out
static __device__ uint32_t g_moe_status;   // one per translation unit

__device__ inline void note_timeout(uint32_t bit) { atomicOr(&g_moe_status, bit); }

// Wait until *p >= v; later LDS reads stay after the poll.
__device__ inline void spin_ge(const uint32_t *p, uint32_t v) {
    uint32_t n = 0;
    for (; lds_ld(p) < v && n < kSpinMax; n++) __builtin_amdgcn_s_sleep(1);
    if (__builtin_expect(n == kSpinMax, 0)) note_timeout(kStConsumer);
    asm volatile("" ::: "memory");
}
__device__ inline void wait_chunk(const Sync *y, uint32_t c) {
    spin_ge(&y->landed[c % kProd], c / kProd + 1);
}

// Producer side of the ring: chunks c = p, p + kProd, ... are issued while
// their slot is free and published (landed[p]++) in order.  A slot is free
// once the consumers finished every item of the chunk it held (cons[s]).
// The producer never waits on a slot while one of its own issued chunks is
// unpublished, so it cannot hold back a chunk the consumers are waiting for.
template <class IssueFn, class ItemsFn>
__device__ inline void produce(Sync *y, uint32_t *ends, uint32_t p, uint32_t C, uint32_t S,
                               uint32_t ahead, uint32_t &issued, IssueFn issue, ItemsFn items
#ifdef Q4MI_TRACE
                               , unsigned long long *q4tr = nullptr, uint32_t q4kern = 0
#endif
                               ) {
#ifdef Q4MI_TRACE
    const uint32_t q4bid = blockIdx.x;
#endif
    uint32_t next = p, pub = p;    // next chunk to issue / to publish
    // Slot c % S is free for chunk c once chunk c - S (its previous user,
    // possibly another producer's) was issued there and fully consumed.  The
    // owner check matters when S is not a multiple of kProd: the count alone
    // could still be the one left by chunk c - 2S.
    auto slot_free = [&](uint32_t c) {
        return c < S || (lds_ld(&y->owner[c % S]) == c - S &&
                         lds_ld(&y->cons[c % S]) >= items(c - S));
    };
    uint32_t idle = 0;
#ifdef Q4MI_TRACE
    uint32_t npub = 0, nloop = 0;
#endif
#ifdef Q4MI_TRACE
    Q4MI_TR(17, q4kern, p == 0 && (threadIdx.x & 63u) == 0);
#endif
#if !defined(Q4MI_TRACE) && !defined(Q4MI_KNOBS)
    ahead = 1;   // the product's setting, as a constant (one chunk in flight)
#endif
    while (pub < C && idle < kSpinMax) {
        while (next < C && (next < pub + kProd * ahead) && slot_free(next)) {
            if (next >= S) lds_st(&y->cons[next % S], 0);
            lds_st(&y->owner[next % S], next);
            issue(next);
#ifdef Q4MI_TRACE
            if (next / kProd < 3) Q4MI_TR(24 + next / kProd, q4kern, p == 0 && (threadIdx.x & 63u) == 0);
#endif
            ends[(next / kProd) % kMaxS] = issued;
            next += kProd;
        }
#ifdef Q4MI_TRACE
        if (nloop++ == 0) Q4MI_TR(20, q4kern, p == 0 && (threadIdx.x & 63u) == 0);
#endif
        if (pub < next) {
#if !defined(Q4MI_TRACE) && !defined(Q4MI_KNOBS)
            asm volatile("s_waitcnt vmcnt(0)" ::: "memory");   // its only chunk in flight
#else
            wait_vm(issued - ends[(pub / kProd) % kMaxS]);
#endif
            lds_st(&y->landed[p], pub / kProd + 1);
#ifdef Q4MI_TRACE
            if (npub < 4) Q4MI_TR(21 + npub, q4kern, p == 0 && (threadIdx.x & 63u) == 0);
            npub++;
#endif
            pub += kProd;
        } else {
            __builtin_amdgcn_s_sleep(1);   // every own chunk published; wait for a slot
            idle++;
        }
    }
    if (__builtin_expect(pub < C, 0)) note_timeout(kStProducer);
    wait_vm(0);
}

template <uint32_t TY>
__device__ inline void build_tables(uint8_t *smem, uint32_t code, uint32_t ct) {
    if constexpr (TY == Q4MI_T_IQ3_S)
        build_stab((uint32_t *)smem, code, ct);
    else if constexpr (tab_bytes<TY>() != 0)
        FmtOf<TY>::F::init(smem, ct, kCons);
}

// ------------------------------------------------------------- gate / up
// Roles: waves 0..kProd-1 produce (issue the weight copies global -> LDS),
// the other waves consume (build the IQ3_S table, quantize x, compute).  The
// block's share of (u, r) pairs is cut into chunks of `ch` pairs that flow
// through a ring of S LDS slots; consumer team j (TPR lanes) computes pairs
// j, j + teams, ... as soon as their chunk has landed.
//
// LDS: [stab 32 KB] (IQ3_S) Plan Sync | xq [NT][K] | xd [NT][K/32] | ring of
//      S slots, slot = gate rows[ch] then up rows[ch].
//
// Block `bid` of `nblk` takes pairs [share_lo(bid), share_lo(bid + 1)).
__device__ inline uint32_t share_lo(uint32_t PT, uint32_t bid, uint32_t nblk) {
    // the first PT % nblk blocks take one pair more (one 32-bit division:
    // a 64-bit one is ~100 scalar instructions of start-up code)
    const uint32_t q = PT / nblk, r = PT % nblk;
    return bid * q + min(bid, r);
}

// First pair of block `bid` when the blocks split the pairs by work: a pair
// of unique expert u costs 2 + (tokens that picked u) -- one decode of its
// gate and up rows shared by all of them, one dot per token -- so the
// blocks holding an expert every token picked (the shared expert) get fewer
// pairs.  Every wave computes the same value (lane u: expert u).
__device__ inline void share_weighted(const Plan *P, uint32_t nu, uint32_t n_ff, uint32_t bid,
                                      uint32_t nblk, uint32_t lane, uint32_t &p0,
                                      uint32_t &p1) {
    const uint32_t c = lane < nu ? 2u + (uint32_t)__popc(P->sel[lane]) : 0u;
    const uint32_t incl = q4mi_wave_incl_scan(c);
    const uint32_t total = (uint32_t)__builtin_amdgcn_readlane((int)incl, 63);
    auto at = [&](uint32_t b) -> uint32_t {
        if (b >= nblk) return nu * n_ff;
        // target in units of 1/n_ff of an expert's cost: t = total * n_ff * b /
        // nblk (< 2^32: total <= 64 * 10, n_ff <= 1024, b < 4096)
        const uint32_t t = total * n_ff * b / nblk;
        // expert u0 = number of experts whose whole cost ends at or before t
        const uint64_t done = __ballot(incl * n_ff <= t && lane < nu);
        const uint32_t u0 = (uint32_t)__popcll(done);
        if (u0 >= nu) return nu * n_ff;
        const uint32_t ex = (uint32_t)__builtin_amdgcn_readlane((int)(incl - c), (int)u0);
        const uint32_t cu = (uint32_t)__builtin_amdgcn_readlane((int)c, (int)u0);
        const uint32_t into = (t - ex * n_ff) / cu;   // pairs of u0 before t
        return u0 * n_ff + min(into, n_ff);
    };
    p0 = at(bid);
    p1 = at(bid + 1);
}

// Producer: issue pairs [p0, p1) of the block (gate rows then up rows per
// chunk).  idv holds expert id u in lane u.
template <uint32_t UNIT>
__device__ inline void gu_produce(const MoeArgs &a, Plan *P, Sync *Y, uint8_t *ring, uint32_t ch,
                                  uint32_t S, int32_t idv, uint32_t p0, uint32_t p1,
                                  uint32_t wave, uint32_t lane) {
    const uint8_t *base = a.base;
    const uint64_t stride = a.stride, og = a.og, ou = a.ou;
    const uint32_t n_ff = a.n_ff, rb = a.rb_gu, slot_bytes = 2u * ch * rb;
    const uint32_t np = p1 - p0, C = (np + ch - 1) / ch;
    uint32_t issued = 0;
    auto issue = [&](uint32_t c) {
        const uint32_t q0 = p0 + c * ch, q1 = min(q0 + ch, p1);
        uint8_t *sg = ring + (size_t)(c % S) * slot_bytes, *su = sg + (size_t)ch * rb;
        for (uint32_t q = q0; q < q1;) {   // one expert's run of rows at a time
            const uint32_t u = q / n_ff, r = q % n_ff;
            const uint32_t n = min(q1 - q, n_ff - r);
            const int32_t id = __builtin_amdgcn_readlane(idv, u);
            const uint8_t *e = base + (uint64_t)id * stride + (uint64_t)r * rb;
            issued += dma1<UNIT>(sg + (size_t)(q - q0) * rb, e + og, n * rb, lane);
#ifdef Q4MI_TRACE
            if (c == 0 && q == q0) {
                unsigned long long *const q4tr = a.trace;
                const uint32_t q4bid = blockIdx.x;
                Q4MI_TR(18, 0, wave == 0 && lane == 0);
            }
#endif
            issued += dma1<UNIT>(su + (size_t)(q - q0) * rb, e + ou, n * rb, lane);
            q += n;
        }
    };
    auto items = [&](uint32_t c) { return min(ch, np - c * ch); };
    produce(Y, P->ends[wave], wave, C, S, a.ahead, issued, issue, items
#ifdef Q4MI_TRACE
            , a.trace, 0
#endif
    );
}

// Consumer prologue: q8 of x (v[k] = quad ct + k kCons, loaded by the
// caller), then wait until every consumer wave finished the shared tables.
template <int NT>
__device__ inline void gu_quant_x(const MoeArgs &a, Sync *Y, int8_t *xq, float *xd,
                                  const float4 (&v0)[kXPre<NT>], uint32_t ct, uint32_t lane) {
    const uint32_t nq = a.src.n_tok * a.K / 4;
    const float4 *xg = (const float4 *)a.x;
#pragma unroll
    for (uint32_t k = 0; k < kXPre<NT>; k++)
        if (ct + k * kCons < nq) quant_quad(v0[k], ct + k * kCons, xq, xd);
    // further quads (many tokens or a wide row) four loads in flight at a
    // time; rare, so laid out after the common path
    if (__builtin_expect(ct + kXPre<NT> * kCons < nq, 0))
    for (uint32_t i0 = ct + kXPre<NT> * kCons; i0 < nq; i0 += 4 * kCons) {
        float4 v[4];
#pragma unroll
        for (int k = 0; k < 4; k++) {
            const uint32_t i = i0 + k * kCons;
            v[k] = i < nq ? xg[i] : make_float4(0.f, 0.f, 0.f, 0.f);
        }
#pragma unroll
        for (int k = 0; k < 4; k++)
            if (i0 + k * kCons < nq) quant_quad(v[k], i0 + k * kCons, xq, xd);
    }
    if (lane == 0) atomicAdd(&Y->ready, 1u);
    spin_ge(&Y->ready, kConsW);                     // table and q8(x) complete
}

// Consumers: h[u][t][r] of pairs [p0, p0 + np) as their chunks land.
template <uint32_t TY, int NT, int TPR, int GPT>
__device__ inline void gu_compute(const MoeArgs &a, const uint32_t *stab, const Plan *P, Sync *Y,
                                  const int8_t *xq, const float *xd, const uint8_t *ring,
                                  uint32_t ch, uint32_t S, uint32_t p0, uint32_t np, bool uniq,
                                  uint32_t ct, uint32_t cw) {
    const uint32_t nt = a.src.n_tok, K = a.K, n_ff = a.n_ff, rb = a.rb_gu;
    const uint32_t slot_bytes = 2u * ch * rb;
    constexpr uint32_t kTeams = kCons / TPR, kTpw = 64 / TPR;
    const uint32_t gi = ct % TPR, sub = (ct & 63u) / TPR;
    // IQ3_S with an even group count per lane: lane gi takes the adjacent
    // groups GPT*gi + m, decoded in pairs that share their superblock reads
    constexpr bool kPair = TY == Q4MI_T_IQ3_S && GPT % 2 == 0;
    // five groups per lane at several tokens (80-group rows, 16 x 5): x is
    // read from LDS per group, for the selected tokens only, since five
    // groups of every token's x do not fit the registers
    constexpr bool kXL = NT >= 2 && GPT == 5;
    XRegs<NT, GPT> xr;
    // a layout may cover more groups than the row has (TPR * GPT > G):
    // lanes past the row skip their groups
    const uint32_t G = K / 32;
    if constexpr (!kXL) load_xregs<NT, GPT, TPR, kPair>(xr, xq, xd, K, nt, gi, G);
    float *hout = a.h;
#ifdef Q4MI_TRACE
    unsigned long long *const q4tr = a.trace;
    const uint32_t q4bid = blockIdx.x;
    uint32_t round = 0;
#endif
    for (uint32_t b = cw * kTpw; b < np; b += kTeams) {   // b: this wave's first pair
        const uint32_t bl = min(b + kTpw, np) - 1;
        for (uint32_t c = b / ch; c <= bl / ch; c++) wait_chunk(Y, c);
#ifdef Q4MI_TRACE
        if (round < 8) Q4MI_TR(5 + round, 0, ct == 0);
        round++;
#endif
        const uint32_t i = b + sub;
#ifdef Q4MI_TRACE
        if ((a.dbg & 1u) && i < np) {   // stream only: count the pair consumed
            if (gi == TPR - 1) atomicAdd(&Y->cons[(i / ch) % S], 1u);
            continue;
        }
#endif
        if (i < np) {
            const uint32_t c = i / ch, j = i % ch;
            const uint8_t *tile = ring + (size_t)(c % S) * slot_bytes;
            const uint32_t *tw = (const uint32_t *)tile;
            const uint32_t p = p0 + i, u = p / n_ff, r = p % n_ff;
            const uint32_t sel = uniq ? 1u : P->sel[u];
            float ag[NT], au[NT];
#pragma unroll
            for (int t = 0; t < NT; t++) ag[t] = au[t] = 0.f;
            auto dotx = [&](const auto &X, int m, int which, const int32_t (&w)[8], int mult,
                            int mult2, float d) __attribute__((always_inline)) {
#pragma unroll
                for (int t = 0; t < NT; t++) {
                    if (!((sel >> t) & 1u)) continue;
                    const int s = tsum<TY>(w, X.q[m][t], mult, mult2);
                    const float f = (float)s * (d * X.d[m][t]);
                    if (which == 0) ag[t] += f;
                    else au[t] += f;
                }
            };
            auto dot = [&](int m, int which, const int32_t (&w)[8], int mult, int mult2,
                           float d) __attribute__((always_inline)) {
                dotx(xr, m, which, w, mult, mult2, d);
            };
            if constexpr (kPair) {
#pragma unroll
                for (int m = 0; m < GPT; m += 2) {
                    const uint32_t g = GPT * gi + m;
                    if (g >= G) continue;   // (G is even: both groups or neither)
#pragma unroll
                    for (int which = 0; which < 2; which++) {
                        int32_t wa[8], wb[8];
                        int ma, mb;
                        float d;
                        iq3s_group2(stab, tile, tw, __umul24(which * ch + j, rb), g, wa, wb, ma, mb, d);
                        dot(m, which, wa, ma, ma, d);
                        dot(m + 1, which, wb, mb, mb, d);
                    }
                }
            } else {
#pragma unroll
                for (int m = 0; m < GPT; m++) {
                    const uint32_t g = gi + TPR * m;
                    if (g >= G) continue;
                    XRegs<NT, 1> xl;
                    if constexpr (kXL) {
#pragma unroll
                        for (int t = 0; t < NT; t++) {
                            if (!((sel >> t) & 1u)) continue;
                            const int4 qa = *(const int4 *)(xq + (size_t)t * K + 32u * g);
                            const int4 qb = *(const int4 *)(xq + (size_t)t * K + 32u * g + 16u);
                            xl.q[0][t][0] = qa.x; xl.q[0][t][1] = qa.y; xl.q[0][t][2] = qa.z;
                            xl.q[0][t][3] = qa.w; xl.q[0][t][4] = qb.x; xl.q[0][t][5] = qb.y;
                            xl.q[0][t][6] = qb.z; xl.q[0][t][7] = qb.w;
                            xl.d[0][t] = xd[(size_t)t * G + g];
                        }
                    }
#pragma unroll
                    for (int which = 0; which < 2; which++) {
                        int32_t w[8];
                        int mult, mult2;
                        float d;
                        group_w<TY>(stab, tile, tw, __umul24(which * ch + j, rb), g, w, mult, mult2, d);
                        if constexpr (kXL) dotx(xl, 0, which, w, mult, mult2, d);
                        else dot(m, which, w, mult, mult2, d);
                    }
                }
            }
#pragma unroll
            for (int t = 0; t < NT; t++) {
                if (!((sel >> t) & 1u)) continue;
                const float gs = q4mi_rsum<TPR>(ag[t]), us = q4mi_rsum<TPR>(au[t]);
                if (gi == TPR - 1) hout[((size_t)u * kMaxT + t) * n_ff + r] = silu_f(gs) * us;
            }
            if (gi == TPR - 1) atomicAdd(&Y->cons[c % S], 1u);   // rows of pair i read
        }
    }
}

// SRC: kSrcDev device lists, kSrcHost a host list in the kernel arguments
// (one token), kSrcLogits router logits (one token).  Separate
// instantiations, so that each kernel carries only its own list code: the
// start-up runs with a cold instruction cache, on the critical path.
template <uint32_t TY, int NT, int TPR, int GPT, uint32_t UNIT, int SRC>
__global__ __launch_bounds__(kT) void moe_gu_k(MoeArgs a) {
    extern __shared__ __align__(16) uint8_t smem[];
    const uint32_t bid = blockIdx.x, nblk = gridDim.x, ch = a.chunk, S = a.slots;
    Q4MI_TR_DECL(bid);
    Q4MI_TR(31, 0, threadIdx.x == 0);
    constexpr bool kIq = TY == Q4MI_T_IQ3_S;
    uint32_t *stab = (uint32_t *)smem;
    Plan *P = (Plan *)(smem + tab_bytes<TY>());
    Sync *Y = (Sync *)(P + 1);
    int8_t *xq = (int8_t *)(smem + al16((size_t)((uint8_t *)(Y + 1) - smem)));
    float *xd = (float *)(xq + NT * a.K);
    uint8_t *ring = smem + al16((size_t)((uint8_t *)(xd + NT * (a.K / 32)) - smem));
    const uint32_t tid = threadIdx.x, lane = tid & 63u;
    const uint32_t wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const KArgs ka = kargs();
    constexpr bool uniq = SRC == kSrcHost;
    // the host list's ids, loaded while the block starts up (lane u: id u)
    const int32_t hid = (uniq && wave < kProd) ? host_ids(ka, a.src.n_fixed) : -1;
    // consumers issue their prologue loads (codebook entry, first x quad)
    // as their wave starts, ahead of the weight stream the producers begin
    // after the barrier
    const uint32_t nq = a.src.n_tok * a.K / 4;
    uint32_t code = 0u;
    float4 v0[kXPre<NT>];
#pragma unroll
    for (uint32_t k = 0; k < kXPre<NT>; k++) v0[k] = make_float4(0.f, 0.f, 0.f, 0.f);
    if (wave >= kProd) {
        const uint32_t c0 = tid - kProd * 64;
        if (kIq && c0 < 512) code = q4mi_iq3s_code_dev[c0];
        // every x quad of up to kXPre<NT> passes: loads issued after the
        // barrier queue behind the weight stream and return when it drains
#pragma unroll
        for (uint32_t k = 0; k < kXPre<NT>; k++)
            if (c0 + k * kCons < nq) v0[k] = ((const float4 *)a.x)[c0 + k * kCons];
    }
    if (tid < sizeof(Sync) / 4) ((uint32_t *)Y)[tid] = 0;
    if (!uniq && tid < 64) build_plan<SRC == kSrcLogits>(P, a.src, tid, (uint32_t *)ring);
    Q4MI_TR(13, 0, tid == 0);
    Q4MI_TR(14, 0, tid == kProd * 64);
    __syncthreads();                 // the only block-wide barrier: Sync zeroed, plan built
    Q4MI_TR(15, 0, tid == 0);
    if (!uniq && bid == 0 && wave == kProd) {   // the down launch reuses this plan
        for (uint32_t i = lane; i < sizeof(Plan) / 16; i += 64)
            ((uint4 *)a.gplan)[i] = ((const uint4 *)P)[i];
    }
    const uint32_t nu = uniq ? a.src.n_fixed : P->nu;
    const uint32_t PT = nu * a.n_ff;
    uint32_t p0, p1;
    if (NT == 1 || uniq) {
        p0 = share_lo(PT, bid, nblk);
        p1 = share_lo(PT, bid + 1, nblk);
    } else {   // shares of equal work: an expert picked by more tokens costs more
        share_weighted(P, nu, a.n_ff, bid, nblk, lane, p0, p1);
    }

    if (wave < kProd) {
        // every expert id in one register (lane u holds id u): a segment's id
        // is then one v_readlane, not a memory round trip
        const int32_t idv = uniq ? hid : (lane < nu ? P->uid[lane] : -1);
        Q4MI_TR(0, 0, tid == 0);
        gu_produce<UNIT>(a, P, Y, ring, ch, S, idv, p0, p1, wave, lane);
        Q4MI_TR(2, 0, tid == 0);
        return;
    }
    const uint32_t ct = tid - kProd * 64;
    build_tables<TY>(smem, code, ct);
    gu_quant_x<NT>(a, Y, xq, xd, v0, ct, lane);
    Q4MI_TR(4, 0, ct == 0);
    gu_compute<TY, NT, TPR, GPT>(a, stab, P, Y, xq, xd, ring, ch, S, p0, p1 - p0, uniq, ct,
                                 wave - kProd);
    Q4MI_TR(30, 0, ct == 0);
#ifdef Q4MI_TRACE
    if (lane == 0 && atomicAdd(&Y->ready, 1u) == 2 * kConsW - 1) Q4MI_TR(29, 0, true);
#endif
}

// ---------------------------------------------------------------- down
// Same roles.  Items are (expert u, output row rr); the chunks are runs of
// `ch` experts (dn_rows rows each).  The consumers quantize every selected
// h row (q8, 32-value groups) into LDS before computing.
//
// LDS: [stab] Plan Sync | part [kMaxU][NT][dn_rows] | hq [nsel_cap][n_ff] |
//      hd [nsel_cap][n_ff/32] | ring of S slots, slot = ch experts x dn_rows
//      rows.
//
// Block `bid` owns output rows dn_rows*bid .. dn_rows*bid + dn_rows - 1.
template <uint32_t UNIT>
__device__ inline void dn_produce(const MoeArgs &a, Plan *P, Sync *Y, uint8_t *ring, uint32_t ch,
                                  uint32_t S, int32_t idv, uint32_t nu, uint32_t r0, uint32_t nr,
                                  uint32_t wave, uint32_t lane) {
    const uint8_t *base = a.base;
    const uint64_t stride = a.stride_d, od = a.od;
    const uint32_t rb = a.rb_dn, slot_bytes = ch * a.dn_rows * rb;
    const uint32_t C = (nu + ch - 1) / ch;
    uint32_t issued = 0;
    auto issue = [&](uint32_t c) {
        const uint32_t e0 = c * ch, e1 = min(e0 + ch, nu);
        uint8_t *dst = ring + (size_t)(c % S) * slot_bytes;
        for (uint32_t u = e0; u < e1; u++) {
            const int32_t id = __builtin_amdgcn_readlane(idv, u);
            const uint8_t *e = base + (uint64_t)id * stride + od + (uint64_t)r0 * rb;
            issued += dma1<UNIT>(dst + (size_t)(u - e0) * nr * rb, e, nr * rb, lane);
#ifdef Q4MI_TRACE
            if (c == 0 && u == e0) {
                unsigned long long *const q4tr = a.trace;
                const uint32_t q4bid = blockIdx.x;
                Q4MI_TR(18, 1, wave == 0 && lane == 0);
            }
#endif
        }
    };
    auto items = [&](uint32_t c) { return min(ch, nu - c * ch) * nr; };
    produce(Y, P->ends[wave], wave, C, S, a.ahead, issued, issue, items
#ifdef Q4MI_TRACE
            , a.trace, 1
#endif
    );
}

// Consumers: q8 of every selected h row, the (expert, row) dots as their
// chunks land, then y[t][r0 + rr] = yv + sum_u w[u][t] * part[u][t][rr].
// With `pre`, quads ct and ct + kCons of the host list's h rows are already
// in v0, v1; yv is the old y of output ct / 8 (lanes with ct % 8 == 7).
template <uint32_t TY, int NT, int TPR, int GPT>
__device__ inline void dn_compute(const MoeArgs &a, const uint32_t *stab, Plan *P, Sync *Y,
                                  float *part, int8_t *hq, float *hd, const uint8_t *ring,
                                  uint32_t ch, uint32_t S, uint32_t r0, uint32_t nr, uint32_t nu,
                                  uint32_t nsel, bool uniq, float wv, float yv, float4 v0,
                                  float4 v1, bool pre, uint32_t ct, uint32_t cw, uint32_t lane) {
    const uint32_t n_ff = a.n_ff, rb = a.rb_dn, nt = a.src.n_tok;
    const uint32_t dr = a.dn_rows, slot_bytes = ch * dr * rb;
    const float *hg = a.h;
    const uint32_t qpr = n_ff / 4;
    // host list: its weights go to Plan::w[0] for the final sum
    if (uniq && cw == 0 && lane < nu) P->w[0][lane] = wv;
    // q8 of every selected h row; pair slot s holds h[u][t] (slots of u are
    // its selected tokens in order).  Every prologue load is issued before
    // any is used.
    const uint32_t nq = nsel * qpr;
    auto hquad = [&](uint32_t i) -> float4 {
        const uint32_t s = i / qpr;
        const uint32_t row = uniq ? s * kMaxT : P->prow[s];
        return ((const float4 *)(hg + (size_t)row * n_ff))[i % qpr];
    };
    // device lists: the rows are known only now, and these loads queue
    // behind the weight stream, so the first batch takes eight quads per
    // thread (a window's 44 rows in one round trip)
    uint32_t i0 = ct;
    if (pre) {
        if (ct < nq) quant_quad(v0, ct, hq, hd);
        if (ct + kCons < nq) quant_quad(v1, ct + kCons, hq, hd);
        i0 = ct + 2 * kCons;
    }
    // further quads eight loads in flight at a time (with the prologue's
    // quads, only for many or long rows: laid out after the common path)
    if (__builtin_expect(i0 < nq, !pre))
    for (; i0 < nq; i0 += 8 * kCons) {
        float4 v[8];
#pragma unroll
        for (int k = 0; k < 8; k++) {
            const uint32_t i = i0 + k * kCons;
            v[k] = i < nq ? hquad(i) : make_float4(0.f, 0.f, 0.f, 0.f);
        }
#pragma unroll
        for (int k = 0; k < 8; k++)
            if (i0 + k * kCons < nq) quant_quad(v[k], i0 + k * kCons, hq, hd);
    }
    if (lane == 0) atomicAdd(&Y->ready, 1u);
    spin_ge(&Y->ready, kConsW);                     // table and q8(h) complete
#ifdef Q4MI_TRACE
    unsigned long long *const q4tr = a.trace;
    const uint32_t q4bid = blockIdx.x;
    Q4MI_TR(5, 1, ct == 0);
#endif
    constexpr uint32_t kTeams = kCons / TPR, kTpw = 64 / TPR;
    const uint32_t gi = ct % TPR, sub = (ct & 63u) / TPR;
    const uint32_t ni = nu * nr;                    // items, expert-major
    const uint32_t ipc = ch * nr;                   // items per chunk
    for (uint32_t b = cw * kTpw; b < ni; b += kTeams) {
        const uint32_t bl = min(b + kTpw, ni) - 1;
        for (uint32_t c = b / ipc; c <= bl / ipc; c++) wait_chunk(Y, c);
        const uint32_t it = b + sub;
        if (it < ni) {
            const uint32_t c = it / ipc, jj = it % ipc;
            const uint8_t *tile = ring + (size_t)(c % S) * slot_bytes;
            const uint32_t *tw = (const uint32_t *)tile;
            const uint32_t u = it / nr, rr = it % nr;
            const uint32_t sel = uniq ? 1u : P->sel[u];
            const uint32_t ps = uniq ? u : P->pslot[u];
            float acc[NT];
#pragma unroll
            for (int t = 0; t < NT; t++) acc[t] = 0.f;
            auto dot = [&](uint32_t g, const int32_t (&w)[8], int mult, int mult2, float d)
                __attribute__((always_inline)) {
                uint32_t s2 = ps;
#pragma unroll
                for (int t = 0; t < NT; t++) {
                    if (!((sel >> t) & 1u)) continue;
                    const int4 qa = *(const int4 *)(hq + (size_t)s2 * n_ff + 32 * g);
                    const int4 qb = *(const int4 *)(hq + (size_t)s2 * n_ff + 32 * g + 16);
                    const int32_t q[8] = {qa.x, qa.y, qa.z, qa.w, qb.x, qb.y, qb.z, qb.w};
                    const int s = tsum<TY>(w, q, mult, mult2);
                    acc[t] = fmaf((float)s, d * hd[(size_t)s2 * (n_ff / 32) + g], acc[t]);
                    s2++;
                }
            };
            // IQ3_S with an even group count per lane: adjacent groups
            // GPT*gi + m, decoded in pairs sharing their superblock reads
            if constexpr (TY == Q4MI_T_IQ3_S && GPT % 2 == 0) {
#pragma unroll
                for (int m = 0; m < GPT; m += 2) {
                    const uint32_t g = GPT * gi + m;
                    int32_t wa[8], wb[8];
                    int ma, mb;
                    float d;
                    iq3s_group2(stab, tile, tw, __umul24(jj, rb), g, wa, wb, ma, mb, d);
                    dot(g, wa, ma, ma, d);
                    dot(g + 1, wb, mb, mb, d);
                }
            } else {
#pragma unroll
                for (int m = 0; m < GPT; m++) {
                    const uint32_t g = gi + TPR * m;
                    int32_t w[8];
                    int mult, mult2;
                    float d;
                    group_w<TY>(stab, tile, tw, __umul24(jj, rb), g, w, mult, mult2, d);
                    dot(g, w, mult, mult2, d);
                }
            }
#pragma unroll
            for (int t = 0; t < NT; t++) {
                const float v = ((sel >> t) & 1u) ? q4mi_rsum<TPR>(acc[t]) : 0.f;
                if (gi == TPR - 1) part[((size_t)u * NT + t) * dr + rr] = v;
            }
            if (gi == TPR - 1) atomicAdd(&Y->cons[c % S], 1u);
        }
    }
#ifdef Q4MI_TRACE
    Q4MI_TR(6, 1, ct == 0);
#endif
    if (lane == 0) atomicAdd(&Y->fin, 1u);
    spin_ge(&Y->fin, kConsW);                       // every partial sum written
#ifdef Q4MI_TRACE
    Q4MI_TR(7, 1, ct == 0);
#endif
    // y[t][r] += sum_u w[u][t] * part[u][t][r]: lane sl of an output's
    // 8 lanes takes experts u = sl, sl + 8, ... in plan order, then a fixed
    // DPP tree joins the 8 partial sums (deterministic)
    for (uint32_t c8 = ct; c8 < 8 * nt * nr; c8 += kCons) {   // whole 8-lane groups
        const uint32_t o = c8 >> 3, sl = c8 & 7u, t = o / nr, rr = o % nr;
        float s = 0.f;
        for (uint32_t u = sl; u < nu; u += 8)
            if (uniq || ((P->sel[u] >> t) & 1u)) s += P->w[t][u] * part[((size_t)u * NT + t) * dr + rr];
        s = q4mi_rsum<8>(s);
        // outputs past the first kCons / 8 read their old y here
        const float y0 = c8 == ct ? yv : a.y[(size_t)t * a.n_embd + r0 + rr];
        if (sl == 7u) a.y[(size_t)t * a.n_embd + r0 + rr] = y0 + s;
    }
}

// The old y of output o = ct / 8 (t = o / nr, row r0 + o % nr) in the lane
// that stores it (ct % 8 == 7), loaded early.
__device__ inline float dn_y_early(const MoeArgs &a, uint32_t c0, uint32_t r0, uint32_t nr) {
    if ((c0 & 7u) == 7u && (c0 >> 3) < a.src.n_tok * nr) {
        const uint32_t o = c0 >> 3;
        return a.y[(size_t)(o / nr) * a.n_embd + r0 + o % nr];
    }
    return 0.f;
}

template <uint32_t TY, int NT, int TPR, int GPT, uint32_t UNIT, int SRC>
__global__ __launch_bounds__(kT) void moe_dn_k(MoeArgs a) {
    extern __shared__ __align__(16) uint8_t smem[];
    const uint32_t bid = blockIdx.x, ch = a.chunk, S = a.slots;
    Q4MI_TR_DECL(bid);
    Q4MI_TR(31, 1, threadIdx.x == 0);
    constexpr bool kIq = TY == Q4MI_T_IQ3_S;
    uint32_t *stab = (uint32_t *)smem;
    Plan *P = (Plan *)(smem + tab_bytes<TY>());
    Sync *Y = (Sync *)(P + 1);
    float *part = (float *)(smem + al16((size_t)((uint8_t *)(Y + 1) - smem)));   // [kMaxU][NT][dn_rows]
    int8_t *hq = (int8_t *)(part + kMaxU * NT * a.dn_rows);
    const uint32_t n_ff = a.n_ff, cap = a.nsel_cap;
    float *hd = (float *)(hq + (size_t)cap * n_ff);
    uint8_t *ring = smem + al16((size_t)((uint8_t *)(hd + (size_t)cap * (n_ff / 32)) - smem));
    const uint32_t tid = threadIdx.x, lane = tid & 63u;
    const uint32_t wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const uint32_t r0 = bid * a.dn_rows;
    const uint32_t nr = min(a.dn_rows, a.n_embd - r0);
    const KArgs ka = kargs();
    constexpr bool uniq = SRC == kSrcHost;
    // the host list's ids (producers) or weights (consumers), loaded while
    // the block starts up (lane u: entry u)
    const int32_t hword = !uniq ? 0 : wave < kProd ? host_ids(ka, a.src.n_fixed)
                                                  : __builtin_bit_cast(int32_t, host_weights(ka, a.src.n_fixed));
    // consumers issue their prologue loads (codebook entry, y, and for a
    // host list the first h quads) as their wave starts, ahead of the weight
    // stream the producers begin after the barrier
    const uint32_t qpr = n_ff / 4;
    uint32_t code = 0u;
    float yv = 0.f;
    float4 v0 = make_float4(0.f, 0.f, 0.f, 0.f), v1 = v0;
    if (wave >= kProd) {
        const uint32_t c0 = tid - kProd * 64;
        if (kIq && c0 < 512) code = q4mi_iq3s_code_dev[c0];
        yv = dn_y_early(a, c0, r0, nr);
        if (uniq) {   // pair slot s = h row s * kMaxT
            const uint32_t nq0 = a.src.n_fixed * qpr;
            auto hq0 = [&](uint32_t i) {
                return ((const float4 *)(a.h + (size_t)(i / qpr) * kMaxT * n_ff))[i % qpr];
            };
            if (c0 < nq0) v0 = hq0(c0);
            if (c0 + kCons < nq0) v1 = hq0(c0 + kCons);
        }
    }
    if (tid < sizeof(Sync) / 4) ((uint32_t *)Y)[tid] = 0;
    if (!uniq && tid < 64) {
        if (a.plan_in) {   // the plan the gate/up launch of this call published
            for (uint32_t i = tid; i < sizeof(Plan) / 16; i += 64)
                ((uint4 *)P)[i] = ((const uint4 *)a.gplan)[i];
        } else {
            build_plan<false>(P, a.src, tid, (uint32_t *)ring);
        }
    }
    __syncthreads();                 // the only block-wide barrier: Sync zeroed, plan built
    const uint32_t nu = uniq ? a.src.n_fixed : P->nu;
    const uint32_t nsel = uniq ? nu : P->nsel;

    if (wave < kProd) {
        const int32_t idv = uniq ? hword : (lane < nu ? P->uid[lane] : -1);
        Q4MI_TR(0, 1, tid == 0);
        dn_produce<UNIT>(a, P, Y, ring, ch, S, idv, nu, r0, nr, wave, lane);
        Q4MI_TR(2, 1, tid == 0);
        return;
    }
    const uint32_t ct = tid - kProd * 64;
    build_tables<TY>(smem, code, ct);
    dn_compute<TY, NT, TPR, GPT>(a, stab, P, Y, part, hq, hd, ring, ch, S, r0, nr, nu, nsel, uniq,
                                 __builtin_bit_cast(float, hword), yv, v0, v1, uniq, ct,
                                 wave - kProd, lane);
    Q4MI_TR(30, 1, ct == 0);
}

// ------------------------------------------------------------------ host
constexpr size_t kLdsCap = 160 * 1024;

// LDS budget of a decode block (the measurement build can lower it;
// moe_decode.hip).
size_t lds_cap();

// bytes build_plan uses at the start of the ring: its 1024-bucket table,
// then (router logits) one token's 64 picks and probabilities
constexpr size_t kPlanTable = 4096 + 512;

static size_t head_bytes(uint32_t ty) {
    const size_t tab = ty == Q4MI_T_IQ3_S   ? tab_bytes<Q4MI_T_IQ3_S>()
                     : ty == Q4MI_T_IQ2_S   ? tab_bytes<Q4MI_T_IQ2_S>()
                     : ty == Q4MI_T_IQ2_XXS ? tab_bytes<Q4MI_T_IQ2_XXS>()
                     : ty == Q4MI_T_IQ2_XS  ? tab_bytes<Q4MI_T_IQ2_XS>()
                     : ty == Q4MI_T_IQ3_XXS ? tab_bytes<Q4MI_T_IQ3_XXS>() : 0;
    return al16(tab + sizeof(Plan) + sizeof(Sync));
}

// Chunk size and ring slots of the gate/up kernel for `grid` blocks within
// `cap` bytes of LDS; returns the LDS bytes (0: does not fit).
template <int NT>
static size_t gu_plan(const MoeArgs &a, uint32_t nu_host, uint32_t grid, size_t cap,
                      uint32_t &ch, uint32_t &S, uint32_t ty, uint32_t tpw) {
    // one chunk per producer wave when it fits (a producer publishes a chunk
    // only after issuing everything before it, so a second chunk would
    // delay the first); device lists (unknown share) use small chunks, so
    // the window's larger shares land chunk by chunk while the consumers
    // work: 4 pairs, or two waves' worth when a wave takes more than two
    // pairs a round (tpw).  Measured, 4-token windows: configs[2] (2 pairs
    // per wave) 4 / 8 / 16 pairs 34.5 / 34.8 / 35.6 us; at hidden 2560,
    // IQ3_S (1 pair per wave) 4 / 8 pairs 29.0 / 29.8 us gate/up, IQ3_XXS and
    // IQ2_S (4 pairs per wave) 27.9 / 26.2 and 26.1 / 24.5 us.
    const uint32_t pairs = nu_host ? nu_host * a.n_ff : kMaxU * a.n_ff;
    const uint32_t share = (pairs + grid - 1) / grid;
    ch = nu_host ? std::max<uint32_t>(1, (share + kProd - 1) / kProd) : std::max<uint32_t>(4, 2 * tpw);
#if defined(Q4MI_TRACE) || defined(Q4MI_KNOBS)
    if (getenv("Q4MI_CHUNK")) ch = std::max(1, atoi(getenv("Q4MI_CHUNK")));
#endif
    const size_t fixed = head_bytes(ty) + al16((size_t)NT * a.K + (size_t)NT * (a.K / 32) * 4);
    S = 0;
    // A consumer wave waits for every chunk its two pairs touch (at most
    // two), so a reused ring needs three slots to always make progress.
    for (;; ch = (ch + 1) / 2) {
        const size_t slot = 2ull * ch * a.rb_gu;
        S = fixed < cap ? (uint32_t)std::min<size_t>(kMaxS, (cap - fixed) / slot) : 0;
        if (S >= 3 || ch == 1) break;
    }
    const uint32_t C = (share + ch - 1) / ch;
    if (S < 3 && S < C) return 0;
    S = std::min<uint32_t>(S, std::max<uint32_t>(1, C));
    // the ring's first 4 KB hold the device-list plan's bucket table first
    return std::max(fixed + (size_t)S * 2 * ch * a.rb_gu, fixed + kPlanTable);
}

// Same for the down kernel (sets a.nsel_cap).
template <int NT>
static size_t dn_plan(MoeArgs &a, uint32_t nu_host, size_t cap_bytes, uint32_t &ch, uint32_t &S,
                      uint32_t ty) {
    const uint32_t cap = nu_host ? nu_host : kMaxU;   // selected pairs (<= 64)
    const size_t fixed = head_bytes(ty) + (size_t)kMaxU * NT * a.dn_rows * 4 +
                         al16((size_t)cap * a.n_ff + (size_t)cap * (a.n_ff / 32) * 4);
    // host lists: one chunk per producer; device lists (up to kMaxU experts)
    // 2 experts, so a window's chunks land one after another and the items
    // start before the last (4-token window: 2 / 3 / 4 / 16 experts per chunk
    // 33.5 / 33.6 / 33.7 / 34.8 us with 8-pair gate/up chunks; at hidden 2560
    // with IQ4_NL down, 2 / 3 / 5: 21.2 / 21.8 / 23.3 us)
    const uint32_t nu_est = nu_host ? nu_host : kMaxU;
    ch = nu_host ? std::max<uint32_t>(1, (nu_est + kProd - 1) / kProd) : 2;
#if defined(Q4MI_TRACE) || defined(Q4MI_KNOBS)
    if (getenv("Q4MI_DNCHUNK")) ch = std::max(1, atoi(getenv("Q4MI_DNCHUNK")));
#endif
    S = 0;
    for (;; ch = (ch + 1) / 2) {
        const size_t slot = (size_t)ch * a.dn_rows * a.rb_dn;
        S = fixed < cap_bytes ? (uint32_t)std::min<size_t>(kMaxS, (cap_bytes - fixed) / slot) : 0;
        if (S >= 2 || ch == 1) break;
    }
    // a consumer wave's 64/TPR consecutive items may touch several chunks (it waits for each)
    const uint32_t C = (nu_est + ch - 1) / ch;
    if (S < 2 && S < C) return 0;
    S = std::min<uint32_t>(S, std::max<uint32_t>(1, C));
    a.nsel_cap = cap;
    return std::max(fixed + (size_t)S * ch * a.dn_rows * a.rb_dn, fixed + kPlanTable);
}

template <uint32_t TY, int NT, int TPR, int GPT>
static bool launch_gu(MoeArgs a, uint32_t nu_host) {
    const uint32_t grid = (uint32_t)cu_count();
    uint32_t ch, S;
    const size_t lds = gu_plan<NT>(a, nu_host, grid, lds_cap(), ch, S, TY, 64u / TPR);
    if (!lds) {
        set_error("moe_gu_k: LDS limit");
        return false;
    }
    a.chunk = ch;
    a.slots = S;
    const bool wide = ((((uintptr_t)a.base) | a.stride | a.og | a.ou | a.rb_gu) & 15u) == 0;
    auto go = [&](auto kern) {
        if (hipFuncSetAttribute((const void *)kern, hipFuncAttributeMaxDynamicSharedMemorySize,
                                (int)lds) != hipSuccess) {
            set_error("moe_gu_k: LDS limit (%zu)", lds);
            return false;
        }
        kern<<<dim3(grid), dim3(kT), lds, stream()>>>(a);
        return launch_ok("moe_gu_k");
    };
    if constexpr (NT == 1) {
        if (a.src.lg)   // router logits
            return wide ? go(moe_gu_k<TY, NT, TPR, GPT, 16, kSrcLogits>)
                        : go(moe_gu_k<TY, NT, TPR, GPT, 4, kSrcLogits>);
        if (a.src.unique)   // host list
            return wide ? go(moe_gu_k<TY, NT, TPR, GPT, 16, kSrcHost>)
                        : go(moe_gu_k<TY, NT, TPR, GPT, 4, kSrcHost>);
    } else if (a.src.lg || a.src.unique) {
        set_error("moe_gu_k: host lists and router logits take one token");
        return false;
    }
    return wide ? go(moe_gu_k<TY, NT, TPR, GPT, 16, kSrcDev>)
                : go(moe_gu_k<TY, NT, TPR, GPT, 4, kSrcDev>);
}

template <uint32_t TY, int NT, int TPR, int GPT>
static bool launch_dn(MoeArgs a, uint32_t nu_host) {
    // rows per block: 8, or more (up to 16) when 8 would need more blocks
    // than CUs (hidden 2560: 10 rows, 256 blocks; 4096: 16)
    const uint32_t cus = (uint32_t)cu_count();
    a.dn_rows = kDnRows;
    if ((a.n_embd + kDnRows - 1) / kDnRows > cus)
        a.dn_rows = std::min(kDnRowsMax, (a.n_embd + cus - 1) / cus);
    uint32_t ch, S;
    const size_t lds = dn_plan<NT>(a, nu_host, lds_cap(), ch, S, TY);
    if (!lds) {
        set_error("moe_dn_k: LDS limit");
        return false;
    }
    a.chunk = ch;
    a.slots = S;
    // a block copies one contiguous run of dn_rows rows per expert: 16-byte
    // units need that run (not each row) 16-byte aligned and sized
    const bool wide = ((((uintptr_t)a.base) | a.stride_d | a.od | ((uint64_t)a.dn_rows * a.rb_dn)) & 15u) == 0 &&
                      a.n_embd % a.dn_rows == 0;
    const uint32_t grid = (a.n_embd + a.dn_rows - 1) / a.dn_rows;
    auto go = [&](auto kern) {
        if (hipFuncSetAttribute((const void *)kern, hipFuncAttributeMaxDynamicSharedMemorySize,
                                (int)lds) != hipSuccess) {
            set_error("moe_dn_k: LDS limit (%zu)", lds);
            return false;
        }
        kern<<<dim3(grid), dim3(kT), lds, stream()>>>(a);
        return launch_ok("moe_dn_k");
    };
    if constexpr (NT == 1) {
        if (a.src.unique)   // host list
            return wide ? go(moe_dn_k<TY, NT, TPR, GPT, 16, kSrcHost>)
                        : go(moe_dn_k<TY, NT, TPR, GPT, 4, kSrcHost>);
    } else if (a.src.unique) {
        set_error("moe_dn_k: host lists take one token");
        return false;
    }
    return wide ? go(moe_dn_k<TY, NT, TPR, GPT, 16, kSrcDev>)
                : go(moe_dn_k<TY, NT, TPR, GPT, 4, kSrcDev>);
}

// Gate/up lanes per pair: 32 (two or more groups per lane, two pairs per
// wave, so each wave has two pairs' chains in flight) while the activation
// registers stay small (groups x tokens <= 4, or 2 groups x 4 tokens), else
// the row layout.
static RowLayout gu_layout(uint32_t G, int NT, uint32_t ty) {
    const uint32_t gn = (G / 32) * (uint32_t)NT;
    if (G >= 64 && G % 32 == 0 && (gn <= 4 || (NT == 4 && G == 64))) return RowLayout{32, (int)(G / 32)};
    // 80 groups (hidden 2560) for several tokens.  IQ3_S: 64 lanes x 2
    // adjacent groups (its paired decode) with the last 48 slots idle, x in
    // registers; the other types: 16 lanes x 5 groups, every slot busy, x
    // read from LDS per group (five groups of every token's x would spill).
    // 4-token window at the reference model's shapes, gate/up alone: IQ3_S
    // 28.9 / 30.1 us, IQ3_XXS 31.6 / 27.8 us, IQ2_S 31.0 / 25.9 us (64 x 2 /
    // 16 x 5).
    if (G == 80 && NT >= 2) return ty == Q4MI_T_IQ3_S ? RowLayout{64, 2} : RowLayout{16, 5};
    return layout_for(G);
}

template <uint32_t TY, int NT>
static bool gu_dispatch(const MoeArgs &a, uint32_t nu_host) {
    const RowLayout L = gu_layout(a.K / 32, NT, TY);
#define Q4MI_L(T, P) \
    if (L.tpr == T && L.gpt == P) return launch_gu<TY, NT, T, P>(a, nu_host);
    Q4MI_L(8, 1) Q4MI_L(16, 1) Q4MI_L(32, 1) Q4MI_L(64, 1) Q4MI_L(64, 2) Q4MI_L(64, 4)
    Q4MI_L(16, 5)
    if constexpr (NT <= 4) { Q4MI_L(32, 2) }
    if constexpr (NT == 1) { Q4MI_L(32, 4) }
#undef Q4MI_L
    return false;
}

// Down lanes per item: 8 lanes with two groups each for 16-group rows, so
// 96 teams cover a block's (expert, row) items in one round; else the row
// layout.
static RowLayout dn_layout(uint32_t G, int NT) {
    // 8 lanes x 2 groups: a one-token block's 88 items in one round of 96
    // teams.  (4 lanes x 4 groups for windows measured slower: 36.0 against
    // 35.1 us for 4 tokens.)
    if (G == 16 && NT <= 4) return RowLayout{8, 2};
    return layout_for(G);
}

template <uint32_t TY, int NT>
static bool dn_dispatch(const MoeArgs &a, uint32_t nu_host) {
    const RowLayout L = dn_layout(a.n_ff / 32, NT);
#define Q4MI_L(T, P) \
    if (L.tpr == T && L.gpt == P) return launch_dn<TY, NT, T, P>(a, nu_host);
    Q4MI_L(8, 1) Q4MI_L(16, 1) Q4MI_L(32, 1) Q4MI_L(64, 1) Q4MI_L(64, 2) Q4MI_L(64, 4)
    Q4MI_L(4, 5)
    if constexpr (NT <= 4) { Q4MI_L(8, 2) }
#undef Q4MI_L
    return false;
}


// Dispatch of the types instantiated outside moe_decode.hip (moe_fmt_*.hip).
bool moe_fmt_gu(uint32_t ty, int nt, const MoeArgs &a, uint32_t nu_host);
bool moe_fmt_dn(uint32_t ty, int nt, const MoeArgs &a, uint32_t nu_host);
// Their translation units' timeout words (see q4mi_device_status).
uint32_t moe_fmt_status(int clear);
uint32_t moe_fmt_status_dn(int clear);

}  // namespace q4mi
