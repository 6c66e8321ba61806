// Device decoders of the weight formats beside IQ3_S / Q8_0 that the
// reference's models mix into their routed experts and LM head: IQ4_NL and
// Q2_0 (down projections of the verify window, src/q4_rocm.cu:7378-7386),
// IQ2_S (gate/up) and Q6_K (LM head, wgv_q6_k_k src/q4_rocm.cu:2525).
//
// Every decoder turns one 32-value group of a row held in LDS into eight
// signed int8 quads (values 4k..4k+3 in quad k, natural order), the integer
// multipliers of quads 0-3 (m1) and 4-7 (m2), and the float block scale d,
// so that the group's exact integer sum against q8 codes q is
//   S = m1 * sum_{k<4} dot4(w_k, q_k) + m2 * sum_{k>=4} dot4(w_k, q_k)
// and its value is d * d_x * S.  Block layouts (reference src/q4_quant.c):
//   IQ4_NL  18 B / 32:  d | qs[16]: value j = kv[qs[j] & 15], j+16 = kv[qs[j] >> 4]
//   Q2_0    18 B / 64:  d | qs[16]: value j = ((qs[j/4] >> 2(j%4)) & 3) - 1
//   IQ2_S   82 B / 256: d | qs[32] grid index low bits | signs[32] | qh[8] |
//                       scales[8]; group ib: entries l = 0..3 of
//                       grid[qs[4ib+l] | ((qh[ib] << (8-2l)) & 0x300)], sign
//                       bit j of signs[4ib+l] negates value j; multiplier
//                       2*nibble+1 (low nibble: values 0-15), d * 0.125
//   IQ2_XXS 66 B / 256: d | per group ib a u32 of four grid bytes (8
//                       values each, {8, 25, 43}) and a u32 of four 7-bit
//                       sign indexes (bit 7 of the sign byte = parity) and
//                       the 4-bit scale s in its top nibble; multiplier
//                       2s+1, d * 0.125
//   IQ2_XS  74 B / 256: d | qs[32] u16 = 9-bit grid index | 7-bit sign
//                       index << 9 | scales[8]: low nibble values 0-15,
//                       high 16-31, multipliers 2*nibble+1, d * 0.125
//   IQ3_XXS 98 B / 256: d | qs[64] grid bytes (4 values each, {4 .. 62}) |
//                       per group a u32 of four 7-bit sign indexes (8 values
//                       each) and the scale s in its top nibble; multiplier
//                       2s+1, d * 0.25
//   IQ4_XS 136 B / 256: d | scales_h u16 | scales_l[4] | qs[128]: group ib
//                       as IQ4_NL's nibbles at qs[16 ib], multiplier
//                       ls - 32, ls = 4 bits of scales_l | 2 of scales_h
//   Q6_K   210 B / 256: ql[128] | qh[64] | int8 sc[16] | d: half h (128
//                       values), group gq = 0..3 of it, value l = (4-bit
//                       from ql[64h + 32(gq&1) + l] (high nibble when gq&2)
//                       | 2 bits (qh[32h + l] >> 2gq) << 4) - 32, sub-block
//                       scales sc[8h + 2gq] (values 0-15), sc[8h + 2gq + 1]
#pragma once
#include "q4mi_common.h"
#include "../../include/q4mi_iq2s_grid.h"
#include "../../include/q4mi_iqxx_grids.h"

#define Q4MI_T_Q6_K 14u
#define Q4MI_T_IQ2_XXS 16u
#define Q4MI_T_IQ2_XS 17u
#define Q4MI_T_IQ3_XXS 18u
#define Q4MI_T_IQ4_XS 23u
#define Q4MI_T_IQ4_NL 20u
#define Q4MI_T_IQ2_S 22u
#define Q4MI_T_Q2_0 42u

namespace q4mi {

struct WGroup {
    int32_t w[8];
    int m1, m2;
    float d;
};

__constant__ uint16_t q4mi_iq2s_code_dev[1024] = {Q4MI_IQ2S_CODES};
__constant__ uint16_t q4mi_iq2xxs_code_dev[256] = {Q4MI_IQ2XXS_CODES};
__constant__ uint16_t q4mi_iq2xs_code_dev[512] = {Q4MI_IQ2XS_CODES};
__constant__ uint16_t q4mi_iq3xxs_code_dev[256] = {Q4MI_IQ3XXS_CODES};

// Four consecutive dwords (any 2-byte-aligned LDS byte offset) as u32.
__device__ inline void lds_dwords(const uint32_t *lw, uint32_t off, uint32_t (&o)[4]) {
    const uint32_t i = off >> 2, sh = off & 3u;
    const uint32_t a = lw[i], b = lw[i + 1], c = lw[i + 2], d = lw[i + 3], e = lw[i + 4];
    o[0] = __builtin_amdgcn_alignbyte(b, a, sh);
    o[1] = __builtin_amdgcn_alignbyte(c, b, sh);
    o[2] = __builtin_amdgcn_alignbyte(d, c, sh);
    o[3] = __builtin_amdgcn_alignbyte(e, d, sh);
}

// ------------------------------------------------------------------ IQ4_NL
// 16-entry value table in four dwords; a byte selector 0..15 picks through
// two v_perm_b32 (entries 0-7 and 8-15) and bit 3 chooses between them.
__device__ inline int32_t iq4nl_map(uint32_t sel) {
    constexpr uint32_t T0 = 0xBFAD9881u;   // -127, -104, -83, -65
    constexpr uint32_t T1 = 0xF6EADDCFu;   //  -49,  -35, -22, -10
    constexpr uint32_t T2 = 0x26190D01u;   //    1,   13,  25,  38
    constexpr uint32_t T3 = 0x71594535u;   //   53,   69,  89, 113
    const uint32_t lo3 = sel & 0x07070707u;
    const uint32_t a = __builtin_amdgcn_perm(T1, T0, lo3);
    const uint32_t b = __builtin_amdgcn_perm(T3, T2, lo3);
    const uint32_t m = (sel >> 3) & 0x01010101u;
    const uint32_t m8 = (m << 8) - m;                       // 0xff where bit 3 set
    return (int32_t)((a & ~m8) | (b & m8));
}

struct FmtIQ4NL {
    static constexpr uint32_t kType = Q4MI_T_IQ4_NL;
    static constexpr uint32_t kTabBytes = 0;
    static constexpr bool kTwo = false;
    __device__ static inline void init(void *, uint32_t, uint32_t) {}
    __device__ static inline void decode(const void *, const uint8_t *lb, const uint32_t *lw,
                                         uint32_t row, uint32_t g, WGroup &o) {
        const uint32_t B = row + 18u * g;
        o.d = q4mi_h2f(lds_u16_at(lb, B));
        o.m1 = o.m2 = 1;
        uint32_t q[4];
        lds_dwords(lw, B + 2u, q);
#pragma unroll
        for (int k = 0; k < 4; k++) {
            o.w[k] = iq4nl_map(q[k] & 0x0F0F0F0Fu);
            o.w[k + 4] = iq4nl_map((q[k] >> 4) & 0x0F0F0F0Fu);
        }
    }
};

// -------------------------------------------------------------------- Q2_0
// Byte b of the codes holds quad b: its four 2-bit codes spread to the four
// bytes by two shift-or steps, then c - 1 through a v_perm byte table.
__device__ inline int32_t q20_quad(uint32_t byte) {
    const uint32_t t1 = (byte << 6) | byte;
    const uint32_t t2 = (t1 << 12) | t1;
    return (int32_t)__builtin_amdgcn_perm(0u, 0x020100FFu, t2 & 0x03030303u);
}

struct FmtQ20 {
    static constexpr uint32_t kType = Q4MI_T_Q2_0;
    static constexpr uint32_t kTabBytes = 0;
    static constexpr bool kTwo = false;
    __device__ static inline void init(void *, uint32_t, uint32_t) {}
    __device__ static inline void decode(const void *, const uint8_t *lb, const uint32_t *lw,
                                         uint32_t row, uint32_t g, WGroup &o) {
        const uint32_t B = row + 18u * (g >> 1);
        o.d = q4mi_h2f(lds_u16_at(lb, B));
        o.m1 = o.m2 = 1;
        const uint32_t c0 = lds_u32_at(lw, B + 2u + 8u * (g & 1u));
        const uint32_t c1 = lds_u32_at(lw, B + 6u + 8u * (g & 1u));
#pragma unroll
        for (int k = 0; k < 4; k++) {
            o.w[k] = q20_quad((c0 >> (8 * k)) & 0xffu);
            o.w[k + 4] = q20_quad((c1 >> (8 * k)) & 0xffu);
        }
    }
};

// ------------------------------------------------------------------- IQ2_S
// LDS: the 1024-entry grid (two magnitude dwords per entry) and the sign
// byte -> two byte-mask dwords table, 10 KB.
struct Iq2sLds {
    uint2 grid[1024];
    uint2 smask[256];
};

struct FmtIQ2S {
    static constexpr uint32_t kType = Q4MI_T_IQ2_S;
    static constexpr uint32_t kTabBytes = sizeof(Iq2sLds);
    static constexpr bool kTwo = true;
    __device__ static inline void init(void *tab, uint32_t tid, uint32_t n) {
        Iq2sLds *t = (Iq2sLds *)tab;
        for (uint32_t i = tid; i < 1024; i += n) {
            const uint32_t c = q4mi_iq2s_code_dev[i];
            uint32_t lo = 0, hi = 0;
#pragma unroll
            for (int j = 0; j < 4; j++) {
                const uint32_t a = (c >> (2 * j)) & 3u, b = (c >> (2 * j + 8)) & 3u;
                lo |= (a == 0 ? 8u : a == 1 ? 25u : 43u) << (8 * j);
                hi |= (b == 0 ? 8u : b == 1 ? 25u : 43u) << (8 * j);
            }
            t->grid[i] = make_uint2(lo, hi);
        }
        for (uint32_t i = tid; i < 256; i += n)
            t->smask[i] = make_uint2(q4mi_expand4(i & 15u), q4mi_expand4(i >> 4));
    }
    __device__ static inline void decode(const void *tab, const uint8_t *lb, const uint32_t *lw,
                                         uint32_t row, uint32_t g, WGroup &o) {
        const Iq2sLds *t = (const Iq2sLds *)tab;
        const uint32_t B = row + 82u * (g >> 3), ib = g & 7u;
        o.d = q4mi_h2f(lds_u16_at(lb, B)) * 0.125f;
        const uint32_t qs = lds_u32_at(lw, B + 2u + 4u * ib);
        const uint32_t sg = lds_u32_at(lw, B + 34u + 4u * ib);
        const uint32_t qh = lds_u8_at(lb, B + 66u + ib);
        const uint32_t sc = lds_u8_at(lb, B + 74u + ib);
        o.m1 = 2 * (int)(sc & 15u) + 1;
        o.m2 = 2 * (int)(sc >> 4) + 1;
#pragma unroll
        for (int l = 0; l < 4; l++) {
            const uint32_t idx = ((qs >> (8 * l)) & 0xffu) | ((qh << (8 - 2 * l)) & 0x300u);
            const uint2 e = t->grid[idx];
            const uint2 m = t->smask[(sg >> (8 * l)) & 0xffu];
            // magnitudes <= 43: (g ^ m) + (m & 1) stays inside each byte
            o.w[2 * l] = q4mi_sign4(e.x, m.x);
            o.w[2 * l + 1] = q4mi_sign4(e.y, m.y);
        }
    }
};

// -------------------------------------------------------------------- Q6_K
// 6-bit codes c -> int8 c - 32 per byte: t = c ^ 0x20 is c - 32 when bit 5
// of c was set, else c + 32, whose bit 5 is then set: fill bits 6 and 7.
__device__ inline int32_t q6_sub32(uint32_t c) {
    const uint32_t t = c ^ 0x20202020u;
    const uint32_t m = t & 0x20202020u;
    return (int32_t)(t | (m << 1) | (m << 2));
}

struct FmtQ6K {
    static constexpr uint32_t kType = Q4MI_T_Q6_K;
    static constexpr uint32_t kTabBytes = 0;
    static constexpr bool kTwo = true;
    __device__ static inline void init(void *, uint32_t, uint32_t) {}
    __device__ static inline void decode(const void *, const uint8_t *lb, const uint32_t *lw,
                                         uint32_t row, uint32_t g, WGroup &o) {
        const uint32_t B = row + 210u * (g >> 3), j = g & 7u, h = j >> 2, gq = j & 3u;
        o.d = q4mi_h2f(lds_u16_at(lb, B + 208u));
        const uint32_t sc = lds_u16_at(lb, B + 192u + 8u * h + 2u * gq);
        o.m1 = (int)(int8_t)(sc & 0xffu);
        o.m2 = (int)(int8_t)(sc >> 8);
        uint32_t ql[4], qh[4];
#pragma unroll
        for (int half = 0; half < 2; half++) {
            lds_dwords(lw, B + 64u * h + 32u * (gq & 1u) + 16u * half, ql);
            lds_dwords(lw, B + 128u + 32u * h + 16u * half, qh);
#pragma unroll
            for (int k = 0; k < 4; k++) {
                const uint32_t lo = ((gq & 2u) ? (ql[k] >> 4) : ql[k]) & 0x0F0F0F0Fu;
                const uint32_t hi = (qh[k] >> (2 * gq)) & 0x03030303u;
                o.w[4 * half + k] = q6_sub32(lo | (hi << 4));
            }
        }
    }
};


// ------------------------------------------- IQ2_XXS, IQ2_XS, IQ3_XXS
// LDS: the grid as magnitude dwords and the 7-bit sign index -> two byte-mask
// dwords table (the sign byte's bit 7 is the parity of the other seven).
__device__ inline uint2 iqxx_sign_masks(uint32_t i) {
    const uint32_t sb = i | ((__popc(i) & 1u) << 7);
    return make_uint2(q4mi_expand4(sb & 15u), q4mi_expand4(sb >> 4));
}
__device__ inline uint32_t iq2_level_dev(uint32_t c) { return c == 0 ? 8u : c == 1 ? 25u : 43u; }

template <uint32_t N>
struct Iq2xLds {
    uint2 grid[N];
    uint2 smask[128];
};

template <uint32_t N>
__device__ inline void iq2x_init(Iq2xLds<N> *t, const uint16_t *codes, uint32_t tid, uint32_t n) {
    for (uint32_t i = tid; i < N; i += n) {
        const uint32_t c = codes[i];
        uint32_t lo = 0, hi = 0;
#pragma unroll
        for (int j = 0; j < 4; j++) {
            lo |= iq2_level_dev((c >> (2 * j)) & 3u) << (8 * j);
            hi |= iq2_level_dev((c >> (2 * j + 8)) & 3u) << (8 * j);
        }
        t->grid[i] = make_uint2(lo, hi);
    }
    for (uint32_t i = tid; i < 128; i += n) t->smask[i] = iqxx_sign_masks(i);
}

struct FmtIQ2XXS {
    static constexpr uint32_t kType = Q4MI_T_IQ2_XXS;
    static constexpr uint32_t kTabBytes = sizeof(Iq2xLds<256>);
    static constexpr bool kTwo = false;
    __device__ static inline void init(void *tab, uint32_t tid, uint32_t n) {
        iq2x_init((Iq2xLds<256> *)tab, q4mi_iq2xxs_code_dev, tid, n);
    }
    __device__ static inline void decode(const void *tab, const uint8_t *lb, const uint32_t *lw,
                                         uint32_t row, uint32_t g, WGroup &o) {
        const Iq2xLds<256> *t = (const Iq2xLds<256> *)tab;
        const uint32_t B = row + 66u * (g >> 3), ib = g & 7u;
        o.d = q4mi_h2f(lds_u16_at(lb, B)) * 0.125f;
        const uint32_t gi = lds_u32_at(lw, B + 2u + 8u * ib);
        const uint32_t aux = lds_u32_at(lw, B + 6u + 8u * ib);
        o.m1 = o.m2 = 2 * (int)(aux >> 28) + 1;
#pragma unroll
        for (int l = 0; l < 4; l++) {
            const uint2 e = t->grid[(gi >> (8 * l)) & 0xffu];
            const uint2 m = t->smask[(aux >> (7 * l)) & 127u];
            o.w[2 * l] = q4mi_sign4(e.x, m.x);
            o.w[2 * l + 1] = q4mi_sign4(e.y, m.y);
        }
    }
};

struct FmtIQ2XS {
    static constexpr uint32_t kType = Q4MI_T_IQ2_XS;
    static constexpr uint32_t kTabBytes = sizeof(Iq2xLds<512>);
    static constexpr bool kTwo = true;
    __device__ static inline void init(void *tab, uint32_t tid, uint32_t n) {
        iq2x_init((Iq2xLds<512> *)tab, q4mi_iq2xs_code_dev, tid, n);
    }
    __device__ static inline void decode(const void *tab, const uint8_t *lb, const uint32_t *lw,
                                         uint32_t row, uint32_t g, WGroup &o) {
        const Iq2xLds<512> *t = (const Iq2xLds<512> *)tab;
        const uint32_t B = row + 74u * (g >> 3), ib = g & 7u;
        o.d = q4mi_h2f(lds_u16_at(lb, B)) * 0.125f;
        const uint32_t v01 = lds_u32_at(lw, B + 2u + 8u * ib);
        const uint32_t v23 = lds_u32_at(lw, B + 6u + 8u * ib);
        const uint32_t sc = lds_u8_at(lb, B + 66u + ib);
        o.m1 = 2 * (int)(sc & 15u) + 1;
        o.m2 = 2 * (int)(sc >> 4) + 1;
#pragma unroll
        for (int l = 0; l < 4; l++) {
            const uint32_t v = ((l < 2 ? v01 : v23) >> (16 * (l & 1))) & 0xffffu;
            const uint2 e = t->grid[v & 511u];
            const uint2 m = t->smask[v >> 9];
            o.w[2 * l] = q4mi_sign4(e.x, m.x);
            o.w[2 * l + 1] = q4mi_sign4(e.y, m.y);
        }
    }
};

struct Iq3xxsLds {
    uint32_t grid[256];
    uint2 smask[128];
};

struct FmtIQ3XXS {
    static constexpr uint32_t kType = Q4MI_T_IQ3_XXS;
    static constexpr uint32_t kTabBytes = sizeof(Iq3xxsLds);
    static constexpr bool kTwo = false;
    __device__ static inline void init(void *tab, uint32_t tid, uint32_t n) {
        Iq3xxsLds *t = (Iq3xxsLds *)tab;
        for (uint32_t i = tid; i < 256; i += n) {
            const uint32_t c = q4mi_iq3xxs_code_dev[i];
            uint32_t v = 0;
#pragma unroll
            for (int j = 0; j < 4; j++) {
                const uint32_t k = (c >> (3 * j)) & 7u;
                v |= (k == 7u ? 62u : 8u * k + 4u) << (8 * j);
            }
            t->grid[i] = v;
        }
        for (uint32_t i = tid; i < 128; i += n) t->smask[i] = iqxx_sign_masks(i);
    }
    __device__ static inline void decode(const void *tab, const uint8_t *lb, const uint32_t *lw,
                                         uint32_t row, uint32_t g, WGroup &o) {
        const Iq3xxsLds *t = (const Iq3xxsLds *)tab;
        const uint32_t B = row + 98u * (g >> 3), ib = g & 7u;
        o.d = q4mi_h2f(lds_u16_at(lb, B)) * 0.25f;
        const uint32_t q0 = lds_u32_at(lw, B + 2u + 8u * ib);
        const uint32_t q1 = lds_u32_at(lw, B + 6u + 8u * ib);
        const uint32_t aux = lds_u32_at(lw, B + 66u + 4u * ib);
        o.m1 = o.m2 = 2 * (int)(aux >> 28) + 1;
#pragma unroll
        for (int k = 0; k < 8; k++) {
            const uint32_t gb = ((k < 4 ? q0 : q1) >> (8 * (k & 3))) & 0xffu;
            const uint2 m = t->smask[(aux >> (7 * (k >> 1))) & 127u];
            o.w[k] = q4mi_sign4(t->grid[gb], (k & 1) ? m.y : m.x);
        }
    }
};

// ------------------------------------------------------------------ IQ4_XS
struct FmtIQ4XS {
    static constexpr uint32_t kType = Q4MI_T_IQ4_XS;
    static constexpr uint32_t kTabBytes = 0;
    static constexpr bool kTwo = false;
    __device__ static inline void init(void *, uint32_t, uint32_t) {}
    __device__ static inline void decode(const void *, const uint8_t *lb, const uint32_t *lw,
                                         uint32_t row, uint32_t g, WGroup &o) {
        const uint32_t B = row + 136u * (g >> 3), ib = g & 7u;
        o.d = q4mi_h2f(lds_u16_at(lb, B));
        const uint32_t sh = lds_u16_at(lb, B + 2u);
        const uint32_t sl = lds_u8_at(lb, B + 4u + (ib >> 1));
        const int ls = (int)(((sl >> (4 * (ib & 1u))) & 15u) | (((sh >> (2 * ib)) & 3u) << 4));
        o.m1 = o.m2 = ls - 32;
        uint32_t q[4];
        lds_dwords(lw, B + 8u + 16u * ib, q);
#pragma unroll
        for (int k = 0; k < 4; k++) {
            o.w[k] = iq4nl_map(q[k] & 0x0F0F0F0Fu);
            o.w[k + 4] = iq4nl_map((q[k] >> 4) & 0x0F0F0F0Fu);
        }
    }
};

template <uint32_t TY>
struct FmtOf;
template <>
struct FmtOf<Q4MI_T_IQ4_NL> {
    using F = FmtIQ4NL;
};
template <>
struct FmtOf<Q4MI_T_Q2_0> {
    using F = FmtQ20;
};
template <>
struct FmtOf<Q4MI_T_IQ2_S> {
    using F = FmtIQ2S;
};
template <>
struct FmtOf<Q4MI_T_Q6_K> {
    using F = FmtQ6K;
};
template <>
struct FmtOf<Q4MI_T_IQ2_XXS> {
    using F = FmtIQ2XXS;
};
template <>
struct FmtOf<Q4MI_T_IQ2_XS> {
    using F = FmtIQ2XS;
};
template <>
struct FmtOf<Q4MI_T_IQ3_XXS> {
    using F = FmtIQ3XXS;
};
template <>
struct FmtOf<Q4MI_T_IQ4_XS> {
    using F = FmtIQ4XS;
};

}  // namespace q4mi
