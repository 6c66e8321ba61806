// Int8-activation row-dot engine for decode (MMVQ), wave64 / gfx950.
//
// A 256-thread block stages a tile of weight rows into LDS with coalesced
// 16-byte loads (IQ3_S rows are 110-byte superblocks, not 16-byte aligned
// units, so they are decoded from LDS, never straight from global memory).
// TPR lanes cooperate on one row; lane gi owns the row's 32-value groups
// gi, gi+TPR, ... (GPT of them), so its q8 activations for those groups stay
// in registers for every row of the tile.  Per group the lane decodes the
// weights to signed int8 quads, takes v_dot4_i32_i8 against the activation
// quads, scales the exact int32 group sum by (2s+1) and accumulates
// float(S) * (d_w * d_x).  A DPP reduction over the TPR lanes finishes
// the row.
#pragma once
#include "formats.h"
#include "q4mi_common.h"

namespace q4mi {

// Formats of the engine: kType, kTabBytes (LDS tables before the tile),
// kTwo (two multipliers per group, quads 0-3 and 4-7), init (build the
// tables), decode (one 32-value group of a row in LDS, formats.h's WGroup).
struct FmtIQ3S {
    static constexpr uint32_t kType = Q4MI_T_IQ3_S;
    static constexpr uint32_t kTabBytes = sizeof(Iq3sLds);
    static constexpr bool kTwo = false;
    __device__ static inline void init(void *tab, uint32_t tid, uint32_t n) {
        q4mi_iq3s_tables_init((Iq3sLds *)tab, (int)tid, (int)n);
    }
    __device__ static inline void decode(const void *tab, const uint8_t *lb,
                                         const uint32_t *lw, uint32_t row, uint32_t g,
                                         WGroup &o) {
        Iq3sGroup q;
        q4mi_iq3s_decode((const Iq3sLds *)tab, lb, lw, row, g, q);
#pragma unroll
        for (int k = 0; k < 8; k++) o.w[k] = q.w[k];
        o.m1 = o.m2 = q.mult;
        o.d = q.d;
    }
};

struct FmtQ80 {
    static constexpr uint32_t kType = Q4MI_T_Q8_0;
    static constexpr uint32_t kTabBytes = 0;
    static constexpr bool kTwo = false;
    __device__ static inline void init(void *, uint32_t, uint32_t) {}
    __device__ static inline void decode(const void *, const uint8_t *lb,
                                         const uint32_t *lw, uint32_t row, uint32_t g,
                                         WGroup &o) {
        const uint32_t B = row + g * Q80_BYTES;
        o.d = q4mi_h2f(lds_u16_at(lb, B));
        o.m1 = o.m2 = 1;
        const uint32_t i0 = (B + 2u) >> 2, sh = (B + 2u) & 3u;
        uint32_t prev = lw[i0];
#pragma unroll
        for (int k = 0; k < 8; k++) {
            const uint32_t nx = lw[i0 + 1 + k];
            o.w[k] = (int32_t)__builtin_amdgcn_alignbyte(nx, prev, sh);
            prev = nx;
        }
    }
};

// Exact group sum against one token's eight activation quads.
template <class F>
__device__ inline int group_sum(const WGroup &w, const int32_t (&q)[8]) {
    if constexpr (F::kTwo) {
        int a = 0, b = 0;
#pragma unroll
        for (int k = 0; k < 4; k++) a = q4mi_sdot4(w.w[k], q[k], a);
#pragma unroll
        for (int k = 4; k < 8; k++) b = q4mi_sdot4(w.w[k], q[k], b);
        return __mul24(a, w.m1) + __mul24(b, w.m2);
    } else {
        int s = 0;
#pragma unroll
        for (int k = 0; k < 8; k++) s = q4mi_sdot4(w.w[k], q[k], s);
        return __mul24(s, w.m1);
    }
}

// q8 activations of this lane's GPT groups for NT tokens.
template <int NT, int GPT>
struct XRegs {
    int32_t q[GPT][NT][8];
    float d[GPT][NT];
};

// xq: [nt][K] int8, xd: [nt][K/32] (global or LDS); tokens >= nt read as 0.
// Lane gi's groups: gi + TPR*m, or with ADJ the adjacent GPT*gi + m.
// (G: the row's group count when TPR * GPT covers more groups than the row
// has; the lanes past it hold zeros)
template <int NT, int GPT, int TPR, bool ADJ = false>
__device__ inline void load_xregs(XRegs<NT, GPT> &x, const int8_t *xq, const float *xd,
                                  uint32_t K, uint32_t nt, uint32_t gi, uint32_t G = ~0u) {
#pragma unroll
    for (int m = 0; m < GPT; m++) {
        const uint32_t g = ADJ ? GPT * gi + m : gi + TPR * m;
#pragma unroll
        for (int t = 0; t < NT; t++) {
            if ((uint32_t)t < nt && g < G) {
                const int4 a = *(const int4 *)(xq + (size_t)t * K + 32u * g);
                const int4 b = *(const int4 *)(xq + (size_t)t * K + 32u * g + 16u);
                x.q[m][t][0] = a.x; x.q[m][t][1] = a.y; x.q[m][t][2] = a.z; x.q[m][t][3] = a.w;
                x.q[m][t][4] = b.x; x.q[m][t][5] = b.y; x.q[m][t][6] = b.z; x.q[m][t][7] = b.w;
                x.d[m][t] = xd[(size_t)t * (K / 32) + g];
            } else {
#pragma unroll
                for (int k = 0; k < 8; k++) x.q[m][t][k] = 0;
                x.d[m][t] = 0.f;
            }
        }
    }
}

// Partial dot of one row (this lane's groups) for NT tokens, added to acc.
// sums (optional): per-token int32 group sums, sums[t * sum_tstride + g].
template <class F, int NT, int GPT, int TPR>
__device__ inline void row_dot(const void *tab, const uint8_t *lb, const uint32_t *lw,
                               uint32_t row, uint32_t gi, const XRegs<NT, GPT> &x,
                               float (&acc)[NT], int32_t *sums, size_t sum_tstride) {
#pragma unroll
    for (int m = 0; m < GPT; m++) {
        const uint32_t g = gi + TPR * m;
        WGroup w;
        F::decode(tab, lb, lw, row, g, w);
#pragma unroll
        for (int t = 0; t < NT; t++) {
            const int s = group_sum<F>(w, x.q[m][t]);
            acc[t] = fmaf((float)s, w.d * x.d[m][t], acc[t]);
            if (sums) sums[(size_t)t * sum_tstride + g] = s;
        }
    }
}

// Wait until at most n VMEM operations of this wave are outstanding.  The
// count is an instruction immediate, so a runtime n selects among literal
// waits; n beyond the 6-bit field waits for more than asked, never less.
__device__ inline void wait_vm(uint32_t n) {
    switch (__builtin_amdgcn_readfirstlane(n)) {
    case 0: asm volatile("s_waitcnt vmcnt(0)" ::: "memory"); break;
    case 1: asm volatile("s_waitcnt vmcnt(1)" ::: "memory"); break;
    case 2: asm volatile("s_waitcnt vmcnt(2)" ::: "memory"); break;
    case 3: asm volatile("s_waitcnt vmcnt(3)" ::: "memory"); break;
    case 4: asm volatile("s_waitcnt vmcnt(4)" ::: "memory"); break;
    case 5: asm volatile("s_waitcnt vmcnt(5)" ::: "memory"); break;
    case 6: asm volatile("s_waitcnt vmcnt(6)" ::: "memory"); break;
    case 7: asm volatile("s_waitcnt vmcnt(7)" ::: "memory"); break;
    case 8: asm volatile("s_waitcnt vmcnt(8)" ::: "memory"); break;
    case 9: asm volatile("s_waitcnt vmcnt(9)" ::: "memory"); break;
    case 10: asm volatile("s_waitcnt vmcnt(10)" ::: "memory"); break;
    case 11: asm volatile("s_waitcnt vmcnt(11)" ::: "memory"); break;
    case 12: asm volatile("s_waitcnt vmcnt(12)" ::: "memory"); break;
    case 13: asm volatile("s_waitcnt vmcnt(13)" ::: "memory"); break;
    case 14: asm volatile("s_waitcnt vmcnt(14)" ::: "memory"); break;
    case 15: asm volatile("s_waitcnt vmcnt(15)" ::: "memory"); break;
    case 16: asm volatile("s_waitcnt vmcnt(16)" ::: "memory"); break;
    case 17: asm volatile("s_waitcnt vmcnt(17)" ::: "memory"); break;
    case 18: asm volatile("s_waitcnt vmcnt(18)" ::: "memory"); break;
    case 19: asm volatile("s_waitcnt vmcnt(19)" ::: "memory"); break;
    case 20: asm volatile("s_waitcnt vmcnt(20)" ::: "memory"); break;
    case 21: asm volatile("s_waitcnt vmcnt(21)" ::: "memory"); break;
    case 22: asm volatile("s_waitcnt vmcnt(22)" ::: "memory"); break;
    case 23: asm volatile("s_waitcnt vmcnt(23)" ::: "memory"); break;
    case 24: asm volatile("s_waitcnt vmcnt(24)" ::: "memory"); break;
    case 25: asm volatile("s_waitcnt vmcnt(25)" ::: "memory"); break;
    case 26: asm volatile("s_waitcnt vmcnt(26)" ::: "memory"); break;
    case 27: asm volatile("s_waitcnt vmcnt(27)" ::: "memory"); break;
    case 28: asm volatile("s_waitcnt vmcnt(28)" ::: "memory"); break;
    case 29: asm volatile("s_waitcnt vmcnt(29)" ::: "memory"); break;
    case 30: asm volatile("s_waitcnt vmcnt(30)" ::: "memory"); break;
    case 31: asm volatile("s_waitcnt vmcnt(31)" ::: "memory"); break;
    case 32: asm volatile("s_waitcnt vmcnt(32)" ::: "memory"); break;
    case 33: asm volatile("s_waitcnt vmcnt(33)" ::: "memory"); break;
    case 34: asm volatile("s_waitcnt vmcnt(34)" ::: "memory"); break;
    case 35: asm volatile("s_waitcnt vmcnt(35)" ::: "memory"); break;
    case 36: asm volatile("s_waitcnt vmcnt(36)" ::: "memory"); break;
    case 37: asm volatile("s_waitcnt vmcnt(37)" ::: "memory"); break;
    case 38: asm volatile("s_waitcnt vmcnt(38)" ::: "memory"); break;
    case 39: asm volatile("s_waitcnt vmcnt(39)" ::: "memory"); break;
    case 40: asm volatile("s_waitcnt vmcnt(40)" ::: "memory"); break;
    case 41: asm volatile("s_waitcnt vmcnt(41)" ::: "memory"); break;
    case 42: asm volatile("s_waitcnt vmcnt(42)" ::: "memory"); break;
    case 43: asm volatile("s_waitcnt vmcnt(43)" ::: "memory"); break;
    case 44: asm volatile("s_waitcnt vmcnt(44)" ::: "memory"); break;
    case 45: asm volatile("s_waitcnt vmcnt(45)" ::: "memory"); break;
    case 46: asm volatile("s_waitcnt vmcnt(46)" ::: "memory"); break;
    case 47: asm volatile("s_waitcnt vmcnt(47)" ::: "memory"); break;
    case 48: asm volatile("s_waitcnt vmcnt(48)" ::: "memory"); break;
    case 49: asm volatile("s_waitcnt vmcnt(49)" ::: "memory"); break;
    case 50: asm volatile("s_waitcnt vmcnt(50)" ::: "memory"); break;
    case 51: asm volatile("s_waitcnt vmcnt(51)" ::: "memory"); break;
    case 52: asm volatile("s_waitcnt vmcnt(52)" ::: "memory"); break;
    case 53: asm volatile("s_waitcnt vmcnt(53)" ::: "memory"); break;
    case 54: asm volatile("s_waitcnt vmcnt(54)" ::: "memory"); break;
    case 55: asm volatile("s_waitcnt vmcnt(55)" ::: "memory"); break;
    case 56: asm volatile("s_waitcnt vmcnt(56)" ::: "memory"); break;
    case 57: asm volatile("s_waitcnt vmcnt(57)" ::: "memory"); break;
    case 58: asm volatile("s_waitcnt vmcnt(58)" ::: "memory"); break;
    case 59: asm volatile("s_waitcnt vmcnt(59)" ::: "memory"); break;
    case 60: asm volatile("s_waitcnt vmcnt(60)" ::: "memory"); break;
    case 61: asm volatile("s_waitcnt vmcnt(61)" ::: "memory"); break;
    case 62: asm volatile("s_waitcnt vmcnt(62)" ::: "memory"); break;
    default: asm volatile("s_waitcnt vmcnt(63)" ::: "memory"); break;
    }
}

// One 16-byte-per-lane global -> LDS copy of the calling wave (gfx950
// global_load_lds_dwordx4): lane i's 16 bytes at g land at LDS byte address
// lds + 16 i.  Inline asm, so the compiler adds no waits of its own.
__device__ inline void lds_dma16(const void *g, uint32_t lds) {
    lds = __builtin_amdgcn_readfirstlane(lds);
    asm volatile("s_mov_b32 m0, %1\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %0, off"
                 :: "v"(g), "s"(lds) : "memory", "m0");
}

// Start copying nbytes (even) from global src to LDS dst with the widest
// aligned accesses the addresses allow; all threads of the block take part.
// 16-byte-aligned spans go by global -> LDS DMA and stay in flight (the
// caller waits with vmcnt(0) and a barrier); other spans are copied through
// registers before this returns (visible after the caller's barrier).
__device__ inline void stage_tile_issue(uint8_t *dst, const uint8_t *src, uint32_t nbytes,
                                        uint32_t tid, uint32_t nthr) {
    const uintptr_t a = (uintptr_t)src | nbytes;
    // (the register-copy fallbacks are laid out after the common path)
    if (__builtin_expect((a & 15u) == 0, 1)) {
        // every copy of the block in flight at once (1 KB per wave op)
        const uint32_t lane = tid & 63u, nw = nthr / 64;
        const uint32_t w = __builtin_amdgcn_readfirstlane(tid >> 6);
        const uint32_t l0 = (uint32_t)(uintptr_t)dst;   // LDS offset: low half of the flat address
        for (uint32_t j = w; j < (nbytes + 1023) / 1024; j += nw) {
            const uint32_t off = 1024u * j + 16u * lane;
            if (off < nbytes) lds_dma16(src + off, l0 + 1024u * j);
        }
    } else if ((a & 3u) == 0) {
        const uint32_t *s = (const uint32_t *)src;
        uint32_t *d = (uint32_t *)dst;
        for (uint32_t i = tid; i < nbytes / 4; i += nthr) d[i] = s[i];
    } else {
        const uint16_t *s = (const uint16_t *)src;
        uint16_t *d = (uint16_t *)dst;
        for (uint32_t i = tid; i < nbytes / 2; i += nthr) d[i] = s[i];
    }
}

// Row totals by a DPP tree: valid in the row's last lane (gi == TPR - 1).
template <int TPR, int NT>
__device__ inline void reduce_acc(float (&acc)[NT]) {
#pragma unroll
    for (int t = 0; t < NT; t++) acc[t] = q4mi_rsum<TPR>(acc[t]);
}

// Layout of lanes over a row of G = K/32 groups: TPR lanes (a power of two,
// the DPP row-sum tree) with GPT groups each, TPR * GPT = G.  Besides the
// power-of-two rows, the reference model's hidden 2560 (80 groups: 16 x 5)
// and expert intermediate 640 (20 groups: 4 x 5).
struct RowLayout {
    int tpr, gpt;
};
inline RowLayout layout_for(uint32_t G) {
    if (G == 8 || G == 16 || G == 32 || G == 64) return {(int)G, 1};
    if (G == 128) return {64, 2};
    if (G == 256) return {64, 4};
    if (G == 80) return {16, 5};
    if (G == 20) return {4, 5};
    return {0, 0};
}

// Rows per block so that a tile is about `target` bytes, a multiple of the
// rows one pass covers (256 / tpr).
inline uint32_t tile_rows(uint32_t rb, int tpr, uint32_t target, uint32_t nthr = 256) {
    const uint32_t rpp = nthr / (uint32_t)tpr;
    uint32_t r = target / rb;
    r = r / rpp * rpp;
    if (r < rpp) r = rpp;
    return r;
}

}  // namespace q4mi
