// Expert-sorted prefill MMQ on MFMA (gfx950).
//
// Routed rows are packed per expert (ragged bounds[e]..bounds[e+1]).  For
// each (expert, 128-row token tile, 128-row weight tile) a 256-thread block
// walks K one IQ3_S superblock (256 values) at a time:
//   * weights: the raw blocks are copied to LDS; each lane decodes its MFMA
//     operands in registers: IQ3_S -> exact integers w*(2s+1) (|v| <= 465)
//     as fp16; Q8_0 -> its int8 values as fp16;
//   * activations: q8 codes (exact fp16 copies made by the quantizer) and
//     their fp32 group scales;
//   * per 32-value group: two v_mfma_f32_32x32x16_f16 produce the exact
//     int32 group sums S (every partial sum is an integer below 2^24, so the
//     fp32 accumulation is exact), then inner += S * d_x(token, group);
//     per superblock acc += inner * d_w(row).
// Folding the sub-block multiplier into the operand leaves one FMA per
// output element per group.  The int8-MFMA alternative needs a convert, a
// scale product and an FMA per element per group, which on this chip makes
// the VALU, not the matrix core, the limit (3 wave64 VALU ops, 12 cycles per
// element-group, against 32 cycles of i8 MFMA per 32x32x32 tile: about 3x).
//
// C ABI: the reference's q4_mmq_* wrapper contract (src/q4.h:1150-1175,
// src/q4_mmq.cu:341-438): q4_mmq_q8_bytes, q4_mmq_quantize,
// q4_mmq_mul_id (expert e owns rows [bounds[e], bounds[e+1]), weights at
// w + e*expert_stride_bytes, dst rows in xq order), q4_mmq_swiglu.
#include <stdlib.h>

#include <algorithm>

#include "formats.h"
#include "q4mi_common.h"
#include "q4mi_internal.h"

typedef _Float16 half8_t __attribute__((ext_vector_type(8)));
typedef _Float16 half2_t __attribute__((ext_vector_type(2)));
typedef float f32x16_t __attribute__((ext_vector_type(16)));

namespace q4mi {

constexpr int MT = 128;         // largest tile height (token rows); a call may use 64 or 32

// ------------------------------------------------------------ quantizer
// MMQ activation buffer layout: codes as fp16 [rows][cols], then fp32 group
// scales [rows][cols/32].  The codes are the CPU expert path's int8 codes,
// exactly (an fp16 holds every integer in -128..127).
__global__ __launch_bounds__(256) void mmq_quant_k(const float *__restrict__ x,
                                                   const int32_t *__restrict__ ids,
                                                   uint64_t rows, uint32_t cols,
                                                   _Float16 *__restrict__ q,
                                                   float *__restrict__ d) {
    const uint32_t gpr = cols / 32;
    const uint64_t gid = (uint64_t)blockIdx.x * 32 + (threadIdx.x >> 3);
    if (gid >= rows * gpr) return;
    const uint64_t r = gid / gpr;
    const uint32_t g = (uint32_t)(gid % gpr);
    const uint32_t sub = threadIdx.x & 7u;
    const uint64_t src = ids ? (uint64_t)ids[r] : r;
    const float4 v = *(const float4 *)(x + src * cols + 32u * g + 4u * sub);
    float dd;
    int bs;
    const uint32_t p = q4mi_quant_team8(v, &dd, &bs);
    _Float16 h[4];
#pragma unroll
    for (int j = 0; j < 4; j++) h[j] = (_Float16)(float)(int8_t)(p >> (8 * j));
    *(uint2 *)(q + r * cols + 32u * g + 4u * sub) = *(const uint2 *)h;
    if (sub == 0) d[gid] = dd;
}

// --------------------------------------------------------------- tiles
// One tile list, tiles[i] = (expert, first row), *count = its length.  Every
// whole 128-row tile of an expert is listed; its remaining rows (if any)
// form one more tile that the kernel runs with just enough 32-row
// sub-tiles, so a tail of a few rows costs a 32-row tile, not a 128-row
// one.  The list is ordered by tile size, largest first (longest work is
// scheduled first).
//
// One block, thread e = expert e.  The four classes' tile counts of an
// expert are packed into one 64-bit word (16 bits per class, class 3 = the
// 128-row class in the top field), so a single exclusive scan over the
// experts gives every class's offsets at once: a wave scan, then one step
// across the 16 waves.  Field sums stay below 2^16 (at most
// total_rows/mt + n_exp <= 65535 tiles, checked by the caller).  mt (128,
// 64 or 32) is the tile height: whole tiles are mt rows (class mt/32 - 1).
__global__ __launch_bounds__(1024) void mmq_tiles_k(const int32_t *__restrict__ bounds,
                                                   uint32_t n_exp, uint32_t mt,
                                                   int4 *__restrict__ tiles,
                                                   uint32_t *__restrict__ count, uint32_t cap) {
    __shared__ uint64_t wsum[16];
    const uint32_t e = threadIdx.x, lane = e & 63u, w = e >> 6;
    uint32_t n = 0;
    int32_t b0 = 0;
    if (e < n_exp) {
        b0 = bounds[e];
        const int32_t v = bounds[e + 1] - b0;
        n = v > 0 ? (uint32_t)v : 0u;
    }
    const uint32_t nfull = n / mt, tail = n % mt, fcls = mt / 32 - 1;
    const uint32_t tcls = tail ? (tail + 31) / 32 - 1 : 4u;   // 4 = no tail tile
    auto field = [](uint32_t c) { return 16u * c; };
    uint64_t mine = (uint64_t)nfull << field(fcls);
    if (tcls < 4) mine += 1ull << field(tcls);
    // every field's sums stay below 2^16, so the two 32-bit halves scan
    // independently (no carry crosses bit 32)
    const uint64_t incl = (uint64_t)q4mi_wave_incl_scan((uint32_t)mine) |
                          ((uint64_t)q4mi_wave_incl_scan((uint32_t)(mine >> 32)) << 32);
    if (lane == 63) wsum[w] = incl;
    __syncthreads();
    uint64_t before = 0, total = 0;
#pragma unroll
    for (uint32_t k = 0; k < 16; k++) {
        const uint64_t v = wsum[k];
        if (k < w) before += v;
        total += v;
    }
    const uint64_t excl = before + incl - mine;
    auto get = [&](uint64_t v, uint32_t c) { return (uint32_t)(v >> field(c)) & 0xFFFFu; };
    // classes laid out largest first: 3, 2, 1, 0
    uint32_t cbase[4];
    cbase[3] = 0;
    cbase[2] = get(total, 3);
    cbase[1] = cbase[2] + get(total, 2);
    cbase[0] = cbase[1] + get(total, 1);
    const uint32_t all = cbase[0] + get(total, 0);
    uint32_t start = cbase[fcls] + get(excl, fcls);
    uint32_t k = 0;
    // entry: expert, first packed row, rows
    for (; k < nfull && start + k < cap; k++)
        tiles[start + k] = make_int4((int)e, b0 + (int)(k * mt), (int)mt, 0);
    if (tcls < 4) {
        const uint32_t at = tcls == fcls ? start + nfull : cbase[tcls] + get(excl, tcls);
        if (at < cap) tiles[at] = make_int4((int)e, b0 + (int)(nfull * mt), (int)tail, 0);
    }
    if (e == 0) *count = min(all, cap);
}

// --------------------------------------------------------------- kernel
// Block = 256 threads (4 waves), tile = 128 weight rows x 128 token rows.
// Wave w owns weight rows [32w, 32w+32) of the tile and every token of it
// (four 32-token sub-tiles, skipped when empty).  Each K superblock:
//   1. the 128 rows' raw block bytes are copied to LDS with dword loads;
//   2. per 64-value stage the 128 token rows' fp16 codes (and group scales)
//      are copied to LDS, double-buffered;
//   3. per 32-value group each lane decodes the 16 weight values its MFMA A
//      operand needs straight from the raw bytes (lane half kh takes values
//      8kh..8kh+7 and 16+8kh..+7), then two 32x32x16 MFMAs per token sub-tile.
// Fused gate/up mode: tile rows 0..63 are gate rows n0..n0+63 and 64..127
// the matching up rows F+n0..; each gate/up wave pair (w, w+2) exchanges
// half of its accumulators through LDS, and each wave forms h = silu(g)*u
// and its q8 codes for half of the token sub-tiles (the 32 h columns of a
// q8 group are in the lane and its partner lane l^32).
constexpr int MMQ_NB = 128;      // weight rows per block
constexpr int MMQ_MB = 128;      // token rows per block

// Raw superblock slots in LDS.  A row's slot holds the dwords covering its
// superblock, which starts 0 or 2 bytes into a dword (rows are 4-byte
// multiples, so the offset is the same for every row of a tile).
//   IQ3_S: 28 data dwords + 1 pad = 29 per row.  29 is odd, so the 32 rows
//          one wave decodes at a common byte offset fall on 32 banks, and
//          one 58-lane copy fills two whole rows.
//   Q8_0:  the dwords rounded to an even count, copied as one linear run.
//   IQ4_NL, Q2_0, IQ2_S: like Q8_0 (8 x 18, 4 x 18 and 82 bytes per 256).
template <uint32_t TY>
struct RawSpec {
    static constexpr uint32_t SB = TY == Q4MI_T_IQ3_S    ? 110u
                                   : TY == Q4MI_T_Q8_0   ? 8u * 34u
                                   : TY == Q4MI_T_IQ4_NL ? 8u * 18u
                                   : TY == Q4MI_T_Q2_0   ? 4u * 18u
                                                         : 82u;   // IQ2_S
    static constexpr uint32_t SS = TY == Q4MI_T_IQ3_S ? 29u * 4u
                                                      : ((SB + 2u + 3u) / 4u + 1u) / 2u * 8u;
};

// Per-format facts of the MMQ operand decode:
//   kSuper  the block scale is per superblock (IQ3_S, IQ2_S: the exact group
//           sums times d_x accumulate in `inner`, times d_w once per
//           superblock), else per 32 or 64 values (d_w folded per group);
//   kTab    entries of the LDS decode table g16 (IQ3_S: codebook as fp16
//           magnitudes; IQ2_S: codebook as fp16 magnitudes, two entries of
//           four per grid point; IQ4_NL: byte -> fp16 values of its two
//           nibbles; Q2_0: byte -> its four fp16 values c - 1).
template <uint32_t TY>
struct MmqFmt {
    static constexpr bool kSuper = TY == Q4MI_T_IQ3_S || TY == Q4MI_T_IQ2_S;
    static constexpr uint32_t kTab = TY == Q4MI_T_IQ3_S    ? 512u
                                     : TY == Q4MI_T_IQ2_S  ? 2048u
                                     : TY == Q4MI_T_IQ4_NL ? 256u
                                     : TY == Q4MI_T_Q2_0   ? 256u
                                                           : 1u;
    // byte offset of group j's scale inside the superblock, and its factor
    __device__ static inline uint32_t doff(uint32_t j) {
        return TY == Q4MI_T_Q8_0 ? 34u * j : TY == Q4MI_T_IQ4_NL ? 18u * j
             : TY == Q4MI_T_Q2_0 ? 18u * (j >> 1) : 0u;
    }
    static constexpr float kDScale = TY == Q4MI_T_IQ2_S ? 0.125f : 1.f;
};

// Double-buffered stages of 64 K values (two q8 groups).  Activation rows
// are 128 B (64 fp16 codes) with their eight 16-byte chunks XOR-swizzled by
// the row index (chunk c of row r sits at c ^ (r & 7)), so one 1 KB copy
// fills 8 whole rows and the MFMA operand reads of 32 rows hit distinct
// banks.  Raw weight bytes are double-buffered per superblock.
template <uint32_t TY>
struct MmqLds {
    _Float16 act[2][MMQ_MB][64];            // 32 KB; reused for the fused hand-off
    float dx[2][MMQ_MB][2];                 // group scales of each staged pair
    uint8_t raw[2][MMQ_NB][RawSpec<TY>::SS];  // raw weight bytes per superblock
    uint2 g16[MmqFmt<TY>::kTab];            // decode table (MmqFmt)
    uint2 sm16[16];                         // sign nibble -> fp16 sign masks
};

struct MmqArgs {
    const uint8_t *w;
    const uint8_t *wx;      // optional: base of expert ex (else w + ex * estride)
    const uint8_t *wx_up;   // fused mode: expert ex's up rows (with wx)
    uint64_t up_off;        // fused mode: expert e's up rows at w + e*estride + up_off
    uint32_t ex;
    uint64_t estride;       // bytes between experts
    uint32_t rb;            // bytes per weight row
    uint32_t K;             // w_cols
    uint32_t n_ff;          // fused mode: gate rows = up rows = n_ff
    const _Float16 *xq;     // [xrows][K] fp16 codes
    const float *xd;        // [xrows][K/32]
    const int32_t *act_row; // optional: activation row of packed row p
    const int32_t *bounds;  // [n_exp+1]
    const int4 *tiles;      // (expert, first packed row, rows, -)
    const uint32_t *ntiles;
    uint32_t mt;            // tile height (token rows): 128, 64 or 32
    float *dst;             // plain mode: [rows][ld]
    uint64_t ld;
    _Float16 *hq;           // fused mode: [rows][n_ff] fp16 codes of h
    float *hd;              // fused mode: [rows][n_ff/32]
    uint32_t wide;          // one- and two-sub-tile tiles use 256 / 128-value stages
    uint32_t ko;            // measurement build: knockout bits (timing studies only)
    uint32_t xcd;           // XCD-grouped block order (grid rows a multiple of 8)
};

// Knockouts of a timing-study build (-DQ4MI_MMQ_KO=bits):
// parts of the tile loop switched off to time what each costs.  Results are
// garbage with any bit set; the product library compiles them out.
#ifdef Q4MI_MMQ_KO
#define MMQ_KO(a, bit) (((Q4MI_MMQ_KO) >> (bit)) & 1u)
#else
#define MMQ_KO(a, bit) false
#endif

__device__ inline uint32_t lds_u16(const uint8_t *p) { return *(const uint16_t *)p; }

typedef _Float16 half4_t __attribute__((ext_vector_type(4)));

// Lane's A operands of group j for one weight row: A0 = values 8kh..8kh+7,
// A1 = values 16+8kh..16+8kh+7 (IQ3_S entries 2kh, 2kh+1 / 4+2kh, 5+2kh).
// XG mode (fp16 activations, the reference's q4_xg): the operand is the
// dequantized weight times kXgWs in fp16 -- the exact integer times the
// block scale kXgWs * d_w (* (2s+1)) rounded to fp16 -- and the MFMA
// accumulates the whole K; the epilogue divides kXgWs out.
constexpr float kXgWs = 256.f;

template <uint32_t TY, bool XG = false>
__device__ inline void decode_a(const MmqLds<TY> &L, const uint8_t *R, uint32_t j,
                                uint32_t kh, half8_t &A0, half8_t &A1) {
    if constexpr (TY == Q4MI_T_IQ3_S) {
#if defined(Q4MI_MMQ_KO) && ((Q4MI_MMQ_KO >> 9) & 1)
        const uint32_t lv = (uint32_t)(uintptr_t)R;
        const uint32_t qa = (lv * 7u + j) & 0xffffu, qb = (lv * 13u + j) & 0xffffu;
        const uint32_t qh = (lv >> 3) & 0xffu, sa = (lv >> 5) & 0xffu, sb = (lv >> 7) & 0xffu;
        const uint32_t sc = (lv >> 2) & 0xffu;
#else
        const uint32_t qa = lds_u16(R + 2 + 8 * j + 2 * kh);       // qs entries 2kh, 2kh+1
        const uint32_t qb = lds_u16(R + 2 + 8 * j + 4 + 2 * kh);   // 4+2kh, 5+2kh
        const uint32_t qh = R[66 + j];
        const uint32_t sa = R[74 + 4 * j + kh];                    // sign nibbles 2kh, 2kh+1
        const uint32_t sb = R[74 + 4 * j + 2 + kh];                // 4+2kh, 5+2kh
        const uint32_t sc = R[106 + (j >> 1)];
#endif
        float m = (float)(2u * ((j & 1u) ? (sc >> 4) : (sc & 15u)) + 1u);
        if constexpr (XG) m = q4mi_h2f(lds_u16(R)) * m * kXgWs;
        const half2_t mm = {(_Float16)m, (_Float16)m};
        uint32_t o[8];
#pragma unroll
        for (int q = 0; q < 4; q++) {
            const uint32_t e = (q < 2 ? 2 * kh : 4 + 2 * kh) + (q & 1);  // entry index
            const uint32_t qs8 = ((q < 2 ? qa : qb) >> (8 * (q & 1))) & 0xffu;
            const uint32_t idx = qs8 | (((qh >> e) & 1u) << 8);
            const uint32_t nib = ((q < 2 ? sa : sb) >> (4 * (q & 1))) & 15u;
#if defined(Q4MI_MMQ_KO) && ((Q4MI_MMQ_KO >> 8) & 1)
            const uint2 g = make_uint2(idx * 0x00010001u, idx * 0x00030001u);
            const uint2 s = make_uint2(nib << 15, nib << 31);
#else
            const uint2 g = L.g16[idx];
            const uint2 s = L.sm16[nib];
#endif
            half2_t a = __builtin_bit_cast(half2_t, g.x ^ s.x) * mm;
            half2_t b = __builtin_bit_cast(half2_t, g.y ^ s.y) * mm;
            o[2 * q] = __builtin_bit_cast(uint32_t, a);
            o[2 * q + 1] = __builtin_bit_cast(uint32_t, b);
        }
        A0 = __builtin_bit_cast(half8_t, make_uint4(o[0], o[1], o[2], o[3]));
        A1 = __builtin_bit_cast(half8_t, make_uint4(o[4], o[5], o[6], o[7]));
    } else if constexpr (TY == Q4MI_T_IQ4_NL) {
        // block j: qs at 18j+2; values 8kh+k (low nibble of qs[8kh+k], in A0)
        // and 16+8kh+k (its high nibble, in A1); the table gives both as fp16
        const uint8_t *qs = R + 18 * j + 2 + 8 * kh;
        uint32_t t[8];
#pragma unroll
        for (int k = 0; k < 8; k += 2) {
            const uint32_t b2 = lds_u16(qs + k);
            t[k] = L.g16[b2 & 0xffu].x;
            t[k + 1] = L.g16[b2 >> 8].x;
        }
        uint32_t o0[4], o1[4];
#pragma unroll
        for (int k = 0; k < 4; k++) {
            o0[k] = __builtin_amdgcn_perm(t[2 * k + 1], t[2 * k], 0x05040100u);
            o1[k] = __builtin_amdgcn_perm(t[2 * k + 1], t[2 * k], 0x07060302u);
        }
        A0 = __builtin_bit_cast(half8_t, make_uint4(o0[0], o0[1], o0[2], o0[3]));
        A1 = __builtin_bit_cast(half8_t, make_uint4(o1[0], o1[1], o1[2], o1[3]));
        if constexpr (XG) {   // times fp16(d * kXgWs), rounded to fp16
            const _Float16 ws = (_Float16)(q4mi_h2f(lds_u16(R + 18 * j)) * kXgWs);
            A0 = A0 * ws;
            A1 = A1 * ws;
        }
    } else if constexpr (TY == Q4MI_T_Q2_0) {
        // group j = half j&1 of block j>>1; code byte b holds values 4b..4b+3:
        // A0 = bytes 2kh, 2kh+1; A1 = bytes 4+2kh, 5+2kh
        const uint8_t *cs = R + 18 * (j >> 1) + 2 + 8 * (j & 1u);
        const uint32_t a = lds_u16(cs + 2 * kh), b = lds_u16(cs + 4 + 2 * kh);
        const uint2 t0 = L.g16[a & 0xffu], t1 = L.g16[a >> 8];
        const uint2 t2 = L.g16[b & 0xffu], t3 = L.g16[b >> 8];
        A0 = __builtin_bit_cast(half8_t, make_uint4(t0.x, t0.y, t1.x, t1.y));
        A1 = __builtin_bit_cast(half8_t, make_uint4(t2.x, t2.y, t3.x, t3.y));
        if constexpr (XG) {   // times fp16(d * kXgWs), rounded to fp16
            const _Float16 ws = (_Float16)(q4mi_h2f(lds_u16(R + 18 * (j >> 1))) * kXgWs);
            A0 = A0 * ws;
            A1 = A1 * ws;
        }
    } else if constexpr (TY == Q4MI_T_IQ2_S) {
        // group j: grid points l = 0..3 (8 values each), index qs[4j+l] with
        // 2 bits of qh[j]; A0 = point kh (multiplier of values 0-15), A1 =
        // point 2+kh (values 16-31).  The table holds each point's eight
        // magnitudes as fp16; the sign masks come from the sign byte.
        const uint32_t qs4 = lds_u16(R + 2 + 4 * j) | (lds_u16(R + 4 + 4 * j) << 16);
        const uint32_t sg4 = lds_u16(R + 34 + 4 * j) | (lds_u16(R + 36 + 4 * j) << 16);
        const uint32_t qh = R[66 + j], sc = R[74 + j];
        auto point = [&](uint32_t l, uint32_t mult, half8_t &A) __attribute__((always_inline)) {
            const uint32_t idx = ((qs4 >> (8 * l)) & 0xffu) | ((qh << (8 - 2 * l)) & 0x300u);
            const uint2 g0 = L.g16[2 * idx], g1 = L.g16[2 * idx + 1];
            const uint32_t sg = (sg4 >> (8 * l)) & 0xffu;
            const uint2 m0 = L.sm16[sg & 15u], m1 = L.sm16[sg >> 4];
            // XG: the multiplier becomes fp16(d / 8 * (2s+1) * kXgWs)
            const float mf = XG ? q4mi_h2f(lds_u16(R)) * 0.125f * (float)mult * kXgWs
                                : (float)mult;
            const half2_t mm = {(_Float16)mf, (_Float16)mf};
            const uint32_t o0 = __builtin_bit_cast(uint32_t, __builtin_bit_cast(half2_t, g0.x ^ m0.x) * mm);
            const uint32_t o1 = __builtin_bit_cast(uint32_t, __builtin_bit_cast(half2_t, g0.y ^ m0.y) * mm);
            const uint32_t o2 = __builtin_bit_cast(uint32_t, __builtin_bit_cast(half2_t, g1.x ^ m1.x) * mm);
            const uint32_t o3 = __builtin_bit_cast(uint32_t, __builtin_bit_cast(half2_t, g1.y ^ m1.y) * mm);
            A = __builtin_bit_cast(half8_t, make_uint4(o0, o1, o2, o3));
        };
        point(kh, 2u * (sc & 15u) + 1u, A0);
        point(2 + kh, 2u * (sc >> 4) + 1u, A1);
    } else {
        // Q8_0 block j of the superblock: qs at 34j+2; values 8kh.. and 16+8kh..
        const uint8_t *qs = R + 34 * j + 2;
        uint32_t v[4];
#pragma unroll
        for (int q = 0; q < 4; q++) {
            const uint32_t off = (q < 2 ? 8 * kh : 16 + 8 * kh) + 4 * (q & 1);
            v[q] = lds_u16(qs + off) | (lds_u16(qs + off + 2) << 16);
        }
        uint32_t o[8];
        // XG: the block's fp16 d times kXgWs, then the product rounded to fp16
        const _Float16 ws = XG ? (_Float16)(q4mi_h2f(lds_u16(R + 34 * j)) * kXgWs) : (_Float16)1;
#pragma unroll
        for (int q = 0; q < 4; q++) {
#pragma unroll
            for (int b = 0; b < 2; b++) {
                _Float16 lo = (_Float16)(float)(int8_t)(v[q] >> (16 * b));
                _Float16 hi = (_Float16)(float)(int8_t)(v[q] >> (16 * b + 8));
                if constexpr (XG) {
                    lo = lo * ws;
                    hi = hi * ws;
                }
                o[2 * q + b] = (uint32_t)__builtin_bit_cast(uint16_t, lo) |
                               ((uint32_t)__builtin_bit_cast(uint16_t, hi) << 16);
            }
        }
        A0 = __builtin_bit_cast(half8_t, make_uint4(o[0], o[1], o[2], o[3]));
        A1 = __builtin_bit_cast(half8_t, make_uint4(o[4], o[5], o[6], o[7]));
    }
}

// gfx950 global -> LDS copy of one wave (lane i's UNIT bytes land at LDS
// address m0 + i*UNIT), as inline asm: the compiler does not track it, so
// its conservative wait before every later LDS read (it would wait for all
// copies in flight) is not emitted; this kernel waits with exact counts.
template <uint32_t UNIT>
__device__ inline void mmq_copy(const void *g, uint32_t lds_addr) {
    lds_addr = __builtin_amdgcn_readfirstlane(lds_addr);
    if constexpr (UNIT == 16)
        asm volatile("s_mov_b32 m0, %1\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %0, off"
                     :: "v"(g), "s"(lds_addr) : "memory", "m0");
    else
        asm volatile("s_mov_b32 m0, %1\n\ts_nop 0\n\tglobal_load_lds_dword %0, off"
                     :: "v"(g), "s"(lds_addr) : "memory", "m0");
}
// LDS address of a generic pointer into LDS: the low half of a flat
// address in the LDS aperture is the LDS offset (an address-space cast would
// add a null check to every copy)
__device__ inline uint32_t mmq_lds(const void *p) { return (uint32_t)(uintptr_t)p; }
// wait until at most N of this wave's copies are in flight
template <uint32_t N>
__device__ inline void mmq_wait() {
    static_assert(N <= 63, "vmcnt holds 6 bits");
    asm volatile("s_waitcnt vmcnt(%0)" ::"n"(N) : "memory");
}
// workgroup barrier that leaves this kernel's copies in flight
__device__ inline void mmq_bar() { asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory"); }
// barrier that also leaves this wave's LDS reads in flight (the caller knows
// none of them reads a buffer another wave refills after it)
__device__ inline void mmq_bar_rd() { asm volatile("s_barrier" ::: "memory"); }

// One (expert, weight block, token tile) of NSUB 32-row token sub-tiles.
// KS = K values per stage: 64 for three or four token sub-tiles; one- and
// two-sub-tile tiles take 256 / 128 (the same 16 KB of activation rows per
// buffer), so their short per-stage compute waits for a memory round trip 4x
// / 2x less often.
template <uint32_t TY, bool FUSED, int NSUB, bool XG = false, uint32_t KS = 64>
__device__ __attribute__((always_inline)) inline void mmq_tile(const MmqArgs a, uint8_t *smem,
                                                               const int4 tinfo, uint32_t cblk) {
    MmqLds<TY> &L = *(MmqLds<TY> *)smem;
    constexpr uint32_t SB = RawSpec<TY>::SB;
    constexpr uint32_t SSD = RawSpec<TY>::SS / 4;             // raw slot dwords
    constexpr bool kIq = TY == Q4MI_T_IQ3_S;
    // dword copies per superblock: IQ3_S two rows per copy, else linear
    constexpr uint32_t RAW_OPS = kIq ? MMQ_NB / 2 : (MMQ_NB * SSD + 63) / 64;
    constexpr uint32_t RAW_PER_WAVE = (RAW_OPS + 3) / 4;
    constexpr uint32_t GPS = KS / 32;                         // q8 groups per stage
    constexpr uint32_t SPS = 256 / KS;                        // stages per superblock
    constexpr uint32_t RPO = 512 / KS;                        // activation rows per 1 KB copy
    constexpr uint32_t CPR = KS / 8;                          // 16-byte chunks per row
    constexpr uint32_t AOPS = NSUB * KS / 64;                 // activation copies per wave
    static_assert(32 * NSUB * KS <= MMQ_MB * 64 && 32 * NSUB * GPS <= 2 * MMQ_MB, "stage fits");
    // copies per stage per wave: the activation rows and (q8 mode) their scales
    constexpr uint32_t ST_OPS = AOPS + (XG ? 0 : 1);
    _Float16 *const actb = &L.act[0][0][0];                   // [2][32 NSUB][KS] per buffer
    float *const dxb = &L.dx[0][0][0];                        // [2][32 NSUB][GPS]
    constexpr uint32_t kActBuf = MMQ_MB * 64, kDxBuf = MMQ_MB * 2;
    const uint32_t tid = threadIdx.x, lane = tid & 63u, kh = lane >> 5;
    const uint32_t wv = __builtin_amdgcn_readfirstlane(tid >> 6);
    const uint32_t e = (uint32_t)tinfo.x;
    const int32_t rbase = tinfo.y;
    const uint32_t mrows = min((uint32_t)tinfo.z, 32u * NSUB);
    const bool isx = a.wx && e == a.ex;
    const uint8_t *We = isx ? a.wx : a.w + (uint64_t)e * a.estride;
    // fused mode: the expert's up rows (after its gate rows in a packed
    // expert; another tensor in the GGUF layout)
    const uint8_t *Wu = isx ? a.wx_up : We + a.up_off;
    // weight row (within the gate or up matrix) of tile row r
    const uint32_t nblk = FUSED ? cblk * 64 : cblk * MMQ_NB;
    auto wsrc = [&](uint32_t r, uint32_t sbi) -> const uint8_t * {
        const uint8_t *m = (FUSED && r >= 64) ? Wu : We;
        const uint32_t wr = (FUSED && r >= 64) ? nblk + (r - 64) : nblk + r;
        return m + (uint64_t)wr * a.rb + (uint64_t)sbi * SB;
    };

    // the codebook entries this thread converts (loaded now, stored into
    // LDS once the first copies are in flight)
    uint32_t code[2] = {0u, 0u};
    if (TY == Q4MI_T_IQ3_S) {
        code[0] = q4mi_iq3s_code_dev[tid];
        code[1] = q4mi_iq3s_code_dev[tid + 256];
    }
    // copies of superblock sbi's raw weight bytes into buffer sbi & 1
    // IQ3_S copy lanes: lane < 29 -> dword `lane` of the first row, 29..57 ->
    // dword lane-29 of the second row (the pad dword re-reads dword 27)
    const uint32_t rsel = lane >= 29u ? 1u : 0u;
    const uint32_t lofs = rsel * a.rb + 4u * min(lane - 29u * rsel, 27u);
    auto issue_raw = [&](uint32_t sbi) __attribute__((always_inline)) {
        const uint32_t buf = sbi & 1u;
        uint8_t *base = &L.raw[buf][0][0];
        if constexpr (kIq) {
            // rows 2j, 2j+1 are adjacent in memory (gate/up halves split at
            // an even row): one wave-uniform base per copy
            const uint32_t roff = (uint32_t)((uintptr_t)wsrc(0, sbi) & 3u);
#pragma unroll
            for (uint32_t m = 0; m < RAW_PER_WAVE; m++) {
                const uint32_t j = wv + 4 * m;
                const uint8_t *rb0 = wsrc(2 * j, sbi) - roff;
                if (lane < 58u) mmq_copy<4>(rb0 + lofs, mmq_lds(base + 2u * j * RawSpec<TY>::SS));
            }
            return;
        }
#pragma unroll
        for (uint32_t m = 0; m < RAW_PER_WAVE; m++) {
            const uint32_t j = wv + 4 * m;
            uint32_t d = 64 * j + lane;                // slot dword, row-major
            // opaque: recompute the source address per copy instead of
            // keeping 14 hoisted row pointers live across the K loop
            asm volatile("" : "+v"(d));
            const uint32_t r = min(d / SSD, (uint32_t)MMQ_NB - 1u), dw = d % SSD;
            const uint8_t *rs = wsrc(r, sbi);
            const uint32_t nd = ((uint32_t)((uintptr_t)rs & 3u) + SB + 3u) / 4u;
            const uint32_t *s32 = (const uint32_t *)((uintptr_t)rs & ~(uintptr_t)3);
            // dwords past the slice re-read its first dword (stay in bounds)
            const uint32_t *src = (j < RAW_OPS && dw < nd) ? s32 + dw : s32;
            mmq_copy<4>(src, mmq_lds(base + 256u * j));
        }
    };

    issue_raw(0);   // needs only the expert: goes out before the activation rows resolve

    // source rows of this lane's copies: activation op m covers tile rows
    // RPO(wv + 4m) .. +RPO-1 (lane / CPR picks the row), the scale op the
    // dwords 64wv .. 64wv+63 of the stage's [rows][GPS] scales (rows past
    // the tile's end copy the last row's bytes: their outputs are never
    // stored, and the copy stays one instruction)
    const _Float16 *arow_src[AOPS];
#pragma unroll
    for (uint32_t m = 0; m < AOPS; m++) {
        const uint32_t r = RPO * (wv + 4 * m) + lane / CPR;
        const int32_t p = rbase + (int32_t)min(r, mrows - 1);
        const int64_t xr = a.act_row ? a.act_row[p] : p;
        arow_src[m] = a.xq + (uint64_t)xr * a.K;
    }
    const float *drow_src = nullptr;
    if constexpr (!XG) {
        const uint32_t r = (64 * wv + lane) / GPS;
        const int32_t p = rbase + (int32_t)min(r, mrows - 1);
        const int64_t xr = a.act_row ? a.act_row[p] : p;
        drow_src = a.xd + (uint64_t)xr * (a.K / 32) + (64 * wv + lane) % GPS;
    }
    const uint32_t nsb = a.K / 256;
    const uint32_t nst = SPS * nsb;                   // KS-value stages

    // copies of stage s (activation codes + scales) into buffer s & 1
    auto issue_stage = [&](uint32_t s) __attribute__((always_inline)) {
        const uint32_t buf = s & 1u;
#pragma unroll
        for (uint32_t m = 0; m < AOPS; m++) {
            const uint32_t j = wv + 4 * m;            // RPO rows per op
            const uint32_t r = RPO * j + lane / CPR;
            // logical chunk stored at slot lane % CPR (its low 3 bits
            // swizzled by the row)
            const uint32_t c = (lane % CPR) ^ (r & 7u);
            const _Float16 *src = arow_src[m] + s * KS + c * 8;
            mmq_copy<16>(src, mmq_lds(actb + buf * kActBuf + RPO * j * KS));
        }
        if constexpr (!XG) {
            mmq_copy<4>(drow_src + s * GPS, mmq_lds(dxb + buf * kDxBuf + 64 * wv));
        }
    };
    f32x16_t acc[NSUB], inner[NSUB];
#pragma unroll
    for (int t = 0; t < NSUB; t++) {
        acc[t] = f32x16_t{};
        inner[t] = f32x16_t{};
    }
    const uint32_t arow = 32 * wv + (lane & 31u);    // this lane's weight row in the tile
    // Byte offsets inside a stage buffer of this lane's B operand chunks
    // (token row lane % 32 of sub-tile 0; sub-tile t adds 32 rows, a
    // constant) and of its group scales: loop invariant, so each read is a
    // per-stage base plus an immediate.
    const uint32_t l31 = lane & 31u;
    uint32_t boff[GPS][2];
#pragma unroll
    for (uint32_t gl = 0; gl < GPS; gl++)
#pragma unroll
        for (uint32_t hf = 0; hf < 2; hf++) {
            const uint32_t c = 4 * gl + 2 * hf + kh;             // logical 16-byte chunk
            boff[gl][hf] = 2u * (l31 * KS + 8u * (c ^ (l31 & 7u)));
        }
    const uint32_t dxoff = 4u * l31 * GPS;
    issue_stage(0);
    if constexpr (TY == Q4MI_T_IQ3_S) {   // tables (read after the first barrier pair)
#pragma unroll
        for (int h2 = 0; h2 < 2; h2++) {
            const uint32_t c = code[h2];
            uint32_t h[4];
#pragma unroll
            for (int jj = 0; jj < 4; jj++) {
                const _Float16 f = (_Float16)(float)(2u * ((c >> (3 * jj)) & 7u) + 1u);
                h[jj] = __builtin_bit_cast(uint16_t, f);
            }
            L.g16[tid + 256 * h2] = make_uint2(h[0] | (h[1] << 16), h[2] | (h[3] << 16));
        }
    }
    if constexpr (TY == Q4MI_T_IQ2_S) {   // codebook magnitudes as fp16
        for (uint32_t i = tid; i < 1024; i += 256) {
            const uint32_t c = q4mi_iq2s_code_dev[i];
            uint32_t h[8];
#pragma unroll
            for (int jj = 0; jj < 8; jj++) {
                const uint32_t v = (c >> (2 * jj)) & 3u;
                h[jj] = __builtin_bit_cast(uint16_t, (_Float16)(v == 0 ? 8.f : v == 1 ? 25.f : 43.f));
            }
            L.g16[2 * i] = make_uint2(h[0] | (h[1] << 16), h[2] | (h[3] << 16));
            L.g16[2 * i + 1] = make_uint2(h[4] | (h[5] << 16), h[6] | (h[7] << 16));
        }
    }
    if constexpr (TY == Q4MI_T_IQ4_NL) {   // byte -> fp16 of both nibbles' values
        constexpr int8_t kv[16] = {-127, -104, -83, -65, -49, -35, -22, -10,
                                   1,    13,   25,  38,  53,  69,  89,  113};
        const uint32_t lo = __builtin_bit_cast(uint16_t, (_Float16)(float)kv[tid & 15u]);
        const uint32_t hi = __builtin_bit_cast(uint16_t, (_Float16)(float)kv[tid >> 4]);
        L.g16[tid] = make_uint2(lo | (hi << 16), 0u);
    }
    if constexpr (TY == Q4MI_T_Q2_0) {   // byte -> its four fp16 values c - 1
        uint32_t h[4];
#pragma unroll
        for (int jj = 0; jj < 4; jj++)
            h[jj] = __builtin_bit_cast(uint16_t, (_Float16)(float)((int)((tid >> (2 * jj)) & 3u) - 1));
        L.g16[tid] = make_uint2(h[0] | (h[1] << 16), h[2] | (h[3] << 16));
    }
    if (MmqFmt<TY>::kSuper && tid < 16) {   // sign nibble -> fp16 sign masks
        uint32_t sgn[4];
#pragma unroll
        for (int jj = 0; jj < 4; jj++) sgn[jj] = ((tid >> jj) & 1u) ? 0x8000u : 0u;
        L.sm16[tid] = make_uint2(sgn[0] | (sgn[1] << 16), sgn[2] | (sgn[3] << 16));
    }
    for (uint32_t s = 0; s < nst; s++) {
        const uint32_t sbi = s / SPS, q = s % SPS;
        // the row's raw bytes start at the same offset inside its slot as
        // in memory (the slot begins at the enclosing dword)
        const uint32_t roff = (uint32_t)((uintptr_t)wsrc(0, sbi) & 3u);   // same for every row
        // Weight operands of the stage's two groups.  Past stage 0 they are
        // decoded ahead of the barriers: superblock sbi's raw bytes are in
        // LDS since stage 4 sbi - 3 (stage 0 waits for them below), and
        // their buffer is refilled only after the first barrier of stage
        // 4 sbi + 4.
        half8_t A[GPS][2];
        auto decode = [&]() __attribute__((always_inline)) {
            const uint8_t *R = &L.raw[sbi & 1u][arow][roff];
#pragma unroll
            for (uint32_t gl = 0; gl < GPS; gl++)
                decode_a<TY, XG>(L, R, GPS * q + gl, kh, A[gl][0], A[gl][1]);
        };
        // (one stage per superblock: its raw bytes land only with this
        // stage's wait, so the decode follows the barriers)
        const bool ahead = SPS >= 2 && s != 0;
        if (ahead && !MMQ_KO(a, 2)) decode();
        // every wave is done with stage s-1 (and at a superblock start with
        // superblock sbi-1): their buffers may be refilled.  The reads in
        // flight here are the decode's, of a buffer nobody refills now.
        if (!MMQ_KO(a, 0)) mmq_bar_rd();
        // issue the next copies, then wait for this wave's part of stage s
        // (the copies just issued stay in flight)
        const bool nraw = q == 0 && sbi + 1 < nsb, nstage = s + 1 < nst;
        if (!MMQ_KO(a, 5)) {
            if (nraw && !MMQ_KO(a, 6)) issue_raw(sbi + 1);
            if (nstage && !MMQ_KO(a, 7)) issue_stage(s + 1);
        }
        if (MMQ_KO(a, 1) || MMQ_KO(a, 5)) {
        } else if (nraw && nstage) mmq_wait<RAW_PER_WAVE + ST_OPS>();
        else if (nstage) mmq_wait<ST_OPS>();
        else if (nraw) mmq_wait<RAW_PER_WAVE>();
        else mmq_wait<0>();
        if (!MMQ_KO(a, 0)) mmq_bar();                 // everyone's part is
        const uint32_t buf = s & 1u;
        if (MMQ_KO(a, 2)) {
#pragma unroll
            for (uint32_t gl = 0; gl < GPS; gl++) {
                A[gl][0] = half8_t{} + (_Float16)(float)(lane + gl);
                A[gl][1] = half8_t{} + (_Float16)(float)(lane + 3 * gl);
            }
        } else if (!ahead) decode();
        // The stage's 2*NSUB products n = (group gl, token sub-tile t): an
        // exact-integer MFMA pair, then one scale FMA per output.  Product
        // n+1's pair is issued before product n's FMAs, so the FMAs never
        // wait on the pair right before them.
        const uint8_t *actc8 = (const uint8_t *)(actb + buf * kActBuf);
        const uint8_t *dxc8 = (const uint8_t *)(dxb + buf * kDxBuf) + dxoff;
        auto prod = [&](int n, float &dxo) __attribute__((always_inline)) {
            const int gl = n / NSUB, t = n % NSUB;
            half8_t B0, B1;
            if (MMQ_KO(a, 3)) {
                const uint32_t tok = 32 * t + l31;
                B0 = half8_t{} + (_Float16)(float)(tok + gl);
                B1 = half8_t{} + (_Float16)(float)(tok + t);
                dxo = (float)n;
            } else {
                B0 = *(const half8_t *)(actc8 + boff[gl][0] + 64u * KS * t);
                B1 = *(const half8_t *)(actc8 + boff[gl][1] + 64u * KS * t);
                dxo = *(const float *)(dxc8 + 4u * (32u * GPS * t + gl));
            }
            f32x16_t r = __builtin_amdgcn_mfma_f32_32x32x16_f16(A[gl][0], B0, f32x16_t{}, 0, 0, 0);
            return __builtin_amdgcn_mfma_f32_32x32x16_f16(A[gl][1], B1, r, 0, 0, 0);
        };
        auto scale = [&](int n, const f32x16_t &sacc, float dxv) __attribute__((always_inline)) {
            const int gl = n / NSUB, t = n % NSUB;
            if constexpr (MmqFmt<TY>::kSuper) {
                if (MMQ_KO(a, 4)) {   // two VALU ops instead of sixteen FMAs
                    inner[t][n & 15] = fmaf(sacc[0] + sacc[15], dxv, inner[t][n & 15]);
                } else {
#pragma unroll
                    for (int i = 0; i < 16; i++) inner[t][i] = fmaf(sacc[i], dxv, inner[t][i]);
                }
            } else {
                const uint32_t j = GPS * q + gl;
#pragma unroll
                for (int i = 0; i < 16; i++) {
                    const uint32_t nr = 32 * wv + 8 * (i / 4) + 4 * kh + (i % 4);
                    const float dw = q4mi_h2f(
                        lds_u16(&L.raw[sbi & 1u][nr][roff] + MmqFmt<TY>::doff(j)));
                    acc[t][i] = fmaf(sacc[i], dxv * dw, acc[t][i]);
                }
            }
        };
        if constexpr (XG) {
            // the MFMA accumulates across K straight into acc
#pragma unroll
            for (int n = 0; n < (int)GPS * NSUB; n++) {
                const int gl = n / NSUB, t = n % NSUB;
                const half8_t B0 = *(const half8_t *)(actc8 + boff[gl][0] + 64u * KS * t);
                const half8_t B1 = *(const half8_t *)(actc8 + boff[gl][1] + 64u * KS * t);
                acc[t] = __builtin_amdgcn_mfma_f32_32x32x16_f16(A[gl][0], B0, acc[t], 0, 0, 0);
                acc[t] = __builtin_amdgcn_mfma_f32_32x32x16_f16(A[gl][1], B1, acc[t], 0, 0, 0);
            }
            continue;
        }
        float dcur;
        f32x16_t cur = prod(0, dcur);
#pragma unroll
        for (int n = 0; n < (int)GPS * NSUB; n++) {
            float dnext = 0.f;
            f32x16_t nxt{};
            if (n + 1 < (int)GPS * NSUB) nxt = prod(n + 1, dnext);
            scale(n, cur, dcur);
            cur = nxt;
            dcur = dnext;
        }
        if (MmqFmt<TY>::kSuper && q == SPS - 1) {   // superblock done: acc += inner * d_w
#pragma unroll
            for (int i = 0; i < 16; i++) {
                const uint32_t n = 32 * wv + 8 * (i / 4) + 4 * kh + (i % 4);
                const float dw = q4mi_h2f(lds_u16(&L.raw[sbi & 1u][n][roff])) *
                                 MmqFmt<TY>::kDScale;
#pragma unroll
                for (int t = 0; t < NSUB; t++) {
                    acc[t][i] = fmaf(inner[t][i], dw, acc[t][i]);
                    inner[t][i] = 0.f;
                }
            }
        }
    }
    if constexpr (XG) {
#pragma unroll
        for (int t = 0; t < NSUB; t++)
#pragma unroll
            for (int i = 0; i < 16; i++) acc[t][i] *= 1.f / kXgWs;   // exact (power of 2)
    }
    if (MMQ_KO(a, 10)) {   // no epilogue: one guarded store keeps the results live
        float z = 0.f;
#pragma unroll
        for (int t = 0; t < NSUB; t++)
#pragma unroll
            for (int i = 0; i < 16; i++) z += acc[t][i];
        float *o = FUSED ? a.hd : a.dst;
        if (z == 1234.5f) o[tid] = z;
        return;
    }
    if (!FUSED) {
        // lane: token column 32t + lane%32, weight rows 32wv + 8b + 4kh + 0..3
#pragma unroll
        for (int t = 0; t < NSUB; t++) {
            const uint32_t p = 32 * t + (lane & 31u);
            if (p < mrows) {
                float *o = a.dst + (uint64_t)(rbase + (int32_t)p) * a.ld + nblk + 32 * wv + 4 * kh;
#pragma unroll
                for (int b = 0; b < 4; b++)
                    *(float4 *)(o + 8 * b) = make_float4(acc[t][4 * b], acc[t][4 * b + 1],
                                                         acc[t][4 * b + 2], acc[t][4 * b + 3]);
            }
        }
        return;
    }
    // fused: wave w < 2 holds gate rows 32w..32w+31 of h's columns, wave
    // w + 2 the matching up rows.  The pair splits the token sub-tiles: the
    // gate wave forms h for t < TS, the up wave for t >= TS, each taking the
    // other half's accumulators through LDS.
    constexpr int TS = (NSUB + 1) / 2;
    __syncthreads();
    // [4 waves][2 slots][16 i][64 lanes] = 32 KB; sub-tile t uses slot
    // t < TS ? t : t - TS (a wave hands over at most two sub-tiles)
    float *ex = (float *)&L.act[0][0][0];
    static_assert(sizeof(MmqLds<TY>::act) >= 4 * 2 * 16 * 64 * sizeof(float), "hand-off space");
    auto slot = [&](int t) { return t < TS ? t : t - TS; };
    const bool gate_w = wv < 2;
#pragma unroll
    for (int t = 0; t < NSUB; t++) {
        if ((t < TS) != gate_w) {           // the half the partner wave finishes
#pragma unroll
            for (int i = 0; i < 16; i++) ex[((wv * 2 + slot(t)) * 16 + i) * 64 + lane] = acc[t][i];
        }
    }
    __syncthreads();
    const uint32_t pw = wv ^ 2u;            // partner wave
    const uint32_t col = 32 * (wv & 1u);    // h columns of this pair: col + 0..31
#pragma unroll
    for (int t = 0; t < NSUB; t++) {
        if ((t < TS) != gate_w) continue;
        const uint32_t p = 32 * t + (lane & 31u);
        float h[16];
        float amax = 0.f;
#pragma unroll
        for (int i = 0; i < 16; i++) {
            const float other = ex[((pw * 2 + slot(t)) * 16 + i) * 64 + lane];
            const float g = gate_w ? acc[t][i] : other;
            const float u = gate_w ? other : acc[t][i];
            // silu(g) * u with the hardware exp2 / reciprocal (a few ulp of
            // h; the q8 scale below stays correctly rounded)
            h[i] = g * u * __builtin_amdgcn_rcpf(1.f + __expf(-g));
            amax = fmaxf(amax, fabsf(h[i]));
        }
        if constexpr (XG) {   // h as fp16 rows [rows][n_ff] (the XG down's input)
            if (p < mrows) {
                const uint64_t prow = (uint64_t)(rbase + (int32_t)p);
                _Float16 *o = a.hq + prow * a.n_ff + nblk + col + 4 * kh;
#pragma unroll
                for (int b = 0; b < 4; b++) {
                    half4_t v;
#pragma unroll
                    for (int c = 0; c < 4; c++) v[c] = (_Float16)h[4 * b + c];
                    *(half4_t *)(o + 8 * b) = v;
                }
            }
            continue;
        }
        // the q8 group = h columns col + 0..31 of token p: this lane has
        // columns 8b + 4kh + 0..3, the partner lane (lane ^ 32) the rest
        amax = fmaxf(amax, __shfl_xor(amax, 32));
        const float d = __fdiv_rn(amax, 127.f);
        const float sc = amax > 0.f ? __fdiv_rn(127.f, amax) : 0.f;
        if (p < mrows) {
            const uint64_t prow = (uint64_t)(rbase + (int32_t)p);
            _Float16 *o = a.hq + prow * a.n_ff + nblk + col + 4 * kh;
#pragma unroll
            for (int b = 0; b < 4; b++) {
                half4_t v;
#pragma unroll
                for (int c = 0; c < 4; c++) v[c] = (_Float16)(float)q4mi_q8_code(h[4 * b + c] * sc);
                *(half4_t *)(o + 8 * b) = v;
            }
            if (kh == 0) a.hd[prow * (a.n_ff / 32) + (nblk + col) / 32] = d;
        }
    }
}

__global__ __launch_bounds__(256) void swiglu_k(const float *__restrict__ gu,
                                                float *__restrict__ h, uint64_t rows,
                                                uint32_t n_ff) {
    const uint64_t i = (uint64_t)blockIdx.x * 256 + threadIdx.x;
    if (i >= rows * n_ff) return;
    const uint64_t r = i / n_ff, k = i % n_ff;
    const float g = gu[r * 2 * n_ff + k], u = gu[r * 2 * n_ff + n_ff + k];
    h[i] = g / (1.f + expf(-g)) * u;
}

// Block order: the hardware hands workgroups to the 8 XCDs round-robin in
// linear order (x fastest), so with the plain (column block, tile) grid every
// XCD's L2 would fetch every tile's activation rows.  With a.xcd set, linear
// block L runs tile 8 (k / gx) + L % 8 and column block k % gx, k = L / 8:
// all column blocks of a tile run on one XCD and share its activation rows in
// that L2 (and consecutive tiles, largest first, go to different XCDs).
struct MmqBlock {
    uint32_t col, tile;
};
__device__ inline MmqBlock mmq_block(const MmqArgs &a) {
    if (!a.xcd) return MmqBlock{blockIdx.x, blockIdx.y};
    const uint32_t gx = gridDim.x;
    const uint32_t L = blockIdx.x + gx * blockIdx.y, k = L >> 3;
    return MmqBlock{k % gx, 8u * (k / gx) + (L & 7u)};
}

template <uint32_t TY, bool FUSED, bool XG = false>
__global__ __launch_bounds__(256, 2) void mmq_k(MmqArgs a) {
    extern __shared__ __align__(16) uint8_t smem[];
    const MmqBlock mb = mmq_block(a);
    const uint32_t ti = mb.tile;
    const int4 tinfo = a.tiles[ti];          // in bounds: the grid is the list's capacity
    if (ti >= *a.ntiles) return;
    const uint32_t col = mb.col;
    const int32_t rows = tinfo.z;
    if (rows <= 0) return;                   // an empty tile (a rejected XG record)
    // block-uniform choice of the (branch-free) sub-tile count
    switch (rows > 96 ? 4 : rows > 64 ? 3 : rows > 32 ? 2 : 1) {
    case 4: mmq_tile<TY, FUSED, 4, XG>(a, smem, tinfo, col); break;
    case 3: mmq_tile<TY, FUSED, 3, XG>(a, smem, tinfo, col); break;
    case 2:
        if (a.wide) mmq_tile<TY, FUSED, 2, XG, 128>(a, smem, tinfo, col);
        else mmq_tile<TY, FUSED, 2, XG>(a, smem, tinfo, col);
        break;
    default:
        if (a.wide) mmq_tile<TY, FUSED, 1, XG, 256>(a, smem, tinfo, col);
        else mmq_tile<TY, FUSED, 1, XG>(a, smem, tinfo, col);
        break;
    }
}

static int4 *g_tiles = nullptr;
static uint32_t *g_ntiles = nullptr;
static uint32_t g_tiles_cap = 0;

// The tile list grows by the library's scratch policy (scratch_grow): never
// inside a stream capture, and a grown-out list stays allocated, so a graph
// captured before the growth keeps its own list.
static bool ensure_tiles(uint32_t n) {
    if (g_tiles_cap >= n) return true;
    if (!g_ntiles && !scratch_grow((void **)&g_ntiles, sizeof(uint32_t), "mmq tile count"))
        return false;
    if (!scratch_grow((void **)&g_tiles, (size_t)n * sizeof(int4), "mmq tile list")) return false;
    g_tiles_cap = n;
    return true;
}

static bool mmq_type(uint32_t ty) {
    return ty == Q4MI_T_IQ3_S || ty == Q4MI_T_Q8_0 || ty == Q4MI_T_IQ4_NL || ty == Q4MI_T_Q2_0 ||
           ty == Q4MI_T_IQ2_S;
}

bool mmq_supported(uint32_t ty, uint64_t w_rows, uint64_t w_cols) {
    if (!mmq_type(ty)) return false;
    // rows must be 4-byte multiples (IQ3_S: an even number of superblocks)
    return w_rows > 0 && w_rows % MMQ_NB == 0 && w_cols > 0 && w_cols % 256 == 0 &&
           w_cols <= 65536 && q4mi_row_bytes(ty, w_cols) % 4 == 0;
}

bool mmq_quant(const float *x, const int32_t *ids, void *xq, uint64_t cols, uint64_t rows) {
    if (!rows) return true;
    _Float16 *q = (_Float16 *)xq;
    float *d = (float *)((uint8_t *)xq + rows * cols * 2);
    const uint64_t blocks = (rows * (cols / 32) + 31) / 32;
    mmq_quant_k<<<dim3((uint32_t)blocks), dim3(256), 0, stream()>>>(x, ids, rows, (uint32_t)cols,
                                                                    q, d);
    return launch_ok("mmq_quant_k");
}

template <uint32_t TY, bool FUSED, bool XG = false>
static bool set_lds_attr() {
    static bool done = false;
    if (done) return true;
    if (hipFuncSetAttribute((const void *)mmq_k<TY, FUSED, XG>,
                            hipFuncAttributeMaxDynamicSharedMemorySize,
                            (int)sizeof(MmqLds<TY>)) != hipSuccess) {
        set_error("mmq: cannot raise the LDS limit to %zu bytes", sizeof(MmqLds<TY>));
        return false;
    }
    done = true;
    return true;
}

template <uint32_t TY, bool FUSED>
static bool mmq_launch(const MmqArgs &a, dim3 grid) {
    if (!set_lds_attr<TY, FUSED>()) return false;
    mmq_k<TY, FUSED><<<grid, dim3(256), sizeof(MmqLds<TY>), stream()>>>(a);
    return launch_ok("mmq_k");
}

template <uint32_t TY, bool FUSED>
static bool xg_launch(const MmqArgs &a, dim3 grid) {
    if (!set_lds_attr<TY, FUSED, true>()) return false;
    mmq_k<TY, FUSED, true><<<grid, dim3(256), sizeof(MmqLds<TY>), stream()>>>(a);
    return launch_ok("mmq_k (xg)");
}

// The reference's XG tile table {first routed row, rows (<= 128), slot,
// expert} -> this kernel's tile entries (slot as the weight index, first
// row, rows) and the tile count, on the stream (graph-capturable).
// A record with rows outside 1..128 (the tile height) or a negative slot or
// first row becomes an empty tile, which the MMQ kernel skips, and sets
// kStXgTile in g_mmq_status (read by q4mi_device_status).
static __device__ uint32_t g_mmq_status;
constexpr uint32_t kStXgTile = 4u;

__global__ void xg_tiles_k(const int32_t *__restrict__ in, uint32_t n, int4 *__restrict__ out,
                           uint32_t *__restrict__ count) {
    const uint32_t i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i < n) {
        const int32_t row = in[4 * i], rows = in[4 * i + 1], slot = in[4 * i + 2];
        const bool ok = rows >= 1 && rows <= MMQ_MB && slot >= 0 && row >= 0;
        if (!ok) atomicOr(&g_mmq_status, kStXgTile);
        out[i] = make_int4(ok ? slot : 0, ok ? row : 0, ok ? rows : 0, 0);
    }
    if (i == 0) *count = n;
}

// The MMQ status word (kStXgTile), read and optionally cleared after the
// stream drained (q4mi_device_status).
uint32_t mmq_status(int clear) {
    uint32_t v = 0;
    if (hipMemcpyFromSymbol(&v, HIP_SYMBOL(g_mmq_status), sizeof v, 0, hipMemcpyDeviceToHost) !=
        hipSuccess)
        return 0x80000000u;
    if (v && clear) {
        const uint32_t z = 0;
        (void)hipMemcpyToSymbol(HIP_SYMBOL(g_mmq_status), &z, sizeof z, 0, hipMemcpyHostToDevice);
    }
    return v;
}

__global__ void xg_cvt_k(const float4 *__restrict__ x, half4_t *__restrict__ y, uint64_t n4) {
    const uint64_t i = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i < n4) {
        const float4 v = x[i];
        y[i] = half4_t{(_Float16)v.x, (_Float16)v.y, (_Float16)v.z, (_Float16)v.w};
    }
}

// xq holds xrows activation rows; act_row (optional) maps packed row p to
// its activation row.  Plain mode writes dst[p][0..w_rows); fused mode
// (w_rows = 2*n_ff, gate rows then up rows) writes the q8 codes of
// h = silu(gate)*up into hq (the q4_mmq_q8_bytes(total_rows, n_ff) layout).
// wx (optional) is the base of the last expert, n_exp - 1, which then need
// not sit at w + (n_exp - 1) * estride (a shared expert kept apart from the
// routed arena).
// Q4MI_MMQ_WIDE=0 keeps 64-value stages for every tile class (A/B timing).
static const bool g_wide = !(getenv("Q4MI_MMQ_WIDE") && getenv("Q4MI_MMQ_WIDE")[0] == '0');
// XCD-grouped block order (Q4MI_MMQ_XCD=0 restores the plain order for A/B timing).
static const bool g_mmq_xcd = !(getenv("Q4MI_MMQ_XCD") && getenv("Q4MI_MMQ_XCD")[0] == '0');

bool mmq_run(const uint8_t *w, uint32_t ty, uint64_t w_rows, uint64_t w_cols, uint64_t estride,
             uint32_t n_exp, const void *xq, uint64_t xrows, const int32_t *act_row,
             const int32_t *bounds, uint64_t total_rows, float *dst, uint64_t ld, void *hq,
             const uint8_t *wx = nullptr, const uint8_t *w_up = nullptr,
             const uint8_t *wx_up = nullptr) {
    if (!total_rows) return true;
    // tile height: the largest of 128, 64, 32 rows whose block count (from
    // the whole-tile lower bound) still fills two blocks per CU.  Small
    // calls (one shared expert over a prompt) trade sub-tile reuse of the
    // weight decode for using the whole chip.
    const uint64_t colblocks = hq ? w_rows / 2 / 64 : w_rows / MMQ_NB;
    uint32_t mt = MT;
    while (mt > 32 && colblocks * ((total_rows + mt - 1) / mt) < 2ull * (uint64_t)cu_count()) mt /= 2;
    // (a multiple of 8: the XCD-grouped block order maps whole octets)
    const uint32_t max_tiles = (uint32_t)((total_rows / mt + n_exp + 1 + 7) & ~(uint64_t)7);
    if (max_tiles > 65535) {
        set_error("mmq: too many row tiles (%u)", max_tiles);
        return false;
    }
    if (!ensure_tiles(max_tiles)) {
        set_error("mmq: tile buffer allocation failed");
        return false;
    }
    mmq_tiles_k<<<1, 1024, 0, stream()>>>(bounds, n_exp, mt, g_tiles, g_ntiles, max_tiles);
    if (!launch_ok("mmq_tiles_k")) return false;
    MmqArgs a;
    a.w = w;
    a.wx = wx;
    a.ex = n_exp - 1;
    a.estride = estride;
    a.rb = (uint32_t)q4mi_row_bytes(ty, w_cols);
    // packed experts: up rows follow the n_ff gate rows
    a.up_off = w_up ? (uint64_t)(w_up - w) : (w_rows / 2) * a.rb;
    a.wx_up = wx_up ? wx_up : (wx ? wx + (w_rows / 2) * a.rb : nullptr);
    a.K = (uint32_t)w_cols;
    a.n_ff = (uint32_t)(w_rows / 2);
    a.xq = (const _Float16 *)xq;
    a.xd = (const float *)((const uint8_t *)xq + xrows * w_cols * 2);
    a.act_row = act_row;
    a.bounds = bounds;
    a.tiles = g_tiles;
    a.ntiles = g_ntiles;
    a.mt = mt;
    a.wide = g_wide ? 1u : 0u;
    a.ko = 0;
    a.xcd = g_mmq_xcd ? 1u : 0u;
    a.dst = dst;
    a.ld = ld;
    a.hq = (_Float16 *)hq;
    a.hd = hq ? (float *)((uint8_t *)hq + total_rows * a.n_ff * 2) : nullptr;
    if (hq) {
        const dim3 grid((uint32_t)(a.n_ff / 64), max_tiles);
        switch (ty) {
        case Q4MI_T_IQ3_S: return mmq_launch<Q4MI_T_IQ3_S, true>(a, grid);
        case Q4MI_T_Q8_0: return mmq_launch<Q4MI_T_Q8_0, true>(a, grid);
        case Q4MI_T_IQ2_S: return mmq_launch<Q4MI_T_IQ2_S, true>(a, grid);
        case Q4MI_T_IQ4_NL: return mmq_launch<Q4MI_T_IQ4_NL, true>(a, grid);
        default: return mmq_launch<Q4MI_T_Q2_0, true>(a, grid);
        }
    }
    const dim3 grid((uint32_t)(w_rows / MMQ_NB), max_tiles);
    switch (ty) {
    case Q4MI_T_IQ3_S: return mmq_launch<Q4MI_T_IQ3_S, false>(a, grid);
    case Q4MI_T_Q8_0: return mmq_launch<Q4MI_T_Q8_0, false>(a, grid);
    case Q4MI_T_IQ2_S: return mmq_launch<Q4MI_T_IQ2_S, false>(a, grid);
    case Q4MI_T_IQ4_NL: return mmq_launch<Q4MI_T_IQ4_NL, false>(a, grid);
    default: return mmq_launch<Q4MI_T_Q2_0, false>(a, grid);
    }
}

bool swiglu_launch(const float *gu, float *h, uint64_t rows, uint64_t n_ff) {
    if (!rows) return true;
    const uint64_t n = rows * n_ff;
    swiglu_k<<<dim3((uint32_t)((n + 255) / 256)), dim3(256), 0, stream()>>>(gu, h, rows,
                                                                            (uint32_t)n_ff);
    return launch_ok("swiglu_k");
}

}  // namespace q4mi

using namespace q4mi;

extern "C" {

/* Q4_MMQ=0 disables (callers keep another path). */
int q4_mmq_on(void) {
    static int v = -1;
    if (v < 0) {
        const char *e = getenv("Q4_MMQ");
        v = !(e && e[0] == '0');
    }
    return v;
}

/* Token-group cap (Q4_MMQ_GROUP, 512..8192, default 6144 = the reference's
 * default prefill chunk, src/q4_place.c:23-40). */
uint32_t q4_mmq_group(void) {
    static int v = -1;
    if (v < 0) {
        const char *e = getenv("Q4_MMQ_GROUP");
        v = e && e[0] ? atoi(e) : 6144;
        if (v < 512) v = 512;
        if (v > 8192) v = 8192;
    }
    return (uint32_t)v;
}

/* A tile exists for (type, w_rows): IQ3_S or Q8_0, w_rows % 128 == 0. */
bool q4_mmq_supported(uint32_t type, uint64_t w_rows) {
    return mmq_type(type) && w_rows > 0 && w_rows % MMQ_NB == 0;
}

/* Bytes of the activation buffer q4_mmq_quantize fills for rows x cols:
 * fp16 codes + fp32 group scales. */
uint64_t q4_mmq_q8_bytes(uint64_t rows, uint64_t cols) {
    return rows * cols * 2 + rows * (cols / 32) * 4 + 256;
}

/* xq rows = q8 of x[ids[r]] (ids NULL = identity); x rows are `cols`
 * contiguous floats.  w_type is accepted for ABI shape (one layout here). */
bool q4_mmq_quantize(const float *x, const int32_t *ids, void *xq, uint32_t w_type,
                     uint64_t cols, uint64_t rows) {
    (void)w_type;
    if (!x || !xq || !cols || cols % 32 || ((uintptr_t)x & 15) || ((uintptr_t)xq & 15)) {
        set_error("q4_mmq_quantize: bad arguments");
        return false;
    }
    return mmq_quant(x, ids, xq, cols, rows);
}

/* dst[p][0..w_rows) = W_e . xq[p] for p in [bounds[e], bounds[e+1]).
 * max_rows is accepted for ABI shape (tiles are built on the device). */
bool q4_mmq_mul_id(const void *w, uint32_t type, uint64_t w_rows, uint64_t w_cols,
                   uint64_t expert_stride_bytes, uint32_t n_expert, const void *xq,
                   const int32_t *bounds, uint32_t max_rows, uint64_t total_rows, float *dst,
                   uint64_t ld_dst) {
    (void)max_rows;
    if (!w || !xq || !bounds || !dst || !n_expert || n_expert > 512 || !w_cols || !ld_dst ||
        ld_dst % 4 || ((uintptr_t)dst & 15) || ((uintptr_t)xq & 15)) {
        set_error("q4_mmq_mul_id: bad arguments");
        return false;
    }
    if (!mmq_supported(type, w_rows, w_cols)) {
        set_error("q4_mmq_mul_id: type/shape not covered");
        return false;
    }
    return mmq_run((const uint8_t *)w, type, w_rows, w_cols, expert_stride_bytes, n_expert, xq,
                   total_rows, nullptr, bounds, total_rows, dst, ld_dst, nullptr);
}

/* q4_mmq_mul_id with the activation rows gathered through act_row: xq
 * holds xrows rows (e.g. one per token, quantized once) and packed row p
 * reads xq row act_row[p] (e.g. the pack's a_tok).  No reference
 * counterpart: it removes the gathered q8 copy of every routed row. */
bool q4mi_mmq_mul_id_rows(const void *w, uint32_t type, uint64_t w_rows, uint64_t w_cols,
                          uint64_t expert_stride_bytes, uint32_t n_expert, const void *xq,
                          uint64_t xrows, const int32_t *act_row, const int32_t *bounds,
                          uint64_t total_rows, float *dst, uint64_t ld_dst) {
    if (!w || !xq || !bounds || !dst || !n_expert || n_expert > 512 || !w_cols || !ld_dst ||
        ld_dst % 4 || ((uintptr_t)dst & 15) || ((uintptr_t)xq & 15) || !xrows) {
        set_error("q4mi_mmq_mul_id_rows: bad arguments");
        return false;
    }
    if (!mmq_supported(type, w_rows, w_cols)) {
        set_error("q4mi_mmq_mul_id_rows: type/shape not covered");
        return false;
    }
    return mmq_run((const uint8_t *)w, type, w_rows, w_cols, expert_stride_bytes, n_expert, xq,
                   xrows, act_row, bounds, total_rows, dst, ld_dst, nullptr);
}

/* Fused gate/up MMQ: each expert's 2*n_ff x w_cols matrix (gate rows then
 * up rows) against xq rows (gathered through act_row when given); writes the
 * q8 of h = silu(gate)*up straight into hq, the q4_mmq_q8_bytes(total_rows,
 * n_ff) activation buffer the down q4_mmq_mul_id reads.  Replaces the
 * reference's mul_id(gate|up) + q4_mmq_swiglu + q4_mmq_quantize(h) sequence
 * (src/q4_moe.c:3718-3730) with one launch. */
bool q4mi_mmq_gate_up(const void *w, uint32_t type, uint64_t n_ff, uint64_t w_cols,
                      uint64_t expert_stride_bytes, uint32_t n_expert, const void *xq,
                      uint64_t xrows, const int32_t *act_row, const int32_t *bounds,
                      uint64_t total_rows, void *hq) {
    if (!w || !xq || !bounds || !hq || !n_expert || n_expert > 512 || !w_cols || !xrows ||
        ((uintptr_t)hq & 15) || ((uintptr_t)xq & 15) || n_ff % 64) {
        set_error("q4mi_mmq_gate_up: bad arguments");
        return false;
    }
    if (!mmq_supported(type, 2 * n_ff, w_cols)) {
        set_error("q4mi_mmq_gate_up: type/shape not covered");
        return false;
    }
    return mmq_run((const uint8_t *)w, type, 2 * n_ff, w_cols, expert_stride_bytes, n_expert,
                   xq, xrows, act_row, bounds, total_rows, nullptr, 0, hq);
}

/* q4mi_mmq_gate_up / q4_mmq_mul_id over n_expert routed experts at
 * w + e*stride plus one more expert, index n_expert, whose matrix sits at
 * w_extra (a shared expert stored apart from the routed arena).  bounds has
 * n_expert + 2 entries.  One launch covers both, so a shared expert over
 * every token rides in the routed launch instead of its own. */
bool q4mi_mmq_gate_up_x(const void *w, const void *w_extra, uint32_t type, uint64_t n_ff,
                        uint64_t w_cols, uint64_t expert_stride_bytes, uint32_t n_expert,
                        const void *xq, uint64_t xrows, const int32_t *act_row,
                        const int32_t *bounds, uint64_t total_rows, void *hq) {
    if (!w || !w_extra || !xq || !bounds || !hq || !n_expert || n_expert > 1023 || !w_cols ||
        !xrows || ((uintptr_t)hq & 15) || ((uintptr_t)xq & 15) || n_ff % 64) {
        set_error("q4mi_mmq_gate_up_x: bad arguments");
        return false;
    }
    if (!mmq_supported(type, 2 * n_ff, w_cols)) {
        set_error("q4mi_mmq_gate_up_x: type/shape not covered");
        return false;
    }
    return mmq_run((const uint8_t *)w, type, 2 * n_ff, w_cols, expert_stride_bytes, n_expert + 1,
                   xq, xrows, act_row, bounds, total_rows, nullptr, 0, hq,
                   (const uint8_t *)w_extra);
}

bool q4mi_mmq_mul_id_x(const void *w, const void *w_extra, uint32_t type, uint64_t w_rows,
                       uint64_t w_cols, uint64_t expert_stride_bytes, uint32_t n_expert,
                       const void *xq, const int32_t *bounds, uint64_t total_rows, float *dst,
                       uint64_t ld_dst) {
    if (!w || !w_extra || !xq || !bounds || !dst || !n_expert || n_expert > 1023 || !w_cols ||
        !ld_dst || ld_dst % 4 || ((uintptr_t)dst & 15) || ((uintptr_t)xq & 15)) {
        set_error("q4mi_mmq_mul_id_x: bad arguments");
        return false;
    }
    if (!mmq_supported(type, w_rows, w_cols)) {
        set_error("q4mi_mmq_mul_id_x: type/shape not covered");
        return false;
    }
    return mmq_run((const uint8_t *)w, type, w_rows, w_cols, expert_stride_bytes, n_expert + 1, xq,
                   total_rows, nullptr, bounds, total_rows, dst, ld_dst, nullptr,
                   (const uint8_t *)w_extra);
}

/* q4mi_mmq_gate_up over the GGUF expert layout: gate and up are separate
 * stacked tensors (blk.N.ffn_gate_exps / ffn_up_exps), expert e's gate
 * matrix at w_gate + e*expert_stride and its up matrix at w_up +
 * e*expert_stride; with wx_gate / wx_up (a shared expert's own 2-D
 * tensors), expert n_expert is that shared expert over bounds[n_expert] ..
 * bounds[n_expert + 1].  The up base must sit at the same offset within a
 * dword as the gate base. */
bool q4mi_mmq_gate_up_parts(const void *w_gate, const void *w_up, uint32_t type, uint64_t n_ff,
                            uint64_t w_cols, uint64_t expert_stride_bytes, uint32_t n_expert,
                            const void *xq, uint64_t xrows, const int32_t *act_row,
                            const int32_t *bounds, uint64_t total_rows, void *hq,
                            const void *wx_gate, const void *wx_up) {
    if (!w_gate || !w_up || !xq || !bounds || !hq || !n_expert || n_expert > 1023 || !w_cols ||
        !xrows || ((uintptr_t)hq & 15) || ((uintptr_t)xq & 15) || n_ff % 64 ||
        (!wx_gate) != (!wx_up)) {
        set_error("q4mi_mmq_gate_up_parts: bad arguments");
        return false;
    }
    if (((uintptr_t)w_gate ^ (uintptr_t)w_up) & 3u ||
        (wx_gate && (((uintptr_t)wx_gate ^ (uintptr_t)wx_up) & 3u))) {
        set_error("q4mi_mmq_gate_up_parts: up base at another in-dword offset than gate");
        return false;
    }
    if (!mmq_supported(type, 2 * n_ff, w_cols)) {
        set_error("q4mi_mmq_gate_up_parts: type/shape not covered");
        return false;
    }
    return mmq_run((const uint8_t *)w_gate, type, 2 * n_ff, w_cols, expert_stride_bytes,
                   n_expert + (wx_gate ? 1u : 0u), xq, xrows, act_row, bounds, total_rows,
                   nullptr, 0, hq, (const uint8_t *)wx_gate, (const uint8_t *)w_up,
                   (const uint8_t *)wx_up);
}

/* ---------------------------------------------------------- XG prefill
 * fp16-activation prefill GEMMs on the same MFMA tiles (the reference's
 * q4_xg, src/q4_xg.cu, src/q4.h:1177-1199): weights dequantized to fp16
 * (times 256), activations fp16, fp32 accumulation over the whole K; gate/up
 * writes h = silu(g)*u as fp16 rows, down writes fp32 rows.  Here gate/up
 * IQ3_S, Q8_0 or IQ2_S and down IQ3_S, Q8_0, IQ4_NL, Q2_0 or IQ2_S (the
 * reference: gate/up IQ2_S / IQ3_XXS / IQ3_S / IQ4_XS, down IQ4_NL /
 * Q2_0). */
int q4_xg_on(void) {
    static int v = -1;
    if (v < 0) {
        const char *e = getenv("Q4_XG");
        v = !(e && e[0] == '0');
    }
    return v;
}
bool q4_xg_gu_type(uint32_t t) {
    return t == Q4MI_T_IQ3_S || t == Q4MI_T_Q8_0 || t == Q4MI_T_IQ2_S;
}
bool q4_xg_dn_type(uint32_t t) {
    return t == Q4MI_T_IQ3_S || t == Q4MI_T_Q8_0 || t == Q4MI_T_IQ4_NL || t == Q4MI_T_Q2_0 ||
           t == Q4MI_T_IQ2_S;
}
bool q4_xg_shape_ok(uint32_t n_embd, uint32_t n_ff) {
    return n_embd % MMQ_NB == 0 && n_ff % 64 == 0 && n_embd % 512 == 0 && n_ff % 512 == 0 &&
           n_embd <= 65536 && n_ff <= 65536;
}
uint32_t q4_xg_tile_cap(uint32_t rows, uint32_t n_exp) { return rows / MMQ_MB + n_exp; }

/* Host tile table: tiles of <= 128 routed rows per expert,
 * out[4i..] = {first row, rows, slot, expert}; 0 when cap is too small. */
uint32_t q4_xg_tiles(const uint32_t *ek, const uint32_t *ebase, const int32_t *slot,
                     uint32_t n_exp, int32_t *out, uint32_t cap) {
    uint32_t n = 0;
    for (uint32_t e = 0; e < n_exp; e++)
        for (uint32_t t = 0; t < ek[e]; t += MMQ_MB) {
            if (n >= cap) return 0;
            out[4 * n + 0] = (int32_t)(ebase[e] + t);
            out[4 * n + 1] = (int32_t)(ek[e] - t < (uint32_t)MMQ_MB ? ek[e] - t : MMQ_MB);
            out[4 * n + 2] = slot[e];
            out[4 * n + 3] = (int32_t)e;
            n++;
        }
    return n;
}


/* x16[i] = fp16(x[i]), n % 4 == 0. */
bool q4_xg_cvt(const float *x, void *x16, uint64_t n) {
    if (!n) return true;
    if (!x || !x16 || n % 4 || ((uintptr_t)x & 15) || ((uintptr_t)x16 & 7)) {
        set_error("q4_xg_cvt: bad arguments");
        return false;
    }
    const uint64_t n4 = n / 4;
    xg_cvt_k<<<dim3((uint32_t)((n4 + 255) / 256)), dim3(256), 0, stream()>>>(
        (const float4 *)x, (half4_t *)x16, n4);
    return launch_ok("xg_cvt_k");
}

static bool xg_args(uint32_t type, const uint8_t *w, uint64_t astride, uint32_t K,
                    const int32_t *d_tiles, uint32_t n_tiles, MmqArgs &a, const char *who) {
    if (!w || !d_tiles || (((uintptr_t)w) & 3u) || (astride & 3u)) {
        set_error("%s: bad arguments", who);
        return false;
    }
    if (!ensure_tiles(n_tiles)) {
        set_error("%s: tile buffer allocation failed", who);
        return false;
    }
    xg_tiles_k<<<dim3((n_tiles + 255) / 256), dim3(256), 0, stream()>>>(d_tiles, n_tiles,
                                                                       g_tiles, g_ntiles);
    if (!launch_ok("xg_tiles_k")) return false;
    a = MmqArgs{};
    a.w = w;
    a.estride = astride;
    a.rb = (uint32_t)q4mi_row_bytes(type, K);
    a.K = K;
    a.tiles = g_tiles;
    a.ntiles = g_ntiles;
    a.mt = MMQ_MB;
    a.wide = g_wide ? 1u : 0u;
    return true;
}

/* h16[row][n_ff] = fp16(silu(gate . x16[atok[row]]) * (up . x16[atok[row]]))
 * over the tiles; expert weights at abase + slot*astride + og / ou. */
bool q4_xg_gu(uint32_t type, const uint8_t *abase, uint64_t astride, uint64_t og, uint64_t ou,
              uint32_t n_embd, uint32_t n_ff, const int32_t *d_tiles, uint32_t n_tiles,
              const void *x16, const int32_t *d_atok, void *h16) {
    if (!n_tiles) return true;
    if (!q4_xg_gu_type(type) || !q4_xg_shape_ok(n_embd, n_ff) || !x16 || !h16 ||
        ((uintptr_t)x16 & 15) || ((og ^ ou) & 3u)) {
        set_error("q4_xg_gu: type/shape not covered");
        return false;
    }
    MmqArgs a;
    if (!abase || !xg_args(type, abase + og, astride, n_embd, d_tiles, n_tiles, a, "q4_xg_gu"))
        return false;
    a.up_off = ou - og;
    a.n_ff = n_ff;
    a.xq = (const _Float16 *)x16;
    a.act_row = d_atok;
    a.hq = (_Float16 *)h16;
    const dim3 grid(n_ff / 64, n_tiles);
    switch (type) {
    case Q4MI_T_IQ3_S: return xg_launch<Q4MI_T_IQ3_S, true>(a, grid);
    case Q4MI_T_IQ2_S: return xg_launch<Q4MI_T_IQ2_S, true>(a, grid);
    default: return xg_launch<Q4MI_T_Q8_0, true>(a, grid);
    }
}

/* out[row][n_embd] (fp32) = down . h16[row] over the tiles; expert down
 * matrices at abase + slot*astride + od. */
bool q4_xg_dn(uint32_t type, const uint8_t *abase, uint64_t astride, uint64_t od,
              uint32_t n_ff, uint32_t n_embd, const int32_t *d_tiles, uint32_t n_tiles,
              const void *h16, float *out) {
    if (!n_tiles) return true;
    if (!q4_xg_dn_type(type) || !q4_xg_shape_ok(n_embd, n_ff) || !h16 || !out ||
        ((uintptr_t)h16 & 15) || ((uintptr_t)out & 15)) {
        set_error("q4_xg_dn: type/shape not covered");
        return false;
    }
    MmqArgs a;
    if (!abase || !xg_args(type, abase + od, astride, n_ff, d_tiles, n_tiles, a, "q4_xg_dn"))
        return false;
    a.xq = (const _Float16 *)h16;
    a.dst = out;
    a.ld = n_embd;
    const dim3 grid(n_embd / MMQ_NB, n_tiles);
    switch (type) {
    case Q4MI_T_IQ3_S: return xg_launch<Q4MI_T_IQ3_S, false>(a, grid);
    case Q4MI_T_IQ2_S: return xg_launch<Q4MI_T_IQ2_S, false>(a, grid);
    case Q4MI_T_IQ4_NL: return xg_launch<Q4MI_T_IQ4_NL, false>(a, grid);
    case Q4MI_T_Q2_0: return xg_launch<Q4MI_T_Q2_0, false>(a, grid);
    default: return xg_launch<Q4MI_T_Q8_0, false>(a, grid);
    }
}

/* h[r][k] = silu(gu[r][k]) * gu[r][n_ff + k]. */
bool q4_mmq_swiglu(const float *gu, float *h, uint64_t rows, uint64_t n_ff) {
    if (!gu || !h || !n_ff) return false;
    return swiglu_launch(gu, h, rows, n_ff);
}

}  // extern "C"
