// Shared device-side pieces of the MI355X (gfx950, wave64) routed-expert
// library: block formats, the bit-exact q8 group quantizer, LDS codebook
// tables and wave reductions.
#pragma once
#include <hip/hip_runtime.h>
#include <hip/hip_fp16.h>
#include <stdint.h>

#include "../../include/q4mi_iq3s_grid.h"

#define Q4MI_T_Q8_0 8u
#define Q4MI_T_IQ3_S 21u

// IQ3_S superblock: 256 values in 110 bytes (reference src/q4_quant.c:384-422)
//   +0 d (fp16) | +2 qs[64] | +66 qh[8] | +74 signs[32] | +106 scales[4]
// 32-value group j of a superblock: qs[8j..8j+7], qh[j] (bit k = index bit 8
// of qs[8j+k]), signs[4j..4j+3] (bit v = value v negative), scale nibble
// j&1 of scales[j/2] -> multiplier 2*nibble+1.
#define IQ3S_BYTES 110u
// Q8_0 block: fp16 d + int8 qs[32] (reference src/q4_quant.c:131-140)
#define Q80_BYTES 34u

// Row bytes of every format this library reads (0: not covered).  Besides
// IQ3_S and Q8_0: Q6_K (14), IQ4_NL (20), IQ2_S (22), Q2_0 (42), whose
// decoders are in formats.h.
__host__ __device__ inline uint64_t q4mi_row_bytes(uint32_t ty, uint64_t n) {
    switch (ty) {
    case Q4MI_T_IQ3_S: return (n % 256) ? 0 : n / 256 * IQ3S_BYTES;
    case Q4MI_T_Q8_0: return (n % 32) ? 0 : n / 32 * Q80_BYTES;
    case 14u: return n % 256 ? 0 : n / 256 * 210;   // Q6_K
    case 20u: return n % 32 ? 0 : n / 32 * 18;      // IQ4_NL
    case 22u: return n % 256 ? 0 : n / 256 * 82;    // IQ2_S
    case 42u: return n % 64 ? 0 : n / 64 * 18;      // Q2_0
    case 16u: return n % 256 ? 0 : n / 256 * 66;    // IQ2_XXS
    case 17u: return n % 256 ? 0 : n / 256 * 74;    // IQ2_XS
    case 18u: return n % 256 ? 0 : n / 256 * 98;    // IQ3_XXS
    case 23u: return n % 256 ? 0 : n / 256 * 136;   // IQ4_XS
    }
    return 0;
}

__device__ inline float q4mi_h2f(uint32_t h) {
    return __half2float(__ushort_as_half((unsigned short)h));
}

// ---------------------------------------------------------------- q8 quant
// One 32-value group, the CPU expert path's rounding (reference
// src/q4_cpuexp.c:605-637): a = max|x|, d = a/127, q = RNE(x * (127/a)),
// both divisions IEEE round-to-nearest.  A product that does not fit int32
// (or is NaN) becomes -128, as the x86 conversion + saturating pack does.
__device__ inline int q4mi_q8_code(float v) {
    if (!(v >= -2147483648.0f && v < 2147483648.0f)) return -128;
    float r = __builtin_rintf(v);
    r = fminf(fmaxf(r, -128.f), 127.f);
    return (int)r;
}

// Cross-lane step of an 8-lane team as a DPP move (no LDS round trip):
// 0xB1 = quad_perm(1,0,3,2) (lane ^ 1), 0x4E = quad_perm(2,3,0,1)
// (lane ^ 2), 0x141 = row_half_mirror (lane 7 - i within the 8: after the
// two quad steps every lane of a quad holds the same value, so this takes
// the other quad's).  Max and integer sums over the team are then exact and
// every lane holds the result.
template <int CTRL>
__device__ inline int q4mi_team8_swap(int v) {
    return __builtin_amdgcn_update_dpp(0, v, CTRL, 0xF, 0xF, true);
}
template <int CTRL>
__device__ inline float q4mi_team8_swap(float v) {
    return __builtin_bit_cast(float, q4mi_team8_swap<CTRL>(__builtin_bit_cast(int, v)));
}

// Lane-cooperative quantizer: 8 lanes own one group, 4 consecutive values
// each (lane sub = lane & 7 holds values 4*sub..4*sub+3).  Returns the packed
// int8 codes of this lane's 4 values; *d and *bs are valid in every lane of
// the 8-lane team.
__device__ inline uint32_t q4mi_quant_team8(float4 v, float *d, int *bs) {
    float a = fmaxf(fmaxf(fabsf(v.x), fabsf(v.y)), fmaxf(fabsf(v.z), fabsf(v.w)));
    a = fmaxf(a, q4mi_team8_swap<0xB1>(a));    // lane ^ 1
    a = fmaxf(a, q4mi_team8_swap<0x4E>(a));    // lane ^ 2
    a = fmaxf(a, q4mi_team8_swap<0x141>(a));   // the other quad of the team
    *d = __fdiv_rn(a, 127.f);
    const float sc = a > 0.f ? __fdiv_rn(127.f, a) : 0.f;
    const int c0 = q4mi_q8_code(v.x * sc), c1 = q4mi_q8_code(v.y * sc);
    const int c2 = q4mi_q8_code(v.z * sc), c3 = q4mi_q8_code(v.w * sc);
    int s = c0 + c1 + c2 + c3;
    s += q4mi_team8_swap<0xB1>(s);
    s += q4mi_team8_swap<0x4E>(s);
    s += q4mi_team8_swap<0x141>(s);
    *bs = s;
    return (uint32_t)(c0 & 0xff) | ((uint32_t)(c1 & 0xff) << 8) |
           ((uint32_t)(c2 & 0xff) << 16) | ((uint32_t)(c3 & 0xff) << 24);
}

// ------------------------------------------------------------- LDS tables
// grid[512]: IQ3_S codebook magnitudes (4 bytes per entry).
// smask[256]: sign byte -> two 4-byte masks (0xff where the bit is set) for
// the two grid entries that byte covers.
struct Iq3sLds {
    uint32_t grid[512];
    uint2 smask[256];
};

__device__ inline uint32_t q4mi_expand4(uint32_t n) {
    // bit k of n -> byte k = 0xff
    uint32_t b = (n & 1u) | ((n & 2u) << 7) | ((n & 4u) << 14) | ((n & 8u) << 21);
    return b * 0xffu;
}

__constant__ uint16_t q4mi_iq3s_code_dev[512] = {Q4MI_IQ3S_CODES};

__device__ inline void q4mi_iq3s_tables_init(Iq3sLds *t, int tid, int nthreads) {
    // the codebook loads of four entries go out before any is used
    for (int i0 = tid; i0 < 512; i0 += 4 * nthreads) {
        uint32_t c[4];
#pragma unroll
        for (int k = 0; k < 4; k++) c[k] = i0 + k * nthreads < 512 ? q4mi_iq3s_code_dev[i0 + k * nthreads] : 0u;
#pragma unroll
        for (int k = 0; k < 4; k++) {
            const int i = i0 + k * nthreads;
            if (i >= 512) break;
            uint32_t v = 0;
#pragma unroll
            for (int j = 0; j < 4; j++) v |= (2u * ((c[k] >> (3 * j)) & 7u) + 1u) << (8 * j);
            t->grid[i] = v;
        }
    }
    for (int i = tid; i < 256; i += nthreads)
        t->smask[i] = make_uint2(q4mi_expand4(i & 15u), q4mi_expand4(i >> 4));
}

// ----------------------------------------------------- unaligned LDS reads
// LDS byte buffer readers at 2-byte-aligned offsets (IQ3_S fields never sit
// on odd offsets, Q8_0 fields likewise).
__device__ inline uint32_t lds_u32_at(const uint32_t *w, uint32_t off) {
    const uint32_t i = off >> 2;
    return __builtin_amdgcn_alignbyte(w[i + 1], w[i], off & 3u);
}
__device__ inline uint32_t lds_u8_at(const uint8_t *b, uint32_t off) { return b[off]; }
__device__ inline uint32_t lds_u16_at(const uint8_t *b, uint32_t off) {
    return *(const uint16_t *)(b + off);
}

// Signed int8 weights of grid entry gv under a byte mask m (0xff = negate):
// (g ^ m) + (m & 1) per byte; magnitudes are nonzero and below 128 (1..62
// in the IQ grids), so no byte carries out.
__device__ inline int32_t q4mi_sign4(uint32_t gv, uint32_t m) {
    return (int32_t)((gv ^ m) + (m & 0x01010101u));
}

__device__ inline int q4mi_sdot4(int32_t a, int32_t b, int c) {
    return __builtin_amdgcn_sdot4(a, b, c, false);
}

// One IQ3_S 32-value group: decodes the 8 grid entries of group g of the row
// whose bytes start at LDS byte offset `row` and returns, per entry k, the
// signed int8 quad w[k].  *mult = 2s+1, *d = superblock scale.
struct Iq3sGroup {
    int32_t w[8];
    int mult;
    float d;
};

__device__ inline void q4mi_iq3s_decode(const Iq3sLds *tab, const uint8_t *lb,
                                        const uint32_t *lw, uint32_t row, uint32_t g,
                                        Iq3sGroup &o) {
    const uint32_t B = row + (g >> 3) * IQ3S_BYTES;
    const uint32_t j = g & 7u;
    o.d = q4mi_h2f(lds_u16_at(lb, B));
    const uint32_t qo = B + 2u + 8u * j;
    const uint32_t i0 = qo >> 2, sh = qo & 3u;
    const uint32_t w0 = lw[i0], w1 = lw[i0 + 1], w2 = lw[i0 + 2];
    const uint32_t q0 = __builtin_amdgcn_alignbyte(w1, w0, sh);
    const uint32_t q1 = __builtin_amdgcn_alignbyte(w2, w1, sh);
    const uint32_t qh = lds_u8_at(lb, B + 66u + j);
    const uint32_t sg = lds_u32_at(lw, B + 74u + 4u * j);
    const uint32_t sc = lds_u8_at(lb, B + 106u + (j >> 1));
    o.mult = 2 * (int)((j & 1u) ? (sc >> 4) : (sc & 15u)) + 1;
#pragma unroll
    for (int k = 0; k < 8; k++) {
        const uint32_t qb = ((k < 4 ? q0 : q1) >> (8 * (k & 3))) & 0xffu;
        const uint32_t idx = qb | (((qh >> k) & 1u) << 8);
        const uint2 mm = tab->smask[(sg >> (8 * (k >> 1))) & 0xffu];
        o.w[k] = q4mi_sign4(tab->grid[idx], (k & 1) ? mm.y : mm.x);
    }
}

// ---------------------------------------------------------- wave reductions
template <int W>
__device__ inline float q4mi_sum_width(float v) {
#pragma unroll
    for (int o = W / 2; o > 0; o >>= 1) v += __shfl_xor(v, o, W);
    return v;
}

// DPP reduction over aligned groups of W lanes (W = 4, 8, 16, 32, 64); the
// group's total lands in its last lane (lane % W == W-1).
template <int W>
__device__ inline float q4mi_rsum(float v) {
    v += __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), 0x111, 0xF, 0xF, true));
    v += __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), 0x112, 0xF, 0xF, true));
    if (W >= 8)
        v += __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), 0x114, 0xF, 0xF, true));
    if (W >= 16)
        v += __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), 0x118, 0xF, 0xF, true));
    if (W >= 32)
        v += __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), 0x142, 0xA, 0xF, true));
    if (W >= 64)
        v += __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), 0x143, 0xC, 0xF, true));
    return v;
}

// Inclusive prefix sum over the 64 lanes of a wave by DPP (row shifts 1, 2,
// 4, 8 within each 16-lane row, then the row-15 and row-31 broadcasts carry
// the earlier rows' totals forward).
__device__ inline uint32_t q4mi_wave_incl_scan(uint32_t v) {
    v += (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, 0x111, 0xF, 0xF, true);
    v += (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, 0x112, 0xF, 0xF, true);
    v += (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, 0x114, 0xF, 0xF, true);
    v += (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, 0x118, 0xF, 0xF, true);
    v += (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, 0x142, 0xA, 0xF, true);
    v += (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, 0x143, 0xC, 0xF, true);
    return v;
}

#define Q4MI_CHECK_LAUNCH() (hipGetLastError() == hipSuccess)
