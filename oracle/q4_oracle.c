/* q4_oracle.c -- CPU restatement of the reference's quantized routed-expert
 * path.  TEST INFRASTRUCTURE ONLY: tests/, __graft_entry__.smoke() and
 * bench.py's cpu_baseline leg load it as the checker.  The product library
 * (suzuku-engine-q4_amd/) never links, calls or falls back to it.
 *
 * Plain scalar C, no intrinsics, written from the reference's algorithm:
 *
 *   or_f16_to_f32        src/q4_quant.c:21-45
 *   or_quant8            cpx_quant8, src/q4_cpuexp.c:605-637
 *   or_dequant_row       dequant_iq3_s src/q4_quant.c:384-422,
 *                        dequant_q8_0  src/q4_quant.c:131-140
 *   or_group_sums        the exact int32 inside dq8_iq3_s (src/q4_cpuexp.c:
 *                        855-892) and dq8_q8_0 (:1076-1096), one per 32 values
 *   or_dot8              dq8_iq3_s / dq8_q8_0 fp32 result, including the
 *                        8-lane FMA accumulation and the cpx_hsum fold order
 *                        (src/q4_cpuexp.c:39-46)
 *   or_softmax_topk      q4_softmax + q4_topk(renorm) src/q4_quant.c:715-755
 *   or_pack              host pack, src/q4_moe.c:3404-3451 and bounds
 *                        :3558-3571
 *   or_moe_tokens        q4_cpuex_dispatch2 / _win job semantics
 *                        (src/q4_cpuexp.c:2239-2321, :2387-2410, :2503-2753);
 *                        also the MMQ prefill composition q4_moe.c:3697-3748
 *                        + reduce_expert_k q4_rocm.cu:15739-15750 (same math)
 *
 * Pinning (see tests/test_oracle_*.py): or_quant8 and or_dot8 are compared
 * bit-for-bit with the reference kernels compiled from source (oracle/_ref);
 * or_group_sums against a brute-force integer dot over or_dequant_row;
 * or_dequant_row against the reference's closed-form known answer
 * (src/q4_test.c:51-57) and golden vectors; routing/pack against the
 * reference's q4_softmax/q4_topk and the partition invariants of
 * src/q4_test.c:2036-2081.
 */
#include <math.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

#include "../include/q4mi_iq2s_grid.h"
#include "../include/q4mi_iq3s_grid.h"
#include "../include/q4mi_iqxx_grids.h"

#define OR_T_Q8_0 8u
#define OR_T_Q6_K 14u
#define OR_T_IQ2_XXS 16u
#define OR_T_IQ2_XS 17u
#define OR_T_IQ3_XXS 18u
#define OR_T_IQ4_XS 23u
#define OR_T_IQ4_NL 20u
#define OR_T_IQ3_S 21u
#define OR_T_IQ2_S 22u
#define OR_T_Q2_0 42u

/* IQ4_NL value table (the format's, src/q4_quant.c:13-15) */
static const int8_t or_kv_iq4nl[16] = {-127, -104, -83, -65, -49, -35, -22, -10,
                                       1,    13,   25,  38,  53,  69,  89,  113};

float or_f16_to_f32(uint16_t h) {
    uint32_t s = ((uint32_t)h & 0x8000u) << 16;
    uint32_t e = (h >> 10) & 0x1fu;
    uint32_t m = h & 0x3ffu;
    uint32_t u;
    if (e == 0) {
        if (m == 0) {
            u = s;
        } else {
            /* subnormal: normalise the mantissa */
            int ex = 113;
            while (!(m & 0x400u)) {
                m <<= 1;
                ex--;
            }
            u = s | ((uint32_t)ex << 23) | ((m & 0x3ffu) << 13);
        }
    } else if (e == 31) {
        u = s | 0x7f800000u | (m << 13);
    } else {
        u = s | ((e + 112u) << 23) | (m << 13);
    }
    float f;
    memcpy(&f, &u, 4);
    return f;
}

uint64_t or_row_bytes(uint32_t type, uint64_t n) {
    switch (type) {
    case OR_T_IQ3_S: return n % 256 ? 0 : n / 256 * 110;
    case OR_T_Q8_0: return n % 32 ? 0 : n / 32 * 34;
    case OR_T_IQ4_NL: return n % 32 ? 0 : n / 32 * 18;
    case OR_T_Q2_0: return n % 64 ? 0 : n / 64 * 18;
    case OR_T_IQ2_S: return n % 256 ? 0 : n / 256 * 82;
    case OR_T_Q6_K: return n % 256 ? 0 : n / 256 * 210;
    case OR_T_IQ2_XXS: return n % 256 ? 0 : n / 256 * 66;
    case OR_T_IQ2_XS: return n % 256 ? 0 : n / 256 * 74;
    case OR_T_IQ3_XXS: return n % 256 ? 0 : n / 256 * 98;
    case OR_T_IQ4_XS: return n % 256 ? 0 : n / 256 * 136;
    }
    return 0;
}

static float or_h2f_at(const uint8_t *p) {
    uint16_t h;
    memcpy(&h, p, 2);
    return or_f16_to_f32(h);
}

/* Integers of one 32-value group of the non-IQ3_S formats: wi = the signed
 * integer weights, lm[l] = the integer multiplier of values 4l..4l+3, *d =
 * the float block scale (IQ2_S, IQ2_XXS, IQ2_XS: d * 0.125; IQ3_XXS:
 * d * 0.25).  Follows the reference's dequantizers (src/q4_quant.c: Q2_0
 * :177-188, IQ4_NL :273-288, IQ2_S :290-322, IQ2_XS :324-347, IQ2_XXS
 * :356-381, IQ3_XXS :424-453, IQ4_XS :455-477, Q6_K :481-510) and the
 * integer structure of the CPU dots (src/q4_cpuexp.c: dq8_iq2_xs :740-772,
 * dq8_iq2_xxs :777-810, dq8_iq3_xxs :895-935, dq8_iq4_xs :945-975): the value
 * of element i is *d * lm[i/4] * wi[i]. */
static void or_group_other(uint32_t type, const uint8_t *w, uint64_t g, int32_t wi[32],
                           int32_t lm[8], float *d) {
    for (int l = 0; l < 8; l++) lm[l] = 1;
    if (type == OR_T_IQ4_NL) {
        const uint8_t *blk = w + 18 * g;
        *d = or_h2f_at(blk);
        for (int j = 0; j < 16; j++) {
            wi[j] = or_kv_iq4nl[blk[2 + j] & 15];
            wi[j + 16] = or_kv_iq4nl[blk[2 + j] >> 4];
        }
    } else if (type == OR_T_Q2_0) {
        const uint8_t *blk = w + 18 * (g / 2);
        *d = or_h2f_at(blk);
        const uint8_t *qs = blk + 2 + 8 * (g % 2);
        for (int j = 0; j < 32; j++) wi[j] = (int32_t)((qs[j / 4] >> (2 * (j % 4))) & 3) - 1;
    } else if (type == OR_T_IQ2_S) {
        const uint8_t *blk = w + 82 * (g / 8);
        const int ib = (int)(g % 8);
        *d = or_h2f_at(blk) * 0.125f;
        const uint8_t *qs = blk + 2 + 4 * ib, *sg = blk + 34 + 4 * ib;
        const uint32_t qh = blk[66 + ib], sc = blk[74 + ib];
        for (int l = 0; l < 4; l++) {
            const uint64_t e = q4mi_iq2s_entry(qs[l] | ((qh << (8 - 2 * l)) & 0x300));
            for (int j = 0; j < 8; j++) {
                const int mag = (int)((e >> (8 * j)) & 0xff);
                wi[8 * l + j] = ((sg[l] >> j) & 1) ? -mag : mag;
            }
        }
        for (int l = 0; l < 8; l++) lm[l] = 2 * (int32_t)(l < 4 ? (sc & 15) : (sc >> 4)) + 1;
    } else if (type == OR_T_IQ2_XXS) {
        /* group ib: u32 of four grid bytes, u32 of four 7-bit sign indexes
         * and the 4-bit scale in its top nibble; multiplier 2*sc+1 */
        const uint8_t *blk = w + 66 * (g / 8);
        const int ib = (int)(g % 8);
        *d = or_h2f_at(blk) * 0.125f;
        const uint8_t *gb = blk + 2 + 8 * ib;
        uint32_t aux;
        memcpy(&aux, blk + 6 + 8 * ib, 4);
        for (int l = 0; l < 4; l++) {
            const uint64_t e = q4mi_iq2_decode(q4mi_iq2xxs_code[gb[l]]);
            const uint32_t sg = q4mi_iq_sign_byte((aux >> (7 * l)) & 127u);
            for (int j = 0; j < 8; j++) {
                const int mag = (int)((e >> (8 * j)) & 0xff);
                wi[8 * l + j] = ((sg >> j) & 1) ? -mag : mag;
            }
        }
        for (int l = 0; l < 8; l++) lm[l] = 2 * (int32_t)(aux >> 28) + 1;
    } else if (type == OR_T_IQ2_XS) {
        /* group ib: four u16 = 9-bit grid index | 7-bit sign index << 9;
         * scale byte ib: low nibble for values 0-15, high for 16-31 */
        const uint8_t *blk = w + 74 * (g / 8);
        const int ib = (int)(g % 8);
        *d = or_h2f_at(blk) * 0.125f;
        const uint32_t sc = blk[66 + ib];
        for (int l = 0; l < 4; l++) {
            uint16_t v;
            memcpy(&v, blk + 2 + 8 * ib + 2 * l, 2);
            const uint64_t e = q4mi_iq2_decode(q4mi_iq2xs_code[v & 511]);
            const uint32_t sg = q4mi_iq_sign_byte(v >> 9);
            for (int j = 0; j < 8; j++) {
                const int mag = (int)((e >> (8 * j)) & 0xff);
                wi[8 * l + j] = ((sg >> j) & 1) ? -mag : mag;
            }
        }
        for (int l = 0; l < 8; l++) lm[l] = 2 * (int32_t)(l < 4 ? (sc & 15) : (sc >> 4)) + 1;
    } else if (type == OR_T_IQ3_XXS) {
        /* group ib: eight grid bytes (four values each) at 2 + 8ib; u32 at
         * 66 + 4ib: four 7-bit sign indexes (eight values each), scale in
         * the top nibble; value dl = d * (0.5 + sc) * 0.5 = d/4 * (2sc+1) */
        const uint8_t *blk = w + 98 * (g / 8);
        const int ib = (int)(g % 8);
        *d = or_h2f_at(blk) * 0.25f;
        const uint8_t *gb = blk + 2 + 8 * ib;
        uint32_t aux;
        memcpy(&aux, blk + 66 + 4 * ib, 4);
        for (int k = 0; k < 8; k++) {
            const uint32_t e = q4mi_iq3xxs_decode(q4mi_iq3xxs_code[gb[k]]);
            const uint32_t sg = q4mi_iq_sign_byte((aux >> (7 * (k / 2))) & 127u);
            for (int j = 0; j < 4; j++) {
                const int mag = (int)((e >> (8 * j)) & 0xff);
                wi[4 * k + j] = ((sg >> (4 * (k & 1) + j)) & 1) ? -mag : mag;
            }
        }
        for (int l = 0; l < 8; l++) lm[l] = 2 * (int32_t)(aux >> 28) + 1;
    } else if (type == OR_T_IQ4_XS) {
        /* group ib: 6-bit scale ls (low 4 bits from scales_l, high 2 from
         * scales_h), multiplier ls - 32; nibbles as IQ4_NL's */
        const uint8_t *blk = w + 136 * (g / 8);
        const int ib = (int)(g % 8);
        *d = or_h2f_at(blk);
        uint16_t sh;
        memcpy(&sh, blk + 2, 2);
        const int ls = ((blk[4 + ib / 2] >> (4 * (ib % 2))) & 15) | (((sh >> (2 * ib)) & 3) << 4);
        const uint8_t *qs = blk + 8 + 16 * ib;
        for (int j = 0; j < 16; j++) {
            wi[j] = or_kv_iq4nl[qs[j] & 15];
            wi[j + 16] = or_kv_iq4nl[qs[j] >> 4];
        }
        for (int l = 0; l < 8; l++) lm[l] = ls - 32;
    } else { /* Q6_K: group g = 32 values of a 256-value superblock */
        const uint8_t *blk = w + 210 * (g / 8);
        const int j = (int)(g % 8), h = j / 4, gq = j % 4;
        *d = or_h2f_at(blk + 208);
        const uint8_t *ql = blk + 64 * h, *qh = blk + 128 + 32 * h;
        const int8_t *sc = (const int8_t *)(blk + 192 + 8 * h);
        for (int l = 0; l < 32; l++) {
            const int lo = (gq & 1) ? ql[l + 32] : ql[l];
            const int q4 = (gq & 2) ? (lo >> 4) : (lo & 15);
            const int q2 = (qh[l] >> (2 * gq)) & 3;
            wi[l] = (q4 | (q2 << 4)) - 32;
        }
        for (int l = 0; l < 8; l++) lm[l] = sc[2 * gq + (l < 4 ? 0 : 1)];
    }
}

/* _mm256_cvtps_epi32 under the default MXCSR: round to nearest even; a value
 * that does not fit int32 (or NaN) becomes INT32_MIN.  The packs that follow
 * saturate to int8. */
static int8_t or_cvt_sat8(float v) {
    if (!(v >= -2147483648.0f && v < 2147483648.0f)) return -128;
    float r = nearbyintf(v);
    if (r > 127.f) return 127;
    if (r < -128.f) return -128;
    return (int8_t)(int)r;
}

/* Per 32 values: a = max|x|; d = a/127; q = RNE(x * (a > 0 ? 127/a : 0));
 * bs = sum(q). */
void or_quant8(const float *x, uint64_t n, int8_t *q, float *d, int32_t *bs) {
    for (uint64_t g = 0; g < n / 32; g++) {
        const float *xb = x + 32 * g;
        float a = 0.f;
        for (int i = 0; i < 32; i++) {
            float v = fabsf(xb[i]);
            if (v > a) a = v;
        }
        d[g] = a / 127.f;
        const float sc = a > 0.f ? 127.f / a : 0.f;
        int32_t s = 0;
        for (int i = 0; i < 32; i++) {
            int8_t c = or_cvt_sat8(xb[i] * sc);
            q[32 * g + i] = c;
            s += c;
        }
        bs[g] = s;
    }
}

/* Float dequantization, in the reference's element order. */
int or_dequant_row(uint32_t type, const uint8_t *w, uint64_t n, float *y) {
    if (type == OR_T_Q8_0) {
        for (uint64_t b = 0; b < n / 32; b++) {
            const uint8_t *blk = w + 34 * b;
            uint16_t dh;
            memcpy(&dh, blk, 2);
            const float d = or_f16_to_f32(dh);
            for (int j = 0; j < 32; j++)
                y[32 * b + j] = (float)(int8_t)blk[2 + j] * d;
        }
        return 1;
    }
    if (type != OR_T_IQ3_S) {
        if (!or_row_bytes(type, n)) return 0;
        int32_t wi[32], lm[8];
        float d;
        for (uint64_t g = 0; g < n / 32; g++) {
            or_group_other(type, w, g, wi, lm, &d);
            for (int i = 0; i < 32; i++) {
                /* the reference's float expression per format */
                float v;
                if (type == OR_T_IQ2_S)   /* dl = d * (0.5 + s) * 0.25 */
                    v = (or_h2f_at(w + 82 * (g / 8)) * (0.5f + (float)((lm[i / 4] - 1) / 2)) *
                         0.25f) * (float)wi[i];
                else if (type == OR_T_IQ2_XXS || type == OR_T_IQ2_XS)
                    /* dl = d * 0.125 * (2s+1); value = dl * mag * sign */
                    v = (d * (float)lm[i / 4]) * (float)wi[i];
                else if (type == OR_T_IQ3_XXS) /* db = d * (0.5 + s) * 0.5 */
                    v = (or_h2f_at(w + 98 * (g / 8)) * (0.5f + (float)((lm[i / 4] - 1) / 2)) *
                         0.5f) * (float)wi[i];
                else if (type == OR_T_IQ4_XS) /* dl = d * (ls - 32) */
                    v = (d * (float)lm[i / 4]) * (float)wi[i];
                else if (type == OR_T_Q6_K) /* d * sc * (q - 32) */
                    v = d * (float)lm[i / 4] * (float)wi[i];
                else
                    v = d * (float)wi[i];
                y[32 * g + i] = v;
            }
        }
        return 1;
    }
    if (n % 256) return 0;
    for (uint64_t b = 0; b < n / 256; b++) {
        const uint8_t *blk = w + 110 * b;
        uint16_t dh;
        memcpy(&dh, blk, 2);
        const float d = or_f16_to_f32(dh);
        float *o = y + 256 * b;
        /* 8 groups of 32: qs 8 bytes, one qh byte, 4 sign bytes, a nibble
         * of scales[g/2] each. */
        for (int g = 0; g < 8; g++) {
            const uint8_t *qs = blk + 2 + 8 * g;
            const uint8_t qh = blk[66 + g];
            const uint8_t *sg = blk + 74 + 4 * g;
            const int nib = (g & 1) ? blk[106 + g / 2] >> 4 : blk[106 + g / 2] & 15;
            const float db = d * (1.f + 2.f * (float)nib);
            for (int k = 0; k < 8; k++) {
                const uint32_t idx = qs[k] | (((qh >> k) & 1u) << 8);
                const uint32_t e = q4mi_iq3s_entry(idx);
                for (int j = 0; j < 4; j++) {
                    const int v = 4 * k + j; /* value index inside the group */
                    const int neg = (sg[v / 8] >> (v % 8)) & 1;
                    o[32 * g + v] =
                        db * (float)((e >> (8 * j)) & 0xff) * (neg ? -1.f : 1.f);
                }
            }
        }
    }
    return 1;
}

/* Signed integer weights of one 32-group and its integer multiplier:
 * IQ3_S: w = +-grid byte, mult = 2s+1; Q8_0: w = int8, mult = 1. */
static void or_group_ints(uint32_t type, const uint8_t *w, uint64_t g,
                          int32_t wi[32], int32_t *mult) {
    if (type == OR_T_Q8_0) {
        const uint8_t *blk = w + 34 * g;
        for (int j = 0; j < 32; j++) wi[j] = (int8_t)blk[2 + j];
        *mult = 1;
        return;
    }
    const uint8_t *blk = w + 110 * (g / 8);
    const int j = (int)(g % 8);
    const uint8_t *qs = blk + 2 + 8 * j;
    const uint32_t h = blk[66 + j];
    const uint32_t sg = (uint32_t)blk[74 + 4 * j] | ((uint32_t)blk[75 + 4 * j] << 8) |
                        ((uint32_t)blk[76 + 4 * j] << 16) |
                        ((uint32_t)blk[77 + 4 * j] << 24);
    const uint8_t s = blk[106 + j / 2];
    *mult = 2 * ((j & 1) ? (s >> 4) : (s & 15)) + 1;
    for (int k = 0; k < 8; k++) {
        const uint32_t e = q4mi_iq3s_entry(qs[k] | (((h >> k) & 1u) << 8));
        for (int b = 0; b < 4; b++) {
            const int v = 4 * k + b;
            const int mag = (int)((e >> (8 * b)) & 0xff);
            wi[v] = ((sg >> v) & 1u) ? -mag : mag;
        }
    }
}

static int or_other(uint32_t type) {
    return type == OR_T_IQ4_NL || type == OR_T_Q2_0 || type == OR_T_IQ2_S || type == OR_T_Q6_K ||
           type == OR_T_IQ2_XXS || type == OR_T_IQ2_XS || type == OR_T_IQ3_XXS ||
           type == OR_T_IQ4_XS;
}

/* Exact per-group sums S_g = sum_l lm_l * sum_{i in quad l} w_i q_i (int32;
 * IQ3_S / Q8_0: one multiplier per group). */
int or_group_sums(uint32_t type, const uint8_t *w, uint64_t n, const int8_t *q,
                  int32_t *s) {
    if (!or_row_bytes(type, n)) return 0;
    int32_t wi[32], mult, lm[8];
    float d;
    for (uint64_t g = 0; g < n / 32; g++) {
        if (or_other(type)) {
            or_group_other(type, w, g, wi, lm, &d);
            int32_t acc = 0;
            for (int i = 0; i < 32; i++) acc += lm[i / 4] * wi[i] * (int32_t)q[32 * g + i];
            s[g] = acc;
            continue;
        }
        or_group_ints(type, w, g, wi, &mult);
        int32_t acc = 0;
        for (int i = 0; i < 32; i++) acc += wi[i] * (int32_t)q[32 * g + i];
        s[g] = acc * mult;
    }
    return 1;
}

/* fp32 row dot with the oracle's accumulation structure: lane l (0..7) of an
 * 8-wide fp32 accumulator receives, per 32-group, fma(d_w*d_x, lane_int, acc)
 * where lane_int = mult * sum of products of values 4l..4l+3; the result is
 * the cpx_hsum fold ((a0+a4)+(a2+a6)) + ((a1+a5)+(a3+a7)). */
float or_dot8(uint32_t type, const uint8_t *w, uint64_t n, const int8_t *q,
              const float *dx) {
    float acc[8] = {0, 0, 0, 0, 0, 0, 0, 0};
    int32_t wi[32], mult, lm[8];
    if (or_other(type)) {
        /* IQ4_NL, IQ2_S (dq8_iq4_nl / dq8_iq2_s, src/q4_cpuexp.c:814-853,
         * :978-1005), and IQ2_XS, IQ2_XXS, IQ3_XXS, IQ4_XS (:740-772,
         * :777-810, :895-935, :945-975): lane l gets
         * fma(d*d_x, lm_l * sum of quad l, .);
         * Q2_0 (dq8_q2_0 :1113-1150): lanes take the unsigned codes
         * (w + 1) and a serial cs = fma(d*d_x, sum(q), cs) is subtracted after the
         * fold.  Q6_K (no CPU expert kernel in the reference) uses the
         * IQ4_NL structure with its int8 sub-block scales. */
        float cs = 0.f, d;
        for (uint64_t g = 0; g < n / 32; g++) {
            or_group_other(type, w, g, wi, lm, &d);
            const float dd = d * dx[g];
            int32_t bs = 0;
            for (int l = 0; l < 8; l++) {
                int32_t li = 0;
                for (int b = 0; b < 4; b++) {
                    const int32_t v = type == OR_T_Q2_0 ? wi[4 * l + b] + 1 : wi[4 * l + b];
                    li += v * (int32_t)q[32 * g + 4 * l + b];
                    bs += q[32 * g + 4 * l + b];
                }
                acc[l] = fmaf(dd, (float)(li * lm[l]), acc[l]);
            }
            /* the reference is built with FMA contraction (gcc -O3 -mfma) */
            if (type == OR_T_Q2_0) cs = fmaf(dd, (float)bs, cs);
        }
        const float l0 = acc[0] + acc[4], l1 = acc[1] + acc[5];
        const float l2 = acc[2] + acc[6], l3 = acc[3] + acc[7];
        return ((l0 + l2) + (l1 + l3)) - cs;
    }
    for (uint64_t g = 0; g < n / 32; g++) {
        or_group_ints(type, w, g, wi, &mult);
        uint16_t dh;
        if (type == OR_T_Q8_0)
            memcpy(&dh, w + 34 * g, 2);
        else
            memcpy(&dh, w + 110 * (g / 8), 2);
        const float dd = or_f16_to_f32(dh) * dx[g];
        for (int l = 0; l < 8; l++) {
            int32_t li = 0;
            for (int b = 0; b < 4; b++) li += wi[4 * l + b] * (int32_t)q[32 * g + 4 * l + b];
            acc[l] = fmaf(dd, (float)(li * mult), acc[l]);
        }
    }
    const float l0 = acc[0] + acc[4], l1 = acc[1] + acc[5];
    const float l2 = acc[2] + acc[6], l3 = acc[3] + acc[7];
    return (l0 + l2) + (l1 + l3);
}

/* y[t*rows + r] = dot of row r with q8(x[t]), nt tokens. */
int or_dot8_rows(uint32_t type, const uint8_t *w, uint64_t rows, uint64_t n,
                 const float *x, uint32_t nt, float *y) {
    const uint64_t rb = or_row_bytes(type, n);
    if (!rb) return 0;
    int8_t *q = (int8_t *)malloc(n);
    float *d = (float *)malloc(n / 32 * sizeof(float));
    int32_t *bs = (int32_t *)malloc(n / 32 * sizeof(int32_t));
    if (!q || !d || !bs) return 0;
    for (uint32_t t = 0; t < nt; t++) {
        or_quant8(x + (uint64_t)t * n, n, q, d, bs);
        for (uint64_t r = 0; r < rows; r++)
            y[(uint64_t)t * rows + r] = or_dot8(type, w + r * rb, n, q, d);
    }
    free(q);
    free(d);
    free(bs);
    return 1;
}

/* or_dot8 over rows with the activations given already quantized: q
 * [nt][n] int8 codes and d [nt][n/32] scales (the down projection fed with
 * another implementation's q8(h), so its exact-integer part is compared
 * independently of how h rounded). */
int or_dot8q_rows(uint32_t type, const uint8_t *w, uint64_t rows, uint64_t n,
                  const int8_t *q, const float *d, uint32_t nt, float *y) {
    const uint64_t rb = or_row_bytes(type, n);
    if (!rb) return 0;
    for (uint32_t t = 0; t < nt; t++)
        for (uint64_t r = 0; r < rows; r++)
            y[(uint64_t)t * rows + r] =
                or_dot8(type, w + r * rb, n, q + (uint64_t)t * n, d + (uint64_t)t * (n / 32));
    return 1;
}

/* Router GEMV (router.hip, q4mi_moe_route): logits[t][e] = W[e] . x[t] for a
 * row type F32 (0), F16 (1) or BF16 (30), in the library's fixed order:
 * lane l (of 64) sums, for i = 0 .. K/256-1, the four products at element
 * 4(64i + l) with fmaf in component order; the 64 lane sums are joined by an
 * xor butterfly over distances 32 .. 1.  The reference's router is the same
 * GEMV (q4_gemv / dot_f32, src/q4_quant.c:583-622, in another order).  With
 * sgw, sg[t] = 1 / (1 + expf(-(sgw . x[t]))) (src/q4_moe.c:297-306), same
 * dot order. */
static float or_rw(uint32_t type, const uint8_t *row, uint64_t i) {
    if (type == 0) {
        float f;
        memcpy(&f, row + 4 * i, 4);
        return f;
    }
    const uint16_t h = (uint16_t)(row[2 * i] | (row[2 * i + 1] << 8));
    if (type == 1) return or_f16_to_f32(h);
    const uint32_t u = (uint32_t)h << 16;
    float f;
    memcpy(&f, &u, 4);
    return f;
}

static float or_lane_dot(uint32_t type, const uint8_t *row, const float *x, uint32_t K) {
    float acc[64], nx[64];
    for (uint32_t l = 0; l < 64; l++) {
        float a = 0.f;
        for (uint32_t i = 0; i < K / 256; i++)
            for (uint32_t c = 0; c < 4; c++) {
                const uint64_t e = 4ull * (64 * i + l) + c;
                a = fmaf(or_rw(type, row, e), x[e], a);
            }
        acc[l] = a;
    }
    for (uint32_t o = 32; o >= 1; o >>= 1) {
        for (uint32_t l = 0; l < 64; l++) nx[l] = acc[l] + acc[l ^ o];
        memcpy(acc, nx, sizeof acc);
    }
    return acc[0];
}

int or_router(uint32_t type, const uint8_t *w, uint32_t n_exp, uint32_t K, const float *x,
              uint32_t T, const float *sgw, float *logits, float *sg) {
    if ((type != 0 && type != 1 && type != 30) || K % 256) return 0;
    const uint64_t rb = (uint64_t)K * (type == 0 ? 4 : 2);
    for (uint32_t t = 0; t < T; t++) {
        const float *xt = x + (uint64_t)t * K;
        for (uint32_t e = 0; e < n_exp; e++)
            logits[(uint64_t)t * n_exp + e] = or_lane_dot(type, w + e * rb, xt, K);
        if (sgw) {
            const float d = or_lane_dot(0, (const uint8_t *)sgw, xt, K);
            sg[t] = 1.f / (1.f + expf(-d));
        }
    }
    return 1;
}

/* q4_softmax (serial sum, index order) then q4_topk with renormalisation:
 * strict '>' so that the earlier index wins ties. */
void or_softmax_topk(const float *logits, uint32_t n, uint32_t k, int32_t *ids,
                     float *wts) {
    float *p = (float *)malloc(n * sizeof(float));
    float m = logits[0];
    for (uint32_t i = 1; i < n; i++)
        if (logits[i] > m) m = logits[i];
    float s = 0.f;
    for (uint32_t i = 0; i < n; i++) {
        p[i] = expf(logits[i] - m);
        s += p[i];
    }
    const float inv = s > 0 ? 1.0f / s : 0.f;
    for (uint32_t i = 0; i < n; i++) p[i] *= inv;
    if (k > n) k = n;
    for (uint32_t i = 0; i < k; i++) {
        ids[i] = -1;
        wts[i] = -INFINITY;
    }
    for (uint32_t i = 0; i < n; i++) {
        const float v = p[i];
        uint32_t pos = k;
        while (pos > 0 && (ids[pos - 1] < 0 || v > wts[pos - 1])) pos--;
        if (pos == k) continue;
        for (uint32_t j = k - 1; j > pos; j--) {
            ids[j] = ids[j - 1];
            wts[j] = wts[j - 1];
        }
        ids[pos] = (int32_t)i;
        wts[pos] = v;
    }
    float t = 0.f;
    for (uint32_t i = 0; i < k; i++) t += wts[i];
    if (t > 0) {
        const float iv = 1.0f / t;
        for (uint32_t i = 0; i < k; i++) wts[i] *= iv;
    }
    free(p);
}

/* Host stable pack per token group of gsz tokens.  Outputs:
 *   ek[g*512+e]   rows of expert e in group g
 *   a_tok[g*gsz*topk + p] token of packed row p (group-local p)
 *   rsrc[t*topk+k] packed row of pick (t,k) (-1 for invalid ids), rw weight
 *   stg[g*512+i], stgn[g]  used experts ascending
 *   bounds[g*(n_exp+1) + e] = exclusive prefix, bounds[.. + n_exp] = rows */
void or_pack(const int32_t *ids, const float *wts, uint32_t n_tok,
             uint32_t topk, uint32_t n_exp, uint32_t gsz, int32_t *a_tok,
             int32_t *rsrc, float *rw, uint32_t *ek, int32_t *stg,
             uint32_t *stgn, int32_t *bounds) {
    const uint32_t n_g = (n_tok + gsz - 1) / gsz;
    uint32_t *cur = (uint32_t *)calloc((size_t)n_g * 512, sizeof(uint32_t));
    memset(ek, 0, (size_t)n_g * 512 * sizeof(uint32_t));
    memset(stgn, 0, n_g * sizeof(uint32_t));
    for (uint32_t t = 0; t < n_tok; t++)
        for (uint32_t k = 0; k < topk; k++) {
            const int32_t e = ids[t * topk + k];
            if (e >= 0 && e < (int32_t)n_exp) ek[(t / gsz) * 512 + e]++;
        }
    for (uint32_t g = 0; g < n_g; g++) {
        uint32_t b = 0;
        for (uint32_t e = 0; e < n_exp; e++) {
            cur[g * 512 + e] = b;
            bounds[g * (n_exp + 1) + e] = (int32_t)b;
            b += ek[g * 512 + e];
        }
        bounds[g * (n_exp + 1) + n_exp] = (int32_t)b;
    }
    for (uint32_t t = 0; t < n_tok; t++) {
        const uint32_t g = t / gsz, seg = g * gsz * topk;
        for (uint32_t k = 0; k < topk; k++) {
            const int32_t e = ids[t * topk + k];
            if (e < 0 || e >= (int32_t)n_exp) {
                rsrc[t * topk + k] = -1;
                rw[t * topk + k] = 0.f;
                continue;
            }
            const uint32_t p = cur[g * 512 + e]++;
            a_tok[seg + p] = (int32_t)t;
            rsrc[t * topk + k] = (int32_t)p;
            rw[t * topk + k] = wts[t * topk + k];
        }
    }
    for (uint32_t g = 0; g < n_g; g++)
        for (uint32_t e = 0; e < n_exp; e++)
            if (ek[g * 512 + e]) stg[g * 512 + stgn[g]++] = (int32_t)e;
    free(cur);
}

static float or_silu(float v) { return v / (1.f + expf(-v)); }

/* Routed-expert FFN over T tokens, the CPU expert job's arithmetic.
 * Experts live at base + id*stride as gate[n_ff][n_embd] | up | down
 * [n_embd][n_ff] (src/q4_expert.c:962-982).  Per token t and pick j
 * (expert ids[t*k+j], weight wts[t*k+j]):
 *   xq = q8(x[t]); h_r = silu(gate_r . xq) * (up_r . xq); hq = q8(h);
 *   pd_r = down_r . hq
 * mode 0 (decode job): y[t][r] accumulates wts*pd_r in pick order, starting
 *   from zero (the reference's CAS adds land in a nondeterministic order).
 * mode 1 (prefill reduce): y[t][r] += sum_j wts*pd_r (sum formed first, in
 *   pick order), as reduce_expert_k does.
 * h_out (optional) receives h for each (t, j): [T*k][n_ff]. */
int or_moe_tokens(uint32_t n_embd, uint32_t n_ff, uint32_t t_gu, uint32_t t_d,
                  const uint8_t *base, uint64_t stride, const float *x,
                  uint32_t T, const int32_t *ids, const float *wts, uint32_t k,
                  float *y, int mode, float *h_out) {
    const uint64_t rg = or_row_bytes(t_gu, n_embd), rd = or_row_bytes(t_d, n_ff);
    if (!rg || !rd) return 0;
    int8_t *xq = (int8_t *)malloc(n_embd);
    float *xd = (float *)malloc(n_embd / 32 * sizeof(float));
    int32_t *bs = (int32_t *)malloc((n_embd / 32 + n_ff / 32) * sizeof(int32_t));
    float *h = (float *)malloc(n_ff * sizeof(float));
    int8_t *hq = (int8_t *)malloc(n_ff);
    float *hd = (float *)malloc(n_ff / 32 * sizeof(float));
    float *acc = (float *)malloc(n_embd * sizeof(float));
    for (uint32_t t = 0; t < T; t++) {
        or_quant8(x + (uint64_t)t * n_embd, n_embd, xq, xd, bs);
        float *yt = y + (uint64_t)t * n_embd;
        if (mode == 0) memset(yt, 0, n_embd * sizeof(float));
        else memset(acc, 0, n_embd * sizeof(float));
        for (uint32_t j = 0; j < k; j++) {
            const int32_t e = ids[t * k + j];
            if (e < 0) continue;
            const float wt = wts[t * k + j];
            const uint8_t *pe = base + (uint64_t)e * stride;
            const uint8_t *wg = pe, *wu = pe + (uint64_t)n_ff * rg;
            const uint8_t *wd = pe + 2ull * n_ff * rg;
            for (uint32_t r = 0; r < n_ff; r++) {
                const float gv = or_dot8(t_gu, wg + r * rg, n_embd, xq, xd);
                const float uv = or_dot8(t_gu, wu + r * rg, n_embd, xq, xd);
                h[r] = or_silu(gv) * uv;
            }
            if (h_out) memcpy(h_out + ((uint64_t)t * k + j) * n_ff, h, n_ff * sizeof(float));
            or_quant8(h, n_ff, hq, hd, bs);
            for (uint32_t r = 0; r < n_embd; r++) {
                const float dv = or_dot8(t_d, wd + r * rd, n_ff, hq, hd);
                if (mode == 0) yt[r] += wt * dv;
                else acc[r] += wt * dv;
            }
        }
        if (mode != 0)
            for (uint32_t r = 0; r < n_embd; r++) yt[r] += acc[r];
    }
    free(xq);
    free(xd);
    free(bs);
    free(h);
    free(hq);
    free(hd);
    free(acc);
    return 1;
}

/* fp32 -> fp16 bits, round to nearest even (overflow to inf). */
static uint16_t or_f32_to_f16(float f) {
    uint32_t x;
    memcpy(&x, &f, 4);
    const uint32_t sign = (x >> 16) & 0x8000u;
    const int32_t e = (int32_t)((x >> 23) & 0xff) - 127 + 15;
    uint32_t m = x & 0x7fffffu;
    if (((x >> 23) & 0xff) == 0xff) return (uint16_t)(sign | 0x7c00u | (m ? 0x200u : 0));
    if (e >= 31) return (uint16_t)(sign | 0x7c00u);
    if (e <= 0) {                       /* subnormal or zero */
        if (e < -10) return (uint16_t)sign;
        m |= 0x800000u;
        const uint32_t shift = (uint32_t)(14 - e);
        uint32_t r = m >> shift;
        const uint32_t rem = m & ((1u << shift) - 1), half = 1u << (shift - 1);
        if (rem > half || (rem == half && (r & 1))) r++;
        return (uint16_t)(sign | r);
    }
    uint32_t r = ((uint32_t)e << 10) | (m >> 13);
    const uint32_t rem = m & 0x1fffu;
    if (rem > 0x1000u || (rem == 0x1000u && (r & 1))) r++;
    return (uint16_t)(sign | r);
}
static float or_fp16_round(float f) { return or_f16_to_f32(or_f32_to_f16(f)); }
uint16_t or_f16_bits(float f) { return or_f32_to_f16(f); }
void or_xg_dequant_row(uint32_t type, const uint8_t *w, uint64_t n, float *o);

/* One row of an XG (fp16) weight matrix: element = fp16(int_w * ws) with
 * ws = fp16(block scale * 256) (IQ3_S: d * (2s+1); Q8_0: d), the reference
 * XG's dequantization (src/q4_xg.cu:29-35, :60-80). */
static void or_xg_row(uint32_t type, const uint8_t *w, uint64_t n, float *o) {
    int32_t wi[32], mult, lm[8];
    for (uint64_t g = 0; g < n / 32; g++) {
        if (or_other(type)) {   /* IQ4_NL, Q2_0: d; IQ2_S: d/8 times the half's (2s+1) */
            float d;
            or_group_other(type, w, g, wi, lm, &d);
            for (int i = 0; i < 32; i++) {
                const float ws = or_fp16_round(type == OR_T_IQ2_S ? d * (float)lm[i / 4] * 256.f
                                                                  : d * 256.f);
                o[32 * g + i] = or_fp16_round((float)wi[i] * ws);
            }
            continue;
        }
        or_group_ints(type, w, g, wi, &mult);
        uint16_t dh;
        memcpy(&dh, type == OR_T_Q8_0 ? w + 34 * g : w + 110 * (g / 8), 2);
        const float ws = or_fp16_round(or_f16_to_f32(dh) * (float)mult * 256.f);
        for (int i = 0; i < 32; i++) o[32 * g + i] = or_fp16_round((float)wi[i] * ws);
    }
}

void or_xg_dequant_row(uint32_t type, const uint8_t *w, uint64_t n, float *o) {
    or_xg_row(type, w, n, o);
}

/* The XG prefill layer (q4_xg_gu + q4_xg_dn + the reduce): x16 = fp16(x);
 * g, u = (W16 . x16) / 256 (exact products, sums in double, rounded to
 * fp32); h16 = fp16(silu(g) * u); pd = (Wd16 . h16) / 256; y[t] += sum_j
 * wts * pd in pick order (mode 1 of or_moe_tokens).  The GPU sums the same
 * products in fp32 in MFMA order: outputs agree to fp32 accumulation error,
 * except where that moves h across an fp16 rounding boundary. */
int or_xg_tokens(uint32_t n_embd, uint32_t n_ff, uint32_t t_gu, uint32_t t_d,
                 const uint8_t *base, uint64_t stride, const float *x, uint32_t T,
                 const int32_t *ids, const float *wts, uint32_t k, float *y) {
    const uint64_t rg = or_row_bytes(t_gu, n_embd), rd = or_row_bytes(t_d, n_ff);
    if (!rg || !rd) return 0;
    float *x16 = (float *)malloc(n_embd * sizeof(float));
    float *wr = (float *)malloc((n_embd > n_ff ? n_embd : n_ff) * sizeof(float));
    float *wr2 = (float *)malloc(n_embd * sizeof(float));
    float *h16 = (float *)malloc(n_ff * sizeof(float));
    float *acc = (float *)malloc(n_embd * sizeof(float));
    for (uint32_t t = 0; t < T; t++) {
        for (uint32_t i = 0; i < n_embd; i++) x16[i] = or_fp16_round(x[(uint64_t)t * n_embd + i]);
        memset(acc, 0, n_embd * sizeof(float));
        for (uint32_t j = 0; j < k; j++) {
            const int32_t e = ids[t * k + j];
            if (e < 0) continue;
            const uint8_t *pe = base + (uint64_t)e * stride;
            for (uint32_t r = 0; r < n_ff; r++) {
                or_xg_row(t_gu, pe + r * rg, n_embd, wr);
                or_xg_row(t_gu, pe + (uint64_t)n_ff * rg + r * rg, n_embd, wr2);
                double sg = 0, su = 0;
                for (uint32_t i = 0; i < n_embd; i++) {
                    sg += (double)wr[i] * x16[i];
                    su += (double)wr2[i] * x16[i];
                }
                const float g = (float)(sg / 256.0), u = (float)(su / 256.0);
                h16[r] = or_fp16_round(g * u / (1.f + expf(-g)));
            }
            for (uint32_t r = 0; r < n_embd; r++) {
                or_xg_row(t_d, pe + 2ull * n_ff * rg + r * rd, n_ff, wr);
                double s = 0;
                for (uint32_t i = 0; i < n_ff; i++) s += (double)wr[i] * h16[i];
                acc[r] += wts[t * k + j] * (float)(s / 256.0);
            }
        }
        for (uint32_t r = 0; r < n_embd; r++) y[(uint64_t)t * n_embd + r] += acc[r];
    }
    free(x16);
    free(wr);
    free(wr2);
    free(h16);
    free(acc);
    return 1;
}

/* The two halves of or_xg_tokens for one expert, to check each GPU launch on
 * its own: h[r] = silu(g) * u before its fp16 rounding (x rounded to fp16
 * first), and pd[r] = (Wd16 . h16) / 256 for given fp16-valued h16. */
int or_xg_gu_row(uint32_t n_embd, uint32_t n_ff, uint32_t t_gu, const uint8_t *pe,
                 const float *x, float *h) {
    const uint64_t rg = or_row_bytes(t_gu, n_embd);
    if (!rg) return 0;
    float *x16 = (float *)malloc(n_embd * sizeof(float));
    float *wr = (float *)malloc(n_embd * sizeof(float));
    float *wr2 = (float *)malloc(n_embd * sizeof(float));
    for (uint32_t i = 0; i < n_embd; i++) x16[i] = or_fp16_round(x[i]);
    for (uint32_t r = 0; r < n_ff; r++) {
        or_xg_row(t_gu, pe + r * rg, n_embd, wr);
        or_xg_row(t_gu, pe + (uint64_t)n_ff * rg + r * rg, n_embd, wr2);
        double sg = 0, su = 0;
        for (uint32_t i = 0; i < n_embd; i++) {
            sg += (double)wr[i] * x16[i];
            su += (double)wr2[i] * x16[i];
        }
        const float g = (float)(sg / 256.0), u = (float)(su / 256.0);
        h[r] = g * u / (1.f + expf(-g));
    }
    free(x16);
    free(wr);
    free(wr2);
    return 1;
}

int or_xg_dn_row(uint32_t n_ff, uint32_t n_embd, uint32_t t_d, const uint8_t *pd_w,
                 const float *h16, float *pd) {
    const uint64_t rd = or_row_bytes(t_d, n_ff);
    if (!rd) return 0;
    float *wr = (float *)malloc(n_ff * sizeof(float));
    for (uint32_t r = 0; r < n_embd; r++) {
        or_xg_row(t_d, pd_w + r * rd, n_ff, wr);
        double s = 0;
        for (uint32_t i = 0; i < n_ff; i++) s += (double)wr[i] * h16[i];
        pd[r] = (float)(s / 256.0);
    }
    free(wr);
    return 1;
}
