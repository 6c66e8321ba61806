// Expert-sorted prefill MMQ on MFMA (gfx950).
//
// Routed rows are packed per expert (ragged bounds[e]..bounds[e+1]).  For
// each (expert, 64-row token tile, 64-row weight tile) a 256-thread block
// walks K one IQ3_S superblock (256 values) at a time:
//   * weights: IQ3_S -> exact integers w*(2s+1) (|v| <= 465), written to LDS
//     as fp16 (exact); Q8_0 -> its int8 values as fp16 (exact);
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

#include "q4mi_common.h"
#include "q4mi_internal.h"

typedef _Float16 half8_t __attribute__((ext_vector_type(8)));
typedef _Float16 half2_t __attribute__((ext_vector_type(2)));
typedef float f32x16_t __attribute__((ext_vector_type(16)));

namespace q4mi {

constexpr int MT = 64;          // token rows per block tile
constexpr int NTW = 64;         // weight rows per block tile
constexpr int KS = 256;         // K values per step (one IQ3_S superblock)
constexpr int LDH = KS + 8;     // fp16 row stride in LDS (16-byte skew)

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
// tiles[i] = (expert, first row of the 64-row tile); tiles[-1 slot] count.
__global__ __launch_bounds__(512) void mmq_tiles_k(const int32_t *__restrict__ bounds,
                                                   uint32_t n_exp, int2 *__restrict__ tiles,
                                                   uint32_t *__restrict__ count,
                                                   uint32_t max_tiles) {
    __shared__ uint32_t s[512];
    const uint32_t e = threadIdx.x;
    uint32_t c = 0;
    if (e < n_exp) {
        const int32_t n = bounds[e + 1] - bounds[e];
        c = n > 0 ? (uint32_t)((n + MT - 1) / MT) : 0u;
    }
    s[e] = c;
    __syncthreads();
    for (uint32_t o = 1; o < 512; o <<= 1) {
        const uint32_t v = e >= o ? s[e - o] : 0u;
        __syncthreads();
        s[e] += v;
        __syncthreads();
    }
    const uint32_t start = s[e] - c;
    for (uint32_t i = 0; i < c && start + i < max_tiles; i++)
        tiles[start + i] = make_int2((int)e, (int)(i * MT));
    if (e == 511) *count = min(s[511], max_tiles);
}

// --------------------------------------------------------------- kernel
struct Fp16Lds {
    _Float16 w[NTW][LDH];    // weights of this K step (fp16 exact integers)
    _Float16 x[MT][LDH];     // activation codes
    float dx[8][MT];         // activation group scales
    float dwg[8][NTW];       // Q8_0: per-group weight scales
    float dwb[NTW];          // IQ3_S: superblock scale per weight row
    uint2 g16[512];          // IQ3_S grid as fp16 magnitudes (4 halves)
    uint2 sm16[16];          // sign nibble -> fp16 sign-bit masks
};

__device__ inline uint32_t ld_u16(const uint8_t *p) { return *(const uint16_t *)p; }

// Decode one IQ3_S 32-group of a weight row (global bytes, 2-aligned) into
// 32 fp16 values w*(2s+1) at dst.
__device__ inline void iq3s_group_f16(const Fp16Lds &L, const uint8_t *blk, uint32_t j,
                                      _Float16 *dst) {
    const uint8_t *qs = blk + 2 + 8 * j;
    const uint32_t q0 = ld_u16(qs) | (ld_u16(qs + 2) << 16);
    const uint32_t q1 = ld_u16(qs + 4) | (ld_u16(qs + 6) << 16);
    const uint32_t qh = blk[66 + j];
    const uint32_t sg = ld_u16(blk + 74 + 4 * j) | (ld_u16(blk + 76 + 4 * j) << 16);
    const uint32_t sc = blk[106 + (j >> 1)];
    const float m = (float)(2u * ((j & 1u) ? (sc >> 4) : (sc & 15u)) + 1u);
    const half2_t mm = {(_Float16)m, (_Float16)m};
    uint4 out[4];
    uint32_t *o = (uint32_t *)out;
#pragma unroll
    for (int k = 0; k < 8; k++) {
        const uint32_t qb = ((k < 4 ? q0 : q1) >> (8 * (k & 3))) & 0xffu;
        const uint32_t idx = qb | (((qh >> k) & 1u) << 8);
        const uint2 g = L.g16[idx];
        const uint2 s = L.sm16[(sg >> (4 * k)) & 15u];
        half2_t a = __builtin_bit_cast(half2_t, g.x ^ s.x);
        half2_t b = __builtin_bit_cast(half2_t, g.y ^ s.y);
        a = a * mm;
        b = b * mm;
        o[2 * k] = __builtin_bit_cast(uint32_t, a);
        o[2 * k + 1] = __builtin_bit_cast(uint32_t, b);
    }
    uint4 *d4 = (uint4 *)dst;
#pragma unroll
    for (int i = 0; i < 4; i++) d4[i] = out[i];
}

struct MmqArgs {
    const uint8_t *w;
    uint64_t estride;       // bytes between experts
    uint32_t rb;            // bytes per weight row
    uint32_t K, N;          // w_cols, w_rows
    const _Float16 *xq;     // [xrows][K]
    const float *xd;        // [xrows][K/32]
    const int32_t *act_row; // optional: activation row of packed row p
    const int32_t *bounds;  // [n_exp+1]
    const int2 *tiles;
    const uint32_t *ntiles;
    float *dst;
    uint64_t ld;
};

template <uint32_t TY>
__global__ __launch_bounds__(256, 2) void mmq_k(MmqArgs a) {
    extern __shared__ __align__(16) uint8_t smem[];
    Fp16Lds &L = *(Fp16Lds *)smem;
    const uint32_t tid = threadIdx.x, lane = tid & 63u, wv = tid >> 6;
    const uint32_t ti = blockIdx.y;
    if (ti >= *a.ntiles) return;
    const int2 tinfo = a.tiles[ti];
    const uint32_t e = (uint32_t)tinfo.x;
    const int32_t rbase = a.bounds[e] + tinfo.y;
    const uint32_t mrows = min((uint32_t)(a.bounds[e + 1] - rbase), (uint32_t)MT);
    const uint32_t n0 = blockIdx.x * NTW;
    const uint8_t *W = a.w + (uint64_t)e * a.estride + (uint64_t)n0 * a.rb;

    if (TY == Q4MI_T_IQ3_S) {
        for (uint32_t i = tid; i < 512; i += 256) {
            const uint32_t c = q4mi_iq3s_code_dev[i];
            uint32_t h[4];
#pragma unroll
            for (int jj = 0; jj < 4; jj++) {
                const _Float16 f = (_Float16)(float)(2u * ((c >> (3 * jj)) & 7u) + 1u);
                h[jj] = __builtin_bit_cast(uint16_t, f);
            }
            L.g16[i] = make_uint2(h[0] | (h[1] << 16), h[2] | (h[3] << 16));
        }
        if (tid < 16) {
            uint32_t s[4];
#pragma unroll
            for (int jj = 0; jj < 4; jj++) s[jj] = ((tid >> jj) & 1u) ? 0x8000u : 0u;
            L.sm16[tid] = make_uint2(s[0] | (s[1] << 16), s[2] | (s[3] << 16));
        }
    }
    // activation rows of this tile (packed row -> source row)
    const uint32_t xr_lane = tid >> 2;      // 64 rows, 4 threads per row
    int64_t xrow = -1;
    if (xr_lane < mrows) {
        const int32_t p = rbase + (int32_t)xr_lane;
        xrow = a.act_row ? a.act_row[p] : p;
    }
    const uint32_t wn = wv & 1u, wm = wv >> 1;   // wave's 32x32 output sub-tile
    f32x16_t acc = {};
    f32x16_t inner = {};
    const uint32_t nsteps = a.K / KS;
    for (uint32_t st = 0; st < nsteps; st++) {
        __syncthreads();   // previous step's LDS reads are done
        // activations: 64 rows x 256 fp16 (512 B per row), 4 threads per row
        {
            const uint32_t part = tid & 3u;
            uint4 *dst = (uint4 *)&L.x[xr_lane][part * 64];
            if (xrow >= 0) {
                const uint4 *src = (const uint4 *)(a.xq + (uint64_t)xrow * a.K + st * KS + part * 64);
#pragma unroll
                for (int i = 0; i < 8; i++) dst[i] = src[i];
            } else {
#pragma unroll
                for (int i = 0; i < 8; i++) dst[i] = make_uint4(0, 0, 0, 0);
            }
            if (part < 2) {
                const uint32_t g0 = part * 4;
#pragma unroll
                for (int gg = 0; gg < 4; gg++)
                    L.dx[g0 + gg][xr_lane] =
                        xrow >= 0 ? a.xd[(uint64_t)xrow * (a.K / 32) + st * 8 + g0 + gg] : 0.f;
            }
        }
        // weights: 64 rows x 8 groups = 512 group decodes, 2 per thread
        for (uint32_t it = tid; it < NTW * 8; it += 256) {
            const uint32_t r = it >> 3, j = it & 7u;
            if (TY == Q4MI_T_IQ3_S) {
                const uint8_t *blk = W + (uint64_t)r * a.rb + (uint64_t)st * IQ3S_BYTES;
                iq3s_group_f16(L, blk, j, &L.w[r][32 * j]);
                if (j == 0) L.dwb[r] = q4mi_h2f(ld_u16(blk));
            } else {
                const uint8_t *blk = W + (uint64_t)r * a.rb + (uint64_t)(st * 8 + j) * Q80_BYTES;
                uint4 out[4];
                uint32_t *o = (uint32_t *)out;
#pragma unroll
                for (int k = 0; k < 16; k++) {
                    const uint32_t pr = ld_u16(blk + 2 + 2 * k);
                    const _Float16 lo = (_Float16)(float)(int8_t)(pr & 0xffu);
                    const _Float16 hi = (_Float16)(float)(int8_t)(pr >> 8);
                    o[k] = (uint32_t)__builtin_bit_cast(uint16_t, lo) |
                           ((uint32_t)__builtin_bit_cast(uint16_t, hi) << 16);
                }
                uint4 *d4 = (uint4 *)&L.w[r][32 * j];
#pragma unroll
                for (int i = 0; i < 4; i++) d4[i] = out[i];
                L.dwg[j][r] = q4mi_h2f(ld_u16(blk));
            }
        }
        __syncthreads();
        const uint32_t kb = (lane >> 5) * 8;   // this lane's 8-value k slice
        const uint32_t rw_ = wn * 32 + (lane & 31u);
        const uint32_t rx = wm * 32 + (lane & 31u);
#pragma unroll
        for (int g = 0; g < 8; g++) {
            const half8_t A0 = *(const half8_t *)&L.w[rw_][32 * g + kb];
            const half8_t B0 = *(const half8_t *)&L.x[rx][32 * g + kb];
            const half8_t A1 = *(const half8_t *)&L.w[rw_][32 * g + 16 + kb];
            const half8_t B1 = *(const half8_t *)&L.x[rx][32 * g + 16 + kb];
            f32x16_t s = {};
            s = __builtin_amdgcn_mfma_f32_32x32x16_f16(A0, B0, s, 0, 0, 0);
            s = __builtin_amdgcn_mfma_f32_32x32x16_f16(A1, B1, s, 0, 0, 0);
            const float dxv = L.dx[g][rx];
            if (TY == Q4MI_T_IQ3_S) {
#pragma unroll
                for (int i = 0; i < 16; i++) inner[i] = fmaf(s[i], dxv, inner[i]);
            } else {
#pragma unroll
                for (int i = 0; i < 16; i++) {
                    const uint32_t n = wn * 32 + 8 * (i / 4) + 4 * (lane >> 5) + (i % 4);
                    acc[i] = fmaf(s[i], dxv * L.dwg[g][n], acc[i]);
                }
            }
        }
        if (TY == Q4MI_T_IQ3_S) {
#pragma unroll
            for (int i = 0; i < 16; i++) {
                const uint32_t n = wn * 32 + 8 * (i / 4) + 4 * (lane >> 5) + (i % 4);
                acc[i] = fmaf(inner[i], L.dwb[n], acc[i]);
                inner[i] = 0.f;
            }
        }
    }
    // write: lane holds token column p = wm*32 + lane%32 and 16 weight rows
    const uint32_t p = wm * 32 + (lane & 31u);
    if (p < mrows) {
        float *o = a.dst + (uint64_t)(rbase + (int32_t)p) * a.ld + n0 + wn * 32 + 4 * (lane >> 5);
#pragma unroll
        for (int b = 0; b < 4; b++)
            *(float4 *)(o + 8 * b) =
                make_float4(acc[4 * b], acc[4 * b + 1], acc[4 * b + 2], acc[4 * b + 3]);
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

static int2 *g_tiles = nullptr;
static uint32_t *g_ntiles = nullptr;
static uint32_t g_tiles_cap = 0;

static bool ensure_tiles(uint32_t n) {
    if (g_tiles_cap >= n) return true;
    if (g_tiles) (void)hipFree(g_tiles);
    if (!g_ntiles && hipMalloc(&g_ntiles, sizeof(uint32_t)) != hipSuccess) return false;
    if (hipMalloc(&g_tiles, (size_t)n * sizeof(int2)) != hipSuccess) {
        g_tiles = nullptr;
        g_tiles_cap = 0;
        return false;
    }
    g_tiles_cap = n;
    return true;
}

bool mmq_supported(uint32_t ty, uint64_t w_rows, uint64_t w_cols) {
    if (ty != Q4MI_T_IQ3_S && ty != Q4MI_T_Q8_0) return false;
    return w_rows > 0 && w_rows % NTW == 0 && w_cols > 0 && w_cols % KS == 0 &&
           w_cols <= 65536;
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

// xq rows = xrows (activation rows); act_row maps packed rows to them.
bool mmq_run(const uint8_t *w, uint32_t ty, uint64_t w_rows, uint64_t w_cols, uint64_t estride,
             uint32_t n_exp, const void *xq, uint64_t xrows, const int32_t *act_row,
             const int32_t *bounds, uint64_t total_rows, float *dst, uint64_t ld) {
    if (!total_rows) return true;
    const uint32_t max_tiles = (uint32_t)(total_rows / MT + n_exp + 1);
    if (!ensure_tiles(max_tiles)) {
        set_error("mmq: tile buffer allocation failed");
        return false;
    }
    mmq_tiles_k<<<1, 512, 0, stream()>>>(bounds, n_exp, g_tiles, g_ntiles, max_tiles);
    if (!launch_ok("mmq_tiles_k")) return false;
    MmqArgs a;
    a.w = w;
    a.estride = estride;
    a.rb = (uint32_t)q4mi_row_bytes(ty, w_cols);
    a.K = (uint32_t)w_cols;
    a.N = (uint32_t)w_rows;
    a.xq = (const _Float16 *)xq;
    a.xd = (const float *)((const uint8_t *)xq + xrows * w_cols * 2);
    a.act_row = act_row;
    a.bounds = bounds;
    a.tiles = g_tiles;
    a.ntiles = g_ntiles;
    a.dst = dst;
    a.ld = ld;
    const dim3 grid((uint32_t)(w_rows / NTW), max_tiles);
    const size_t lds = sizeof(Fp16Lds);
    static bool attr = false;
    if (!attr) {
        // the tile needs more than the default 64 KiB of dynamic LDS
        if (hipFuncSetAttribute((const void *)mmq_k<Q4MI_T_IQ3_S>,
                                hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds) != hipSuccess ||
            hipFuncSetAttribute((const void *)mmq_k<Q4MI_T_Q8_0>,
                                hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds) != hipSuccess) {
            set_error("mmq: cannot raise the LDS limit to %zu bytes", lds);
            return false;
        }
        attr = true;
    }
    if (ty == Q4MI_T_IQ3_S)
        mmq_k<Q4MI_T_IQ3_S><<<grid, dim3(256), lds, stream()>>>(a);
    else
        mmq_k<Q4MI_T_Q8_0><<<grid, dim3(256), lds, stream()>>>(a);
    return launch_ok("mmq_k");
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

/* A tile exists for (type, w_rows): IQ3_S or Q8_0, w_rows % 64 == 0. */
bool q4_mmq_supported(uint32_t type, uint64_t w_rows) {
    return (type == Q4MI_T_IQ3_S || type == Q4MI_T_Q8_0) && w_rows > 0 && w_rows % NTW == 0;
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
                   total_rows, nullptr, bounds, total_rows, dst, ld_dst);
}

/* h[r][k] = silu(gu[r][k]) * gu[r][n_ff + k]. */
bool q4_mmq_swiglu(const float *gu, float *h, uint64_t rows, uint64_t n_ff) {
    if (!gu || !h || !n_ff) return false;
    return swiglu_launch(gu, h, rows, n_ff);
}

}  // extern "C"
