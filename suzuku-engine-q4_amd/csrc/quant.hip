// Bit-exact q8 activation quantizer (per 32 values: int8 codes, fp32 d,
// int32 code sum), the CPU expert path's cpx_quant8 (reference
// src/q4_cpuexp.c:605-637).  Rows may be gathered through an index list.
#include "q4mi_common.h"
#include "q4mi_internal.h"

// 8 lanes per group, 32 groups per 256-thread block; grid.x covers the
// groups of all rows (row-major), so adjacent blocks read adjacent memory.
__global__ __launch_bounds__(256) void q8_quant_k(const float *__restrict__ x,
                                                  const int32_t *__restrict__ ids,
                                                  uint64_t rows, uint32_t cols,
                                                  int8_t *__restrict__ q,
                                                  float *__restrict__ d,
                                                  int32_t *__restrict__ bs) {
    const uint32_t gpr = cols / 32;
    const uint64_t gid = (uint64_t)blockIdx.x * 32 + (threadIdx.x >> 3);
    if (gid >= rows * gpr) return;
    const uint64_t r = gid / gpr;
    const uint32_t g = (uint32_t)(gid % gpr);
    const uint32_t sub = threadIdx.x & 7u;
    const uint64_t src = ids ? (uint64_t)ids[r] : r;
    const float4 v = *(const float4 *)(x + src * cols + 32u * g + 4u * sub);
    float dd;
    int s;
    const uint32_t packed = q4mi_quant_team8(v, &dd, &s);
    *(uint32_t *)(q + r * cols + 32u * g + 4u * sub) = packed;
    if (sub == 0) {
        d[gid] = dd;
        if (bs) bs[gid] = s;
    }
}

namespace q4mi {
bool quant8_launch(const float *x, const int32_t *ids, uint64_t rows, uint32_t cols,
                   int8_t *q, float *d, int32_t *bs) {
    if (!rows) return true;
    const uint64_t groups = rows * (cols / 32);
    const uint64_t blocks = (groups + 31) / 32;
    q8_quant_k<<<dim3((uint32_t)blocks), dim3(256), 0, stream()>>>(x, ids, rows, cols, q, d,
                                                                   bs);
    return launch_ok("q8_quant_k");
}
}  // namespace q4mi

extern "C" {

/* x rows (or x[ids[r]]) of `cols` fp32 -> q[rows][cols] int8,
 * d[rows][cols/32] fp32, bs[rows][cols/32] int32 (bs may be NULL). */
bool q4mi_quant8(const float *d_x, const int32_t *d_ids, uint64_t rows, uint64_t cols,
                 int8_t *d_q, float *d_d, int32_t *d_bs) {
    if (!d_x || !d_q || !d_d || !cols || cols % 32 || cols > (1u << 30)) {
        q4mi::set_error("q4mi_quant8: bad arguments");
        return false;
    }
    if (((uintptr_t)d_x & 15) || ((uintptr_t)d_q & 3)) {
        q4mi::set_error("q4mi_quant8: x must be 16-byte and q 4-byte aligned");
        return false;
    }
    if (rows * (cols / 32) > (uint64_t)0xffffffffu * 32) {
        q4mi::set_error("q4mi_quant8: too many rows");
        return false;
    }
    return q4mi::quant8_launch(d_x, d_ids, rows, (uint32_t)cols, d_q, d_d, d_bs);
}

}  // extern "C"
