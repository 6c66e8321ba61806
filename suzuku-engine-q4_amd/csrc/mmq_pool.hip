// Expert-indexed weight buffers for the prefill MMQ: the reference's L1
// gather path (src/q4_mmq.cu:447-601, declared at src/q4.h:1161-1174).
//
// The reference keeps experts in a slot-indexed VRAM cache and, before a
// prefill layer, copies each used expert's gate|up and down slices into
// buffers indexed by expert id, so that q4_mmq_mul_id can address expert e
// at w + e * stride.  With every expert resident the arena already has that
// form and callers need none of this; it is exported so that an engine
// which still stages experts links and runs unchanged.
//
// Differences from the reference, all on the safe side:
//   - q4_mmq_pad is 0: these MMQ kernels read no byte past an expert's last
//     row (their copies are clamped to the row), so no guard span is needed;
//   - buffers are cleared with a fill kernel, not a memset node, so the
//     calls stay correct when a caller records them into a graph.
#include <hip/hip_runtime.h>
#include <stdint.h>

#include <algorithm>

#include "q4mi_internal.h"

namespace q4mi {

// Copy of ordinal i: expert eid[i]'s slices from arena slot slot[i], in
// units of V (16, 4 or 1 bytes, whichever divides every size and address).
// Units [0, na) are gate|up bytes, [na, na + nd) down bytes, then the two
// zero pads up to the destination strides.
template <typename V>
__global__ __launch_bounds__(256) void gather_k(const uint8_t *__restrict__ abase,
                                                uint64_t astride, uint64_t goff, uint64_t doff,
                                                uint64_t na, uint64_t nd, uint64_t pa,
                                                uint64_t pd, uint64_t gu_dst, uint64_t d_dst,
                                                const int32_t *__restrict__ eid,
                                                const int32_t *__restrict__ slot,
                                                uint8_t *__restrict__ gu,
                                                uint8_t *__restrict__ dn) {
    const uint32_t i = blockIdx.y;
    const int32_t e = eid[i], s = slot[i];
    if (e < 0 || s < 0) return;   // no such expert: nothing to copy
    const V *gs = (const V *)(abase + (uint64_t)s * astride + goff);
    const V *ds = (const V *)(abase + (uint64_t)s * astride + doff);
    V *gd = (V *)(gu + (uint64_t)e * gu_dst);
    V *dd = (V *)(dn + (uint64_t)e * d_dst);
    const uint64_t total = na + nd + pa + pd;
    const V z = {};
    for (uint64_t u = (uint64_t)blockIdx.x * 256 + threadIdx.x; u < total;
         u += (uint64_t)gridDim.x * 256) {
        if (u < na) gd[u] = gs[u];
        else if (u < na + nd) dd[u - na] = ds[u - na];
        else if (u < na + nd + pa) gd[na + (u - na - nd)] = z;
        else dd[nd + (u - na - nd - pa)] = z;
    }
}

__global__ __launch_bounds__(256) void zero_k(uint4 *__restrict__ p, uint64_t n16) {
    for (uint64_t i = (uint64_t)blockIdx.x * 256 + threadIdx.x; i < n16;
         i += (uint64_t)gridDim.x * 256)
        p[i] = make_uint4(0, 0, 0, 0);
}

static uint8_t *g_wgu = nullptr, *g_wdn = nullptr;   // id-indexed gate|up, down
static uint64_t g_wgu_b = 0, g_wdn_b = 0;
static bool g_lend = false;                          // buffers are borrowed

// Zero `bytes` (a multiple of 16, 16-byte aligned) on the library stream.
static bool zero_fill(void *p, uint64_t bytes) {
    if (!bytes) return true;
    const uint64_t n16 = bytes / 16;
    const uint32_t grid = (uint32_t)std::min<uint64_t>((n16 + 255) / 256, 4096);
    zero_k<<<dim3(grid), dim3(256), 0, stream()>>>((uint4 *)p, n16);
    return launch_ok("zero_k");
}

static bool grow(uint8_t *&buf, uint64_t &have, uint64_t need) {
    if (need <= have) return true;
    uint8_t *nb = nullptr;
    // weight-sized buffers: freed when outgrown (not retired), so growth is
    // refused inside a capture like every other library allocation
    if (stream_capturing()) {
        set_error("q4_mmq_wbuf: growing to %llu bytes cannot happen inside a stream capture",
                  (unsigned long long)need);
        return false;
    }
    if (!lib_malloc((void **)&nb, need)) {
        set_error("q4_mmq_wbuf: hipMalloc(%llu) failed", (unsigned long long)need);
        return false;
    }
    if (!zero_fill(nb, need)) {
        (void)hipFree(nb);
        return false;
    }
    if (buf) {
        (void)hipStreamSynchronize(stream());   // earlier gathers may still use it
        (void)hipFree(buf);
    }
    buf = nb;
    have = need;
    return true;
}

}  // namespace q4mi

using namespace q4mi;

extern "C" {

/* Guard bytes each gathered expert needs past its rows: none here (the
 * reference returned at least one MMQ k-span). */
uint64_t q4_mmq_pad(uint64_t row_bytes) {
    (void)row_bytes;
    return 0;
}

/* Library-owned expert-indexed buffers of n_exp * gu_bytes and
 * n_exp * d_bytes, grown on demand and zero-filled when allocated.  In lend
 * mode (after q4_mmq_wbuf_lend) only the borrowed buffers are handed out. */
bool q4_mmq_wbuf(uint64_t gu_bytes, uint64_t d_bytes, uint32_t n_exp, uint8_t **gu,
                 uint8_t **d) {
    if (!gu || !d || !n_exp) {
        set_error("q4_mmq_wbuf: bad arguments");
        return false;
    }
    const uint64_t gneed = (gu_bytes * n_exp + 15) & ~15ull;
    const uint64_t dneed = (d_bytes * n_exp + 15) & ~15ull;
    if (g_lend) {
        if (!g_wgu || !g_wdn || gneed > g_wgu_b || dneed > g_wdn_b) {
            set_error("q4_mmq_wbuf: borrowed buffers missing or too small");
            return false;
        }
    } else if (!grow(g_wgu, g_wgu_b, gneed) || !grow(g_wdn, g_wdn_b, dneed)) {
        return false;
    }
    *gu = g_wgu;
    *d = g_wdn;
    return true;
}

/* Point the buffers at caller memory (zero-filled here) or drop them
 * (NULL).  The first call frees the library's own buffers and switches
 * q4_mmq_wbuf to lend mode for good. */
bool q4_mmq_wbuf_lend(void *gu, uint64_t gu_bytes, void *d, uint64_t d_bytes) {
    if ((gu && ((uintptr_t)gu & 15)) || (d && ((uintptr_t)d & 15))) {
        set_error("q4_mmq_wbuf_lend: buffers must be 16-byte aligned");
        return false;
    }
    if (!g_lend) {
        (void)hipStreamSynchronize(stream());
        if (g_wgu) (void)hipFree(g_wgu);
        if (g_wdn) (void)hipFree(g_wdn);
        g_lend = true;
    }
    g_wgu = (uint8_t *)gu;
    g_wdn = (uint8_t *)d;
    g_wgu_b = gu ? gu_bytes & ~15ull : 0;
    g_wdn_b = d ? d_bytes & ~15ull : 0;
    return zero_fill(gu, g_wgu_b) && zero_fill(d, g_wdn_b);
}

/* For i < n: copy [abase + slot[i]*astride + goff, +gu_bytes) to
 * d_gu + eid[i]*gu_dst and [.. + doff, +d_bytes) to d_d + eid[i]*d_dst,
 * zeroing each destination's tail up to its stride.  Entries with a
 * negative id or slot are skipped. */
bool q4_mmq_gather(const uint8_t *abase, uint64_t astride, uint64_t goff, uint64_t gu_bytes,
                   uint64_t doff, uint64_t d_bytes, uint64_t gu_dst, uint64_t d_dst,
                   const int32_t *d_eid, const int32_t *d_slot, uint32_t n, uint8_t *d_gu,
                   uint8_t *d_d) {
    if (!n) return true;
    if (!abase || !d_eid || !d_slot || !d_gu || !d_d || gu_dst < gu_bytes || d_dst < d_bytes ||
        n > 65535) {
        set_error("q4_mmq_gather: bad arguments");
        return false;
    }
    const uint64_t al = (uintptr_t)abase | astride | goff | gu_bytes | doff | d_bytes | gu_dst |
                        d_dst | (uintptr_t)d_gu | (uintptr_t)d_d;
    const uint64_t unit = (al & 15) == 0 ? 16 : (al & 3) == 0 ? 4 : 1;
    const uint64_t na = gu_bytes / unit, nd = d_bytes / unit;
    const uint64_t pa = (gu_dst - gu_bytes) / unit, pd = (d_dst - d_bytes) / unit;
    const uint64_t total = na + nd + pa + pd;
    const dim3 grid((uint32_t)std::min<uint64_t>((total + 255) / 256, 256), n);
    if (unit == 16)
        gather_k<uint4><<<grid, dim3(256), 0, stream()>>>(abase, astride, goff, doff, na, nd, pa,
                                                         pd, gu_dst, d_dst, d_eid, d_slot, d_gu,
                                                         d_d);
    else if (unit == 4)
        gather_k<uint32_t><<<grid, dim3(256), 0, stream()>>>(abase, astride, goff, doff, na, nd,
                                                            pa, pd, gu_dst, d_dst, d_eid,
                                                            d_slot, d_gu, d_d);
    else
        gather_k<uint8_t><<<grid, dim3(256), 0, stream()>>>(abase, astride, goff, doff, na, nd,
                                                           pa, pd, gu_dst, d_dst, d_eid, d_slot,
                                                           d_gu, d_d);
    return launch_ok("q4_mmq_gather");
}

}  // extern "C"
