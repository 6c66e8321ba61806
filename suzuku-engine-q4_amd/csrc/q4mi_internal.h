// Host-side shared state of the library (one process, one device).
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>
#include <stdio.h>

#include "../../include/q4mi.h"
#ifdef Q4MI_MEASURE
#include "../../include/q4mi_measure.h"
#endif

namespace q4mi {

// Stream every entry point launches on (q4_hip_stream / q4mi_set_stream).
hipStream_t stream();

// Library-owned device scratch, grown on demand.  Growing allocates, so it is
// illegal inside a graph capture; q4_hip_moe_scratch_warm / q4_mmvq_warm
// size everything up front.
struct Scratch {
    float *pd = nullptr;        // MoE decode partials [64][8][n_embd]
    size_t pd_floats = 0;
    uint32_t *tickets = nullptr;  // per-row-tile completion counters
    size_t n_tickets = 0;
    int8_t *xq = nullptr;       // q8 activations for q4_mmvq_n
    float *xd = nullptr;
    size_t xq_elems = 0;
};
Scratch &lib_scratch();
bool ensure_pd(size_t floats);
bool ensure_tickets(size_t n);
bool ensure_xq(size_t elems);

// route_k launch writing per-token lists (route.hip): row t at t*ostride,
// plus expert `shared` with weight sg[t] (or 1) when shared >= 0, and the
// per-token counts nh (optional).
bool route_list_launch(const float *lg, int32_t *ids, float *wts, int32_t *nh, uint32_t n_tok,
                       uint32_t n_exp, uint32_t topk, uint32_t ostride, int32_t shared,
                       const float *sg);

// Compute units of the current device (persistent grids size to it).
int cu_count();

// Error reporting: entry points return false; the last message is kept.
void set_error(const char *fmt, ...);

inline bool launch_ok(const char *what) {
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) {
        set_error("%s: launch failed: %s", what, hipGetErrorString(e));
        return false;
    }
    return true;
}

}  // namespace q4mi
