// Host-side shared state of the library (one process, one device).
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>
#include <stdio.h>

#include <vector>

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

// Grow policy of every library scratch buffer that a captured graph can
// reference (decode partials, GEMV activations, MMQ tile list, pack
// histograms):
//   - no growth while the library stream is being captured: an allocation
//     there would not replay, so the call fails with GrowCapturing and the
//     caller sizes the scratch eagerly first (the warm entry points);
//   - a grown buffer's predecessor is retired, not freed: a graph captured
//     before the growth keeps launching on it, so it must stay valid for the
//     life of the process (the retired bytes stay below the sum of every
//     size asked for, and growth is rare: the warm entry points size the
//     scratch once).
// The hooks are parameters so the policy runs without a device in a test.
enum GrowResult { GrowOk = 0, GrowCapturing = 1, GrowNoMemory = 2 };
template <class Capturing, class Alloc>
inline GrowResult grow_policy(void **p, size_t bytes, Capturing capturing, Alloc alloc,
                              std::vector<void *> &retired) {
    if (capturing()) return GrowCapturing;
    void *n = nullptr;
    if (!alloc(&n, bytes) || !n) return GrowNoMemory;
    if (*p) retired.push_back(*p);
    *p = n;
    return GrowOk;
}
// The device version (library stream, hipMalloc); sets the error text.
bool scratch_grow(void **p, size_t bytes, const char *what);
// Every library allocation goes through lib_malloc, which counts them
// (the measurement build reports the count, q4mi_alloc_count).
bool lib_malloc(void **p, size_t bytes);
uint64_t alloc_count();
void note_alloc();   // counts an allocation made outside lib_malloc (pinned host memory)
bool stream_capturing();
// Status word of the MMQ kernels (rejected XG tile records), for
// q4mi_device_status.
uint32_t mmq_status(int clear);

bool ensure_pd(size_t floats);
bool ensure_tickets(size_t n);
bool ensure_xq(size_t elems);

// route_k launch writing per-token lists (route.hip): row t at t*ostride,
// plus expert `shared` with weight sg[t] (or 1) when shared >= 0, and the
// per-token counts nh (optional).
bool route_list_launch(const float *lg, int32_t *ids, float *wts, int32_t *nh, uint32_t n_tok,
                       uint32_t n_exp, uint32_t topk, uint32_t ostride, int32_t shared,
                       const float *sg);

// Router GEMV of q4mi_moe_route (router.hip); launch = false: checks only.
bool router_front(const void *d_wr, uint32_t wr_type, const float *d_sgw, const float *d_x,
                  uint32_t n_tok, uint32_t n_embd, uint32_t n_exp, uint32_t topk,
                  float *d_logits, uint32_t ostride, int32_t shared_slot, float *d_sg,
                  bool launch);

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
