// Library runtime: stream selection, device scratch and error text.
#include <stdarg.h>
#include <string.h>

#include "q4mi_internal.h"

namespace q4mi {

static hipStream_t g_stream = nullptr;  // null = the device's default stream
static Scratch g_scr;
static char g_err[512];

hipStream_t stream() { return g_stream; }
Scratch &lib_scratch() { return g_scr; }

void set_error(const char *fmt, ...) {
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(g_err, sizeof g_err, fmt, ap);
    va_end(ap);
    if (getenv("Q4MI_VERBOSE")) fprintf(stderr, "q4mi: %s\n", g_err);
}

static uint64_t g_allocs = 0;
static std::vector<void *> g_retired;   // grown-out scratch, kept for earlier graphs

bool lib_malloc(void **p, size_t bytes) {
    if (hipMalloc(p, bytes) != hipSuccess) return false;
    g_allocs++;
    return true;
}
uint64_t alloc_count() { return g_allocs; }
void note_alloc() { g_allocs++; }

bool stream_capturing() {
    hipStreamCaptureStatus st = hipStreamCaptureStatusNone;
    return hipStreamIsCapturing(g_stream, &st) == hipSuccess && st != hipStreamCaptureStatusNone;
}

bool scratch_grow(void **p, size_t bytes, const char *what) {
    const GrowResult r = grow_policy(
        p, bytes, [] { return stream_capturing(); },
        [](void **q, size_t b) { return lib_malloc(q, b); }, g_retired);
    if (r == GrowCapturing)
        set_error("%s: scratch must grow to %zu bytes, which cannot happen inside a stream "
                  "capture; make the largest call (or the warm entry point) before capturing",
                  what, bytes);
    else if (r == GrowNoMemory)
        set_error("%s: hipMalloc(%zu) failed", what, bytes);
    return r == GrowOk;
}

static bool grow(void **p, size_t bytes, const char *what) { return scratch_grow(p, bytes, what); }

bool ensure_pd(size_t floats) {
    if (g_scr.pd_floats >= floats) return true;
    if (!grow((void **)&g_scr.pd, floats * sizeof(float), "pd")) return false;
    g_scr.pd_floats = floats;
    return true;
}

bool ensure_tickets(size_t n) {
    if (g_scr.n_tickets >= n) return true;
    // The counters must start at zero; every kernel that uses them returns
    // them to zero before it exits.
    if (!grow((void **)&g_scr.tickets, n * sizeof(uint32_t), "tickets")) return false;
    if (hipMemset(g_scr.tickets, 0, n * sizeof(uint32_t)) != hipSuccess) return false;
    if (hipDeviceSynchronize() != hipSuccess) return false;
    g_scr.n_tickets = n;
    return true;
}

bool ensure_xq(size_t elems) {
    if (g_scr.xq_elems >= elems) return true;
    if (!grow((void **)&g_scr.xq, elems, "xq")) return false;
    if (!grow((void **)&g_scr.xd, (elems / 32 + 1) * sizeof(float), "xd")) return false;
    g_scr.xq_elems = elems;
    return true;
}

}  // namespace q4mi

extern "C" {

void *q4_hip_stream(void) { return (void *)q4mi::g_stream; }

void q4mi_set_stream(void *s) { q4mi::g_stream = (hipStream_t)s; }

const char *q4mi_last_error(void) { return q4mi::g_err; }

#ifdef Q4MI_MEASURE
/* Measurement build only: library allocations made so far. */
uint64_t q4mi_alloc_count(void) { return q4mi::alloc_count(); }

/* Measurement build only: the scratch grow policy run on host fakes (no
 * device calls); 1 = every case behaves as documented. */
int q4mi_grow_selftest(void) {
    using namespace q4mi;
    std::vector<void *> retired;
    static char a1[16], a2[16];
    void *p = nullptr;
    bool cap = false, fail = false;
    char *next = a1;
    auto capturing = [&] { return cap; };
    auto alloc = [&](void **q, size_t) {
        if (fail) return false;
        *q = next;
        return true;
    };
    // first growth: no predecessor to retire
    if (grow_policy(&p, 16, capturing, alloc, retired) != GrowOk || p != a1 || !retired.empty())
        return 0;
    // refused while capturing: nothing allocated, the buffer unchanged
    cap = true;
    next = a2;
    if (grow_policy(&p, 32, capturing, alloc, retired) != GrowCapturing || p != a1 ||
        !retired.empty())
        return 0;
    // an allocation failure leaves the buffer as it was
    cap = false;
    fail = true;
    if (grow_policy(&p, 32, capturing, alloc, retired) != GrowNoMemory || p != a1 ||
        !retired.empty())
        return 0;
    // growth: the predecessor is retired (kept), never freed
    fail = false;
    if (grow_policy(&p, 32, capturing, alloc, retired) != GrowOk || p != a2 ||
        retired.size() != 1 || retired[0] != a1)
        return 0;
    return 1;
}
#endif

const char *q4mi_status_text(uint32_t bits) {
    static char buf[384];
    if (!bits) return "ok";
    if (bits & 0x80000000u) return "device status not readable";
    buf[0] = 0;
    if (bits & 3u)
        snprintf(buf, sizeof buf, "decode kernel gave up a bounded wait (%s%s%s): results of the "
                 "calls since the last status check are wrong",
                 (bits & 1u) ? "consumer" : "", (bits & 3u) == 3u ? ", " : "",
                 (bits & 2u) ? "producer" : "");
    if (bits & 4u) {
        const size_t l = strlen(buf);
        snprintf(buf + l, sizeof buf - l, "%sXG tile record out of range (rows outside 1..128 or "
                 "a negative slot or row): that tile was skipped, its rows not written",
                 l ? "; " : "");
    }
    return buf;
}

int q4mi_device_ok(void) {
    int n = 0;
    return hipGetDeviceCount(&n) == hipSuccess && n > 0;
}

}  // extern "C"

// ------------------------------------------------------------ device facts
#include "q4mi_common.h"

namespace q4mi {

int cu_count() {
    static int n = 0;
    if (!n) {
        int dev = 0, v = 0;
        if (hipGetDevice(&dev) == hipSuccess &&
            hipDeviceGetAttribute(&v, hipDeviceAttributeMultiprocessorCount, dev) == hipSuccess &&
            v > 0)
            n = v;
        else
            n = 256;
    }
    return n;
}

}  // namespace q4mi
