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

static bool grow(void **p, size_t bytes, const char *what) {
    void *n = nullptr;
    if (hipMalloc(&n, bytes) != hipSuccess) {
        set_error("%s: hipMalloc(%zu) failed", what, bytes);
        return false;
    }
    if (*p) (void)hipFree(*p);
    *p = n;
    return true;
}

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

const char *q4mi_status_text(uint32_t bits) {
    static char buf[256];
    if (!bits) return "ok";
    if (bits & 0x80000000u) return "device status not readable";
    snprintf(buf, sizeof buf, "decode kernel gave up a bounded wait (%s%s%s): results of the "
             "calls since the last status check are wrong",
             (bits & 1u) ? "consumer" : "", (bits & 3u) == 3u ? ", " : "",
             (bits & 2u) ? "producer" : "");
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
