/* Test-only harness around the reference's own CPU expert path.
 *
 * This file is checker infrastructure.  It is compiled (by oracle/Makefile,
 * target `ref`) together with the reference sources where they lie under
 * /root/reference/src, into oracle/_ref/libq4ref.so, which is never
 * committed.  Only tests/, the golden-vector generator and bench.py's
 * cpu_baseline leg load it.  Nothing on the product path links it.
 *
 * The reference's expert store (src/q4_expert.c) is not compiled: it owns a
 * DRAM cache, GGUF reads and GPU residency.  Instead the two lookups the CPU
 * path makes into it -- q4_expert_parts (src/q4_expert.c:962-982) and
 * q4_expert_host_ptr (src/q4_expert.c:1710-1725) -- are answered here from a
 * caller-provided packed arena (gate | up | down per expert, the byte layout
 * q4_expert_parts defines), i.e. every expert is "resident".
 *
 * Exported entry points wrap:
 *   cpx_quant8          src/q4_cpuexp.c:605-637
 *   cpx_dot8 / 8n       src/q4_cpuexp.c:1699-1719, :1962-1979
 *   q4_cpuex_dispatch2  src/q4_cpuexp.c:2503-2611  (+ q4_cpuex_join_tag)
 *   q4_cpuex_dispatch_win src/q4_cpuexp.c:2618-2753
 *   q4_softmax/q4_topk  src/q4_quant.c:715-755
 *   q4_cpx_selftest     src/q4_cpuexp.c:2875-3002
 */
#include "q4_cpuexp.c"

#include <omp.h>

static q4_gguf h_g;
static q4_tensor h_t[3];
static const uint8_t *h_base;
static uint64_t h_stride;

bool q4_expert_parts(const q4_gguf *g, int32_t layer, const q4_tensor **gate,
                     const q4_tensor **up, const q4_tensor **down,
                     uint64_t *off_gate, uint64_t *off_up, uint64_t *off_down,
                     uint64_t *total) {
    (void)g;
    (void)layer;
    const uint64_t sg = h_t[0].nbytes / (uint64_t)h_t[0].n_experts;
    const uint64_t su = h_t[1].nbytes / (uint64_t)h_t[1].n_experts;
    const uint64_t sd = h_t[2].nbytes / (uint64_t)h_t[2].n_experts;
    if (gate) *gate = &h_t[0];
    if (up) *up = &h_t[1];
    if (down) *down = &h_t[2];
    if (off_gate) *off_gate = 0;
    if (off_up) *off_up = sg;
    if (off_down) *off_down = sg + su;
    if (total) *total = sg + su + sd;
    return true;
}

const uint8_t *q4_expert_host_ptr(const q4_expert_cache *c, int32_t layer,
                                  int32_t eid) {
    (void)c;
    (void)layer;
    return h_base + (uint64_t)eid * h_stride;
}

static void h_setup(uint32_t n_embd, uint32_t n_ff, uint32_t t_gu,
                    uint32_t t_d, uint32_t n_exp, const uint8_t *base,
                    uint64_t stride) {
    memset(&h_g, 0, sizeof h_g);
    h_g.n_embd = n_embd;
    h_g.n_ff_exp = n_ff;
    const uint64_t rg = q4_row_bytes(t_gu, n_embd);
    const uint64_t rd = q4_row_bytes(t_d, n_ff);
    for (int i = 0; i < 3; i++) {
        memset(&h_t[i], 0, sizeof h_t[i]);
        h_t[i].n_experts = (int32_t)n_exp;
    }
    h_t[0].ggml_type = h_t[1].ggml_type = t_gu;
    h_t[0].ne[0] = h_t[1].ne[0] = n_embd;
    h_t[0].ne[1] = h_t[1].ne[1] = n_ff;
    h_t[0].nbytes = h_t[1].nbytes = rg * n_ff * n_exp;
    h_t[2].ggml_type = t_d;
    h_t[2].ne[0] = n_ff;
    h_t[2].ne[1] = n_embd;
    h_t[2].nbytes = rd * n_embd * n_exp;
    h_base = base;
    h_stride = stride;
}

/* x[n] -> q[n] int8, d[n/32] fp32, bs[n/32] int32. */
int qref_quant8(const float *x, uint64_t n, int8_t *q, float *d, int32_t *bs) {
    if (n % 32) return 0;
    cpx_q8 *o = (cpx_q8 *)malloc((n / 32) * sizeof(cpx_q8));
    if (!o) return 0;
    cpx_quant8(x, n, o);
    for (uint64_t g = 0; g < n / 32; g++) {
        memcpy(q + 32 * g, o[g].q, 32);
        d[g] = o[g].d;
        bs[g] = o[g].bs;
    }
    free(o);
    return 1;
}

/* y[t][r] = cpx_dot8n(row r, q8(x[t])) for nt tokens (nt == 1: cpx_dot8).
 * threads > 1 splits rows with OpenMP (each row is independent). */
int qref_dot8_rows(uint32_t type, const uint8_t *w, uint64_t rows, uint64_t n,
                   const float *x, uint32_t nt, float *y, int threads) {
    if (n % 32 || !nt || nt > CPX_DQ8N_MAX) return 0;
    const uint64_t rb = q4_row_bytes(type, n);
    if (!rb) return 0;
    const uint64_t ng = n / 32;
    /* the sign-expansion table the IQ2/IQ3_XXS kernels read, set up by the
     * reference's dispatchers before their first dot (src/q4_cpuexp.c:2595) */
    cpx_esigns_init();
    cpx_q8 *xq = (cpx_q8 *)malloc(nt * ng * sizeof(cpx_q8));
    if (!xq) return 0;
    for (uint32_t t = 0; t < nt; t++) cpx_quant8(x + t * n, n, xq + t * ng);
    const cpx_q8 *xs[CPX_DQ8N_MAX];
    for (uint32_t t = 0; t < nt; t++) xs[t] = xq + t * ng;
    int ok = 1;
#pragma omp parallel for num_threads(threads > 0 ? threads : 1) schedule(static)
    for (uint64_t r = 0; r < rows; r++) {
        float o[CPX_DQ8N_MAX];
        if (!cpx_dot8n(type, w + r * rb, xs, nt, n, o)) ok = 0;
        for (uint32_t t = 0; t < nt; t++) y[t * rows + r] = o[t];
    }
    free(xq);
    return ok;
}

/* One decode MoE job on the reference worker pool; y is zeroed and filled. */
int qref_moe_decode(uint32_t n_embd, uint32_t n_ff, uint32_t t_gu,
                    uint32_t t_d, uint32_t n_exp, const uint8_t *base,
                    uint64_t stride, const float *x, const int32_t *ids,
                    const float *wts, uint32_t k, float *y) {
    h_setup(n_embd, n_ff, t_gu, t_d, n_exp, base, stride);
    static q4_expert_cache *c_dummy = (q4_expert_cache *)&h_g;
    uint64_t tag = 0;
    int s;
    while ((s = q4_cpuex_dispatch2(&h_g, c_dummy, 0, x, ids, wts, k, y,
                                   &tag)) == -1)
        q4_cpuex_retire();
    if (s < 0) return 0;
    return q4_cpuex_join_tag(s, tag) ? 1 : 0;
}

/* One 2..8 token window job; ids/wts concatenated in token order, tn[t]
 * per-token counts; y token-major [n_tok][n_embd]. */
int qref_moe_win(uint32_t n_embd, uint32_t n_ff, uint32_t t_gu, uint32_t t_d,
                 uint32_t n_exp, const uint8_t *base, uint64_t stride,
                 const float *x, uint32_t n_tok, const int32_t *ids,
                 const float *wts, const uint32_t *tn, float *y) {
    h_setup(n_embd, n_ff, t_gu, t_d, n_exp, base, stride);
    static q4_expert_cache *c_dummy = (q4_expert_cache *)&h_g;
    uint64_t tag = 0;
    int s;
    while ((s = q4_cpuex_dispatch_win(&h_g, c_dummy, 0, x, n_tok, ids, wts,
                                      tn, y, &tag)) == -1)
        q4_cpuex_retire();
    if (s < 0) return 0;
    return q4_cpuex_join_tag(s, tag) ? 1 : 0;
}

/* Host routing: q4_softmax then q4_topk(..., renormalize = true). */
void qref_softmax_topk(const float *logits, uint32_t n, uint32_t k,
                       int32_t *ids, float *wts) {
    float *p = (float *)malloc(n * sizeof(float));
    memcpy(p, logits, n * sizeof(float));
    q4_softmax(p, n);
    q4_topk(p, n, k, ids, wts, true);
    free(p);
}

int qref_selftest(void) { return q4_cpx_selftest(); }
int qref_has512(void) { return cpx_has512(); }
int qref_threads(void) { return cpx_threads(); }
