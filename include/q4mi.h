/* q4mi.h -- C ABI of the MI355X (gfx950) routed-expert matmul library.
 *
 * Drop-in for the quantized routed-expert path of the reference engine's
 * q4.h: the reference's C host (src/q4_moe.c) links these names unchanged in
 * place of the dispatch in src/q4_rocm.cu / src/q4_mmq.cu / src/q4_mmvq.cu.
 * Plain pointers and sizes only; every pointer named d_* is device memory.
 * All launches are asynchronous on the stream returned by q4_hip_stream().
 * A false return means "not covered / bad arguments": nothing was launched
 * (the reference's reject-before-launch contract, src/q4_rocm.cu:5433-5438),
 * and q4mi_last_error() says why.
 *
 * Weight formats: IQ3_S (ggml type 21, 110-byte superblocks of 256 values)
 * and Q8_0 (type 8, 34-byte blocks of 32).  Experts are resident at
 * base + slot*stride as gate[n_ff][in_dim] | up[n_ff][in_dim] |
 * down[n_embd][n_ff] (reference src/q4_expert.c:962-982).
 */
#ifndef Q4MI_H
#define Q4MI_H

#include <stdbool.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ---------------------------------------------------------------- runtime */

/* Stream of every launch.  Replaces q4_hip_stream (src/q4.h:1137,
 * src/q4_rocm.cu:852). */
void *q4_hip_stream(void);
/* Select the launch stream (hipStream_t; NULL = the default stream).  No
 * reference counterpart: the reference owned one global stream.  The
 * library's scratch (fp32 h, the device-list plan, the staged list, the MMQ
 * buffers) exists once per process, so calls must stay ordered on this one
 * stream: calls from several host threads or streams at once race. */
void q4mi_set_stream(void *stream);
/* Text of the last rejection or launch failure. */
const char *q4mi_last_error(void);
/* 1 when a HIP device is visible. */
int q4mi_device_ok(void);

/* ------------------------------------------------------- q8 activations */

/* Bit-exact CPU-expert quantizer (cpx_quant8, src/q4_cpuexp.c:605-637) on
 * the GPU: rows of `cols` fp32 (row r = x[ids ? ids[r] : r]) -> int8 codes
 * q[rows][cols], fp32 scales d[rows][cols/32], int32 code sums
 * bs[rows][cols/32] (bs may be NULL).  cols % 32 == 0. */
bool q4mi_quant8(const float *d_x, const int32_t *d_ids, uint64_t rows, uint64_t cols,
                 int8_t *d_q, float *d_d, int32_t *d_bs);

/* ---------------------------------------------------------- dense MMVQ */

/* Replaces q4_mmvq_on/_set/_verify/_warm/_hold/_release/q4_mmvq_n
 * (src/q4.h:914-927, src/q4_mmvq.cu:266-349), extended to IQ3_S and Q8_0:
 * y[t*nrows + r] = scale * (W_r . q8(x_t)), t < n (1..8).  A row's result
 * does not depend on n.  ncols/32 in {8,16,32,64,128,256} or 20 / 80 (the
 * reference model's 640 and 2560). */
int q4_mmvq_on(void);
void q4_mmvq_set(int v);
void q4_mmvq_verify(int on);
void q4_mmvq_warm(void);
void q4_mmvq_hold(const float *d_x);
void q4_mmvq_release(void);
bool q4_mmvq_n(uint32_t ty, const uint8_t *d_w, uint64_t nrows, uint64_t ncols,
               const float *d_x, float *d_y, float scale, uint32_t n);
/* Pre-quantized activations (the q4mi_quant8 layout); d_sums (optional)
 * receives the exact int32 group sums (2s+1)*sum(w*q) at
 * [(t*nrows + r)*(ncols/32) + g].  No reference counterpart (debug export of
 * the per-block accumulators the CPU path keeps in registers,
 * src/q4_cpuexp.c:855-892). */
bool q4mi_mmvq(uint32_t ty, const uint8_t *d_w, uint64_t nrows, uint64_t ncols,
               const int8_t *d_xq, const float *d_xd, uint32_t n, float *d_y, float scale,
               int32_t *d_sums);

/* ------------------------------------------------- routed-expert decode */

/* Size library scratch before any graph capture (src/q4.h:958). */
void q4_hip_moe_scratch_warm(void);
/* Drain the library stream and return the decode kernels' timeout word: 0
 * when every bounded in-kernel wait completed; otherwise a wait gave up and
 * the results of the decode calls since the last check are wrong (the bits
 * are described by q4mi_status_text, which also becomes q4mi_last_error()).
 * clear != 0 resets the word.  No reference counterpart (the reference's
 * kernels have no bounded waits). */
uint32_t q4mi_device_status(int clear);
const char *q4mi_status_text(uint32_t bits);
/* Copy the fp32 h = silu(gate.q8(x)) * (up.q8(x)) of the last decode call,
 * [64 unique experts][8 tokens][n_ff], unique experts in first-appearance
 * order, to d_dst (device) on the library stream.  Debug export (the
 * reference keeps h in the caller's d_h, src/q4_rocm.cu:5444-5455). */
bool q4mi_moe_copy_h(float *d_dst, uint32_t n_ff);
/* One token; slots/wts are HOST arrays of n <= 64 experts.
 * d_y[r] += sum_e wts[e] * down_e(q8(silu(gate_e.q8(x)) * up_e.q8(x))).
 * gt == ut; IQ3_S or Q8_0; in_dim == n_embd.  d_h, d_h2, d_down are
 * accepted for ABI compatibility and unused.  Replaces q4_hip_moe_exec
 * (src/q4.h:951-956, src/q4_rocm.cu:5425-5470). */
bool q4_hip_moe_exec(const uint8_t *base, uint64_t stride, const int32_t *slots,
                     const float *wts, uint32_t n, uint32_t gt, uint64_t og, uint32_t ut,
                     uint64_t ou, uint32_t dt, uint64_t od, const float *d_x, float *d_h,
                     float *d_h2, float *d_down, float *d_y, uint32_t n_ff, uint32_t in_dim,
                     uint32_t n_embd);
/* q4_hip_moe_exec that allocates nothing, for callers that cannot allocate
 * (code under graph capture, serving loops that forbid hipMalloc): its
 * intermediates (fp32 h and the list plan) live in a file-scope device
 * array of 2 MiB + 4 KB per GPU, held until the process ends, so n_ff <=
 * 1024 (larger is rejected before any launch).  No counterpart in the
 * reference.  Calls that overlap on one GPU share that array and race; d_y
 * is accumulated as by q4_hip_moe_exec (same kernels, same bits). */
bool q4mi_moe_exec_noalloc(const uint8_t *base, uint64_t stride, const int32_t *slots,
                           const float *wts, uint32_t n, uint32_t gt, uint64_t og, uint32_t ut,
                           uint64_t ou, uint32_t dt, uint64_t od, const float *d_x, float *d_y,
                           uint32_t n_ff, uint32_t in_dim, uint32_t n_embd);
/* Same with device lists (count d_nhit[0]); graph-capturable.  Replaces
 * q4_hip_moe_exec_dev (src/q4.h:1295-1301, src/q4_rocm.cu:6570-6608). */
bool q4_hip_moe_exec_dev(const uint8_t *base, uint64_t stride, const int32_t *d_es,
                         const float *d_ew, const int32_t *d_nhit, uint32_t gt, uint64_t og,
                         uint32_t ut, uint64_t ou, uint32_t dt, uint64_t od, const float *d_x,
                         float *d_h, float *d_h2, float *d_down, float *d_y, uint32_t n_ff,
                         uint32_t in_dim, uint32_t n_embd);
/* Verify window, 2..8 tokens; token t's picks at d_es/d_ew[t*64 ..
 * t*64 + d_nh[t]); experts picked by several tokens are read once.  x, y
 * token-major.  Replaces q4_hip_moe_win_ok / q4_hip_moe_exec_win
 * (src/q4.h:906-913, src/q4_rocm.cu:7369-7531); covers every IQ3_S/Q8_0
 * layer (the reference required an IQ4_NL/Q2_0 down).  Gate/up types: IQ3_S,
 * Q8_0 and the reference window's IQ2_XXS, IQ2_XS, IQ2_S, IQ3_XXS, IQ4_XS;
 * down: IQ3_S, Q8_0, IQ4_NL, Q2_0, IQ2_S.  At most 64 (token, pick) entries
 * per call: entries past the 64th are not read. */
bool q4_hip_moe_win_ok(uint32_t gt, uint32_t ut, uint32_t dt, uint32_t in_dim, uint32_t n_ff,
                       uint32_t n_tok);
bool q4_hip_moe_exec_win(const uint8_t *base, uint64_t stride, const int32_t *d_es,
                         const float *d_ew, const int32_t *d_nh, uint32_t n_tok, uint32_t gt,
                         uint64_t og, uint32_t ut, uint64_t ou, uint32_t dt, uint64_t od,
                         const float *d_x, float *d_h, float *d_y, uint32_t n_ff,
                         uint32_t in_dim, uint32_t n_embd);
/* Decode (n_tok 1) or verify window (2..8) over the GGUF expert layout:
 * gate, up and down are separate stacked tensors (blk.N.ffn_gate_exps,
 * ffn_up_exps, ffn_down_exps), expert e's matrices at gate + e*gu_stride,
 * up + e*gu_stride and down + e*d_stride (gate/up type gt, down type dt).
 * Device lists and y as q4_hip_moe_exec_win.  The slices are the ones the
 * reference's expert loader reads (q4_expert_parts, src/q4_expert.c:
 * 962-982); a shared expert joins the lists once it is placed at index
 * n_exp of the stacked tensors.  No reference counterpart (the reference
 * packed experts into cache slots first). */
bool q4mi_moe_exec_parts(const uint8_t *gate, const uint8_t *up, const uint8_t *down,
                         uint64_t gu_stride, uint64_t d_stride, const int32_t *d_es,
                         const float *d_ew, const int32_t *d_nh, uint32_t n_tok, uint32_t gt,
                         uint32_t dt, const float *d_x, float *d_y, uint32_t n_ff,
                         uint32_t in_dim, uint32_t n_embd);
/* Per-token small batch: token t's picks at d_slots/d_wts[h_off[t] ..
 * h_off[t+1]) (device arrays, host prefix offsets), x and y token-major, y
 * accumulated; nothing is queued when false is returned.  Equal counts run
 * as one window.  d_h, d_h2 unused.  Replaces q4_hip_moe_tok_ok /
 * q4_hip_moe_exec_tok (src/q4.h:893-901, src/q4_rocm.cu:5606-5657). */
bool q4_hip_moe_tok_ok(uint32_t gt, uint32_t ut, uint32_t dt, uint32_t in_dim, uint32_t n_ff);
bool q4_hip_moe_exec_tok(const uint8_t *base, uint64_t stride, const int32_t *d_slots,
                         const float *d_wts, const uint32_t *h_off, uint32_t n_tok, uint32_t gt,
                         uint64_t og, uint32_t ut, uint64_t ou, uint32_t dt, uint64_t od,
                         const float *d_x, float *d_h, float *d_h2, float *d_y, uint32_t n_ff,
                         uint32_t in_dim, uint32_t n_embd);
/* Staged list for graphs: q4_hip_moe_stage copies one token's host list
 * (n <= 64) into pinned memory; q4_hip_moe_exec_staged is q4_hip_moe_exec_dev
 * over that memory, read when the kernels run, so a captured graph replays
 * with the list staged last.  Do not restage while a launch reading the
 * previous list is queued.  Replaces q4_hip_moe_stage /
 * q4_hip_moe_exec_staged (src/q4.h:1306-1311, src/q4_rocm.cu:7548-7590). */
bool q4_hip_moe_stage(const int32_t *slots, const float *wts, uint32_t n);
bool q4_hip_moe_exec_staged(const uint8_t *base, uint64_t stride, uint32_t gt, uint64_t og,
                            uint32_t ut, uint64_t ou, uint32_t dt, uint64_t od,
                            const float *d_x, float *d_h, float *d_h2, float *d_down,
                            float *d_y, uint32_t n_ff, uint32_t in_dim, uint32_t n_embd);

/* ------------------------------------------------------ routing and pack */

/* Per-token softmax + top-k + renormalisation (q4_softmax + q4_topk,
 * src/q4_quant.c:715-755); n_exp <= 512, topk 1..64.  Replaces
 * q4_hip_route_pf (src/q4.h:1278-1280, src/q4_rocm.cu:6383-6549). */
bool q4_hip_route_pf(const float *d_rlog, int32_t *d_ids, float *d_wts, uint32_t n_tok,
                     uint32_t n_exp, uint32_t topk);
/* Device routing of a decode / verify batch, the reference's entry
 * (src/q4.h:1285-1294, src/q4_rocm.cu:6106-6283, called from
 * src/q4_moe.c:2439): per token t < n_tok the softmax top-k of
 * d_rlog[t][n_exp] (bit-exact with q4_hip_route_pf), each pick mapped
 * through devtab (expert -> arena slot, < 0 = not resident).  Hits: slots
 * and renormalised weights at d_es/d_ew[t*64 + i], count d_nh[t] (the device
 * lists q4_hip_moe_exec_win / _dev read).  Misses: published through `mail`,
 * the reference's q4_mail_t prefix (ids/wts/rk in token order, n, ntok,
 * tn[8], hs[8*16] hit slots, hn[8], routed[16] and rseq when d_rseq is
 * given, then seq = ++*d_seq).  With every expert resident the miss list is
 * empty.  d_prof (optional): [0] += the kernel's wall-clock ticks (100 MHz),
 * [1] += 1.  n_exp <= 1024, n_tok 1..8, topk 1..16, n_tok * topk <= 64. */
bool q4_hip_route_dev_n(const float *d_rlog, const int32_t *devtab, int32_t *d_es, float *d_ew,
                        int32_t *d_nh, void *mail, unsigned long long *d_seq,
                        unsigned long long *d_rseq, unsigned long long *d_prof,
                        uint32_t n_exp, uint32_t topk, uint32_t n_tok);
/* Single token variants (src/q4.h:1414-1418, src/q4_rocm.cu:12703-12789). */
bool q4_hip_softmax_topk_launch(const float *d_logits, uint32_t n, uint32_t k, int32_t *d_ids,
                                float *d_wts);
bool q4_hip_softmax_topk(const float *d_logits, uint32_t n, uint32_t k, int32_t *h_ids,
                         float *h_wts);
/* Router front of a MoE layer, one entry for decode, verify windows and
 * prefill: logits[t][e] = W_r[e] . x[t] (the router GEMV; W_r is n_exp rows
 * of n_embd in F32 (type 0), F16 (1) or BF16 (30), dot order fixed so the
 * logits reproduce bit for bit), then softmax + top-k + renormalisation as
 * q4_hip_route_pf into ids/wts rows of ostride entries.  With d_sgw (the
 * shared expert's gate vector, fp32 [n_embd]) also d_sg[t] =
 * sigmoid(d_sgw . x[t]).  With shared_slot >= 0 each token's row gets one
 * more entry after its topk picks: expert shared_slot with weight d_sg[t]
 * (1 without a gate), so the shared expert runs inside the same decode /
 * window launch; d_nh (optional) receives the per-token entry counts.  With
 * ostride 64 the rows are the device lists of q4_hip_moe_exec_win /
 * q4_hip_moe_exec_dev.  n_exp <= 512, topk <= 64, n_embd % 256 == 0 and <=
 * 16384, pointers 16-byte aligned.  Replaces the router q4_hip_gemv_dd +
 * q4_hip_moe_pack sgate dot + route_dev_n_k sequence of q4_moe_gpu_a /
 * q4_moe_gpu_dev (src/q4_moe.c:1360-1440, src/q4_rocm.cu:5930-6060,
 * :15967-15990); the gate is applied as y += sg * shared
 * (src/q4_moe.c:297-306). */
bool q4mi_moe_route(const void *d_wr, uint32_t wr_type, const float *d_sgw, const float *d_x,
                    uint32_t n_tok, uint32_t n_embd, uint32_t n_exp, uint32_t topk,
                    float *d_logits, int32_t *d_ids, float *d_wts, int32_t *d_nh,
                    uint32_t ostride, int32_t shared_slot, float *d_sg);
/* One token's routed decode layer in three launches: q4mi_moe_route's
 * router GEMV (d_logits, and d_sg with a gate vector), then the device-list
 * decode layer of q4_hip_moe_exec_dev whose gate/up blocks take the top-k of
 * d_logits themselves (the same code as q4mi_moe_route's top-k launch, so
 * the same picks and weights bit for bit) instead of a fourth launch.  The
 * lists are still written, with ostride 64 (d_ids, d_wts, d_nh: all three or
 * none).  Arguments as q4mi_moe_route (n_tok 1) and q4_hip_moe_exec_dev
 * (in_dim = n_embd); topk + (shared_slot >= 0) <= 64.  No reference
 * counterpart: it fuses the route_dev_n_k launch of q4_moe_gpu_dev
 * (src/q4_moe.c:2439) into the layer. */
bool q4mi_moe_route_exec(const void *d_wr, uint32_t wr_type, const float *d_sgw,
                         const float *d_x, uint32_t n_embd, uint32_t n_exp, uint32_t topk,
                         float *d_logits, int32_t *d_ids, float *d_wts, int32_t *d_nh,
                         int32_t shared_slot, float *d_sg, const uint8_t *base, uint64_t stride,
                         uint32_t gt, uint64_t og, uint32_t ut, uint64_t ou, uint32_t dt,
                         uint64_t od, float *d_y, uint32_t n_ff);
/* d_y[t] += sigmoid(d_w . d_x[t]) * d_sh[t], t < n_tok: the shared
 * expert's gate applied to its separately computed output, one launch.
 * Replaces q4_hip_sgate_axpy (src/q4.h:1129-1131, src/q4_rocm.cu:15775-15800;
 * src/q4_moe.c:2177).  The dot is q4mi_moe_route's fixed order (so sg has the
 * same bits as its d_sg) for n % 256 == 0 and 16-byte aligned d_w, d_x;
 * any other n or alignment adds the remaining elements lane-strided (any n
 * >= 1, as the reference). */
bool q4_hip_sgate_axpy(float *d_y, const float *d_sh, const float *d_w, const float *d_x,
                       uint32_t n, uint32_t n_tok);
/* *out = sigmoid(a . b) (the one-token sgate scalar).  Replaces
 * q4_hip_dot_sigmoid (src/q4.h:975-976, src/q4_rocm.cu:4890).  Any n >= 1
 * and alignment, the dot in q4_hip_sgate_axpy's order. */
bool q4_hip_dot_sigmoid(const float *a, const float *b, float *out, uint32_t n);
/* Stable expert pack per token group: the host order of src/q4_moe.c:
 * 3404-3451 (the reference's GPU assign_pf_k orders by atomic arrival).
 * Replaces q4_hip_assign_pf (src/q4.h:1281-1285, src/q4_rocm.cu:6483-6563). */
bool q4_hip_assign_pf(const int32_t *d_ids, const float *d_wts, int32_t *d_atok,
                      int32_t *d_rsrc, float *d_rw, int32_t *d_stg, uint32_t *d_stgn,
                      uint32_t *d_ek, uint32_t gsz, uint32_t topk, uint32_t n_exp,
                      uint32_t n_tok);
/* Same plus the MMQ expert bounds [n_g][n_exp+1] the reference built on the
 * host (src/q4_moe.c:3558-3571); d_bounds may be NULL. */
bool q4mi_assign(const int32_t *d_ids, const float *d_wts, int32_t *d_atok, int32_t *d_rsrc,
                 float *d_rw, int32_t *d_stg, uint32_t *d_stgn, uint32_t *d_ek,
                 int32_t *d_bounds, uint32_t gsz, uint32_t topk, uint32_t n_exp,
                 uint32_t n_tok);
/* dy[t] += sum_k rw[t,k] * pd[rsrc[t,k]] in k order (deterministic).
 * Replaces q4_hip_expert_reduce (src/q4.h:1087-1089,
 * src/q4_rocm.cu:15739-15761). */
bool q4_hip_expert_reduce(float *d_y, const float *d_pd, const int32_t *d_rsrc,
                          const float *d_rw, uint32_t n_tok, uint32_t topk, uint32_t n_embd);

/* ------------------------------------------------------------ prefill MMQ */

/* Replaces the q4_mmq_* wrapper around vendored ggml MMQ
 * (src/q4.h:1150-1175, src/q4_mmq.cu:250-610).  Types IQ3_S, Q8_0, IQ4_NL,
 * Q2_0, IQ2_S; w_rows % 128 == 0, w_cols % 256 == 0 with whole-dword rows
 * (IQ3_S: w_cols % 512).  Weight buffers must be readable up
 * to the next 4-byte boundary after their last byte (any hipMalloc'd
 * buffer is).  The activation buffer layout is this
 * library's (q4_mmq_q8_bytes gives its size); its codes are the bit-exact
 * CPU-expert q8 codes.  With every expert resident, MMQ reads it in place at
 * w + e*expert_stride_bytes; the expert-gather helpers below serve engines
 * that still stage experts. */
int q4_mmq_on(void);
uint32_t q4_mmq_group(void);
bool q4_mmq_supported(uint32_t type, uint64_t w_rows);
uint64_t q4_mmq_q8_bytes(uint64_t rows, uint64_t cols);
bool q4_mmq_quantize(const float *x, const int32_t *ids, void *xq, uint32_t w_type,
                     uint64_t cols, uint64_t rows);
bool q4_mmq_mul_id(const void *w, uint32_t type, uint64_t w_rows, uint64_t w_cols,
                   uint64_t expert_stride_bytes, uint32_t n_expert, const void *xq,
                   const int32_t *bounds, uint32_t max_rows, uint64_t total_rows, float *dst,
                   uint64_t ld_dst);
bool q4_mmq_swiglu(const float *gu, float *h, uint64_t rows, uint64_t n_ff);
/* Expert-id-indexed weight buffers (src/q4.h:1161-1174,
 * src/q4_mmq.cu:447-601).  q4_mmq_pad: guard bytes after each gathered
 * expert, 0 here (no kernel reads past an expert's rows).  q4_mmq_wbuf:
 * library buffers of n_exp*gu_bytes and n_exp*d_bytes, grown and zeroed on
 * demand (allocates: not during capture).  q4_mmq_wbuf_lend: use caller
 * memory instead (zeroed; NULL drops it) from then on.  q4_mmq_gather: for
 * i < n, slot d_slot[i]'s [goff, +gu_bytes) and [doff, +d_bytes) go to
 * d_gu + d_eid[i]*gu_dst and d_d + d_eid[i]*d_dst, tails zeroed up to the
 * strides.  q4_mmq_wbuf_size / q4_mmq_wbuf_need read the reference's model
 * struct and stay in the host engine. */
uint64_t q4_mmq_pad(uint64_t row_bytes);
bool q4_mmq_wbuf(uint64_t gu_bytes, uint64_t d_bytes, uint32_t n_exp, uint8_t **gu,
                 uint8_t **d);
bool q4_mmq_wbuf_lend(void *gu, uint64_t gu_bytes, void *d, uint64_t d_bytes);
bool q4_mmq_gather(const uint8_t *abase, uint64_t astride, uint64_t goff, uint64_t gu_bytes,
                   uint64_t doff, uint64_t d_bytes, uint64_t gu_dst, uint64_t d_dst,
                   const int32_t *d_eid, const int32_t *d_slot, uint32_t n, uint8_t *d_gu,
                   uint8_t *d_d);
/* q4_mmq_mul_id with activation rows gathered through act_row: xq holds
 * xrows rows (one per token, quantized once) and packed row p reads row
 * act_row[p] (the pack's a_tok).  No reference counterpart: it removes the
 * per-routed-row q8 copy the reference's quantize(x, ids) makes. */
bool q4mi_mmq_mul_id_rows(const void *w, uint32_t type, uint64_t w_rows, uint64_t w_cols,
                          uint64_t expert_stride_bytes, uint32_t n_expert, const void *xq,
                          uint64_t xrows, const int32_t *act_row, const int32_t *bounds,
                          uint64_t total_rows, float *dst, uint64_t ld_dst);
/* Fused gate/up: each expert's [gate; up] (2*n_ff x w_cols) against xq rows
 * (through act_row when given); writes q8(silu(gate)*up) straight into hq
 * (a q4_mmq_q8_bytes(total_rows, n_ff) buffer for the down mul_id).
 * Replaces mul_id(gate|up) + q4_mmq_swiglu + q4_mmq_quantize(h)
 * (src/q4_moe.c:3718-3730).  n_ff % 64 == 0. */
bool q4mi_mmq_gate_up(const void *w, uint32_t type, uint64_t n_ff, uint64_t w_cols,
                      uint64_t expert_stride_bytes, uint32_t n_expert, const void *xq,
                      uint64_t xrows, const int32_t *act_row, const int32_t *bounds,
                      uint64_t total_rows, void *hq);

/* q4mi_mmq_gate_up / q4_mmq_mul_id over n_expert routed experts at
 * w + e*expert_stride_bytes plus one more expert, index n_expert, read from
 * w_extra; bounds has n_expert + 2 entries.  For a shared expert stored apart
 * from the routed arena (src/q4_moe.c:97-103 names its own tensors): its rows
 * (every token, appended after the routed pack) ride in the routed launches.
 * No reference counterpart. */
bool q4mi_mmq_gate_up_x(const void *w, const void *w_extra, uint32_t type, uint64_t n_ff,
                        uint64_t w_cols, uint64_t expert_stride_bytes, uint32_t n_expert,
                        const void *xq, uint64_t xrows, const int32_t *act_row,
                        const int32_t *bounds, uint64_t total_rows, void *hq);
bool q4mi_mmq_mul_id_x(const void *w, const void *w_extra, uint32_t type, uint64_t w_rows,
                       uint64_t w_cols, uint64_t expert_stride_bytes, uint32_t n_expert,
                       const void *xq, const int32_t *bounds, uint64_t total_rows, float *dst,
                       uint64_t ld_dst);
/* q4mi_mmq_gate_up over the GGUF expert layout: expert e's gate matrix at
 * w_gate + e*expert_stride_bytes and its up matrix at w_up +
 * e*expert_stride_bytes (separate stacked tensors); with wx_gate / wx_up
 * (a shared expert's own tensors, both or neither) expert n_expert is that
 * shared expert (bounds then has n_expert + 2 entries).  w_up must sit at
 * the same offset within a dword as w_gate.  No reference counterpart. */
bool q4mi_mmq_gate_up_parts(const void *w_gate, const void *w_up, uint32_t type, uint64_t n_ff,
                            uint64_t w_cols, uint64_t expert_stride_bytes, uint32_t n_expert,
                            const void *xq, uint64_t xrows, const int32_t *act_row,
                            const int32_t *bounds, uint64_t total_rows, void *hq,
                            const void *wx_gate, const void *wx_up);
/* XG prefill: the same routed-expert GEMMs with fp16 activations on the
 * MFMA tiles (weights dequantized to fp16 times 256, fp32 accumulation over
 * the whole K).  Replaces q4_xg_on / _gu_type / _dn_type / _shape_ok /
 * _tile_cap / _tiles / _cvt / _gu / _dn (src/q4.h:1177-1199,
 * src/q4_xg.cu:514-616), same arguments: tiles {first routed row, rows <=
 * 128, slot, expert}, weights at abase + slot*astride + og/ou/od, x16 / h16
 * fp16 rows, q4_xg_gu writes h = silu(gate.x)*(up.x) as fp16 [rows][n_ff],
 * q4_xg_dn writes fp32 [rows][n_embd] for the expert reduce.  Types here:
 * gate/up IQ3_S, Q8_0, IQ2_S; down IQ3_S, Q8_0, IQ4_NL, Q2_0, IQ2_S (the
 * reference's gate/up IQ2_S / IQ3_XXS / IQ3_S / IQ4_XS, down IQ4_NL / Q2_0).  Numerics are the reference XG's, not the q8
 * path's: this is its A/B. */
int q4_xg_on(void);
bool q4_xg_gu_type(uint32_t type);
bool q4_xg_dn_type(uint32_t type);
bool q4_xg_shape_ok(uint32_t n_embd, uint32_t n_ff);
uint32_t q4_xg_tile_cap(uint32_t rows, uint32_t n_exp);
uint32_t q4_xg_tiles(const uint32_t *ek, const uint32_t *ebase, const int32_t *slot,
                     uint32_t n_exp, int32_t *out, uint32_t cap);
bool q4_xg_cvt(const float *x, void *x16, uint64_t n);
bool q4_xg_gu(uint32_t type, const uint8_t *abase, uint64_t astride, uint64_t og, uint64_t ou,
              uint32_t n_embd, uint32_t n_ff, const int32_t *d_tiles, uint32_t n_tiles,
              const void *x16, const int32_t *d_atok, void *h16);
bool q4_xg_dn(uint32_t type, const uint8_t *abase, uint64_t astride, uint64_t od,
              uint32_t n_ff, uint32_t n_embd, const int32_t *d_tiles, uint32_t n_tiles,
              const void *h16, float *out);
/* q4_hip_expert_reduce plus one extra row per token:
 * d_y[t] += sum_k rw*pd[rsrc] + xw[t]*pd[x_row0 + t] (d_xw NULL: weight 1;
 * the reference applies the shared expert's sigmoid gate there,
 * src/q4_moe.c:306).  No reference counterpart. */
bool q4mi_expert_reduce_x(float *d_y, const float *d_pd, const int32_t *d_rsrc,
                          const float *d_rw, uint32_t n_tok, uint32_t topk, uint32_t n_embd,
                          uint64_t x_row0, const float *d_xw);

#ifdef __cplusplus
}
#endif

#endif /* Q4MI_H */
