/* q4mi_measure.h -- hooks of the measurement build of the library
 * (suzuku-engine-q4_amd/lib/libq4mi_meas.so, compiled with -DQ4MI_MEASURE).
 *
 * The product library (libq4mi.so) does not export these: each changes
 * process-global behaviour (a benchmark that runs only one kernel of the
 * decode pair, a test that shrinks the kernels' LDS), which no production
 * caller may reach.  None has a reference counterpart.
 */
#ifndef Q4MI_MEASURE_H
#define Q4MI_MEASURE_H

#include <stdbool.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Which launches of the decode pair run: 1 = gate/up only, 2 = down only,
 * 3 = both (default).  Lets a benchmark time each kernel alone. */
void q4mi_moe_phases(int mask);
/* Cap the decode kernels' LDS at `bytes` (0: all of it), so their LDS rings
 * get reused within a launch. */
void q4mi_moe_lds_cap(uint32_t bytes);
/* One launch of an MFMA throughput probe on the library stream (kind 0:
 * int8 32x32x32, 1: fp16 32x32x16); *ops = the launch's ops, for a
 * caller-timed rate. */
bool q4mi_mfma_probe(int kind, uint32_t iters, uint64_t *ops);
/* One launch of the stream floor probe: one 1024-thread block per CU whose
 * `waves` producer waves copy per_block bytes (src + block * per_block)
 * into LDS with 1 KB global_load_lds_dwordx4 operations and wait for them;
 * per_block = 0 launches the same grid empty.  *bytes = the launch's
 * total.  The floors of the decode kernels' structure. */
bool q4mi_stream_probe(const void *src, uint32_t per_block, uint32_t waves, uint64_t *bytes);
/* One launch of the plain streaming probe, the chip's own floor: `bytes`
 * (a multiple of 4096 * unroll) read from src by 256-thread blocks with
 * `unroll` (1, 4 or 8) 16-byte register loads per thread, nothing written. */
bool q4mi_plain_stream_probe(const void *src, uint64_t bytes, uint32_t unroll);
/* One launch of the prefill MMQ inner-loop A/B (kind 0: exact-integer fp16
 * MFMA, this library's design; 1: int8 MFMA with the per-row (2s+1)
 * multiplier and d_x applied per output), 2 blocks per CU, each wave 32 x
 * 128 outputs over `groups` (a multiple of 8) 32-value groups, operands in
 * LDS; *ops = the launch's integer ops, for a caller-timed rate. */
bool q4mi_mmq_ab_probe(int kind, uint32_t groups, uint64_t *ops);
/* Library device allocations made so far (every allocating path counts). */
uint64_t q4mi_alloc_count(void);
/* The scratch grow policy (no growth inside a stream capture; an outgrown
 * buffer is retired, not freed) run on host fakes without a device; 1 =
 * every case behaves as documented. */
int q4mi_grow_selftest(void);

#ifdef __cplusplus
}
#endif

#endif /* Q4MI_MEASURE_H */
