/* Register-only matrix-core rate probe (libseqattn_probe.so).
 *
 * No counterpart in the reference: bench.py calls it to report the sustained
 * bf16 MFMA rate of the GPU it runs on beside the update kernel's rate.  It is
 * not part of the attention path and the attention library does not use it.
 */
#ifndef SEQATTN_PROBE_H
#define SEQATTN_PROBE_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Floats the output buffer of sa_probe_mfma must hold (one per thread). */
int64_t sa_probe_mfma_out_elems(void);

/* bf16 MFMA FLOP of one probe launch (2 * M * N * K per MFMA). */
double sa_probe_mfma_flop_per_launch(void);

/* Enqueue `launches` probe launches on `stream` (a hipStream_t, may be null
 * for the null stream).  `out` is device memory of at least
 * sa_probe_mfma_out_elems() floats.  Returns 0, -1 on a bad argument (nothing
 * enqueued) or -2 when a launch fails. */
int32_t sa_probe_mfma(float* out, int64_t out_elems, int32_t launches, uint32_t seed, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* SEQATTN_PROBE_H */
