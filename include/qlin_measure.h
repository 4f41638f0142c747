/* Measurement helper, not part of the quantized linear library's ABI:
 * libqlin_measure.so, built beside libqlinear.so and loaded only by
 * bench.py and its tests. No counterpart in the reference. */
#ifndef QLIN_MEASURE_H
#define QLIN_MEASURE_H

#include <stddef.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef void *qlm_stream_t; /* hipStream_t; NULL = the default stream */

/* Streaming-read ceiling that the decode GEMMs are measured against. Reads
 * `bytes` (a nonzero multiple of 16) at 16-byte aligned `src` once with
 * 16-byte non-temporal loads, 512 workgroups of 512 threads; writes nothing
 * except, never in practice, to `sink` (NULL, or room for 512 unsigned
 * values: a workgroup stores its xor only if it equals one fixed constant,
 * which keeps the loads live). Returns 0, -1 for invalid arguments, -5 when
 * the launch fails. */
int qlm_stream_read(const void *src, size_t bytes, unsigned *sink, qlm_stream_t stream);

#ifdef __cplusplus
}
#endif

#endif
