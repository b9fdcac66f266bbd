/*
 * sas_probe.h - measurement probes of libsas_probe.so (gfx950).
 *
 * Not part of the sampling library's ABI and no counterpart in the
 * reference: bench.py loads this library to measure the streaming bound
 * that the sampling kernels run against.  Each call is one launch on
 * `stream` (a hipStream_t; NULL is HIP's null stream) and returns 0, or a
 * nonzero hipError_t / -1 for a bad argument.
 */
#ifndef SAS_PROBE_H
#define SAS_PROBE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Reads `bytes` (a multiple of 16) at `src` (16-byte aligned) with the
 * parts kernel's access pattern and no other work: `blocks` blocks of 256
 * threads, each a contiguous share, 16-byte nontemporal loads, eight per
 * thread in flight.  `sink`: device, 256 floats, written only with an
 * impossible value (it keeps the loads alive). */
int sasp_read(const void *src, size_t bytes, int32_t blocks, float *sink, void *stream);

/* One pass over `rows` rows of `vocab` fp32 logits (vocab a multiple of
 * 8192) and their packed masks ([rows][vocab / 32] u32), one block per
 * 8192 ids: each thread loads the mask words of its eight float4s, then
 * the float4s, and folds the allowed values into a maximum.
 *   mode 0: every float4 is loaded, the loads issued with the mask's;
 *   mode 5: every float4 is loaded, after the mask words arrived;
 *   modes 1, 4, 3, 2: a float4 is loaded only when its 16-, 32-, 64- or
 *   128-byte aligned span of ids holds an allowed id.
 * `sink` as for sasp_read. */
int sasp_masked_read(const float *logits, const uint32_t *mask, int32_t rows, int32_t vocab, int32_t mode,
                     float *sink, void *stream);

/* Whether hipMemset, which runs on the null stream, is ordered before a
 * kernel launched right after it on a non-blocking stream: `reps` times, a
 * buffer of `bytes` filled with 0xFF (finished), then hipMemset to 0 and at
 * once a kernel on a non-blocking stream that reads 128 of its words.
 * Allocates its own buffers and stream. */
typedef struct sasp_memset_result {
  int32_t reps;
  int32_t stale_runs; /* runs whose kernel read a word the fill had not reached */
  double host_us;     /* average host time of the hipMemset call */
  double fill_us;     /* the same fill, timed on a stream with events */
} sasp_memset_result;
int sasp_memset_order(size_t bytes, int32_t reps, sasp_memset_result *out);

#ifdef __cplusplus
}
#endif

#endif /* SAS_PROBE_H */
