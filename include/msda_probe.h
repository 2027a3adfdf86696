/*
 * libmsda_probe.so: measurement probes for the MSDA library, not part of its drop-in
 * boundary (no counterpart in the reference). bench.py uses them to state the
 * ceilings the MSDA kernels are rated against.
 */
#ifndef MSDA_PROBE_H_
#define MSDA_PROBE_H_

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Random 64-byte row gathers: `blocks` workgroups of 256 threads on `stream` (a
 * hipStream_t), each wave fetching iters * 8 rows of `buffer` (rows * 64 bytes, rows
 * a power of two, device memory) with one 16-byte load per lane, 4 lanes a row.
 * `sink` (device memory) takes one uint32 per thread. Returns 0, or 1 for bad
 * arguments or a failed launch. */
int msda_probe_row_gather(const void* buffer, int64_t rows, int blocks, int iters, void* sink,
                          void* stream);

#ifdef __cplusplus
}
#endif

#endif /* MSDA_PROBE_H_ */
