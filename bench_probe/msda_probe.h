/*
 * bench_probe/libmsda_probe.so: measurement probes for bench.py, not part of the
 * MSDA library or its drop-in boundary (no counterpart in the reference). bench.py
 * uses them to state the ceilings the MSDA kernels are rated against.
 */
#ifndef MSDA_PROBE_H_
#define MSDA_PROBE_H_

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Random row gathers: `blocks` workgroups of 256 threads on `stream` (a
 * hipStream_t). Each lane makes iters * 8 loads of 16 bytes; row_bytes / 16 lanes
 * (4 for 64-byte rows, 8 for 128-byte rows) fetch one pseudo-random row of `buffer`
 * (rows * row_bytes bytes, rows a power of two, device memory) per load, so a wave
 * load gathers 1 KiB either way. `sink` (device memory) takes one uint32 per
 * thread. Returns 0, or 1 for bad arguments (row_bytes other than 64 or 128) or a
 * failed launch. */
int msda_probe_row_gather(const void* buffer, int64_t rows, int row_bytes, int blocks, int iters, void* sink,
                          void* stream);

#ifdef __cplusplus
}
#endif

#endif /* MSDA_PROBE_H_ */
