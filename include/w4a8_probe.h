/*
 * w4a8_probe.h -- measurement probe exported by libw4a8_mi355x.so, not part of the W4A8 path.
 *
 * No counterpart in the reference. bench.py --read-floor uses it to time one launch of a plain
 * streaming-read kernel over B bytes (the floor a decode GEMV call of B weight bytes is read
 * against). Conventions as in w4a8_mi355x.h: device pointers, a hipStream_t as void*, 0 on success.
 */
#ifndef W4A8_PROBE_H
#define W4A8_PROBE_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Read `bytes` (a multiple of 16, under 4 GiB) of buf with 16-byte non-temporal loads,
 * loads_per_thread (1, 4, 8 or 16) per thread and pass, workgroups of `threads` (64, 256, 512 or
 * 1024). grid = 0: a one-shot grid covering the buffer once; grid > 0: that many workgroups striding
 * over it. sink: 4 device bytes a never-taken store may write (it keeps the loads alive). Returns 1
 * on bad arguments, 3 on a launch error. */
int w4a8_probe_read(const void* buf, int64_t bytes, int loads_per_thread, int threads, int grid, uint32_t* sink,
                    void* stream);

#ifdef __cplusplus
}
#endif

#endif
