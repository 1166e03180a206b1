/*
 * moa_bench.h -- measurement support for bench.py (no counterpart in the reference).
 */
#ifndef MOA_BENCH_H
#define MOA_BENCH_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Reads `bytes` (a multiple of 16) from device memory src with `workgroups` workgroups of
 * `threads` threads: workgroup b streams the b-th contiguous slice, each wave 1 KB per load
 * instruction with eight loads in flight per lane (non-temporal). Writes nothing (sink, a device
 * uint32, is only a guard that keeps the loads). bytes = 0 launches the same grid doing nothing:
 * the launch floor of that shape. Asynchronous on `stream`. */
int moa_bench_stream_read(const void* src, uint64_t bytes, int workgroups, int threads, uint32_t* sink, void* stream);

#ifdef __cplusplus
}
#endif
#endif
