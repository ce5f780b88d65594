/* Per-wave timestamps of the decode step: entry points of the profiling build
 * build/librtxllm_timeline.so only (the library proper does not export
 * them). They have no counterpart in the reference, whose profiling is
 * Nsight's; they are for bench.py --timeline and similar tools.
 *
 * The profiling build records s_memrealtime (100 MHz, 10 ns per count, one
 * clock for every CU) per wave at fixed points of the decode step's kernels
 * (batch 1 and the batch launches) into 32 regions x 65536 slots; a launch
 * overwrites the slots of its kernel role, so after one step the array
 * describes the last layer (region and slot layout: csrc/timeline.h). */
#ifndef RTXLLM_TIMELINE_H
#define RTXLLM_TIMELINE_H

#include <hip/hip_runtime_api.h>
#include <stddef.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Copies the whole record, count = 32 * 65536 entries, to host memory; waits
 * for the device copies (not capture-safe). */
hipError_t rtxllm_timeline_read(unsigned long long* host, size_t count);
/* Zeroes every slot (synchronous). */
hipError_t rtxllm_timeline_clear(void);

#ifdef __cplusplus
}
#endif

#endif
