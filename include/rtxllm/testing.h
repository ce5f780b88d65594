/* Test hooks of the decode library: entry points that let a host-side test
 * force a failure condition while every kernel still runs to its end. They
 * have no counterpart in the reference and are not for production callers. */
#ifndef RTXLLM_TESTING_H
#define RTXLLM_TESTING_H

#include <hip/hip_runtime_api.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* rtxllm_gate_up_silu (rtxllm/decode_kernels.h) with every bounded LDS wait of
 * the 16-wave gate/up workgroup given wait_limit reads (>= 1; production:
 * 2^20) and a target raised by wait_bias (production: 0). A bias no counter
 * reaches makes each wait give up after wait_limit reads, so a test can check
 * that RTXLLM_STATUS_WAIT_TIMEOUT reaches *status; the waves then hand over
 * whatever partials are in LDS and finish their rounds (act is not valid). */
hipError_t rtxllm_test_gate_up_silu_waits(int format, const uint8_t* payload, const uint8_t* meta, const void* xq,
                                          const float* sumsq, uint32_t nslots, float eps, float* act, uint32_t rows,
                                          uint32_t cols, uint32_t* status, uint32_t wait_limit, uint32_t wait_bias,
                                          hipStream_t stream);

#ifdef __cplusplus
}
#endif

#endif
