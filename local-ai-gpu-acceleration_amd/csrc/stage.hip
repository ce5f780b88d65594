// Activation staging entry point: fp32 x (times an optional elementwise weight)
// -> 16-value fixed-point groups consumed by the matvec kernels.
#include "rtxllm/decode_kernels.h"
#include "xq.h"

namespace rtxllm {
namespace {

__global__ __launch_bounds__(256) void stage_kernel(const float* __restrict__ x, const float* __restrict__ mul,
                                                    std::uint32_t groups, XQOut out) {
  const std::uint32_t g = blockIdx.x * blockDim.x + threadIdx.x;
  if (g >= groups) return;
  XG v;
  xg_stage(x, mul, g, v);
  xg_store(out, g, v);
}

}  // namespace
}  // namespace rtxllm

using namespace rtxllm;

extern "C" hipError_t rtxllm_stage_activation(const float* x, const float* weight, std::uint32_t cols, void* xq,
                                              hipStream_t stream) {
  if (x == nullptr || xq == nullptr || cols == 0u || (cols % 256u) != 0u) return hipErrorInvalidValue;
  if ((reinterpret_cast<std::uintptr_t>(x) % 16u) != 0u || (reinterpret_cast<std::uintptr_t>(xq) % 16u) != 0u ||
      (weight != nullptr && (reinterpret_cast<std::uintptr_t>(weight) % 16u) != 0u))
    return hipErrorInvalidValue;
  const std::uint32_t groups = cols / kXGroup;
  hipLaunchKernelGGL(stage_kernel, dim3((groups + 255u) / 256u), dim3(256), 0, stream, x, weight, groups,
                     xq_out(xq, cols));
  return hipGetLastError();
}
