// Activation staging entry point: fp32 x (times an optional elementwise weight)
// -> 16-value fixed-point groups consumed by the matvec kernels.
#include "rtxllm/decode_kernels.h"
#include "xq.h"

namespace rtxllm {
namespace {

template <bool ALIGNED>
__global__ __launch_bounds__(256) void stage_kernel(const float* __restrict__ x, const float* __restrict__ mul,
                                                    std::uint32_t groups, XQOut out) {
  const std::uint32_t g = blockIdx.x * blockDim.x + threadIdx.x;
  if (g >= groups) return;
  XG v;
  xg_stage<ALIGNED>(x, mul, g, v);
  xg_store(out, g, v);
}

}  // namespace
}  // namespace rtxllm

using namespace rtxllm;

extern "C" hipError_t rtxllm_stage_activation(const float* x, const float* weight, std::uint32_t cols, void* xq,
                                              hipStream_t stream) {
  if (x == nullptr || xq == nullptr || cols == 0u || (cols % 256u) != 0u) return hipErrorInvalidValue;
  auto align = [](const void* p) { return reinterpret_cast<std::uintptr_t>(p) % 16u; };
  if ((reinterpret_cast<std::uintptr_t>(x) % 4u) != 0u || align(xq) != 0u ||
      (weight != nullptr && (reinterpret_cast<std::uintptr_t>(weight) % 4u) != 0u))
    return hipErrorInvalidValue;
  const std::uint32_t groups = cols / kXGroup;
  const bool vec = align(x) == 0u && (weight == nullptr || align(weight) == 0u);
  if (vec)
    hipLaunchKernelGGL(stage_kernel<true>, dim3((groups + 255u) / 256u), dim3(256), 0, stream, x, weight, groups,
                       xq_out(xq, cols));
  else
    hipLaunchKernelGGL(stage_kernel<false>, dim3((groups + 255u) / 256u), dim3(256), 0, stream, x, weight, groups,
                       xq_out(xq, cols));
  return hipGetLastError();
}
