// Measurement helper, not part of the decode library: a plain streaming read of
// a device buffer, the practical HBM ceiling the decode kernels are compared
// with (bench.py --read-ceiling). Built into its own build/librtxllm_probe.so.
//
// extern "C" hipError_t rtxllm_stream_read(const void* data, size_t bytes,
//     uint32_t* out, uint32_t workgroups, hipStream_t stream): read `bytes` (a
//     multiple of 16, 16-byte aligned) with `workgroups` workgroups of 256
//     threads, each writing the xor of what it read to out[workgroup].
#include <hip/hip_runtime.h>

#include <cstddef>
#include <cstdint>

namespace rtxllm {
namespace {

typedef unsigned u32x4v __attribute__((ext_vector_type(4)));

// Grid-stride read of n16 16-byte vectors, four nontemporal loads in flight per
// lane; every workgroup writes the xor of what it read to out[blockIdx.x].
__global__ __launch_bounds__(256) void stream_read_kernel(const u32x4v* __restrict__ p, std::size_t n16,
                                                          std::uint32_t* __restrict__ out) {
  const std::size_t stride = static_cast<std::size_t>(gridDim.x) * blockDim.x;
  std::size_t i = static_cast<std::size_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  std::uint32_t acc = 0u;
  for (; i + 3u * stride < n16; i += 4u * stride) {
    const u32x4v a = __builtin_nontemporal_load(p + i);
    const u32x4v b = __builtin_nontemporal_load(p + i + stride);
    const u32x4v c = __builtin_nontemporal_load(p + i + 2u * stride);
    const u32x4v d = __builtin_nontemporal_load(p + i + 3u * stride);
    const u32x4v x = (a ^ b) ^ (c ^ d);
    acc ^= x.x ^ x.y ^ x.z ^ x.w;
  }
  for (; i < n16; i += stride) {
    const u32x4v a = __builtin_nontemporal_load(p + i);
    acc ^= a.x ^ a.y ^ a.z ^ a.w;
  }
  for (int o = 32; o > 0; o >>= 1) acc ^= static_cast<std::uint32_t>(__shfl_xor(static_cast<int>(acc), o, 64));
  __shared__ std::uint32_t w[4];
  if ((threadIdx.x & 63u) == 0u) w[threadIdx.x >> 6] = acc;
  __syncthreads();
  if (threadIdx.x == 0u) out[blockIdx.x] = w[0] ^ w[1] ^ w[2] ^ w[3];
}

}  // namespace
}  // namespace rtxllm

extern "C" hipError_t rtxllm_stream_read(const void* data, size_t bytes, uint32_t* out, uint32_t workgroups,
                                         hipStream_t stream) {
  if (data == nullptr || out == nullptr || bytes == 0u || (bytes % 16u) != 0u || workgroups == 0u ||
      (reinterpret_cast<std::uintptr_t>(data) % 16u) != 0u)
    return hipErrorInvalidValue;
  hipLaunchKernelGGL(rtxllm::stream_read_kernel, dim3(workgroups), dim3(256), 0, stream,
                     static_cast<const rtxllm::u32x4v*>(data), bytes / 16u, out);
  return hipGetLastError();
}
