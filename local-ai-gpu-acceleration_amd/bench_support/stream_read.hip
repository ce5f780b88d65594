// Measurement helper, not part of the decode library: a plain streaming read of
// a device buffer, the practical HBM ceiling the decode kernels are compared
// with (bench.py --read-ceiling). Built into its own build/librtxllm_probe.so.
//
// extern "C" hipError_t rtxllm_stream_read(const void* data, size_t bytes,
//     uint32_t* out, uint32_t workgroups, uint32_t mode, hipStream_t stream):
//     read `bytes` (a multiple of 16, 16-byte aligned) with `workgroups`
//     workgroups of 256 threads, each writing the xor of what it read to
//     out[workgroup]. mode 0: grid-stride loop, four nontemporal 16-byte loads
//     in flight per lane; 1: the same with eight; 2: each workgroup reads one
//     contiguous chunk of bytes / workgroups, four loads in flight per lane.
//     Which pattern is fastest depends on the size and grid (on MI355X the
//     361 MB read is fastest chunked at 8192 workgroups, 33-38 MB grid-stride
//     at 2048-8192), so the caller times them all and keeps the best.
#include <hip/hip_runtime.h>

#include <cstddef>
#include <cstdint>

namespace rtxllm {
namespace {

typedef unsigned u32x4v __attribute__((ext_vector_type(4)));

__device__ __forceinline__ void reduce_out(std::uint32_t acc, std::uint32_t* out) {
  for (int o = 32; o > 0; o >>= 1) acc ^= static_cast<std::uint32_t>(__shfl_xor(static_cast<int>(acc), o, 64));
  __shared__ std::uint32_t w[4];
  if ((threadIdx.x & 63u) == 0u) w[threadIdx.x >> 6] = acc;
  __syncthreads();
  if (threadIdx.x == 0u) out[blockIdx.x] = w[0] ^ w[1] ^ w[2] ^ w[3];
}

// Grid-stride read of n16 16-byte vectors, U nontemporal loads in flight per lane.
template <int U>
__global__ __launch_bounds__(256) void stream_read_kernel(const u32x4v* __restrict__ p, std::size_t n16,
                                                          std::uint32_t* __restrict__ out) {
  const std::size_t stride = static_cast<std::size_t>(gridDim.x) * blockDim.x;
  std::size_t i = static_cast<std::size_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  std::uint32_t acc = 0u;
  for (; i + (U - 1) * stride < n16; i += U * stride) {
    u32x4v x = {0u, 0u, 0u, 0u};
#pragma unroll
    for (int k = 0; k < U; ++k) x ^= __builtin_nontemporal_load(p + i + k * stride);
    acc ^= x.x ^ x.y ^ x.z ^ x.w;
  }
  for (; i < n16; i += stride) {
    const u32x4v a = __builtin_nontemporal_load(p + i);
    acc ^= a.x ^ a.y ^ a.z ^ a.w;
  }
  reduce_out(acc, out);
}

// One contiguous chunk per workgroup, four nontemporal loads in flight per lane.
__global__ __launch_bounds__(256) void stream_read_chunk_kernel(const u32x4v* __restrict__ p, std::size_t n16,
                                                                std::uint32_t* __restrict__ out) {
  const std::size_t per = (n16 + gridDim.x - 1u) / gridDim.x;
  const std::size_t b0 = static_cast<std::size_t>(blockIdx.x) * per;
  const std::size_t b1 = b0 + per < n16 ? b0 + per : n16;
  std::size_t i = b0 + threadIdx.x;
  std::uint32_t acc = 0u;
  for (; i + 3u * 256u < b1; i += 4u * 256u) {
    u32x4v x = {0u, 0u, 0u, 0u};
#pragma unroll
    for (int k = 0; k < 4; ++k) x ^= __builtin_nontemporal_load(p + i + k * 256u);
    acc ^= x.x ^ x.y ^ x.z ^ x.w;
  }
  for (; i < b1; i += 256u) {
    const u32x4v a = __builtin_nontemporal_load(p + i);
    acc ^= a.x ^ a.y ^ a.z ^ a.w;
  }
  reduce_out(acc, out);
}

}  // namespace
}  // namespace rtxllm

extern "C" hipError_t rtxllm_stream_read(const void* data, size_t bytes, uint32_t* out, uint32_t workgroups,
                                         uint32_t mode, hipStream_t stream) {
  if (data == nullptr || out == nullptr || bytes == 0u || (bytes % 16u) != 0u || workgroups == 0u || mode > 2u ||
      (reinterpret_cast<std::uintptr_t>(data) % 16u) != 0u)
    return hipErrorInvalidValue;
  const auto* p = static_cast<const rtxllm::u32x4v*>(data);
  if (mode == 0u)
    hipLaunchKernelGGL(rtxllm::stream_read_kernel<4>, dim3(workgroups), dim3(256), 0, stream, p, bytes / 16u, out);
  else if (mode == 1u)
    hipLaunchKernelGGL(rtxllm::stream_read_kernel<8>, dim3(workgroups), dim3(256), 0, stream, p, bytes / 16u, out);
  else
    hipLaunchKernelGGL(rtxllm::stream_read_chunk_kernel, dim3(workgroups), dim3(256), 0, stream, p, bytes / 16u, out);
  return hipGetLastError();
}
