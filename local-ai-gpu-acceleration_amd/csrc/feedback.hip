// Greedy token selection and the reference runner's RMSNorm/SiLU feedback
// family (decode_kernels.cu:122-289, 2993-3073).
//
// Feedback kernels: the reference recomputes sum(logits^2) in every thread
// (O(rows * cols)); here each 1024-thread workgroup reduces it once with wave64
// shuffles and then writes 1024 outputs, so the cost is O(rows * cols / 1024).
#include <cfloat>

#include "common.h"
#include "internal.h"
#include "rtxllm/decode_kernels.h"

namespace rtxllm {
namespace {

constexpr int kFbThreads = 1024;

__device__ float block_sum(float v, float* sh) {
  v = wave_sum(v);
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  if (lane == 0) sh[wave] = v;
  __syncthreads();
  float s = 0.0f;
  const int nw = blockDim.x >> 6;
  for (int i = 0; i < nw; ++i) s += sh[i];
  __syncthreads();
  return s;
}

__device__ float inv_rms(const float* __restrict__ logits, std::uint32_t rows, float eps, float* sh) {
  float s = 0.0f;
  for (std::uint32_t r = threadIdx.x; r < rows; r += blockDim.x) s = fmaf(logits[r], logits[r], s);
  const float total = block_sum(s, sh);
  return rsqrtf(total / static_cast<float>(rows) + eps);
}

__device__ __forceinline__ float silu(float v) {
  const float sig = 1.0f / (1.0f + expf(-v));
  return v * sig;
}

enum FbMode : int {
  kRmsnorm = 0,          // act = n
  kSiluRmsnorm = 1,      // act = silu(n)
  kWithSiluCache = 2,    // act = n, cache = silu(n)
  kGatedSilu = 3,        // act = cache[c % cache_cols] * n
  kSiluCache = 4,        // cache (+)= silu(n)
  kCache = 5,            // cache (+)= n
  kCacheGatedProduct = 6 // up (+)= n; act = gate * up
};

template <int MODE>
__global__ __launch_bounds__(kFbThreads) void feedback_kernel(const float* __restrict__ logits, const float* gate,
                                                              float* cache, float* act, std::uint32_t rows,
                                                              std::uint32_t cache_cols, std::uint32_t cols,
                                                              float eps, std::uint32_t accumulate) {
  __shared__ float sh[kFbThreads / 64];
  if (rows == 0u) return;
  if ((MODE == kGatedSilu || MODE == kCacheGatedProduct) && cache_cols == 0u) return;
  const float inv = inv_rms(logits, rows, eps, sh);
  const std::uint32_t c = blockIdx.x * blockDim.x + threadIdx.x;
  if (c >= cols) return;
  const float n = logits[c % rows] * inv;
  if constexpr (MODE == kRmsnorm) {
    act[c] = n;
  } else if constexpr (MODE == kSiluRmsnorm) {
    act[c] = silu(n);
  } else if constexpr (MODE == kWithSiluCache) {
    act[c] = n;
    cache[c] = silu(n);
  } else if constexpr (MODE == kGatedSilu) {
    act[c] = gate[c % cache_cols] * n;
  } else if constexpr (MODE == kSiluCache) {
    const float v = silu(n);
    cache[c] = accumulate != 0u ? cache[c] + v : v;
  } else if constexpr (MODE == kCache) {
    cache[c] = accumulate != 0u ? cache[c] + n : n;
  } else {
    const float u = accumulate != 0u ? cache[c] + n : n;
    cache[c] = u;
    act[c] = gate[c] * u;
  }
}

template <int MODE>
hipError_t launch_feedback(const float* logits, const float* gate, float* cache, float* act, std::uint32_t rows,
                           std::uint32_t cache_cols, std::uint32_t cols, float eps, std::uint32_t accumulate,
                           hipStream_t stream) {
  // A zero-column launch is an invalid configuration, as the reference's
  // <<<ceil(cols / 256), 256>>> launch would report.
  if (cols == 0u) return hipErrorInvalidConfiguration;
  const dim3 grid((cols + kFbThreads - 1) / kFbThreads);
  hipLaunchKernelGGL(feedback_kernel<MODE>, grid, dim3(kFbThreads), 0, stream, logits, gate, cache, act, rows,
                     cache_cols, cols, eps, accumulate);
  return hipGetLastError();
}

// ---- argmax ---------------------------------------------------------------

__device__ __forceinline__ bool better(float v, std::uint32_t i, float bv, std::uint32_t bi) {
  return v > bv || (v == bv && i < bi);
}

// One workgroup; each thread scans a strided slice keeping the first maximum,
// then a wave64 + LDS tournament keeps the lowest index among equal maxima.
// Initial (value, index) = (-FLT_MAX, 0) as in the reference, so NaNs never win.
__global__ __launch_bounds__(1024) void argmax_token_kernel(const float* __restrict__ logits, std::uint32_t* token,
                                                             std::uint32_t rows, int mode, std::uint32_t vocab,
                                                             std::uint32_t offset) {
  __shared__ float sv[16];
  __shared__ std::uint32_t si[16];
  float bv = -FLT_MAX;
  std::uint32_t bi = 0u;
  for (std::uint32_t r = threadIdx.x; r < rows; r += blockDim.x) {
    const float v = logits[r];
    if (better(v, r, bv, bi)) {
      bv = v;
      bi = r;
    }
  }
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) {
    const float ov = __shfl_xor(bv, o, 64);
    const std::uint32_t oi = __shfl_xor(bi, o, 64);
    if (better(ov, oi, bv, bi)) {
      bv = ov;
      bi = oi;
    }
  }
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  if (lane == 0) {
    sv[wave] = bv;
    si[wave] = bi;
  }
  __syncthreads();
  if (threadIdx.x == 0) {
    const int nw = blockDim.x >> 6;
    for (int i = 1; i < nw; ++i)
      if (better(sv[i], si[i], bv, bi)) {
        bv = sv[i];
        bi = si[i];
      }
    token[0] = mode == 0 ? (bi + token[0] + 1u) % 32000u : (bi + offset) % vocab;
  }
}

}  // namespace

hipError_t launch_argmax_token(const float* logits, std::uint32_t* token, std::uint32_t rows, int mode,
                               std::uint32_t vocab, std::uint32_t offset, hipStream_t stream) {
  hipLaunchKernelGGL(argmax_token_kernel, dim3(1), dim3(1024), 0, stream, logits, token, rows, mode, vocab, offset);
  return hipGetLastError();
}

}  // namespace rtxllm

using namespace rtxllm;

extern "C" hipError_t rtxllm_launch_rmsnorm_feedback(const float* logits, float* activation, std::uint32_t rows,
                                                     std::uint32_t cols, float epsilon, hipStream_t stream) {
  return launch_feedback<kRmsnorm>(logits, nullptr, nullptr, activation, rows, 0u, cols, epsilon, 0u, stream);
}

extern "C" hipError_t rtxllm_launch_silu_rmsnorm_feedback(const float* logits, float* activation,
                                                          std::uint32_t rows, std::uint32_t cols, float epsilon,
                                                          hipStream_t stream) {
  return launch_feedback<kSiluRmsnorm>(logits, nullptr, nullptr, activation, rows, 0u, cols, epsilon, 0u, stream);
}

extern "C" hipError_t rtxllm_launch_rmsnorm_feedback_with_silu_cache(const float* logits, float* activation,
                                                                     float* silu_cache, std::uint32_t rows,
                                                                     std::uint32_t cols, float epsilon,
                                                                     hipStream_t stream) {
  return launch_feedback<kWithSiluCache>(logits, nullptr, silu_cache, activation, rows, 0u, cols, epsilon, 0u,
                                         stream);
}

extern "C" hipError_t rtxllm_launch_gated_silu_rmsnorm_feedback(const float* logits, const float* silu_cache,
                                                                float* activation, std::uint32_t rows,
                                                                std::uint32_t cache_cols, std::uint32_t cols,
                                                                float epsilon, hipStream_t stream) {
  return launch_feedback<kGatedSilu>(logits, silu_cache, nullptr, activation, rows, cache_cols, cols, epsilon, 0u,
                                     stream);
}

extern "C" hipError_t rtxllm_launch_rmsnorm_silu_cache(const float* logits, float* silu_cache, std::uint32_t rows,
                                                       std::uint32_t cache_cols, float epsilon,
                                                       std::uint32_t accumulate, hipStream_t stream) {
  if (cache_cols == 0u) return hipErrorInvalidValue;
  return launch_feedback<kSiluCache>(logits, nullptr, silu_cache, nullptr, rows, cache_cols, cache_cols, epsilon,
                                     accumulate, stream);
}

extern "C" hipError_t rtxllm_launch_rmsnorm_cache(const float* logits, float* cache, std::uint32_t rows,
                                                  std::uint32_t cache_cols, float epsilon, std::uint32_t accumulate,
                                                  hipStream_t stream) {
  if (cache_cols == 0u) return hipErrorInvalidValue;
  return launch_feedback<kCache>(logits, nullptr, cache, nullptr, rows, cache_cols, cache_cols, epsilon,
                                 accumulate, stream);
}

extern "C" hipError_t rtxllm_launch_rmsnorm_cache_and_gated_product(const float* logits, const float* gate_cache,
                                                                    float* up_cache, float* activation,
                                                                    std::uint32_t rows, std::uint32_t cache_cols,
                                                                    std::uint32_t output_cols, float epsilon,
                                                                    std::uint32_t accumulate, hipStream_t stream) {
  if (cache_cols == 0u || output_cols == 0u) return hipErrorInvalidValue;
  return launch_feedback<kCacheGatedProduct>(logits, gate_cache, up_cache, activation, rows, cache_cols,
                                             output_cols, epsilon, accumulate, stream);
}

extern "C" hipError_t rtxllm_launch_output_token_sample(const float* logits, std::uint32_t* token,
                                                        std::uint32_t rows, std::uint32_t vocab_size,
                                                        std::uint32_t token_offset, hipStream_t stream) {
  if (logits == nullptr || token == nullptr || rows == 0u || vocab_size == 0u) return hipErrorInvalidValue;
  return launch_argmax_token(logits, token, rows, 1, vocab_size, token_offset, stream);
}
