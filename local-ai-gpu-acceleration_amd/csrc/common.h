// Device helpers shared by the gfx950 decode kernels: GGUF block field decode,
// wave64 reductions, launch-argument checks.
#pragma once

#include <hip/hip_runtime.h>

#include <cstddef>
#include <cstdint>

#include "synth.h"

namespace rtxllm {

constexpr int kWave = 64;

// IEEE binary16 -> fp32 with the reference's NaN rule (any NaN becomes the
// canonical +quiet NaN, decode_kernels.cu:1665-1676). The hardware conversion is
// exact for every finite and infinite input.
__device__ __forceinline__ float f16_bits_to_f32(std::uint32_t bits) {
  bits &= 0xFFFFu;
  if ((bits & 0x7C00u) == 0x7C00u && (bits & 0x03FFu) != 0u) return __uint_as_float(0x7FC00000u);
  return static_cast<float>(__builtin_bit_cast(_Float16, static_cast<unsigned short>(bits)));
}

// Wave64 sum; every lane receives the total.
__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o, kWave);
  return v;
}

// 6-bit scale / min of sub-block j of a K-quant block from its 12 packed scale
// bytes held as three little-endian words (ggml get_scale_min_k4).
__device__ __forceinline__ void scale_min_k4(int j, std::uint32_t s0, std::uint32_t s1, std::uint32_t s2,
                                             std::uint32_t& sc, std::uint32_t& m) {
  if (j < 4) {
    sc = (s0 >> (8 * j)) & 63u;
    m = (s1 >> (8 * j)) & 63u;
  } else {
    const int jj = j - 4;
    sc = ((s2 >> (8 * jj)) & 15u) | (((s0 >> (8 * jj + 6)) & 3u) << 4);
    m = ((s2 >> (8 * jj + 4)) & 15u) | (((s1 >> (8 * jj + 6)) & 3u) << 4);
  }
}

__device__ __forceinline__ std::uint32_t ld_u8(const std::uint8_t* p) { return *p; }
__device__ __forceinline__ std::uint32_t ld_u16(const std::uint8_t* p) {
  return *reinterpret_cast<const std::uint16_t*>(p);
}
__device__ __forceinline__ std::uint32_t ld_u32(const std::uint8_t* p) {
  return *reinterpret_cast<const std::uint32_t*>(p);
}
__device__ __forceinline__ uint4 ld_u128(const std::uint8_t* p) { return *reinterpret_cast<const uint4*>(p); }

inline bool format_is_q4k(int fmt) {
  return (fmt >= RTXLLM_FMT_Q4K_RAW && fmt <= RTXLLM_FMT_Q4K_SPLIT_NATIVE) || fmt == RTXLLM_FMT_Q4K_RAW_PREDECODED;
}
inline bool format_is_split(int fmt) {
  return fmt >= RTXLLM_FMT_Q4K_SPLIT_PREDECODED && fmt <= RTXLLM_FMT_Q4K_SPLIT_NATIVE;
}

}  // namespace rtxllm
