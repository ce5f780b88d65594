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


// v_permlane32_swap / v_permlane16_swap (gfx950): exchange a's upper 32 (odd
// 16-lane rows') lanes with b's lower 32 (even rows') lanes. Issued as inline
// asm: this compiler's __builtin_amdgcn_permlane{16,32}_swap treats the two
// results as one value (it emitted a + a for the sum of both), so the builtin
// is not usable. The s_nop covers the VALU-write -> permlane-read hazard.
__device__ __forceinline__ void permlane32_swap(float& a, float& b) {
  asm volatile("s_nop 1\n\tv_permlane32_swap_b32 %0, %1" : "+v"(a), "+v"(b));
}
__device__ __forceinline__ void permlane16_swap(float& a, float& b) {
  asm volatile("s_nop 1\n\tv_permlane16_swap_b32 %0, %1" : "+v"(a), "+v"(b));
}

// Wave64 all-reduce of an operation on 32-bit patterns (exact and order-free
// for max, integer sum, or; the fp32 sum below fixes this order): DPP quad xor 1 and xor 2, row half mirror (lane
// i <-> 7 - i), row mirror (i <-> 15 - i), then the 16- and 32-lane permlane
// swaps; every lane receives the result, and no step goes through LDS. G = 8
// stops after the half mirror: the result of each aligned group of 8 lanes.
template <int CTRL>
__device__ __forceinline__ std::uint32_t dpp_bits(std::uint32_t v) {
  return static_cast<std::uint32_t>(__builtin_amdgcn_update_dpp(0, static_cast<int>(v), CTRL, 0xF, 0xF, false));
}
template <int G = 64, class Op>
__device__ __forceinline__ std::uint32_t lanes_reduce_exact(std::uint32_t v, Op op) {
  static_assert(G == 8 || G == 64, "groups of 8 lanes or the wave");
  v = op(v, dpp_bits<0xB1>(v));   // quad_perm [1,0,3,2]
  v = op(v, dpp_bits<0x4E>(v));   // quad_perm [2,3,0,1]
  v = op(v, dpp_bits<0x141>(v));  // row_half_mirror
  if constexpr (G == 64) {
    v = op(v, dpp_bits<0x140>(v));  // row_mirror
    float a = __uint_as_float(v), b = a;
    permlane16_swap(a, b);
    v = op(__float_as_uint(a), __float_as_uint(b));
    a = __uint_as_float(v), b = a;
    permlane32_swap(a, b);
    v = op(__float_as_uint(a), __float_as_uint(b));
  }
  return v;
}

// The value of lane ^ M (the pairing of __shfl_xor with mask M, so sums and
// maxima keep their bits) by DPP or a permlane swap instead of an LDS shuffle.
// M = 4 takes lane - 4 or lane + 4 within the 16-lane row; every lane of the
// wave must be active.
template <int M>
__device__ __forceinline__ float lane_xor(float v) {
  static_assert(M == 1 || M == 2 || M == 4 || M == 8 || M == 16 || M == 32, "a single-bit lane mask");
  const std::uint32_t u = __float_as_uint(v);
  if constexpr (M == 1) {
    return __uint_as_float(dpp_bits<0xB1>(u));  // quad_perm [1,0,3,2]
  } else if constexpr (M == 2) {
    return __uint_as_float(dpp_bits<0x4E>(u));  // quad_perm [2,3,0,1]
  } else if constexpr (M == 4) {
    const std::uint32_t down = dpp_bits<0x114>(u), up = dpp_bits<0x104>(u);  // row_shr:4, row_shl:4
    return __uint_as_float((threadIdx.x & 4u) ? down : up);
  } else if constexpr (M == 8) {
    return __uint_as_float(dpp_bits<0x128>(u));  // row_ror:8
  } else {
    float a = v, b = v;
    if constexpr (M == 16) permlane16_swap(a, b);  // a: rows 0, 0, 2, 2; b: rows 1, 1, 3, 3
    else permlane32_swap(a, b);                     // a: lanes 0-31 twice; b: lanes 32-63 twice
    return (threadIdx.x & static_cast<std::uint32_t>(M)) ? a : b;
  }
}

// Wave64 sum in the order of lanes_reduce_exact (DPP and permlane steps, no
// LDS); every lane receives the same total (each step adds a + b in both
// partners, and fp32 addition commutes).
__device__ __forceinline__ float wave_sum(float v) {
  return __uint_as_float(lanes_reduce_exact(__float_as_uint(v), [](std::uint32_t a, std::uint32_t b) {
    return __float_as_uint(__uint_as_float(a) + __uint_as_float(b));
  }));
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
