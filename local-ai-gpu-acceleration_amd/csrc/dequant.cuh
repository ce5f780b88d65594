// Per-element dequant of the resident-pack layouts with the reference gate's
// expression order (runtime/apps/mixed_sequence_benchmark_runner/main.cpp:
// 1133-1259), compiled without FMA contraction: bit-exact with the CPU gate.
// Used by the dequant entry point and the Q5_K embedding gather.
#pragma once

#include "mv.cuh"

namespace rtxllm {

#pragma clang fp contract(off)
// Value v of a block, with the reference's expression order (main.cpp:1133-1259).
template <int FMT>
__device__ __forceinline__ float dequant_value(const std::uint8_t* p, const std::uint8_t* m, std::uint32_t v) {
  if constexpr (FMT == RTXLLM_FMT_Q5K) {
    const float d = f16_bits_to_f32(ld_u16(p));
    const float dmin = f16_bits_to_f32(ld_u16(p + 2));
    const std::uint32_t g = v >> 6, lane = v & 31u, high = (v & 63u) >= 32u;
    std::uint32_t sc, mn;
    scale_min_k4(static_cast<int>(2u * g + high), ld_u32(p + 4), ld_u32(p + 8), ld_u32(p + 12), sc, mn);
    const std::uint32_t packed = p[48u + 32u * g + lane];
    const std::uint32_t low = high ? (packed >> 4) : (packed & 15u);
    const std::uint32_t quant = low + (((p[16u + lane] >> (2u * g + high)) & 1u) ? 16u : 0u);
    return d * static_cast<float>(sc) * static_cast<float>(quant) - dmin * static_cast<float>(mn);
  } else if constexpr (FMT == RTXLLM_FMT_IQ2S) {
    const std::uint32_t ib32 = v >> 5, grp = (v & 31u) >> 3, lane = v & 7u;
    const float d = f16_bits_to_f32(ld_u16(p));
    const std::uint32_t go = ib32 * 4u + grp;
    const std::uint32_t idx = p[2u + go] | ((static_cast<std::uint32_t>(p[66u + ib32]) << (8u - 2u * grp)) & 0x300u);
    const std::uint32_t grid = 2u * ((kIq2sGridDev[idx] >> (2u * lane)) & 3u) + 1u;
    const std::uint32_t sb = p[74u + ib32];
    const std::uint32_t nib = grp < 2u ? (sb & 15u) : (sb >> 4);
    const float scale = d * (0.5f + static_cast<float>(nib)) * 0.25f;
    const bool neg = (p[34u + go] >> lane) & 1u;
    return scale * static_cast<float>(grid) * (neg ? -1.0f : 1.0f);
  } else if constexpr (FMT == RTXLLM_FMT_IQ3S) {
    const std::uint32_t ib32 = v >> 5, grp = (v & 31u) >> 3, lane = v & 7u, pair = lane >> 2, gl = lane & 3u;
    const float d = f16_bits_to_f32(ld_u16(p));
    const std::uint32_t sel = ib32 * 8u + grp * 2u + pair;
    const std::uint32_t hb = (p[66u + ib32] >> (2u * grp + pair)) & 1u;
    const std::uint32_t idx = p[2u + sel] | (hb << 8);
    const std::uint32_t grid = (kIq3sGridDev[idx] >> (8u * gl)) & 0xFFu;
    const std::uint32_t sb = p[106u + (ib32 >> 1)];
    const std::uint32_t nib = (ib32 & 1u) == 0u ? (sb & 15u) : (sb >> 4);
    const float scale = d * static_cast<float>(1u + 2u * nib);
    const bool neg = (p[74u + ib32 * 4u + grp] >> lane) & 1u;
    return scale * static_cast<float>(grid) * (neg ? -1.0f : 1.0f);
  } else {
    const std::uint32_t g = v >> 6, lane = v & 31u, high = (v & 63u) >= 32u, pair = 2u * g + high;
    const std::uint8_t* qs = (FMT == RTXLLM_FMT_Q4K_RAW || FMT == RTXLLM_FMT_Q4K_RAW_PREDECODED) ? p + 16 : p;
    const std::uint32_t packed = qs[32u * g + lane];
    const float quant = static_cast<float>(high ? (packed >> 4) : (packed & 15u));
    if constexpr (FMT == RTXLLM_FMT_Q4K_SPLIT_PREDECODED || FMT == RTXLLM_FMT_Q4K_RAW_PREDECODED) {
      const float* pm = reinterpret_cast<const float*>(m) + 2u * pair;
      return pm[0] * quant - pm[1];
    } else if constexpr (FMT == RTXLLM_FMT_Q4K_SPLIT_HALF) {
      return f16_bits_to_f32(ld_u16(m + 4u * pair)) * quant - f16_bits_to_f32(ld_u16(m + 4u * pair + 2u));
    } else if constexpr (FMT == RTXLLM_FMT_Q4K_SPLIT_COMPACT) {
      const float d = f16_bits_to_f32(ld_u16(m));
      const float dmin = f16_bits_to_f32(ld_u16(m + 2));
      return d * static_cast<float>(m[4u + pair]) * quant - dmin * static_cast<float>(m[12u + pair]);
    } else {  // native head: split-native metadata or the raw block itself
      const std::uint8_t* h = (FMT == RTXLLM_FMT_Q4K_RAW) ? p : m;
      const float d = f16_bits_to_f32(ld_u16(h));
      const float dmin = f16_bits_to_f32(ld_u16(h + 2));
      std::uint32_t sc, mn;
      scale_min_k4(static_cast<int>(pair), ld_u32(h + 4), ld_u32(h + 8), ld_u32(h + 12), sc, mn);
      return d * static_cast<float>(sc) * quant - dmin * static_cast<float>(mn);
    }
  }
}

// Values [16 t, 16 t + 16) of a Q5_K block (t in [0, 16)) from three aligned
// 16-byte loads: the head (d, dmin, scales), the 16 qh bytes and the 16 qs
// bytes the run uses (the run lies in one 32-value sub-block). Same values,
// bit for bit, as dequant_value<Q5K> for each v in the run. The block must be
// 16-byte aligned (176-byte blocks of a 16-byte aligned table are).
__device__ __forceinline__ void dequant_q5k_run16(const std::uint8_t* blk, std::uint32_t t, float out[16]) {
  const std::uint32_t v0 = 16u * t, g = v0 >> 6, high = (v0 & 63u) >= 32u ? 1u : 0u, lane0 = v0 & 31u;
  const uint4 head = *reinterpret_cast<const uint4*>(blk);
  const uint4 qh4 = *reinterpret_cast<const uint4*>(blk + 16u + lane0);
  const uint4 qs4 = *reinterpret_cast<const uint4*>(blk + 48u + 32u * g + lane0);
  const float d = f16_bits_to_f32(static_cast<std::uint16_t>(head.x & 0xFFFFu));
  const float dmin = f16_bits_to_f32(static_cast<std::uint16_t>(head.x >> 16));
  std::uint32_t sc, mn;
  scale_min_k4(static_cast<int>(2u * g + high), head.y, head.z, head.w, sc, mn);
  const std::uint32_t qh[4] = {qh4.x, qh4.y, qh4.z, qh4.w}, qs[4] = {qs4.x, qs4.y, qs4.z, qs4.w};
  const std::uint32_t hbit = 2u * g + high;
#pragma unroll
  for (int j = 0; j < 16; ++j) {
    const std::uint32_t packed = (qs[j >> 2] >> (8 * (j & 3))) & 0xFFu;
    const std::uint32_t low = high ? (packed >> 4) : (packed & 15u);
    const std::uint32_t quant = low + (((((qh[j >> 2] >> (8 * (j & 3))) & 0xFFu) >> hbit) & 1u) ? 16u : 0u);
    out[j] = d * static_cast<float>(sc) * static_cast<float>(quant) - dmin * static_cast<float>(mn);
  }
}
#pragma clang fp contract(on)

}  // namespace rtxllm
