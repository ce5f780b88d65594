// Host-side split of Q4_K blocks into the resident-pack streams
// (tools/bench/q4k_resident_pack.py:100-145): the 128-byte quant payload, and
// per block the metadata of one split layout - predecoded (8 fp32 pairs
// d*scale, dmin*min), half (the same pairs in fp16, round to nearest even),
// compact (raw d, dmin, then the 8 unpacked scales and 8 unpacked mins) or
// native (the original 16-byte head). Plain C++, no GPU code: the pack
// producer and the C-ABI share it.
#pragma once

#include <cstddef>
#include <cstdint>
#include <cstring>

#include "synth.h"

namespace rtxllm {

// fp16 -> fp32 with the reference gate's rule (main.cpp:1086-1098):
// subnormals exact, infinities kept, every NaN -> +qNaN.
inline float f16_to_f32_host(std::uint16_t h) {
  const std::uint32_t sign = (h & 0x8000u) << 16;
  const std::uint32_t e = (h >> 10) & 0x1Fu, m = h & 0x3FFu;
  std::uint32_t bits;
  if (e == 0u) {
    if (m == 0u) {
      bits = sign;
    } else {  // subnormal: m * 2^-24, exact in fp32
      float v = static_cast<float>(m) * 5.9604644775390625e-08f;
      std::memcpy(&bits, &v, 4);
      bits |= sign;
    }
  } else if (e == 31u) {
    bits = m == 0u ? (sign | 0x7F800000u) : 0x7FC00000u;
  } else {
    bits = sign | ((e + 112u) << 23) | (m << 13);
  }
  float out;
  std::memcpy(&out, &bits, 4);
  return out;
}

inline void scale_min_k4_host(int j, const std::uint8_t* q, std::uint8_t& sc, std::uint8_t& m) {
  if (j < 4) {
    sc = q[j] & 63u;
    m = q[j + 4] & 63u;
  } else {
    sc = static_cast<std::uint8_t>((q[j + 4] & 0x0Fu) | ((q[j - 4] >> 6) << 4));
    m = static_cast<std::uint8_t>((q[j + 4] >> 4) | ((q[j] >> 6) << 4));
  }
}

// One 144-byte block -> its 128 payload bytes and the metadata of `format`
// (an RTXLLM_FMT_Q4K_SPLIT_* id; rtxllm_format_meta_bytes(format) bytes).
inline void q4k_split_block(int format, const std::uint8_t* blk, std::uint8_t* payload, std::uint8_t* m) {
  std::memcpy(payload, blk + 16, 128);
  if (format == RTXLLM_FMT_Q4K_SPLIT_NATIVE) {
    std::memcpy(m, blk, 16);
    return;
  }
  std::uint8_t sc[8], mn[8];
  for (int j = 0; j < 8; ++j) scale_min_k4_host(j, blk + 4, sc[j], mn[j]);
  if (format == RTXLLM_FMT_Q4K_SPLIT_COMPACT) {
    std::memcpy(m, blk, 4);
    std::memcpy(m + 4, sc, 8);
    std::memcpy(m + 12, mn, 8);
    return;
  }
  const float d = f16_to_f32_host(static_cast<std::uint16_t>(blk[0] | (blk[1] << 8)));
  const float dmin = f16_to_f32_host(static_cast<std::uint16_t>(blk[2] | (blk[3] << 8)));
  for (int j = 0; j < 8; ++j) {
    const float s = d * static_cast<float>(sc[j]);  // <= 17 significant bits: exact
    const float mm = dmin * static_cast<float>(mn[j]);
    if (format == RTXLLM_FMT_Q4K_SPLIT_PREDECODED) {
      std::memcpy(m + 8 * j, &s, 4);
      std::memcpy(m + 8 * j + 4, &mm, 4);
    } else {
      const std::uint16_t hs = rtxllm_f32_to_f16_rne(s), hm = rtxllm_f32_to_f16_rne(mm);
      std::memcpy(m + 4 * j, &hs, 2);
      std::memcpy(m + 4 * j + 2, &hm, 2);
    }
  }
}

}  // namespace rtxllm
