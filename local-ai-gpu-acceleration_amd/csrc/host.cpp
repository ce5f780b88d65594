// Host-side helpers of the C-ABI: format sizes, the Q4_K resident-pack split
// (tools/bench/q4k_resident_pack.py:100-145) and the seeded synthetic generator.
#include <algorithm>
#include <cstring>
#include <thread>
#include <vector>

#include "rtxllm/decode_kernels.h"
#include "synth.h"

namespace {

float f16_to_f32_host(std::uint16_t h) {
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

void scale_min_k4_host(int j, const std::uint8_t* q, std::uint8_t& sc, std::uint8_t& m) {
  if (j < 4) {
    sc = q[j] & 63u;
    m = q[j + 4] & 63u;
  } else {
    sc = static_cast<std::uint8_t>((q[j + 4] & 0x0Fu) | ((q[j - 4] >> 6) << 4));
    m = static_cast<std::uint8_t>((q[j + 4] >> 4) | ((q[j] >> 6) << 4));
  }
}

template <class F>
void parallel_for(std::size_t n, int threads, F&& body) {
  unsigned t = threads > 0 ? static_cast<unsigned>(threads) : std::max(1u, std::thread::hardware_concurrency());
  t = static_cast<unsigned>(std::min<std::size_t>(t, std::max<std::size_t>(1, n / 4096)));
  if (t <= 1u) {
    body(std::size_t{0}, n);
    return;
  }
  std::vector<std::thread> pool;
  for (unsigned i = 0; i < t; ++i) {
    const std::size_t a = n * i / t, b = n * (i + 1) / t;
    pool.emplace_back([&body, a, b] { body(a, b); });
  }
  for (auto& th : pool) th.join();
}

}  // namespace

extern "C" std::uint32_t rtxllm_format_payload_block_bytes(int format) { return rtxllm_format_payload_bytes(format); }
extern "C" std::uint32_t rtxllm_format_meta_block_bytes(int format) { return rtxllm_format_meta_bytes(format); }

extern "C" int rtxllm_q4k_split_pack(int format, const std::uint8_t* raw, std::size_t n_blocks,
                                     std::uint8_t* payload, std::uint8_t* meta) {
  if (format < RTXLLM_FMT_Q4K_SPLIT_PREDECODED || format > RTXLLM_FMT_Q4K_SPLIT_NATIVE || raw == nullptr ||
      payload == nullptr || meta == nullptr)
    return -1;
  const std::uint32_t mb = rtxllm_format_meta_bytes(format);
  for (std::size_t b = 0; b < n_blocks; ++b) {
    const std::uint8_t* blk = raw + b * 144u;
    std::memcpy(payload + b * 128u, blk + 16, 128);
    std::uint8_t* m = meta + b * mb;
    if (format == RTXLLM_FMT_Q4K_SPLIT_NATIVE) {
      std::memcpy(m, blk, 16);
      continue;
    }
    std::uint8_t sc[8], mn[8];
    for (int j = 0; j < 8; ++j) scale_min_k4_host(j, blk + 4, sc[j], mn[j]);
    if (format == RTXLLM_FMT_Q4K_SPLIT_COMPACT) {
      std::memcpy(m, blk, 4);
      std::memcpy(m + 4, sc, 8);
      std::memcpy(m + 12, mn, 8);
      continue;
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
  return 0;
}

extern "C" int rtxllm_synth_raw_blocks(int format, std::uint64_t seed, std::size_t n_blocks, float d_lo, float d_hi,
                                       std::uint8_t* out, int threads) {
  if (format != RTXLLM_FMT_Q4K_RAW && format != RTXLLM_FMT_Q5K && format != RTXLLM_FMT_IQ2S &&
      format != RTXLLM_FMT_IQ3S)
    return -1;
  if (out == nullptr) return -1;
  const std::uint32_t bb = rtxllm_format_payload_bytes(format);
  parallel_for(n_blocks, threads, [&](std::size_t a, std::size_t b) {
    rtxllm_synth_raw_blocks(format, seed, a, b - a, d_lo, d_hi, out + a * bb);
  });
  return 0;
}

extern "C" int rtxllm_synth_normal_f32(std::uint64_t seed, std::size_t n, float mean, float stddev, float* out,
                                       int threads) {
  if (out == nullptr) return -1;
  const std::uint64_t s = rtxllm_synth_stream(seed, 3u);
  parallel_for(n, threads, [&](std::size_t a, std::size_t b) {
    for (std::size_t i = a; i < b; ++i) out[i] = mean + stddev * rtxllm_synth_normal(s, i);
  });
  return 0;
}

extern "C" int rtxllm_synth_normal_f16(std::uint64_t seed, std::size_t n, float mean, float stddev,
                                       std::uint16_t* out, int threads) {
  if (out == nullptr) return -1;
  const std::uint64_t s = rtxllm_synth_stream(seed, 3u);
  parallel_for(n, threads, [&](std::size_t a, std::size_t b) {
    for (std::size_t i = a; i < b; ++i) out[i] = rtxllm_f32_to_f16_rne(mean + stddev * rtxllm_synth_normal(s, i));
  });
  return 0;
}
