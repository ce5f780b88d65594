// Host-side helpers of the C-ABI: format sizes, the Q4_K resident-pack split
// (tools/bench/q4k_resident_pack.py:100-145) and the seeded synthetic generator.
#include <algorithm>
#include <cstring>
#include <thread>
#include <vector>

#include "rtxllm/decode_kernels.h"
#include "q4k_split.h"
#include "synth.h"

namespace {

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
  for (std::size_t b = 0; b < n_blocks; ++b)
    rtxllm::q4k_split_block(format, raw + b * 144u, payload + b * 128u, meta + b * mb);
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
