// Device helpers shared by the batch-1 layer kernels (layer.hip) and the
// batched ones (batch.hip): wave max, SiLU, paged-KV addressing, fp16 stores
// and the greedy-argmax key.
#pragma once

#include "common.h"
#include "layer.h"

namespace rtxllm {

__device__ __forceinline__ float wave_max(float v) {
  return __uint_as_float(lanes_reduce_exact(__float_as_uint(v), [](std::uint32_t a, std::uint32_t b) {
    return __float_as_uint(fmaxf(__uint_as_float(a), __uint_as_float(b)));
  }));
}

// SiLU v / (1 + exp(-v)) (main.cpp:1435-1503), as v * sigmoid(v).
__device__ __forceinline__ float silu(float v) {
  const float sig = 1.0f / (1.0f + expf(-v));
  return v * sig;
}

// Element offset of (position pos, kv head) in a layer's paged cache, the
// block table being the sequence's own row.
__device__ __forceinline__ std::size_t kv_offset(const KvLayer& kv, const std::int32_t* table, std::uint32_t pos,
                                                 std::uint32_t head) {
  const std::uint32_t page = static_cast<std::uint32_t>(table[pos / kv.page_size]);
  const std::uint32_t slot = pos % kv.page_size;
  return ((static_cast<std::size_t>(page) * kv.n_kv + head) * kv.page_size + slot) * kHeadDim;
}

// (cos, sin) of the rotary angle of pair i at position pos, from the table of
// positions [0, positions) x kHeadDim / 2 pairs (a position past the table,
// which has no KV slot either, takes the last row).
__device__ __forceinline__ float2 rope_at(const float2* rope, std::uint32_t positions, std::uint32_t pos,
                                          std::uint32_t i) {
  const std::uint32_t p = pos < positions ? pos : positions - 1u;
  return rope[static_cast<std::size_t>(p) * (kHeadDim / 2u) + i];
}

// The rotated query as the attention's matrix-core operand ("q16"): per kv
// head g, 4 instructions j x 64 lanes x 8 fp16, lane l = 16 (d / 32) + n
// holding dims 32 (l / 16) + 8 j + i of column n = 2 h + part (h < group the
// query head within g; part 0 = hi = fp16(x), 1 = lo = fp16(x - hi), x = q /
// sqrt(head_dim)); columns n >= 2 group stay zero. kQ16PerKv values per kv head.
constexpr std::uint32_t kQ16PerKv = 4u * 64u * 8u;
static_assert(2u * kQ16PerKv == kQ16BytesPerKv, "q16 size");

__device__ __forceinline__ std::size_t q16_index(std::uint32_t g, std::uint32_t h, std::uint32_t d,
                                                 std::uint32_t part) {
  const std::uint32_t l = 16u * (d >> 5) + 2u * h + part;
  return ((static_cast<std::size_t>(g) * 4u + ((d >> 3) & 3u)) * 64u + l) * 8u + (d & 7u);
}

// Stores query value q (head `head` of n_heads = group * n_kv, dim d) into q16.
__device__ __forceinline__ void q16_store(_Float16* q16, std::uint32_t head, std::uint32_t group, std::uint32_t d,
                                          float q) {
  const float x = q * 0.08838834764831845f;  // 1 / sqrt(128)
  const _Float16 hi = static_cast<_Float16>(x);
  const std::size_t i = q16_index(head / group, head % group, d, 0u);
  q16[i] = hi;
  q16[i + 8u] = static_cast<_Float16>(x - static_cast<float>(hi));  // column n + 1 = lane + 1
}

__device__ __forceinline__ std::uint16_t f2h(float v) {
  return __builtin_bit_cast(unsigned short, static_cast<_Float16>(v));
}

// Greedy-argmax key: ordered(logit) << 32 | ~row, so the largest key is the
// largest logit at the lowest row (decode_kernels.cu:2993-3031); NaN never
// wins (key 0) and -0 ties with +0.
__device__ __forceinline__ unsigned long long argmax_key(float v, std::uint32_t row) {
  if (v != v) return 0ull;
  if (v == 0.0f) v = 0.0f;
  std::uint32_t u = __float_as_uint(v);
  u = (u & 0x80000000u) ? ~u : (u | 0x80000000u);
  return (static_cast<unsigned long long>(u) << 32) | (0xFFFFFFFFu - row);
}

}  // namespace rtxllm
