// Device helpers shared by the batch-1 layer kernels (layer.hip) and the
// batched ones (batch.hip): wave max, SiLU, paged-KV addressing, fp16 stores
// and the greedy-argmax key.
#pragma once

#include "common.h"
#include "layer.h"

namespace rtxllm {

__device__ __forceinline__ float wave_max(float v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v = fmaxf(v, __shfl_xor(v, o, 64));
  return v;
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
