// Staged batch activation (x16) of the matrix-core matvec: layout and index
// helpers shared by its producers (staging kernels, the fused attention
// combine) and its consumer (mm.cuh).
#pragma once

#include <hip/hip_runtime.h>

#include <cstddef>
#include <cstdint>

namespace rtxllm {

constexpr std::uint32_t kBatchMax = 8;

// Staged batch activation of cols values per sequence (cols % 256 == 0,
// nb = cols / 256 blocks): 16 fp16 columns X[n] (n = 2 s + hi/lo) in operand
// order (x16_index), holding x_s 2^-e[s][b] over block b; then int32
// e[8][nb]; float ss[8][nb]; float eps. With eps >= 0 the vector is
// rmsnorm-staged: its consumer scales W x by 1 / sqrt(sum_b ss[s][b] / cols +
// eps) (ss = the sequence's sums of squares per block); eps < 0: no scale.
__host__ __device__ inline std::size_t x16_bytes(std::uint32_t cols) {
  return 32u * static_cast<std::size_t>(cols) + 8u * kBatchMax * (cols / 256u) + 16u;
}

struct X16Tail {
  int* e;       // [8][nb]
  float* ss;    // [8][nb]
  float* eps;
};

__host__ __device__ inline X16Tail x16_tail(const void* x16, std::uint32_t cols) {
  auto* base = static_cast<std::uint8_t*>(const_cast<void*>(x16)) + 32u * static_cast<std::size_t>(cols);
  const std::size_t n = static_cast<std::size_t>(kBatchMax) * (cols / 256u);
  return {reinterpret_cast<int*>(base), reinterpret_cast<float*>(base + 4u * n), reinterpret_cast<float*>(base + 8u * n)};
}

// Index (in fp16 values) of X[n][c]: the place where lane l = 16 (k / 64) + n
// of instruction j = k / 8 % 8 of block kb = c / 256 holds its eight B values
// (k = c % 256, value i = k % 8).
__host__ __device__ inline std::size_t x16_index(std::uint32_t n, std::uint32_t c) {
  const std::uint32_t k = c & 255u;
  return ((static_cast<std::size_t>(c >> 8) * 8u + ((k >> 3) & 7u)) * 64u + 16u * (k >> 6) + n) * 8u + (k & 7u);
}

}  // namespace rtxllm
