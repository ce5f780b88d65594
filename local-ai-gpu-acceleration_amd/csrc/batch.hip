// Batched (1..8 activation vectors) matvec entry points on the matrix cores
// (mm.cuh), and their activation staging.
#include "internal.h"
#include "mm.cuh"
#include "mv_launch.cuh"

namespace rtxllm {
namespace {

// One workgroup per sequence: e_s from max |x_s|, then the hi / lo fp16 pair
// of x_s 2^-e_s, each at its place in the operand order (x16_index).
// Sequences >= batch get zero columns.
__global__ __launch_bounds__(1024) void stage_batch_kernel(const float* __restrict__ x, std::uint32_t batch,
                                                           std::uint32_t cols, _Float16* __restrict__ x16) {
  __shared__ float part[16];
  const std::uint32_t s = blockIdx.x;
  int* e_out = reinterpret_cast<int*>(x16 + 16u * static_cast<std::size_t>(cols));
  if (s >= batch) {
    for (std::uint32_t c = threadIdx.x; c < cols; c += blockDim.x) {
      const std::size_t i = x16_index(2u * s, c);
      x16[i] = x16[i + 8u] = static_cast<_Float16>(0.0f);
    }
    if (threadIdx.x == 0u) e_out[s] = 0;
    return;
  }
  const float* xs = x + static_cast<std::size_t>(s) * cols;
  float m = 0.0f;
  for (std::uint32_t c = threadIdx.x; c < cols; c += blockDim.x) m = fmaxf(m, fabsf(xs[c]));
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) m = fmaxf(m, __shfl_xor(m, o, 64));
  if ((threadIdx.x & 63u) == 0u) part[threadIdx.x >> 6] = m;
  __syncthreads();
  m = 0.0f;
  for (std::uint32_t i = 0; i < blockDim.x / 64u; ++i) m = fmaxf(m, part[i]);
  int e = 0;
  if (m > 0.0f && m <= 3.0e38f) frexpf(m, &e);  // m = f 2^e, f in [0.5, 1)
  for (std::uint32_t c = threadIdx.x; c < cols; c += blockDim.x) {
    const float v = ldexpf(xs[c], -e);
    const _Float16 h = static_cast<_Float16>(v);
    const std::size_t i = x16_index(2u * s, c);
    x16[i] = h;
    x16[i + 8u] = static_cast<_Float16>(v - static_cast<float>(h));  // column 2 s + 1: lane + 1
  }
  if (threadIdx.x == 0u) e_out[s] = e;
}

// Workgroups of mm_kernel<FMT> of `threads` threads resident per CU (0 if the
// query fails), cached per format and size.
template <int FMT>
int mm_resident_fmt(std::uint32_t threads) {
  static int cache[kMaxPanels + 1] = {};
  const std::uint32_t w = threads / 64u;
  if (w == 0u || w > kMaxPanels) return 0;
  if (cache[w] == 0) {
    int n = 0;
    if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&n, reinterpret_cast<const void*>(&mm_kernel<FMT>),
                                                     static_cast<int>(threads), 0) != hipSuccess || n <= 0)
      return 0;
    cache[w] = n;
  }
  return cache[w];
}

inline int mm_resident(int fmt, std::uint32_t threads) {
  switch (fmt) {
    case RTXLLM_FMT_IQ2S: return mm_resident_fmt<RTXLLM_FMT_IQ2S>(threads);
    case RTXLLM_FMT_IQ3S: return mm_resident_fmt<RTXLLM_FMT_IQ3S>(threads);
    case RTXLLM_FMT_Q5K: return mm_resident_fmt<RTXLLM_FMT_Q5K>(threads);
    case RTXLLM_FMT_Q4K_RAW: return mm_resident_fmt<RTXLLM_FMT_Q4K_RAW>(threads);
    case RTXLLM_FMT_Q4K_SPLIT_NATIVE: return mm_resident_fmt<RTXLLM_FMT_Q4K_SPLIT_NATIVE>(threads);
    default: return 0;
  }
}

struct MmGeom {
  std::uint32_t ppg, groups, grid;
};

inline bool mm_geom(int fmt, std::uint32_t rows, std::uint32_t cols, MmGeom& g) {
  if (!fmt_mm_supported(fmt) || rows == 0u || cols == 0u || (cols % kPanel) != 0u) return false;
  const std::uint32_t panels = cols / kPanel;
  g.ppg = 1u;
  for (std::uint32_t d = kMaxPanels; d >= 1u; --d)
    if (panels % d == 0u) {
      g.ppg = d;
      break;
    }
  g.groups = panels / g.ppg;
  const std::uint32_t tiles = (rows + 15u) / 16u;
  // persistent: the workgroups resident at once, shared by the panel groups,
  // every workgroup taking the same number of tiles (but the last few)
  const int resident = mm_resident(fmt, 64u * g.ppg);
  const std::uint32_t per_cu = resident > 0 ? static_cast<std::uint32_t>(resident) : 1u;
  const std::uint32_t cap = std::max(1u, per_cu * static_cast<std::uint32_t>(num_cus()) / g.groups);
  const std::uint32_t rounds = (tiles + cap - 1u) / cap;
  g.grid = (tiles + rounds - 1u) / rounds;
  return true;
}

template <int FMT>
hipError_t launch_mm_fmt(const QTensor& w, const void* x16, std::uint32_t batch, float* y, float* work,
                         std::size_t work_bytes, hipStream_t stream) {
  MmGeom g;
  if (!mm_geom(FMT, w.rows, w.cols, g)) return hipErrorInvalidValue;
  const std::uint64_t blocks = static_cast<std::uint64_t>(w.rows) * (w.cols / 256u);
  if (blocks * FmtBytes<FMT>::payload > 0xFFFFFFFFull || blocks * FmtBytes<FMT>::meta > 0xFFFFFFFFull)
    return hipErrorInvalidValue;
  const std::size_t n = static_cast<std::size_t>(batch) * w.rows;
  float* out = y;
  if (g.groups > 1u) {
    if (work == nullptr || work_bytes < 4u * n * g.groups) return hipErrorInvalidValue;
    out = work;
  }
  hipLaunchKernelGGL(mm_kernel<FMT>, dim3(g.grid, g.groups), dim3(64u * g.ppg), 0, stream, w, x16, batch, out,
                     w.rows);
  hipError_t st = hipGetLastError();
  if (st != hipSuccess || g.groups == 1u) return st;
  hipLaunchKernelGGL(mm_reduce_kernel, dim3(static_cast<unsigned>((n + 255u) / 256u)), dim3(256), 0, stream, work,
                     g.groups, static_cast<std::uint32_t>(n), y);
  return hipGetLastError();
}

}  // namespace
}  // namespace rtxllm

using namespace rtxllm;

extern "C" size_t rtxllm_x16_bytes(uint32_t cols) { return x16_bytes(cols); }

extern "C" hipError_t rtxllm_stage_batch(const float* x, uint32_t batch, uint32_t cols, void* x16,
                                         hipStream_t stream) {
  if (x == nullptr || x16 == nullptr || batch == 0u || batch > kBatchMax || cols == 0u || (cols % 256u) != 0u)
    return hipErrorInvalidValue;
  hipLaunchKernelGGL(stage_batch_kernel, dim3(kBatchMax), dim3(1024), 0, stream, x, batch, cols,
                     static_cast<_Float16*>(x16));
  return hipGetLastError();
}

extern "C" size_t rtxllm_matvec_batch_workspace(int format, uint32_t rows, uint32_t cols) {
  MmGeom g;
  if (!mm_geom(format, rows, cols, g) || g.groups == 1u) return 0u;
  return 4u * static_cast<std::size_t>(kBatchMax) * rows * g.groups;
}

extern "C" hipError_t rtxllm_matvec_batch(int format, const uint8_t* payload, const uint8_t* meta, const void* x16,
                                          float* y, uint32_t rows, uint32_t cols, uint32_t batch, void* workspace,
                                          size_t workspace_bytes, hipStream_t stream) {
  if (payload == nullptr || x16 == nullptr || y == nullptr || batch == 0u || batch > kBatchMax ||
      ((format == RTXLLM_FMT_Q4K_SPLIT_NATIVE) && meta == nullptr))
    return hipErrorInvalidValue;
  const QTensor w{payload, meta, rows, cols};
  float* work = static_cast<float*>(workspace);
  switch (format) {
    case RTXLLM_FMT_IQ2S: return launch_mm_fmt<RTXLLM_FMT_IQ2S>(w, x16, batch, y, work, workspace_bytes, stream);
    case RTXLLM_FMT_IQ3S: return launch_mm_fmt<RTXLLM_FMT_IQ3S>(w, x16, batch, y, work, workspace_bytes, stream);
    case RTXLLM_FMT_Q5K: return launch_mm_fmt<RTXLLM_FMT_Q5K>(w, x16, batch, y, work, workspace_bytes, stream);
    case RTXLLM_FMT_Q4K_RAW:
      return launch_mm_fmt<RTXLLM_FMT_Q4K_RAW>(w, x16, batch, y, work, workspace_bytes, stream);
    case RTXLLM_FMT_Q4K_SPLIT_NATIVE:
      return launch_mm_fmt<RTXLLM_FMT_Q4K_SPLIT_NATIVE>(w, x16, batch, y, work, workspace_bytes, stream);
    default: return hipErrorInvalidValue;
  }
}
