// Batched (1..8 activation vectors) matvec entry points on the matrix cores
// (mm.cuh), their activation staging, and the batch decode step's kernels:
// residual + RMSNorm + staging per sequence, and the matvec epilogues of the
// qkv (RoPE + KV append), gate/up (SiLU-gate) and LM-head (logits + argmax
// keys) projections.
#include <algorithm>
#include <mutex>

#include "dequant.cuh"
#include "internal.h"
#include "layer.h"
#include "layer_common.cuh"
#include "mm.cuh"
#include "mv_launch.cuh"
#include "rtxllm/decode_kernels.h"

namespace rtxllm {
namespace {

// ---- staging: one workgroup of 256 per (block b of 256 values, sequence s) ----

constexpr std::uint32_t kStageThreads = 256;

// Sum (is_max false) or maximum over the 256 threads; every thread gets it.
__device__ __forceinline__ float block_reduce(float v, float* part, bool is_max) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) {
    const float t = __shfl_xor(v, o, 64);
    v = is_max ? fmaxf(v, t) : v + t;
  }
  __syncthreads();  // part may still be read by a previous reduction
  if ((threadIdx.x & 63u) == 0u) part[threadIdx.x >> 6] = v;
  __syncthreads();
  const float r0 = part[0], r1 = part[1], r2 = part[2], r3 = part[3];
  return is_max ? fmaxf(fmaxf(r0, r1), fmaxf(r2, r3)) : (r0 + r1) + (r2 + r3);
}

// x (already normalised or plain) of thread c of block b, sequence s: e[s][b]
// from the block's max |x|, then the hi / lo fp16 pair of x 2^-e at its place
// in the operand order.
__device__ __forceinline__ void stage_block_value(float x, std::uint32_t s, std::uint32_t b, std::uint32_t c,
                                                  std::uint32_t cols, _Float16* x16, float* part) {
  const float m = block_reduce(fabsf(x), part, true);
  int e = 0;
  if (m > 0.0f && m <= 3.0e38f) frexpf(m, &e);  // m = f 2^e, f in [0.5, 1)
  const float v = ldexpf(x, -e);
  const _Float16 hi = static_cast<_Float16>(v);
  const std::size_t i = x16_index(2u * s, c);
  x16[i] = hi;
  x16[i + 8u] = static_cast<_Float16>(v - static_cast<float>(hi));  // column 2 s + 1: lane + 1
  if (threadIdx.x == 0u) x16_tail(x16, cols).e[s * (cols / 256u) + b] = e;
}

// Sequences >= batch: zero columns, exponent 0, sum of squares 0.
__device__ __forceinline__ void stage_block_zero(std::uint32_t s, std::uint32_t b, std::uint32_t c,
                                                 std::uint32_t cols, _Float16* x16) {
  const std::size_t i = x16_index(2u * s, c);
  x16[i] = x16[i + 8u] = static_cast<_Float16>(0.0f);
  if (threadIdx.x == 0u) {
    const X16Tail t = x16_tail(x16, cols);
    t.e[s * (cols / 256u) + b] = 0;
    t.ss[s * (cols / 256u) + b] = 0.0f;
  }
}

// Plain staging of x [batch][cols]; grid (cols / 256, 8).
__global__ __launch_bounds__(kStageThreads) void stage_batch_kernel(const float* __restrict__ x, std::uint32_t batch,
                                                                    std::uint32_t cols, _Float16* __restrict__ x16) {
  __shared__ float part[kStageThreads / 64u];
  const std::uint32_t b = blockIdx.x, s = blockIdx.y, c = 256u * b + threadIdx.x;
  if (b == 0u && s == 0u && threadIdx.x == 0u) *x16_tail(x16, cols).eps = -1.0f;
  if (s >= batch) {
    stage_block_zero(s, b, c, cols, x16);
    return;
  }
  stage_block_value(x[static_cast<std::size_t>(s) * cols + c], s, b, c, cols, x16, part);
}

// Residual + RMSNorm staging of one batch step: v = embed ? dequant(embed
// [token[s]]) : h[s] (+ the panel groups' partial sums res[g][s] in group
// order, when res is set); h[s] = v; x16 = rmsnorm-staged v * w (the block's
// sum of v^2 in ss, the 1 / rms left to the consumer).
struct RmsStageArgs {
  float* h;              // [batch][cols]
  const float* res;      // [groups][batch][cols] or null
  std::uint32_t groups;
  const std::uint8_t* embed;  // Q5_K [vocab][cols] or null
  const std::uint32_t* token;
  std::uint32_t vocab;
  const float* w;        // [cols] or null
  float eps;
  std::uint32_t cols, batch;
  _Float16* x16;
};

__global__ __launch_bounds__(kStageThreads) void rms_stage_batch_kernel(RmsStageArgs a) {
  __shared__ float part[kStageThreads / 64u];
  const std::uint32_t b = blockIdx.x, s = blockIdx.y, c = 256u * b + threadIdx.x, cols = a.cols;
  const int tl_r = a.res != nullptr && a.groups == 1u ? kTlRmsStageO : kTlRmsStageOther;
  const std::uint32_t tl_slot = ((s * gridDim.x + b) * (kStageThreads / 64u) + (threadIdx.x >> 6)) * 2u;
  tl_stamp(tl_r, tl_slot);
  if (b == 0u && s == 0u && threadIdx.x == 0u) *x16_tail(a.x16, cols).eps = a.eps;
  if (s >= a.batch) {
    stage_block_zero(s, b, c, cols, a.x16);
    return;
  }
  float* const hs = a.h + static_cast<std::size_t>(s) * cols;
  const float wmul = a.w != nullptr ? a.w[c] : 1.0f;  // read before the reductions' barriers
  float x;
  if (a.embed != nullptr) {
    const std::uint32_t tok = a.token[s] < a.vocab ? a.token[s] : a.vocab - 1u;
    const std::uint8_t* blk = a.embed + (static_cast<std::size_t>(tok) * (cols / 256u) + b) * 176u;
    x = dequant_value<RTXLLM_FMT_Q5K>(blk, nullptr, threadIdx.x);
  } else {
    x = hs[c];
  }
  if (a.res != nullptr) {
    // the panel groups' partials, up to eight read at once (a runtime loop
    // would wait for each before reading the next), added in group order
    typedef float f32x8 __attribute__((ext_vector_type(8)));
    f32x8 r;
#pragma unroll
    for (int g = 0; g < 8; ++g) {
      const std::uint32_t gg = static_cast<std::uint32_t>(g) < a.groups ? static_cast<std::uint32_t>(g) : a.groups - 1u;
      r[g] = a.res[(static_cast<std::size_t>(gg) * a.batch + s) * cols + c];
    }
#pragma unroll
    for (int g = 0; g < 8; ++g) x = static_cast<std::uint32_t>(g) < a.groups ? x + r[g] : x;
    for (std::uint32_t g = 8; g < a.groups; ++g) x += a.res[(static_cast<std::size_t>(g) * a.batch + s) * cols + c];
  }
  if (a.embed != nullptr || a.res != nullptr) hs[c] = x;
  const float ss = block_reduce(x * x, part, false);
  if (threadIdx.x == 0u) x16_tail(a.x16, cols).ss[s * (cols / 256u) + b] = ss;
  stage_block_value(a.w != nullptr ? x * wmul : x, s, b, c, cols, a.x16, part);
  tl_stamp(tl_r, tl_slot + 1u);
}

// ---- batch epilogues --------------------------------------------------------

// q | k | v rows (q_rows + 2 kv_rows): RoPE at the sequence's position on q and
// k (pairs of adjacent rows), q -> q[s], k and v -> the fp16 cache slot of
// (sequence s, its position); the rule of the batch-1 qkv epilogue.
struct MmQkv {
  static constexpr int tl_region(int) { return kTlMmQkv; }
  std::uint32_t q_rows, kv_rows, batch, table_stride, rope_positions, group;
  const float2* rope;
  const std::uint32_t* pos_ptr;
  _Float16* q;  // q16 of sequence 0; sequence s kv.n_kv * kQ16PerKv values on
  KvLayer kv;
  std::uint32_t pos;
  __device__ __forceinline__ void init(std::uint32_t s) { pos = s < batch ? pos_ptr[s] : 0u; }
  __device__ __forceinline__ void operator()(std::uint32_t row, std::uint32_t s, float y, float partner) const {
    if (row >= q_rows && pos >= kv.capacity) return;  // no slot for this position
    const std::int32_t* table = kv.block_table + static_cast<std::size_t>(s) * table_stride;
    if (row < q_rows + kv_rows) {
      const std::uint32_t d = row & (kHeadDim - 1u);
      const float2 r = rope_at(rope, rope_positions, pos, d >> 1);
      const float out = (d & 1u) ? (partner * r.y + y * r.x) : (y * r.x - partner * r.y);
      if (row < q_rows) {
        q16_store(q + static_cast<std::size_t>(s) * kv.n_kv * kQ16PerKv, row / kHeadDim, group, d, out);
      } else {
        const std::uint32_t kr = row - q_rows;
        kv.k[kv_offset(kv, table, pos, kr / kHeadDim) + (kr & (kHeadDim - 1u))] = f2h(out);
      }
    } else {
      const std::uint32_t vr = row - q_rows - kv_rows;
      kv.v[kv_offset(kv, table, pos, vr / kHeadDim) + (vr & (kHeadDim - 1u))] = f2h(y);
    }
  }
  __device__ __forceinline__ void finish(std::uint32_t, std::uint32_t, std::uint32_t) {}
};

// Interleaved gate / up rows: act[s][i] = silu(gate_i) * up_i.
struct MmGateUp {
  static constexpr int tl_region(int) { return kTlMmGateUp; }
  float* act;
  std::uint32_t stride;
  __device__ __forceinline__ void init(std::uint32_t) {}
  __device__ __forceinline__ void operator()(std::uint32_t row, std::uint32_t s, float y, float partner) const {
    if ((row & 1u) == 0u) act[static_cast<std::size_t>(s) * stride + (row >> 1)] = silu(y) * partner;
  }
  __device__ __forceinline__ void finish(std::uint32_t, std::uint32_t, std::uint32_t) {}
};

// Logits of every sequence and, per workgroup and sequence, four argmax keys
// (one per epilogue wave slot) at keys[s * key_stride + 4 blockIdx.x + w].
// A thread keeps the best key of its rows; lanes 8 s .. 8 s + 3 of a wave are
// sequence s's.
struct MmLogits {
  static constexpr int tl_region(int) { return kTlMmLogits; }
  float* logits;
  std::uint32_t stride, batch;
  unsigned long long* keys;
  std::uint32_t key_stride;
  unsigned long long best;
  __device__ __forceinline__ void init(std::uint32_t) { best = 0ull; }
  __device__ __forceinline__ void operator()(std::uint32_t row, std::uint32_t s, float y, float) {
    logits[static_cast<std::size_t>(s) * stride + row] = y;
    const unsigned long long k = argmax_key(y, row);
    best = k > best ? k : best;
  }
  __device__ __forceinline__ void finish(std::uint32_t wave, std::uint32_t lane, std::uint32_t nw) const {
    unsigned long long k = best, o = __shfl_xor(k, 1, 64);
    k = o > k ? o : k;
    o = __shfl_xor(k, 2, 64);
    k = o > k ? o : k;
    const std::uint32_t s = (lane >> 3) & 7u;
    if ((lane & 7u) != 0u || s >= batch) return;
    unsigned long long* slot = keys + static_cast<std::size_t>(s) * key_stride + 4u * blockIdx.x;
    if (wave < 4u) slot[wave] = k;
    if (wave == 0u)
      for (std::uint32_t w2 = nw; w2 < 4u; ++w2) slot[w2] = 0ull;  // slots of waves the workgroup lacks
  }
};

// Workgroups of mm_kernel<FMT, Epi> of `threads` threads resident per CU (0 if
// the query fails), cached per size.
template <int FMT, class Epi, bool SELF = false>
int mm_resident(std::uint32_t threads) {
  static int cache[kMaxPanels + 1] = {};
  const std::uint32_t w = threads / 64u;
  if (w == 0u || w > kMaxPanels) return 0;
  if (cache[w] == 0) {
    int n = 0;
    if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&n, reinterpret_cast<const void*>(&mm_kernel<FMT, Epi, SELF>),
                                                     static_cast<int>(threads), 0) != hipSuccess || n <= 0)
      return 0;
    cache[w] = n;
  }
  return cache[w];
}

struct MmGeom {
  std::uint32_t ppg, groups, grid;
};

// Panel split of a matrix: panels of 512 columns, ppg of them per workgroup
// (the largest divisor <= 8 of the panel count), groups = panels / ppg.
inline bool mm_split(int fmt, std::uint32_t rows, std::uint32_t cols, MmGeom& g) {
  if (!fmt_mm_supported(fmt) || rows == 0u || cols == 0u || (cols % kPanel) != 0u) return false;
  const std::uint32_t panels = cols / kPanel;
  g.ppg = 1u;
  for (std::uint32_t d = kMaxPanels; d >= 1u; --d)
    if (panels % d == 0u) {
      g.ppg = d;
      break;
    }
  g.groups = panels / g.ppg;
  return true;
}

// Persistent grid: the workgroups resident at once, shared by the panel groups,
// every workgroup taking the same number of tiles (but the last few).
template <int FMT, class Epi, bool SELF = false>
bool mm_geom(std::uint32_t rows, std::uint32_t cols, MmGeom& g) {
  if (!mm_split(FMT, rows, cols, g)) return false;
  const std::uint32_t tiles = (rows + 15u) / 16u;
  const int resident = mm_resident<FMT, Epi, SELF>(64u * g.ppg);
  const std::uint32_t per_cu = resident > 0 ? static_cast<std::uint32_t>(resident) : 1u;
  const std::uint32_t cap = std::max(1u, per_cu * static_cast<std::uint32_t>(num_cus()) / g.groups);
  const std::uint32_t rounds = (tiles + cap - 1u) / cap;
  g.grid = (tiles + rounds - 1u) / rounds;
  return true;
}

template <int FMT, bool SELF = false, class Epi>
hipError_t launch_mm_epi(const QTensor& w, const void* x16, std::uint32_t batch, const Epi& epi, bool one_group,
                         MmGeom* geom, hipStream_t stream) {
  MmGeom g;
  if (!mm_geom<FMT, Epi, SELF>(w.rows, w.cols, g) || batch == 0u || batch > kBatchMax || x16 == nullptr ||
      (one_group && g.groups != 1u))
    return hipErrorInvalidValue;
  const std::uint64_t blocks = static_cast<std::uint64_t>(w.rows) * (w.cols / 256u);
  if (blocks * FmtBytes<FMT>::payload > 0xFFFFFFFFull || blocks * FmtBytes<FMT>::meta > 0xFFFFFFFFull)
    return hipErrorInvalidValue;
  if (geom != nullptr) *geom = g;
  hipLaunchKernelGGL((mm_kernel<FMT, Epi, SELF>), dim3(g.grid, g.groups), dim3(64u * g.ppg), 0, stream, w, x16, batch,
                     epi);
  return hipGetLastError();
}

// SELF: x16 is the fp32 activation [batch][cols] (the kernel stages it).
template <class Epi, bool SELF = false>
hipError_t launch_mm(int fmt, const QTensor& w, const void* x16, std::uint32_t batch, const Epi& epi, bool one_group,
                     MmGeom* geom, hipStream_t stream) {
  switch (fmt) {
    case RTXLLM_FMT_IQ2S: return launch_mm_epi<RTXLLM_FMT_IQ2S, SELF>(w, x16, batch, epi, one_group, geom, stream);
    case RTXLLM_FMT_IQ3S: return launch_mm_epi<RTXLLM_FMT_IQ3S, SELF>(w, x16, batch, epi, one_group, geom, stream);
    case RTXLLM_FMT_Q5K: return launch_mm_epi<RTXLLM_FMT_Q5K, SELF>(w, x16, batch, epi, one_group, geom, stream);
    case RTXLLM_FMT_Q4K_RAW: return launch_mm_epi<RTXLLM_FMT_Q4K_RAW, SELF>(w, x16, batch, epi, one_group, geom, stream);
    case RTXLLM_FMT_Q4K_SPLIT_NATIVE:
      return launch_mm_epi<RTXLLM_FMT_Q4K_SPLIT_NATIVE, SELF>(w, x16, batch, epi, one_group, geom, stream);
    default: return hipErrorInvalidValue;
  }
}

template <class Epi>
bool mm_geometry(int fmt, std::uint32_t rows, std::uint32_t cols, MmGeom& g) {
  switch (fmt) {
    case RTXLLM_FMT_IQ2S: return mm_geom<RTXLLM_FMT_IQ2S, Epi>(rows, cols, g);
    case RTXLLM_FMT_IQ3S: return mm_geom<RTXLLM_FMT_IQ3S, Epi>(rows, cols, g);
    case RTXLLM_FMT_Q5K: return mm_geom<RTXLLM_FMT_Q5K, Epi>(rows, cols, g);
    case RTXLLM_FMT_Q4K_RAW: return mm_geom<RTXLLM_FMT_Q4K_RAW, Epi>(rows, cols, g);
    case RTXLLM_FMT_Q4K_SPLIT_NATIVE: return mm_geom<RTXLLM_FMT_Q4K_SPLIT_NATIVE, Epi>(rows, cols, g);
    default: return false;
  }
}

}  // namespace
}  // namespace rtxllm

using namespace rtxllm;

namespace rtxllm {

std::size_t mm_batch_workspace_bytes(int fmt, std::uint32_t rows, std::uint32_t cols) {
  MmGeom g;
  if (!mm_split(fmt, rows, cols, g) || g.groups == 1u) return 0u;
  return 4u * static_cast<std::size_t>(kBatchMax) * rows * g.groups;
}

std::uint32_t mm_panel_groups(int fmt, std::uint32_t rows, std::uint32_t cols) {
  MmGeom g;
  return mm_split(fmt, rows, cols, g) ? g.groups : 0u;
}

hipError_t launch_mm_batch(int fmt, const std::uint8_t* payload, const std::uint8_t* meta, std::uint32_t rows,
                           std::uint32_t cols, const void* x16, std::uint32_t batch, float* out, hipStream_t stream) {
  if (payload == nullptr || out == nullptr || (fmt == RTXLLM_FMT_Q4K_SPLIT_NATIVE && meta == nullptr))
    return hipErrorInvalidValue;
  const QTensor w{payload, meta, rows, cols};
  return launch_mm(fmt, w, x16, batch, MmStore{out, rows, batch}, false, nullptr, stream);
}

hipError_t launch_mm_batch_self(int fmt, const std::uint8_t* payload, const std::uint8_t* meta, std::uint32_t rows,
                                std::uint32_t cols, const float* x, std::uint32_t batch, float* out,
                                hipStream_t stream) {
  if (payload == nullptr || out == nullptr || (fmt == RTXLLM_FMT_Q4K_SPLIT_NATIVE && meta == nullptr) ||
      (reinterpret_cast<std::uintptr_t>(x) % 16u) != 0u)
    return hipErrorInvalidValue;
  const QTensor w{payload, meta, rows, cols};
  return launch_mm<MmStore, true>(fmt, w, x, batch, MmStore{out, rows, batch}, false, nullptr, stream);
}

hipError_t launch_mm_qkv_batch(int fmt, const std::uint8_t* payload, const std::uint8_t* meta, std::uint32_t cols,
                               const void* x16, std::uint32_t batch, std::uint32_t q_rows, std::uint32_t kv_rows,
                               const float2* rope, std::uint32_t rope_positions, const std::uint32_t* pos,
                               void* q_out, const KvLayer& kv, std::uint32_t table_stride, hipStream_t stream) {
  if (payload == nullptr || (fmt == RTXLLM_FMT_Q4K_SPLIT_NATIVE && meta == nullptr) || (q_rows % kHeadDim) != 0u ||
      (kv_rows % kHeadDim) != 0u || kv.page_size == 0u || table_stride < kv.capacity / kv.page_size ||
      rope == nullptr || rope_positions == 0u || kv.n_kv == 0u || q_rows % (kHeadDim * kv.n_kv) != 0u)
    return hipErrorInvalidValue;
  const QTensor w{payload, meta, q_rows + 2u * kv_rows, cols};
  MmQkv e{};
  e.q_rows = q_rows, e.kv_rows = kv_rows, e.batch = batch, e.table_stride = table_stride;
  e.rope = rope, e.rope_positions = rope_positions, e.pos_ptr = pos, e.q = static_cast<_Float16*>(q_out), e.kv = kv;
  e.group = q_rows / kHeadDim / kv.n_kv;
  return launch_mm(fmt, w, x16, batch, e, true, nullptr, stream);
}

hipError_t launch_mm_gate_up_batch(int fmt, const std::uint8_t* payload, const std::uint8_t* meta,
                                   std::uint32_t rows, std::uint32_t cols, const void* x16, std::uint32_t batch,
                                   float* act, hipStream_t stream) {
  if (payload == nullptr || (fmt == RTXLLM_FMT_Q4K_SPLIT_NATIVE && meta == nullptr) || (rows % 2u) != 0u)
    return hipErrorInvalidValue;
  const QTensor w{payload, meta, rows, cols};
  return launch_mm(fmt, w, x16, batch, MmGateUp{act, rows / 2u}, true, nullptr, stream);
}

std::uint32_t mm_logits_key_slots(int fmt, std::uint32_t rows, std::uint32_t cols) {
  MmGeom g;
  if (!mm_geometry<MmLogits>(fmt, rows, cols, g)) return 0u;
  return 4u * g.grid;
}

hipError_t launch_mm_logits_batch(int fmt, const std::uint8_t* payload, const std::uint8_t* meta, std::uint32_t rows,
                                  std::uint32_t cols, const void* x16, std::uint32_t batch, float* logits,
                                  unsigned long long* keys, std::uint32_t key_stride, std::uint32_t* key_count,
                                  hipStream_t stream) {
  const std::uint32_t slots = mm_logits_key_slots(fmt, rows, cols);
  if (payload == nullptr || (fmt == RTXLLM_FMT_Q4K_SPLIT_NATIVE && meta == nullptr) || keys == nullptr ||
      slots == 0u || slots > key_stride)
    return hipErrorInvalidValue;
  if (key_count != nullptr) *key_count = slots;
  const QTensor w{payload, meta, rows, cols};
  MmLogits e{};
  e.logits = logits, e.stride = rows, e.batch = batch, e.keys = keys, e.key_stride = key_stride;
  return launch_mm(fmt, w, x16, batch, e, true, nullptr, stream);
}

hipError_t launch_rms_stage_batch(float* h, const float* res, std::uint32_t groups, const std::uint8_t* embed,
                                  const std::uint32_t* token, std::uint32_t vocab, const float* w, float eps,
                                  std::uint32_t cols, std::uint32_t batch, void* x16, hipStream_t stream) {
  if (h == nullptr || x16 == nullptr || cols == 0u || (cols % 256u) != 0u || batch == 0u || batch > kBatchMax ||
      (res != nullptr && groups == 0u) || (embed != nullptr && (token == nullptr || vocab == 0u)) || !(eps >= 0.0f))
    return hipErrorInvalidValue;
  const RmsStageArgs a{h, res, groups, embed, token, vocab, w, eps, cols, batch, static_cast<_Float16*>(x16)};
  hipLaunchKernelGGL(rms_stage_batch_kernel, dim3(cols / 256u, kBatchMax), dim3(kStageThreads), 0, stream, a);
  return hipGetLastError();
}

hipError_t launch_stage_batch(const float* x, std::uint32_t batch, std::uint32_t cols, void* x16,
                              hipStream_t stream) {
  if (x == nullptr || x16 == nullptr || batch == 0u || batch > kBatchMax || cols == 0u || (cols % 256u) != 0u)
    return hipErrorInvalidValue;
  hipLaunchKernelGGL(stage_batch_kernel, dim3(cols / 256u, kBatchMax), dim3(kStageThreads), 0, stream, x, batch, cols,
                     static_cast<_Float16*>(x16));
  return hipGetLastError();
}

}  // namespace rtxllm

extern "C" size_t rtxllm_x16_bytes(uint32_t cols) { return x16_bytes(cols); }

extern "C" hipError_t rtxllm_stage_batch(const float* x, uint32_t batch, uint32_t cols, void* x16,
                                         hipStream_t stream) {
  return launch_stage_batch(x, batch, cols, x16, stream);
}

extern "C" size_t rtxllm_matvec_batch_workspace(int format, uint32_t rows, uint32_t cols) {
  return mm_batch_workspace_bytes(format, rows, cols);
}

namespace {

// x16 is the staged buffer, or with self_stage the fp32 activation [batch][cols].
hipError_t matvec_batch(int format, const uint8_t* payload, const uint8_t* meta, const void* x, bool self_stage,
                        float* y, uint32_t rows, uint32_t cols, uint32_t batch, void* workspace,
                        size_t workspace_bytes, hipStream_t stream) {
  if (y == nullptr || batch == 0u || batch > kBatchMax) return hipErrorInvalidValue;
  const std::uint32_t groups = mm_panel_groups(format, rows, cols);
  if (groups == 0u) return hipErrorInvalidValue;
  const std::size_t n = static_cast<std::size_t>(batch) * rows;
  float* out = y;
  if (groups > 1u) {
    if (workspace == nullptr || workspace_bytes < 4u * n * groups) return hipErrorInvalidValue;
    out = static_cast<float*>(workspace);
  }
  hipError_t st = self_stage ? launch_mm_batch_self(format, payload, meta, rows, cols, static_cast<const float*>(x),
                                                    batch, out, stream)
                             : launch_mm_batch(format, payload, meta, rows, cols, x, batch, out, stream);
  if (st != hipSuccess || groups == 1u) return st;
  hipLaunchKernelGGL(mm_reduce_kernel, dim3(static_cast<unsigned>((n + 255u) / 256u)), dim3(256), 0, stream,
                     static_cast<const float*>(workspace), groups, static_cast<std::uint32_t>(n), y);
  return hipGetLastError();
}

}  // namespace

extern "C" hipError_t rtxllm_matvec_batch(int format, const uint8_t* payload, const uint8_t* meta, const void* x16,
                                          float* y, uint32_t rows, uint32_t cols, uint32_t batch, void* workspace,
                                          size_t workspace_bytes, hipStream_t stream) {
  return matvec_batch(format, payload, meta, x16, false, y, rows, cols, batch, workspace, workspace_bytes, stream);
}

// ---- allocation-free batched matvec ------------------------------------------
// The panel groups' partial sums of rtxllm_matvec_batch_noalloc go to this
// file-scope array instead of a caller's workspace: each GPU the library runs on
// holds its own copy until the process ends. Host code never passes the array's
// name to a kernel (on the host it is only a stand-in for the symbol); it
// passes the device address hipGetSymbolAddress returns for the current
// device, looked up on the entry point's first call on that device.
static __device__ __align__(256) std::uint8_t scratch[RTXLLM_NOALLOC_SCRATCH_BYTES];

namespace {

constexpr int kMaxDevices = 64;
std::mutex g_scratch_mu;
void* g_scratch[kMaxDevices] = {};

hipError_t scratch_address(void** out) {
  int dev = 0;
  hipError_t st = hipGetDevice(&dev);
  if (st != hipSuccess) return st;
  if (dev < 0 || dev >= kMaxDevices) return hipErrorInvalidDevice;
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (g_scratch[dev] == nullptr) {
    void* p = nullptr;
    st = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (st != hipSuccess) return st;
    if (p == nullptr) return hipErrorInvalidSymbol;
    g_scratch[dev] = p;
  }
  *out = g_scratch[dev];
  return hipSuccess;
}

}  // namespace

extern "C" hipError_t rtxllm_matvec_batch_noalloc(int format, const uint8_t* payload, const uint8_t* meta,
                                                  const void* x16, float* y, uint32_t rows, uint32_t cols,
                                                  uint32_t batch, hipStream_t stream) {
  if (batch == 0u || batch > kBatchMax) return hipErrorInvalidValue;
  const std::uint32_t groups = mm_panel_groups(format, rows, cols);
  if (groups == 0u) return hipErrorInvalidValue;
  const std::size_t need = groups > 1u ? 4u * static_cast<std::size_t>(batch) * rows * groups : 0u;
  if (need > RTXLLM_NOALLOC_SCRATCH_BYTES) return hipErrorInvalidValue;  // beyond the scratch array
  void* ws = nullptr;
  const hipError_t st = scratch_address(&ws);
  if (st != hipSuccess) return st;
  return matvec_batch(format, payload, meta, x16, false, y, rows, cols, batch, ws, RTXLLM_NOALLOC_SCRATCH_BYTES,
                      stream);
}

extern "C" hipError_t rtxllm_matvec_batch_f32(int format, const uint8_t* payload, const uint8_t* meta, const float* x,
                                              float* y, uint32_t rows, uint32_t cols, uint32_t batch, void* workspace,
                                              size_t workspace_bytes, hipStream_t stream) {
  if (x == nullptr) return hipErrorInvalidValue;
  return matvec_batch(format, payload, meta, x, true, y, rows, cols, batch, workspace, workspace_bytes, stream);
}

#ifdef RTXLLM_TIMELINE
namespace rtxllm {
hipError_t timeline_read_batch(unsigned long long* host) {
  return hipMemcpyFromSymbol(host, HIP_SYMBOL(g_timeline), sizeof(g_timeline), 0, hipMemcpyDeviceToHost);
}
hipError_t timeline_clear_batch() {
  void* p = nullptr;
  const hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(g_timeline));
  if (e != hipSuccess) return e;
  return hipMemset(p, 0, sizeof(g_timeline));
}
}  // namespace rtxllm
#endif
