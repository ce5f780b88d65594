// Llama decode-layer kernels for gfx950: the matvec epilogues that fuse RMSNorm
// scaling, RoPE, the fp16 KV-cache append, SiLU-gate multiply, residual add and
// next-norm staging into the producing matvec, plus the Q5_K embedding gather,
// split-context GQA attention and the greedy-token finalisation.
//
// The reference runtime has no Llama layer (its feedback kernels are
// unweighted RMSNorm / SiLU stand-ins, decode_kernels.cu:122-289, and its
// attention kernels are synthetic windows); the formulas here are the
// textbook Llama ones, restated on the CPU in oracle/rtxllm_oracle.c, with the
// reference's pieces where it has them: RMSNorm eps handling and inv-rms
// (main.cpp:1363-1382), SiLU v / (1 + exp(-v)) (main.cpp:1435-1503), the
// rotate-pair arithmetic (decode_kernels.cu:327-343) and the lowest-index
// argmax (decode_kernels.cu:2993-3031).
#include <cfloat>

#include "dequant.cuh"
#include "layer.h"
#include "layer_common.cuh"
#include "mv_launch.cuh"
#include "mvq.cuh"
#include "x16.h"

namespace rtxllm {
namespace {

__device__ __forceinline__ int wave_sum_i(int v) {
  return static_cast<int>(lanes_reduce_exact(static_cast<std::uint32_t>(v), [](std::uint32_t a, std::uint32_t b) {
    return a + b;  // two's complement: the same bits as the int sum
  }));
}

// 1 / sqrt(sum / n + eps) from the producer's partial sums of squares, in two
// steps so that the matvec's prologue issues its own loads behind these:
// rms_issue reads the first 256 partials (four per lane, not yet used; the
// launchers refuse nslots = 0, so the clamped index stays in the array) and
// rms_finish adds them, and any further ones, once the prologue has waited for
// its loads. Every lane (and every wave of every kernel) adds the partials in
// the same order, sumsq[lane], sumsq[lane + 64], ..., so all consumers see the
// same value.
struct RmsPartials {
  float v[4];
};
__device__ __forceinline__ RmsPartials rms_issue(const float* __restrict__ sumsq, std::uint32_t nslots,
                                                 std::uint32_t lane) {
  RmsPartials p;
#pragma unroll
  for (std::uint32_t j = 0; j < 4u; ++j) {
    const std::uint32_t i = lane + 64u * j;
    p.v[j] = sumsq[i < nslots ? i : nslots - 1u];  // masked in rms_finish
  }
  return p;
}
__device__ __forceinline__ float rms_finish(const RmsPartials& p, const float* __restrict__ sumsq,
                                            std::uint32_t nslots, std::uint32_t n, float eps, std::uint32_t lane) {
  float s = 0.0f;
  if (lane < nslots) {
#pragma unroll
    for (std::uint32_t j = 0; j < 4u; ++j) s += lane + 64u * j < nslots ? p.v[j] : 0.0f;
  }
  for (std::uint32_t i0 = lane + 256u; i0 < nslots; i0 += 256u) {
    float v[4];
#pragma unroll
    for (std::uint32_t j = 0; j < 4u; ++j) {
      const std::uint32_t i = i0 + 64u * j;
      const float t = sumsq[i < nslots ? i : nslots - 1u];
      v[j] = i < nslots ? t : 0.0f;
    }
#pragma unroll
    for (std::uint32_t j = 0; j < 4u; ++j) s += v[j];
  }
  s = wave_sum(s);
  return 1.0f / sqrtf(s / static_cast<float>(n) + eps);
}

// Stage one 16-value group held by the 16 lanes with owner = true (lane i of
// them holds value x of index `idx`; non-owners pass x = 0): the quant16 rule,
// evaluated with wave reductions (max and integer sum are order independent,
// so the digits equal quant16's). g0 = first index of the group.
__device__ __forceinline__ void stage_group16(const XQOut& xq, std::uint32_t g0, std::uint32_t idx, float x,
                                              bool owner, std::uint32_t lane) {
  const float m = wave_max(fabsf(x));
  const bool nan = __ballot(owner && x != x) != 0ull;
  const XScale sc = xq_scale(m, nan);
  const int X = xq_fixed(x, sc);
  int H, M, L;
  xq_digits(X, H, M, L);
  const int total = wave_sum_i(owner ? X : 0);
  if (owner) {
    xq.h[idx] = static_cast<std::int8_t>(H);
    xq.m[idx] = static_cast<std::int8_t>(M);
    xq.l[idx] = static_cast<std::int8_t>(L);
  }
  if (lane == 0u) {
    const std::uint32_t t = g0 / kXGroup;
    xq.s[t] = sc.s;
    xq.sum[t] = sc.s * static_cast<float>(total);
  }
}

// ---- epilogues (TILE 4: row r of a tile in lanes [16 r, 16 r + 16)) ---------

struct EpiQkv {
  static constexpr int tl_region(int) { return kTlQkv; }
  static constexpr int kTile = 4;
  const float* sumsq;
  std::uint32_t nslots, n;
  float eps;
  std::uint32_t q_rows, kv_rows, rope_positions, group;
  const float2* rope;
  const std::uint32_t* pos_ptr;
  _Float16* q;  // q16 operand order
  KvLayer kv;
  float scale;
  std::uint32_t pos;
  RmsPartials rp;
  __device__ __forceinline__ void init(std::uint32_t lane) {
    rp = rms_issue(sumsq, nslots, lane);
    pos = *pos_ptr;
  }
  __device__ __forceinline__ void ready(std::uint32_t lane) { scale = rms_finish(rp, sumsq, nslots, n, eps, lane); }
  __device__ __forceinline__ void operator()(std::uint32_t row0, float v, std::uint32_t lane, std::uint32_t rows) const {
    const std::uint32_t row = row0 + (lane >> 4);
    const float y = v * scale;
    const float partner = __shfl_xor(y, 16, 64);  // row ^ 1: the other element of a rotary pair
    if ((lane & 15u) != 0u || row >= rows) return;
    if (row >= q_rows && pos >= kv.capacity) return;  // no slot for this position
    if (row < q_rows + kv_rows) {
      const std::uint32_t d = row & (kHeadDim - 1u);
      const float2 r = rope_at(rope, rope_positions, pos, d >> 1);  // (cos, sin)
      // (e, o) -> (e c - o s, e s + o c)
      const float out = (d & 1u) ? (partner * r.y + y * r.x) : (y * r.x - partner * r.y);
      if (row < q_rows) {
        q16_store(q, row / kHeadDim, group, d, out);
      } else {
        const std::uint32_t kr = row - q_rows;
        kv.k[kv_offset(kv, kv.block_table, pos, kr / kHeadDim) + (kr & (kHeadDim - 1u))] = f2h(out);
      }
    } else {
      const std::uint32_t vr = row - q_rows - kv_rows;
      kv.v[kv_offset(kv, kv.block_table, pos, vr / kHeadDim) + (vr & (kHeadDim - 1u))] = f2h(y);
    }
  }
};

struct EpiGateUp {
  static constexpr int kTile = 4;
  const float* sumsq;
  std::uint32_t nslots, n;
  float eps;
  float* act;
  float scale;
  RmsPartials rp;
  __device__ __forceinline__ void init(std::uint32_t lane) { rp = rms_issue(sumsq, nslots, lane); }
  __device__ __forceinline__ void ready(std::uint32_t lane) { scale = rms_finish(rp, sumsq, nslots, n, eps, lane); }
  __device__ __forceinline__ void operator()(std::uint32_t row0, float v, std::uint32_t lane, std::uint32_t rows) const {
    const std::uint32_t row = row0 + (lane >> 4);
    const float y = v * scale;
    const float up = __shfl_xor(y, 16, 64);
    if ((lane & 31u) == 0u && row < rows) act[row >> 1] = silu(y) * up;
  }
};

// The same epilogue for hidden sizes of at most kShareXCols: workgroups of up
// to 16 waves (one per CU at the 8B shapes) share one LDS copy of the staged
// input and of the codebook, their row groups handing over column-split
// partials pairwise (a hand-over wait that runs out sets kStatusWaitTimeout in
// *wait.status).
struct EpiGateUpWide : EpiGateUp {
  static constexpr std::uint32_t kWaves = 16;
  static constexpr bool kShareX = true;
  PairWait wait;
};

// Logits and the greedy argmax: each row group keeps the best key of its tiles
// in a register and stores it once, after its last tile, into its own slot;
// the finalize kernel reduces the slots (no atomics, no per-tile reads).
struct EpiLogits {
  static constexpr int tl_region(int) { return kTlLogits; }
  static constexpr int kTile = 4;
  static constexpr bool kFinish = true;
  const float* sumsq;
  std::uint32_t nslots, n;
  float eps;
  float* logits;
  unsigned long long* keys;
  float scale;
  unsigned long long best;
  RmsPartials rp;
  __device__ __forceinline__ void init(std::uint32_t lane) {
    rp = rms_issue(sumsq, nslots, lane);
    best = 0ull;
  }
  __device__ __forceinline__ void ready(std::uint32_t lane) { scale = rms_finish(rp, sumsq, nslots, n, eps, lane); }
  __device__ __forceinline__ void operator()(std::uint32_t row0, float v, std::uint32_t lane, std::uint32_t rows) {
    const std::uint32_t row = row0 + (lane >> 4);
    const float y = v * scale;
    const bool ok = row < rows;
    if ((lane & 15u) == 0u && ok) logits[row] = y;
    unsigned long long key = ok ? argmax_key(y, row) : 0ull;
    unsigned long long other = __shfl_xor(key, 16, 64);
    key = other > key ? other : key;
    other = __shfl_xor(key, 32, 64);
    key = other > key ? other : key;  // every lane: the tile's best
    best = key > best ? key : best;
  }
  __device__ __forceinline__ void finish(std::uint32_t slot, std::uint32_t lane) const {
    if (lane == 0u) keys[slot] = best;
  }
};

// Residual add and next-norm staging over 16-row groups (one staged group of
// the next matvec's input): lane i < 16 of wave 0 owns row row0 + i.
struct EpiResidual {
  static constexpr int tl_region(int fmt) { return fmt_is_iq(fmt) ? kTlResidualIq : kTlResidualK; }
  static constexpr int kTile = 4;
  static constexpr std::uint32_t kGroupRows = kXGroup;
  float* h;
  const float* w_next;
  XQOut xq;
  float* sumsq;
  // h and w_next of the workgroup's first group (group blockIdx.x), read at
  // the kernel's start so that its epilogue waits on no load
  std::uint32_t pf_row0;
  float pf_h, pf_w;
  __device__ __forceinline__ void init(std::uint32_t lane) {
    pf_row0 = blockIdx.x * kXGroup;
    const std::uint32_t row = pf_row0 + (lane < kXGroup ? lane : 0u);
    pf_h = h[row];
    pf_w = w_next != nullptr ? w_next[row] : 1.0f;
  }
  __device__ __forceinline__ void group(std::uint32_t row0, const float* vals, std::uint32_t lane,
                                        std::uint32_t) const {
    const bool owner = lane < kXGroup;
    const std::uint32_t row = row0 + (owner ? lane : 0u);
    const bool pf = row0 == pf_row0;
    const float h0 = pf ? pf_h : h[row];
    const float wn = pf ? pf_w : (w_next != nullptr ? w_next[row] : 1.0f);
    const float hn = h0 + (owner ? vals[lane] : 0.0f);
    if (owner) h[row] = hn;
    const float sq = wave_sum(owner ? hn * hn : 0.0f);
    // stage the 16-value group h * w_next (w_next null: h itself, times 1)
    const float x = owner ? hn * wn : 0.0f;
    stage_group16(xq, row0, row, x, owner, lane);
    if (lane == 0u) sumsq[row0 / kXGroup] = sq;
  }
};

// ---- embedding gather ----------------------------------------------------------

// One workgroup, thread g handles values [16 g, 16 g + 16) of the row.
__global__ __launch_bounds__(1024) void embed_q5k_kernel(const std::uint8_t* __restrict__ table, std::uint32_t cols,
                                                         std::uint32_t vocab, const std::uint32_t* __restrict__ token,
                                                         float* __restrict__ h,
                                                         const float* __restrict__ wnorm, XQOut xq,
                                                         float* __restrict__ sumsq, std::uint32_t nslots) {
  __shared__ float part[16];
  const std::uint32_t g = threadIdx.x, groups = cols / kXGroup;
  float sq = 0.0f;
  if (g < groups) {
    const std::uint32_t c0 = kXGroup * g;
    float v[16];
    if (table != nullptr) {
      const std::size_t row = token[0] < vocab ? token[0] : vocab - 1u;
      const std::uint8_t* blk = table + (row * (cols / 256u) + c0 / 256u) * 176u;
      dequant_q5k_run16(blk, (c0 & 255u) / 16u, v);
#pragma unroll
      for (int j = 0; j < 16; j += 4)
        *reinterpret_cast<float4*>(h + c0 + j) = make_float4(v[j], v[j + 1], v[j + 2], v[j + 3]);
    } else {
#pragma unroll
      for (int j = 0; j < 16; ++j) v[j] = h[c0 + j];
    }
    float x[16];
#pragma unroll
    for (int j = 0; j < 16; ++j) {
      sq += v[j] * v[j];
      x[j] = wnorm != nullptr ? v[j] * wnorm[c0 + j] : v[j];
    }
    XG st;
    quant16(x, st);
    xg_store(xq, g, st);
  }
  sq = wave_sum(sq);
  if ((threadIdx.x & 63u) == 0u) part[threadIdx.x >> 6] = sq;
  __syncthreads();
  for (std::uint32_t i = threadIdx.x + 1u; i < nslots; i += blockDim.x) sumsq[i] = 0.0f;
  if (threadIdx.x == 0u) {
    float s = 0.0f;
    for (std::uint32_t i = 0; i < blockDim.x / 64u; ++i) s += part[i];
    sumsq[0] = s;
  }
}

// ---- attention -------------------------------------------------------------------

constexpr std::uint32_t kAttnWaves = 8;                // waves per workgroup
constexpr std::uint32_t kAttnSub = 16;                 // positions per wave
constexpr std::uint32_t kAttnChunk = kAttnWaves * kAttnSub;  // positions per workgroup
constexpr std::uint32_t kMaxGroup = 8;

// One workgroup of 8 waves per (chunk c of 128 positions, kv head g): the
// `GROUP` query heads of g over positions [128 c, 128 c + 128) ∩ [0, pos]. Wave
// w takes positions [128 c + 16 w, +16); all its K and V loads are issued up
// front. Then:
//  * scores on the matrix cores: S = K q^T for the 16 positions and every head
//    at once, four v_mfma_f32_16x16x32_f16 over the 128 dims. A = the K rows
//    (lane = (position r = l % 16, dims [32 (l / 16), +32)), fp16 as stored);
//    B = q / sqrt(128) of head n / 2 as an fp16 hi (n even) / lo (n odd) pair,
//    column n of 16 (columns >= 2 GROUP zero), so every product is exact and
//    the pair carries ~22 bits of q; C[position][n] summed over the pair;
//  * softmax of every head at once: the lanes of column 2 h hold head h's
//    scores for positions 4 (l / 16) + i, i < 4: max and sum over i and two
//    xor-shuffles;
//  * o = sum_p p_p v_p: lane = dimension pair, V rows coalesced (256 B per
//    position), p_p taken by readlane;
//  * the 8 wave records merge in LDS into the chunk's record (m, l, o[128]) per
//    head: M = max m_w, l = sum e^{m_w - M} l_w, o = sum e^{m_w - M} o_w.
//
// Sequence blockIdx.z of a batch: its q, block-table row, position and
// partial records are q_stride floats, table_stride entries, one word and
// part_stride floats past those of sequence 0.
//
// EARLY_V (the batch launches): the V loads are issued before the scores,
// which then wait for K and q only; measured faster for eight sequences and
// slower for one.
template <int GROUP, bool EARLY_V>
__global__ __launch_bounds__(64 * kAttnWaves) void attn_partial_kernel(const _Float16* __restrict__ q, KvLayer kv,
                                                                       const std::uint32_t* __restrict__ pos_ptr,
                                                                       std::uint32_t nchunks,
                                                                       float* __restrict__ partials,
                                                                       std::uint32_t q_stride,
                                                                       std::uint32_t table_stride,
                                                                       std::uint32_t part_stride) {
  typedef _Float16 half8 __attribute__((ext_vector_type(8)));
  typedef float f32x4 __attribute__((ext_vector_type(4)));
  __shared__ float wrec[kAttnWaves][GROUP][kHeadDim + 2u];
  const std::uint32_t c = blockIdx.x, g = blockIdx.y, lane = threadIdx.x & 63u;
  const int tl_r = gridDim.z == 1u ? kTlAttnPartial : kTlAttnPartialB;
  const std::uint32_t tl_slot =
      (((blockIdx.z * gridDim.y + blockIdx.y) * gridDim.x + blockIdx.x) * kAttnWaves + (threadIdx.x >> 6)) * 4u;
  tl_stamp(tl_r, tl_slot);
  const std::uint32_t seq = blockIdx.z;
  q += static_cast<std::size_t>(seq) * q_stride;
  partials += static_cast<std::size_t>(seq) * part_stride;
  const std::int32_t* const table = kv.block_table + static_cast<std::size_t>(seq) * table_stride;
  const std::uint32_t wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const std::uint32_t p0 = c * kAttnChunk;
  const std::uint32_t wp0 = p0 + kAttnSub * wave;
  const std::uint32_t r = lane & 15u, qq = lane >> 4;
  // B operands, staged by the qkv epilogue (q16): column n = lane % 16 is
  // head n / 2 (hi n even, lo n odd), rows = dims 32 qq + 8 j + i (A's order).
  // Read first: they depend on nothing below.
  uint4 qb[4];
  {
    const uint4* qr = reinterpret_cast<const uint4*>(q + static_cast<std::size_t>(g) * kQ16PerKv) + lane;
#pragma unroll
    for (int j = 0; j < 4; ++j) qb[j] = qr[64 * j];
  }
  // The lane's position and the chunk's first position, clamped into the
  // cache, and their block-table entries are read together with the position:
  // none of these loads waits for another.
  const std::uint32_t pc = p0 < kv.capacity ? p0 : kv.capacity - 1u;
  const std::uint32_t pr = wp0 + r < kv.capacity ? wp0 + r : kv.capacity - 1u;
  const std::uint32_t page_c = static_cast<std::uint32_t>(table[pc / kv.page_size]);
  const std::uint32_t page_r = static_cast<std::uint32_t>(table[pr / kv.page_size]);
  const std::uint32_t pos = pos_ptr[seq] < kv.capacity ? pos_ptr[seq] : kv.capacity - 1u;
  float* rec = partials + (static_cast<std::size_t>(g) * nchunks + c) * GROUP * (kHeadDim + 2u);
  if (p0 > pos) {  // chunk beyond the context (uniform over the workgroup): empty record
    for (std::uint32_t i = threadIdx.x; i < GROUP * (kHeadDim + 2u); i += blockDim.x)
      rec[i] = (i % (kHeadDim + 2u)) == 0u ? -INFINITY : 0.0f;
    tl_stamp(tl_r, tl_slot + 3u);
    return;
  }
  // K / V row offset (elements; the host checks that a layer's cache has fewer
  // than 2^32 of them). A position past the context reads the chunk's first
  // row (inside the context, so finite data) and is weighted 0.
  auto row_of = [&](std::uint32_t page, std::uint32_t p) {
    return static_cast<std::uint32_t>(((static_cast<std::size_t>(page) * kv.n_kv + g) * kv.page_size +
                                       p % kv.page_size) * kHeadDim);
  };
  const std::uint32_t row_off = wp0 + r <= pos ? row_of(page_r, pr) : row_of(page_c, pc);
  uint4 ka[4];  // A operands: K[position r][32 qq + 8 j + i]
  {
    const uint4* kr = reinterpret_cast<const uint4*>(kv.k + row_off + 32u * qq);
#pragma unroll
    for (int j = 0; j < 4; ++j) ka[j] = kr[j];
  }
  if constexpr (EARLY_V) __builtin_amdgcn_sched_barrier(0);  // K ahead of V: the scores wait for no V load
  std::uint32_t vw[kAttnSub];
#pragma unroll
  for (int j = 0; j < static_cast<int>(kAttnSub); ++j) {
    const std::uint32_t off = static_cast<std::uint32_t>(__builtin_amdgcn_readlane(static_cast<int>(row_off), j));
    vw[j] = *reinterpret_cast<const std::uint32_t*>(kv.v + off + 2u * lane);
  }
  if constexpr (EARLY_V) __builtin_amdgcn_sched_barrier(0);  // every V load issued before the scores
  f32x4 sc = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
  for (int j = 0; j < 4; ++j)
    sc = __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(half8, ka[j]), __builtin_bit_cast(half8, qb[j]), sc,
                                                0, 0, 0);
  // lane: column n, positions 4 qq + i; head hq's score = the hi + lo columns
  float s4[4], p4[4];
  float m = -INFINITY;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const float t = sc[i] + lane_xor<1>(sc[i]);
    const bool valid = wp0 + 4u * qq + static_cast<std::uint32_t>(i) <= pos;
    s4[i] = valid ? t : -INFINITY;
    m = fmaxf(m, s4[i]);
  }
  m = fmaxf(m, lane_xor<16>(m));
  m = fmaxf(m, lane_xor<32>(m));  // head max over the wave's positions (-inf: none)
  float l = 0.0f;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    p4[i] = s4[i] == -INFINITY ? 0.0f : expf(s4[i] - m);
    l += p4[i];
  }
  l += lane_xor<16>(l);
  l += lane_xor<32>(l);
  tl_stamp(tl_r, tl_slot + 1u);
  float o0[GROUP], o1[GROUP];
#pragma unroll
  for (int h = 0; h < GROUP; ++h) o0[h] = o1[h] = 0.0f;
#pragma unroll
  for (int j = 0; j < static_cast<int>(kAttnSub); ++j) {
    const float v0 = h2f(vw[j]), v1 = h2f(vw[j] >> 16);
#pragma unroll
    for (int h = 0; h < GROUP; ++h) {
      // p of position j, head h: lane 16 (j / 4) + 2 h, register j % 4
      const float p = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, p4[j & 3]),
                                                                          16 * (j >> 2) + 2 * h));
      o0[h] += p * v0;
      o1[h] += p * v1;
    }
  }
#pragma unroll
  for (int h = 0; h < GROUP; ++h)
    *reinterpret_cast<float2*>(&wrec[wave][h][2u + 2u * lane]) = make_float2(o0[h], o1[h]);
  if (lane < 2u * GROUP && (lane & 1u) == 0u) {
    wrec[wave][lane >> 1][0] = m;
    wrec[wave][lane >> 1][1] = l;
  }
  tl_stamp(tl_r, tl_slot + 2u);
  __syncthreads();
  // wave h merges head h's records
  if (wave >= static_cast<std::uint32_t>(GROUP)) {
    tl_stamp(tl_r, tl_slot + 3u);
    return;
  }
  {
    const std::uint32_t h = wave;
    float M = wrec[0][h][0];  // finite: wave 0 holds position p0
#pragma unroll
    for (std::uint32_t w = 1; w < kAttnWaves; ++w) M = fmaxf(M, wrec[w][h][0]);
    float L = 0.0f, a0 = 0.0f, a1 = 0.0f;
#pragma unroll
    for (std::uint32_t w = 0; w < kAttnWaves; ++w) {
      const float f = expf(wrec[w][h][0] - M);  // 0 for a wave without positions
      const float2 o = *reinterpret_cast<const float2*>(&wrec[w][h][2u + 2u * lane]);
      L += f * wrec[w][h][1];
      a0 += f * o.x;
      a1 += f * o.y;
    }
    float* rr = rec + h * (kHeadDim + 2u);
    *reinterpret_cast<float2*>(rr + 2u + 2u * lane) = make_float2(a0, a1);
    if (lane == 0u) {
      rr[0] = M;
      rr[1] = L;
    }
  }
  tl_stamp(tl_r, tl_slot + 3u);
}

constexpr std::uint32_t kCombinePass = 32;  // chunk records per combine pass

// Merge the chunk records (m_c, l_c, o_c) of one query head (head of its kv
// head's group) into the lane's two dimensions 2 lane, 2 lane + 1 of att =
// sum_c e^{m_c - M} o_c / sum_c e^{m_c - M} l_c; one wave. Per pass of 32
// chunks every load is issued up front: lane c reads chunk c's (m, l) (wave max
// / sum) and, as lane = dimension pair, the pass's 32 o_c rows; the weights are
// taken by readlane. Running sums are rescaled when a later pass raises the
// maximum.
__device__ __forceinline__ float2 combine_head(const float* __restrict__ partials, std::uint32_t group,
                                               std::uint32_t nchunks, std::uint32_t head, std::uint32_t lane) {
  const std::uint32_t g = head / group, hh = head % group;
  // every chunk record is merged: chunks past the context hold (-inf, 0, 0),
  // so the kernel needs no position and starts loading at once
  const std::uint32_t n = nchunks;
  const std::size_t stride = static_cast<std::size_t>(group) * (kHeadDim + 2u);
  const float* base = partials + static_cast<std::size_t>(g) * nchunks * stride + hh * (kHeadDim + 2u);
  float M = -INFINITY, L = 0.0f, o0 = 0.0f, o1 = 0.0f;
  for (std::uint32_t c0 = 0; c0 < n; c0 += kCombinePass) {
    const std::uint32_t cnt = n - c0 < kCombinePass ? n - c0 : kCombinePass;
    const std::uint32_t c = c0 + (lane < cnt ? lane : cnt - 1u);  // lanes >= cnt: masked below
    const float m_raw = base[c * stride], l_raw = base[c * stride + 1u];
    float2 ov[kCombinePass];
#pragma unroll
    for (std::uint32_t j = 0; j < kCombinePass; ++j) {
      const std::uint32_t cj = c0 + (j < cnt ? j : cnt - 1u);
      ov[j] = *reinterpret_cast<const float2*>(base + cj * stride + 2u + 2u * lane);
    }
    __builtin_amdgcn_sched_barrier(0);  // keep every load of the pass ahead of the reductions
    const bool ok = lane < cnt;
    const float m = ok ? m_raw : -INFINITY;
    const float Mn = fmaxf(M, wave_max(m));  // finite: chunk 0 always holds position 0
    const float r = expf(M - Mn);            // 0 on the first pass
    L *= r, o0 *= r, o1 *= r;
    const float w = ok ? expf(m - Mn) : 0.0f;
    L += wave_sum(ok ? w * l_raw : 0.0f);
    M = Mn;
#pragma unroll
    for (std::uint32_t j = 0; j < kCombinePass; ++j) {
      const float wj = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, w), static_cast<int>(j)));
      o0 += wj * ov[j].x;  // wj = 0 for j >= cnt
      o1 += wj * ov[j].y;
    }
  }
  return make_float2(o0 / L, o1 / L);
}

// One wave per query head (blockIdx.x): att of the head. Sequence blockIdx.y
// of a batch reads its records part_stride floats on and writes att (n_heads *
// head_dim per sequence) further on; xq (batch 1 only) is skipped when null.
__global__ __launch_bounds__(64) void attn_combine_kernel(const float* __restrict__ partials, std::uint32_t group,
                                                          std::uint32_t nchunks, float* __restrict__ att, XQOut xq,
                                                          std::uint32_t part_stride) {
  const std::uint32_t head = blockIdx.x, lane = threadIdx.x;
  partials += static_cast<std::size_t>(blockIdx.y) * part_stride;
  att += static_cast<std::size_t>(blockIdx.y) * gridDim.x * kHeadDim;
  const int tl_r = gridDim.y == 1u ? kTlAttnCombine : -1;
  tl_stamp(tl_r, head * 4u);
  const float2 a = combine_head(partials, group, nchunks, head, lane);
  tl_stamp(tl_r, head * 4u + 1u);
  const float a0 = a.x, a1 = a.y;
  const std::uint32_t d0 = head * kHeadDim + 2u * lane;
  *reinterpret_cast<float2*>(att + d0) = make_float2(a0, a1);
  if (xq.h == nullptr) return;  // the whole grid: a batch stages att separately
  // Stage att for the o projection: the 16-value group of dims [16 k, 16 k + 16)
  // is held by lanes [8 k, 8 k + 8), two values each (the quant16 rule; max and
  // integer sum are order independent, so the digits equal quant16's).
  // the group's max |att|, NaN flag and integer sum over its 8 lanes (DPP, no LDS)
  const float m = __uint_as_float(lanes_reduce_exact<8>(__float_as_uint(fmaxf(fabsf(a0), fabsf(a1))),
                                                        [](std::uint32_t a, std::uint32_t b) {
                                                          return __float_as_uint(fmaxf(__uint_as_float(a), __uint_as_float(b)));
                                                        }));
  const std::uint32_t nan = lanes_reduce_exact<8>(__builtin_isunordered(a0, a1) ? 1u : 0u,
                                                  [](std::uint32_t a, std::uint32_t b) { return a | b; });
  const XScale sc = xq_scale(m, nan != 0);
  const int X0 = xq_fixed(a0, sc), X1 = xq_fixed(a1, sc);
  int H0, M0, L0, H1, M1, L1;
  xq_digits(X0, H0, M0, L0);
  xq_digits(X1, H1, M1, L1);
  const int total = static_cast<int>(lanes_reduce_exact<8>(static_cast<std::uint32_t>(X0 + X1),
                                                           [](std::uint32_t a, std::uint32_t b) { return a + b; }));
  auto pair = [](int lo, int hi) {
    return static_cast<std::uint16_t>((static_cast<std::uint32_t>(lo) & 0xFFu) |
                                      ((static_cast<std::uint32_t>(hi) & 0xFFu) << 8));
  };
  *reinterpret_cast<std::uint16_t*>(xq.h + d0) = pair(H0, H1);
  *reinterpret_cast<std::uint16_t*>(xq.m + d0) = pair(M0, M1);
  *reinterpret_cast<std::uint16_t*>(xq.l + d0) = pair(L0, L1);
  if ((lane & 7u) == 0u) {
    const std::uint32_t t = d0 / kXGroup;
    xq.s[t] = sc.s;
    xq.sum[t] = sc.s * static_cast<float>(total);
  }
  tl_stamp(tl_r, head * 4u + 2u);
}

// Batch form with the o projection's staging fused: wave w of workgroup
// (b, s) combines head 2 b + w of sequence s, so the workgroup holds the 256
// columns of x16 block b (two heads): att, then the block's exponent from its
// max |att| and the hi / lo fp16 pairs in operand order (the rule of the batch
// staging kernel, no norm). Sequences s >= batch (grid y is 8) write zero
// columns and exponent 0.
__global__ __launch_bounds__(128) void attn_combine_x16_kernel(const float* __restrict__ partials, std::uint32_t group,
                                                               std::uint32_t nchunks, std::uint32_t batch,
                                                               float* __restrict__ att, _Float16* __restrict__ x16,
                                                               std::uint32_t part_stride) {
  __shared__ float pm[2];
  const std::uint32_t lane = threadIdx.x & 63u, wave = threadIdx.x >> 6;
  const std::uint32_t b = blockIdx.x, s = blockIdx.y, head = 2u * b + wave;
  const std::uint32_t cols = 2u * gridDim.x * kHeadDim, c0 = head * kHeadDim + 2u * lane;
  const std::uint32_t tl_slot = ((s * gridDim.x + b) * 2u + wave) * 2u;
  tl_stamp(kTlCombineB, tl_slot);
  const X16Tail tail = x16_tail(x16, cols);
  if (b == 0u && s == 0u && threadIdx.x == 0u) *tail.eps = -1.0f;
  if (s >= batch) {
#pragma unroll
    for (std::uint32_t j = 0; j < 2u; ++j) {
      const std::size_t i = x16_index(2u * s, c0 + j);
      x16[i] = x16[i + 8u] = static_cast<_Float16>(0.0f);
    }
    if (threadIdx.x == 0u) {
      tail.e[s * (cols / 256u) + b] = 0;
      tail.ss[s * (cols / 256u) + b] = 0.0f;
    }
    return;
  }
  const float2 a = combine_head(partials + static_cast<std::size_t>(s) * part_stride, group, nchunks, head, lane);
  *reinterpret_cast<float2*>(att + static_cast<std::size_t>(s) * cols + c0) = a;
  float m = wave_max(fmaxf(fabsf(a.x), fabsf(a.y)));
  if (lane == 0u) pm[wave] = m;
  __syncthreads();
  m = fmaxf(pm[0], pm[1]);
  int e = 0;
  if (m > 0.0f && m <= 3.0e38f) frexpf(m, &e);  // m = f 2^e, f in [0.5, 1)
  const float v[2] = {ldexpf(a.x, -e), ldexpf(a.y, -e)};
#pragma unroll
  for (std::uint32_t j = 0; j < 2u; ++j) {
    const _Float16 hi = static_cast<_Float16>(v[j]);
    const std::size_t i = x16_index(2u * s, c0 + j);
    x16[i] = hi;
    x16[i + 8u] = static_cast<_Float16>(v[j] - static_cast<float>(hi));  // column 2 s + 1
  }
  if (threadIdx.x == 0u) tail.e[s * (cols / 256u) + b] = e;
  tl_stamp(kTlCombineB, tl_slot + 1u);
}

// One workgroup of 256 per sequence (blockIdx.x, keys key_stride apart): the
// maximum of count keys, then token and position. A step that ran at a
// position >= capacity had no KV slot for its token: its token and position
// are left as they were and status gets kStatusContextFull.
__global__ __launch_bounds__(256) void argmax_finalize_kernel(const unsigned long long* __restrict__ keys,
                                                              std::uint32_t count, std::uint32_t* token,
                                                              std::uint32_t* pos, std::uint32_t advance,
                                                              std::uint32_t key_stride, std::uint32_t capacity,
                                                              std::uint32_t* status) {
  __shared__ unsigned long long part[4];
  keys += static_cast<std::size_t>(blockIdx.x) * key_stride;
  token += blockIdx.x;
  if (pos != nullptr) pos += blockIdx.x;
  if (status != nullptr) status += blockIdx.x;
  // the position, read before the reduction (only this kernel writes it, below)
  const std::uint32_t p_now = (threadIdx.x == 0u && pos != nullptr) ? pos[0] : 0u;
  unsigned long long best = 0ull;
  for (std::uint32_t i0 = threadIdx.x; i0 < count; i0 += 256u * 8u) {
    unsigned long long k[8];
#pragma unroll
    for (std::uint32_t j = 0; j < 8u; ++j) {
      const std::uint32_t i = i0 + 256u * j;
      k[j] = i < count ? keys[i] : 0ull;
    }
#pragma unroll
    for (std::uint32_t j = 0; j < 8u; ++j) best = k[j] > best ? k[j] : best;
  }
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) {
    const unsigned long long other = __shfl_xor(best, o, 64);
    best = other > best ? other : best;
  }
  if ((threadIdx.x & 63u) == 0u) part[threadIdx.x >> 6] = best;
  __syncthreads();
  if (threadIdx.x != 0u) return;
  for (int w = 1; w < 4; ++w) best = part[w] > best ? part[w] : best;
  if (pos != nullptr && p_now >= capacity) {
    if (status != nullptr) status[0] |= kStatusContextFull;
    return;
  }
  token[0] = best == 0ull ? 0u : 0xFFFFFFFFu - static_cast<std::uint32_t>(best & 0xFFFFFFFFull);
  if (pos != nullptr) pos[0] = p_now + advance;
}

// ---- device-side synthetic packs ------------------------------------------------

__global__ void synth_raw_kernel(int fmt, std::uint64_t seed, std::size_t n_blocks, float d_lo, float d_hi,
                                 std::uint8_t* out) {
  const std::size_t b = blockIdx.x * static_cast<std::size_t>(blockDim.x) + threadIdx.x;
  if (b >= n_blocks) return;
  const std::uint32_t bb = rtxllm_format_payload_bytes(fmt);
  rtxllm_synth_raw_blocks(fmt, seed, b, 1, d_lo, d_hi, out + b * bb);
}

__global__ void synth_q4k_native_kernel(std::uint64_t seed, std::size_t n_blocks, float d_lo, float d_hi,
                                        std::uint8_t* payload, std::uint8_t* meta) {
  const std::size_t b = blockIdx.x * static_cast<std::size_t>(blockDim.x) + threadIdx.x;
  if (b >= n_blocks) return;
  std::uint8_t blk[144];
  rtxllm_synth_raw_blocks(RTXLLM_FMT_Q4K_RAW, seed, b, 1, d_lo, d_hi, blk);
  for (int i = 0; i < 16; ++i) meta[b * 16u + i] = blk[i];
  for (int i = 0; i < 128; ++i) payload[b * 128u + i] = blk[16 + i];
}

}  // namespace

hipError_t launch_embed_q5k(const std::uint8_t* table, std::uint32_t cols, std::uint32_t vocab,
                            const std::uint32_t* token, float* h, const float* wnorm, void* xq, float* sumsq,
                            std::uint32_t nslots, hipStream_t stream) {
  if (cols == 0u || (cols % 256u) != 0u || cols > 16384u || nslots == 0u || vocab == 0u) return hipErrorInvalidValue;
  // the gather reads 16-byte fields of the 176-byte blocks and writes h by float4
  if ((reinterpret_cast<std::uintptr_t>(table) | reinterpret_cast<std::uintptr_t>(h)) % 16u != 0u)
    return hipErrorInvalidValue;
  const std::uint32_t threads = ((cols / kXGroup + 63u) / 64u) * 64u;  // whole waves
  hipLaunchKernelGGL(embed_q5k_kernel, dim3(1), dim3(threads), 0, stream, table, cols, vocab, token, h, wnorm,
                     xq_out(xq, cols), sumsq, nslots);
  return hipGetLastError();
}

hipError_t launch_qkv(int fmt, const std::uint8_t* payload, const std::uint8_t* meta, std::uint32_t cols,
                      const NormIn& in, std::uint32_t q_rows, std::uint32_t kv_rows, const float2* rope,
                      std::uint32_t rope_positions, const std::uint32_t* pos, void* q_out, const KvLayer& kv,
                      hipStream_t stream) {
  if (rope == nullptr || rope_positions == 0u || kv.n_kv == 0u || kv.page_size == 0u || in.nslots == 0u ||
      q_rows % (kHeadDim * kv.n_kv) != 0u)
    return hipErrorInvalidValue;
  const QTensor w{payload, meta, q_rows + 2u * kv_rows, cols};
  EpiQkv e{};
  e.sumsq = in.sumsq, e.nslots = in.nslots, e.n = in.n, e.eps = in.eps;
  e.q_rows = q_rows, e.kv_rows = kv_rows, e.rope = rope, e.rope_positions = rope_positions;
  e.group = q_rows / kHeadDim / kv.n_kv;
  e.pos_ptr = pos, e.q = static_cast<_Float16*>(q_out), e.kv = kv;
  return launch_mv<false>(fmt, w, staged_src(xq_view(in.xq, cols)), w.rows, e, stream);
}

std::size_t attention_partials_floats(std::uint32_t n_heads, std::uint32_t n_kv, std::uint32_t span) {
  const std::uint32_t nchunks = (span + kAttnChunk - 1u) / kAttnChunk;
  return static_cast<std::size_t>(n_kv) * nchunks * (n_heads / n_kv) * (kHeadDim + 2u);
}

hipError_t launch_attention_batch(const void* q, const KvLayer& kv, std::uint32_t n_heads, const std::uint32_t* pos,
                                  std::uint32_t span, std::uint32_t batch, std::uint32_t table_stride,
                                  float* partials, float* att, void* xq_att, void* x16_att, hipStream_t stream) {
  if (kv.n_kv == 0u || n_heads % kv.n_kv != 0u || n_heads / kv.n_kv > kMaxGroup || kv.capacity == 0u ||
      span == 0u || span > kv.capacity || kv.page_size == 0u || kv.capacity % kv.page_size != 0u || batch == 0u ||
      batch > 65535u || (batch > 1u && (xq_att != nullptr || table_stride < kv.capacity / kv.page_size)))
    return hipErrorInvalidValue;
  if (x16_att != nullptr && (xq_att != nullptr || batch > kBatchMax || (n_heads * kHeadDim) % 256u != 0u))
    return hipErrorInvalidValue;
  // element offsets of a layer's K / V cache (every sequence's pages) fit 32 bits
  if (static_cast<std::uint64_t>(kv.capacity) * batch * kv.n_kv * kHeadDim > 0xFFFFFFFFull) return hipErrorInvalidValue;
  const std::uint32_t group = n_heads / kv.n_kv;
  const std::uint32_t nchunks = (span + kAttnChunk - 1u) / kAttnChunk;
  const std::size_t part = attention_partials_floats(n_heads, kv.n_kv, span);
  if (part > 0xFFFFFFFFull) return hipErrorInvalidValue;
  const std::uint32_t part_stride = static_cast<std::uint32_t>(part), q_stride = kv.n_kv * kQ16PerKv;
  const dim3 grid(nchunks, kv.n_kv, batch), block(64 * kAttnWaves);
#define RTXLLM_ATTN_CASE(G)                                                                                      \
  case G:                                                                                                        \
    if (batch > 1u)                                                                                              \
      hipLaunchKernelGGL((attn_partial_kernel<G, true>), grid, block, 0, stream, static_cast<const _Float16*>(q), \
                         kv, pos, nchunks, partials, q_stride, table_stride, part_stride);                      \
    else                                                                                                         \
      hipLaunchKernelGGL((attn_partial_kernel<G, false>), grid, block, 0, stream, static_cast<const _Float16*>(q), \
                         kv, pos, nchunks, partials, q_stride, table_stride, part_stride);                      \
    break;
  switch (group) {
    RTXLLM_ATTN_CASE(1)
    RTXLLM_ATTN_CASE(2)
    RTXLLM_ATTN_CASE(4)
    RTXLLM_ATTN_CASE(8)
    default: return hipErrorInvalidValue;
  }
#undef RTXLLM_ATTN_CASE
  hipError_t st = hipGetLastError();
  if (st != hipSuccess) return st;
  if (x16_att != nullptr) {
    hipLaunchKernelGGL(attn_combine_x16_kernel, dim3(n_heads / 2u, kBatchMax), dim3(128), 0, stream, partials, group,
                       nchunks, batch, att, static_cast<_Float16*>(x16_att), part_stride);
    return hipGetLastError();
  }
  const XQOut xq = xq_att != nullptr ? xq_out(xq_att, n_heads * kHeadDim) : XQOut{};
  hipLaunchKernelGGL(attn_combine_kernel, dim3(n_heads, batch), dim3(64), 0, stream, partials, group, nchunks, att, xq,
                     part_stride);
  return hipGetLastError();
}

hipError_t launch_attention(const void* q, const KvLayer& kv, std::uint32_t n_heads, const std::uint32_t* pos,
                            std::uint32_t span, float* partials, float* att, void* xq_att, hipStream_t stream) {
  if (xq_att == nullptr) return hipErrorInvalidValue;
  return launch_attention_batch(q, kv, n_heads, pos, span, 1u, 0u, partials, att, xq_att, nullptr, stream);
}

hipError_t launch_residual(int fmt, const std::uint8_t* payload, const std::uint8_t* meta, std::uint32_t rows,
                           std::uint32_t cols, const void* xq_in, const float* x_in, float* h, const float* w_next,
                           void* xq_next, float* sumsq_next, hipStream_t stream) {
  if ((rows % kXGroup) != 0u || (xq_in == nullptr) == (x_in == nullptr)) return hipErrorInvalidValue;
  const QTensor w{payload, meta, rows, cols};
  const EpiResidual e{h, w_next, xq_out(xq_next, rows), sumsq_next};
  if (xq_in != nullptr) return launch_mv<false>(fmt, w, staged_src(xq_view(xq_in, cols)), rows, e, stream);
  return launch_mv<true>(fmt, w, self_src(x_in), rows, e, stream);
}

hipError_t launch_gate_up(int fmt, const std::uint8_t* payload, const std::uint8_t* meta, std::uint32_t rows,
                          std::uint32_t cols, const NormIn& in, float* act, std::uint32_t* status,
                          hipStream_t stream, std::uint32_t wait_limit, std::uint32_t wait_bias) {
  if ((rows % 4u) != 0u || in.nslots == 0u) return hipErrorInvalidValue;
  const QTensor w{payload, meta, rows, cols};
  EpiGateUp e{};
  e.sumsq = in.sumsq, e.nslots = in.nslots, e.n = in.n, e.eps = in.eps, e.act = act;
  if (mvq_fits(fmt, rows, cols)) return launch_mvq(fmt, w, xq_view(in.xq, cols), rows, e, stream);
  if (cols <= kShareXCols) {
    EpiGateUpWide ew{};
    static_cast<EpiGateUp&>(ew) = e;
    ew.wait.status = status, ew.wait.limit = wait_limit, ew.wait.bias = wait_bias;
    return launch_mv<false>(fmt, w, staged_src(xq_view(in.xq, cols)), rows, ew, stream);
  }
  return launch_mv<false>(fmt, w, staged_src(xq_view(in.xq, cols)), rows, e, stream);
}

std::uint32_t logits_key_slots(int fmt, std::uint32_t rows, std::uint32_t cols) {
  MvGeom g;
  if (!mv_geometry<false, EpiLogits>(fmt, rows, cols, g)) return 0u;
  return g.grid * g.nrg;
}

hipError_t launch_logits(int fmt, const std::uint8_t* payload, const std::uint8_t* meta, std::uint32_t rows,
                         std::uint32_t cols, const NormIn& in, float* logits, unsigned long long* keys,
                         std::uint32_t key_capacity, std::uint32_t* key_count, hipStream_t stream) {
  const std::uint32_t slots = logits_key_slots(fmt, rows, cols);
  if (slots == 0u || slots > key_capacity || keys == nullptr || in.nslots == 0u) return hipErrorInvalidValue;
  if (key_count != nullptr) *key_count = slots;
  const QTensor w{payload, meta, rows, cols};
  EpiLogits e{};
  e.sumsq = in.sumsq, e.nslots = in.nslots, e.n = in.n, e.eps = in.eps, e.logits = logits, e.keys = keys;
  return launch_mv<false>(fmt, w, staged_src(xq_view(in.xq, cols)), rows, e, stream);
}

hipError_t launch_argmax_finalize(const unsigned long long* keys, std::uint32_t count, std::uint32_t* token,
                                  std::uint32_t* pos, std::uint32_t advance, std::uint32_t capacity,
                                  std::uint32_t* status, hipStream_t stream) {
  return launch_argmax_finalize_batch(keys, 0u, count, 1u, token, pos, advance, capacity, status, stream);
}

hipError_t launch_argmax_finalize_batch(const unsigned long long* keys, std::uint32_t key_stride,
                                        std::uint32_t count, std::uint32_t batch, std::uint32_t* token,
                                        std::uint32_t* pos, std::uint32_t advance, std::uint32_t capacity,
                                        std::uint32_t* status, hipStream_t stream) {
  if (keys == nullptr || token == nullptr || batch == 0u || (batch > 1u && key_stride < count))
    return hipErrorInvalidValue;
  hipLaunchKernelGGL(argmax_finalize_kernel, dim3(batch), dim3(256), 0, stream, keys, count, token, pos, advance,
                     key_stride, capacity, status);
  return hipGetLastError();
}

hipError_t launch_synth_raw(int fmt, std::uint64_t seed, std::size_t n_blocks, float d_lo, float d_hi,
                            std::uint8_t* out, hipStream_t stream) {
  if (fmt != RTXLLM_FMT_Q4K_RAW && fmt != RTXLLM_FMT_Q5K && fmt != RTXLLM_FMT_IQ2S && fmt != RTXLLM_FMT_IQ3S)
    return hipErrorInvalidValue;
  if (n_blocks == 0u) return hipSuccess;
  hipLaunchKernelGGL(synth_raw_kernel, dim3(static_cast<unsigned>((n_blocks + 255u) / 256u)), dim3(256), 0, stream,
                     fmt, seed, n_blocks, d_lo, d_hi, out);
  return hipGetLastError();
}

hipError_t launch_synth_q4k_native(std::uint64_t seed, std::size_t n_blocks, float d_lo, float d_hi,
                                   std::uint8_t* payload, std::uint8_t* meta, hipStream_t stream) {
  if (n_blocks == 0u) return hipSuccess;
  hipLaunchKernelGGL(synth_q4k_native_kernel, dim3(static_cast<unsigned>((n_blocks + 255u) / 256u)), dim3(256), 0,
                     stream, seed, n_blocks, d_lo, d_hi, payload, meta);
  return hipGetLastError();
}

}  // namespace rtxllm

#ifdef RTXLLM_TIMELINE
#include "rtxllm/timeline.h"

extern "C" hipError_t rtxllm_timeline_read(unsigned long long* host, size_t count) {
  constexpr size_t kPerUnit = static_cast<size_t>(rtxllm::kTlRegions) * rtxllm::kTlRegion;
  if (host == nullptr || count != 2u * kPerUnit) return hipErrorInvalidValue;
  const hipError_t e = hipMemcpyFromSymbol(host, HIP_SYMBOL(rtxllm::g_timeline), sizeof(rtxllm::g_timeline), 0,
                                           hipMemcpyDeviceToHost);
  if (e != hipSuccess) return e;
  return rtxllm::timeline_read_batch(host + kPerUnit);
}

extern "C" hipError_t rtxllm_timeline_clear(void) {
  void* p = nullptr;
  hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(rtxllm::g_timeline));
  if (e == hipSuccess) e = hipMemset(p, 0, sizeof(rtxllm::g_timeline));
  if (e != hipSuccess) return e;
  return rtxllm::timeline_clear_batch();
}
#endif
