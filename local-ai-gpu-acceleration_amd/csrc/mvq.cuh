// Batch-1 matvec of the IQ unit layouts (IQ2S_UNITS, IQ3S_UNITS) with the
// integer dot products on the matrix cores.
//
// mv_kernel meets each lane's signed int8 weight words with the three digits
// of the staged activation in 24 v_dot4 per 32-value unit, about a third of
// its VALU work. Here one v_mfma_i32_16x16x64_i8 does them for 16 rows at once:
//  * B operand (weights): lane l = row l & 15 of a 16-row tile and slice
//    q = l >> 4; per instruction the lane supplies 16 values of its row (half
//    a unit) as four signed int8 words, decoded as mv_kernel's unit_lookup
//    decodes them;
//  * A operand (activation): A row m = 4 s + d carries digit d (H, M, L) of the
//    16-value group that slice s of the B lanes holds, in slice s only, and
//    zeros elsewhere (A rows 4 s + 3 are all zero);
//  * C[m][n] = sum over slices and bytes of A[m] B[n]: the A rows of slice s
//    meet only slice s, so C[4 q + d][n] is the dot of row n's 16 weights in
//    slice q with digit d of their group. Lane l holds C[4 (l >> 4) + i][l &
//    15] in result register i, i.e. the H, M and L sums of its own 16 weights,
//    and ((H 256) + M) 256 + L is the same exact integer dot16 forms.
// The lane layout of the instruction (A lane l: row l & 15, slice l >> 4; B
// lane l: column l & 15, slice l >> 4, the same byte order in both; result
// register i of lane l: C[4 (l >> 4) + i][l & 15]) was checked on the MI355X
// with random operands. The scaling after the dot is mv_kernel's, per unit.
//
// Work split: a wave covers a panel of 512 columns (4 consecutive units per
// slice and lane) of a 16-row tile; a workgroup of P = cols / 512 waves covers
// the whole row. Each wave reduces its 16 row partials over the slices, the
// waves meet in LDS (double buffered, one barrier per tile), and the 16 rows
// go to the epilogue 4 at a time in its usual lane layout (row r of 4 in lanes
// [16 r, 16 r + 16)). Persistent grid, one tile of weights in flight per wave.
#pragma once

#include "mv.cuh"

namespace rtxllm {

typedef int i32x4 __attribute__((ext_vector_type(4)));

constexpr std::uint32_t kMqRows = 16;    // rows per tile
constexpr std::uint32_t kMqUnits = 4;    // consecutive units per lane and tile (the group-scale reads assume 4)
constexpr std::uint32_t kMqPanel = 4u * kMqUnits * 32u;  // columns per wave
constexpr std::uint32_t kMqMaxWaves = 16;

// One tile's bytes of a lane: the qs / sign fields of its 4 units (8 or 12 B
// each), their (qh | scale << 8) pairs and the block's d.
template <int FMT>
struct MqRaw {
  static constexpr int kPieces = fmt_is_iq2s(FMT) ? 2 : 3;
  u32x4 q[kPieces];
  u32x2 p;
  std::uint32_t d;
  __device__ __forceinline__ std::uint32_t word(int j) const { return q[j >> 2][j & 3]; }
};

// Per-lane scale factors of unit i's two 16-value groups: IQ2_S (0.5 + n) / 4
// s = n a + b (a = s / 4, b = s / 8); IQ3_S uses the group scales s directly.
struct MqScale {
  float a0, b0, a1, b1;
};

// Unit i's share of the lane's sum before the block's d, from its two group
// dots (mv_kernel's unit_dot_iq without the d factor).
template <int FMT>
__device__ __forceinline__ float mq_unit(std::uint32_t pair, int i, int D0, int D1, const MqScale& ls) {
  if constexpr (fmt_is_iq2s(FMT)) {
    const float f0 = __builtin_fmaf(static_cast<float>((pair >> 8) & 15u), ls.a0, ls.b0);
    const float f1 = __builtin_fmaf(static_cast<float>((pair >> 12) & 15u), ls.a1, ls.b1);
    return __builtin_fmaf(f1, static_cast<float>(D1), f0 * static_cast<float>(D0));
  } else {
    // the unit's scale nibble: low for even units, high for odd (each unit's
    // pair holds a copy of the block's scale byte)
    const float m = __builtin_fmaf(static_cast<float>((pair >> (8 + 4 * (i & 1))) & 15u), 2.0f, 1.0f);
    return m * __builtin_fmaf(ls.a1, static_cast<float>(D1), ls.a0 * static_cast<float>(D0));
  }
}

// A unit's codebook reads, issued one unit ahead of their use so that the
// LDS latency of unit i + 1 overlaps unit i's work: gw = grid entries (IQ2_S:
// four 8-byte entries, IQ3_S: eight 4-byte ones), sw = the matching sign masks.
struct MqFetch {
  std::uint32_t gw[8];
  std::uint32_t sw[8];
};

template <int FMT>
__device__ __forceinline__ void mq_fetch(const std::uint32_t* a, std::uint32_t pair, const IqLds<FMT>* t,
                                         MqFetch& f) {
  const std::uint32_t qh = pair & 0xFFu;
  if constexpr (fmt_is_iq2s(FMT)) {
    // as unit_lookup: the high index bits of group g, (qh >> 2 g) & 3, in byte g
    const std::uint32_t s6 = (qh << 6) | qh;
    const std::uint32_t hb = ((s6 << 12) | s6) & 0x03030303u;
#pragma unroll
    for (int grp = 0; grp < 4; ++grp) {
      const std::uint32_t idx = __builtin_amdgcn_perm(hb, a[0], 0x0C0C0400u + 0x101u * static_cast<std::uint32_t>(grp));
      const uint2 gm = t->grid2[idx];
      const uint2 sm = t->sign[(a[1] >> (8 * grp)) & 0xFFu];
      f.gw[2 * grp] = gm.x, f.gw[2 * grp + 1] = gm.y;
      f.sw[2 * grp] = sm.x, f.sw[2 * grp + 1] = sm.y;
    }
  } else {
    const std::uint32_t s7 = (qh << 7) | qh;
    const std::uint32_t s14 = (s7 << 14) | s7;
    const std::uint32_t hb0 = s14 & 0x01010101u, hb1 = (s14 >> 4) & 0x01010101u;
#pragma unroll
    for (int grp = 0; grp < 4; ++grp) {
      const uint2 sm = t->sign[(a[2] >> (8 * grp)) & 0xFFu];
#pragma unroll
      for (int half = 0; half < 2; ++half) {
        const int sel = 2 * grp + half;
        const std::uint32_t idx = __builtin_amdgcn_perm(sel < 4 ? hb0 : hb1, a[sel >> 2],
                                                        0x0C0C0400u + 0x101u * static_cast<std::uint32_t>(sel & 3));
        f.gw[sel] = t->grid3[idx];
        f.sw[sel] = half ? sm.y : sm.x;
      }
    }
  }
}

__device__ __forceinline__ int mq_digits(const i32x4& c) {
  const std::uint32_t hm = (static_cast<std::uint32_t>(c.x) << 8) + static_cast<std::uint32_t>(c.y);
  return static_cast<int>((hm << 8) + static_cast<std::uint32_t>(c.z));
}

template <int FMT, class Epi>
__global__ __launch_bounds__(64 * kMqMaxWaves) void mvq_kernel(QTensor w, XQ xq, std::uint32_t rows, Epi epi_arg) {
  static_assert(fmt_is_units(FMT), "unit layouts");
  static_assert(Epi::kTile == 4, "epilogue tile of 4 rows");
  static_assert(EpiGroupRows<Epi>::value == 0u && !EpiHasFinish<Epi>::value, "plain epilogues");
  Epi epi = epi_arg;
  const std::uint32_t tl_slot = (blockIdx.x * kMqMaxWaves + (threadIdx.x >> 6)) * 8u;
  tl_stamp(kTlGateUpMq, tl_slot);
  __shared__ float part[2][kMqMaxWaves][kMqRows];
  const std::uint32_t lane = threadIdx.x & 63u;
  const std::uint32_t wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const std::uint32_t nw = blockDim.x >> 6;  // panels = cols / 512
  const std::uint32_t bpr = w.cols >> 8, nb = rows * bpr;
  const std::uint32_t n = lane & 15u, q = lane >> 4;
  // the lane's units: k0 .. k0 + 3 of its row (within one block: k0 % 8 is 0 or 4)
  const std::uint32_t k0 = wave * 16u + q * kMqUnits, b = k0 >> 3, uk0 = k0 & 7u;
  constexpr std::uint32_t kQB = fmt_is_iq2s(FMT) ? 64u : 96u;  // qs / sign bytes per block
  constexpr std::uint32_t kUB = kQB / 8u;                       // ... per unit
  const std::uint32_t rowb = n * bpr + b;                       // blocks before the lane's block, within the tile
  const std::uint32_t o_q = kQB * rowb + kUB * uk0;
  const std::uint32_t o_p = kQB * nb + 16u * rowb + 2u * uk0;
  const std::uint32_t o_d = (kQB + 16u) * nb + 2u * rowb;
  const Rsrc rs = make_rsrc(w.payload, nb * FmtBytes<FMT>::payload);
  constexpr int P = load_policy<FMT>();
  const std::uint32_t tiles = rows / kMqRows, G = gridDim.x;
  const std::uint32_t rounds = (tiles - blockIdx.x + G - 1u) / G;  // >= 1: the host keeps G <= tiles
  const std::uint32_t tile_blocks = kMqRows * bpr;

  auto load_tile = [&](std::uint32_t s, MqRaw<FMT>& r) {
    std::uint32_t t = blockIdx.x + s * G;
    t = __builtin_amdgcn_readfirstlane(t < tiles ? t : tiles - 1u);
    const std::uint32_t tb = t * tile_blocks;
#pragma unroll
    for (int j = 0; j < MqRaw<FMT>::kPieces; ++j) r.q[j] = bld_u128<P>(rs, o_q + 16u * j, kQB * tb);
    r.p = bld_u64<P>(rs, o_p, 16u * tb);
    r.d = bld_u16<P>(rs, o_d, 2u * tb);
  };

  // Prologue: epilogue set-up, codebook grid (registers), the wave's slice of
  // the staged activation, first tile; then the activation and the codebook go
  // to LDS (one barrier), and each lane reads its operands from there.
  epi.init(lane);
  IqLds<FMT>& tables = iq_lds<FMT>();
  LdsGridStage<IqLds<FMT>, 512u> grid_stage;
  lds_grid_issue(grid_stage, iq_image<FMT>(), threadIdx.x, blockDim.x);
  // The wave's panel of the staged activation: its 32 groups' digits in each
  // plane (H, M, L: cols bytes each, in that order from xq.h; 512 bytes per
  // plane and panel) and their 32 scales, three 8-byte and one 4-byte load per
  // lane. In LDS: the three planes' 512 bytes (pieces 0-95), the scales
  // (96-103) and 128 zero bytes (104-111).
  __shared__ uint4 xst[kMqMaxWaves][112];
  const Rsrc rx = make_rsrc(xq.h, 3u * w.cols);
  u32x2 xd[3];
#pragma unroll
  for (std::uint32_t d = 0; d < 3u; ++d) xd[d] = bld_u64<0>(rx, d * w.cols + 512u * wave + 8u * lane, 0u);
  const float xsc = xq.s[32u * wave + (lane & 31u)];
  __builtin_amdgcn_sched_barrier(0);
  MqRaw<FMT> buf[2];
  load_tile(0u, buf[0]);
  {
    std::uint8_t* xw = reinterpret_cast<std::uint8_t*>(xst[wave]);
#pragma unroll
    for (std::uint32_t d = 0; d < 3u; ++d) *reinterpret_cast<u32x2*>(xw + 512u * d + 8u * lane) = xd[d];
    reinterpret_cast<float*>(xw + 1536u)[lane & 31u] = xsc;
    reinterpret_cast<std::uint32_t*>(xw + 1664u)[lane & 31u] = 0u;
  }
  lds_grid_commit(tables, grid_stage, iq_image<FMT>(), threadIdx.x, blockDim.x);
  tl_stamp(kTlGateUpMq, tl_slot + 1u);
  if constexpr (EpiHasReady<Epi>::value) epi.ready(lane);
  // A operand: lane (m = lane & 15, s = lane >> 4) holds digit m & 3 of the
  // group of unit i, half h, of slice s when m >> 2 == s and m & 3 < 3, else
  // zeros (read from the zero pieces).
  const std::uint32_t am = lane & 15u, as = lane >> 4;
  const bool adata = (am >> 2) == as && (am & 3u) < 3u;
  const uint4* xa_src = xst[wave] + (adata ? 32u * (am & 3u) + 8u * as : 104u);
  i32x4 xa[kMqUnits][2];
  MqScale ls[kMqUnits];
  // the group scales of the B lane's own eight groups (slice q)
  const float4 xs03 = reinterpret_cast<const float4*>(xst[wave] + 96u + 2u * q)[0];
  const float4 xs47 = reinterpret_cast<const float4*>(xst[wave] + 96u + 2u * q)[1];
  const float xs[kMqUnits][2] = {{xs03.x, xs03.y}, {xs03.z, xs03.w}, {xs47.x, xs47.y}, {xs47.z, xs47.w}};
#pragma unroll
  for (std::uint32_t i = 0; i < kMqUnits; ++i) {
#pragma unroll
    for (std::uint32_t h = 0; h < 2u; ++h) {
      const uint4 v = xa_src[2u * i + h];
      xa[i][h] = i32x4{static_cast<int>(v.x), static_cast<int>(v.y), static_cast<int>(v.z), static_cast<int>(v.w)};
    }
    if constexpr (fmt_is_iq2s(FMT)) {
      ls[i] = MqScale{0.25f * xs[i][0], 0.125f * xs[i][0], 0.25f * xs[i][1], 0.125f * xs[i][1]};
    } else {
      ls[i] = MqScale{xs[i][0], 0.0f, xs[i][1], 0.0f};
    }
  }

  auto round = [&](std::uint32_t s, const MqRaw<FMT>& r) {
    switch ((4u * s) / rounds) {  // wave priority by progress, as in mv_kernel
      case 0: __builtin_amdgcn_s_setprio(3); break;
      case 1: __builtin_amdgcn_s_setprio(2); break;
      case 2: __builtin_amdgcn_s_setprio(1); break;
      default: __builtin_amdgcn_s_setprio(0); break;
    }
    constexpr int kW = fmt_is_iq2s(FMT) ? 2 : 3;  // qs / sign words per unit
    auto pair_of = [&](int i) -> std::uint32_t { return i & 1 ? r.p[i >> 1] >> 16 : r.p[i >> 1]; };
    auto fetch = [&](int i, MqFetch& f) {
      std::uint32_t a[3];
#pragma unroll
      for (int j = 0; j < kW; ++j) a[j] = r.word(kW * i + j);
      mq_fetch<FMT>(a, pair_of(i), &tables, f);
    };
    float acc = 0.0f;
    MqFetch fq[2];
    fetch(0, fq[0]);
#pragma unroll
    for (int i = 0; i < static_cast<int>(kMqUnits); ++i) {
      if (i + 1 < static_cast<int>(kMqUnits)) fetch(i + 1, fq[(i + 1) & 1]);
      __builtin_amdgcn_sched_barrier(0);  // unit i + 1's reads ahead of unit i's work
      const std::uint32_t pair = pair_of(i);
      const MqFetch& f = fq[i & 1];
      std::uint32_t wv[8];
#pragma unroll
      for (int j = 0; j < 8; ++j) wv[j] = (f.gw[j] ^ f.sw[j]) | kIqLowBits;
      const i32x4 w0{static_cast<int>(wv[0]), static_cast<int>(wv[1]), static_cast<int>(wv[2]),
                     static_cast<int>(wv[3])};
      const i32x4 w1{static_cast<int>(wv[4]), static_cast<int>(wv[5]), static_cast<int>(wv[6]),
                     static_cast<int>(wv[7])};
      const i32x4 c0 = __builtin_amdgcn_mfma_i32_16x16x64_i8(xa[i][0], w0, i32x4{0, 0, 0, 0}, 0, 0, 0);
      const i32x4 c1 = __builtin_amdgcn_mfma_i32_16x16x64_i8(xa[i][1], w1, i32x4{0, 0, 0, 0}, 0, 0, 0);
      acc += mq_unit<FMT>(pair, i, mq_digits(c0), mq_digits(c1), ls[i]);
    }
    // the row's sum over the four slices (lanes n, n + 16, n + 32, n + 48):
    // with both operands v, a permlane swap leaves v and its partner 16 (32)
    // lanes away in the two registers
    float v = acc * h2f(r.d);
    {
      float a = v, b = v;
      permlane16_swap(a, b);
      v = a + b;
      a = v, b = v;
      permlane32_swap(a, b);
      v = a + b;
    }
    const std::uint32_t par = s & 1u;
    if (lane < kMqRows) part[par][wave][lane] = v;
    __syncthreads();
    const std::uint32_t t = blockIdx.x + s * G;  // < tiles: s < rounds
    for (std::uint32_t j = wave; j < 4u; j += nw) {
      const std::uint32_t rr = 4u * j + (lane >> 4);
      float y = part[par][0][rr];
      for (std::uint32_t k = 1; k < nw; ++k) y += part[par][k][rr];
      epi(t * kMqRows + 4u * j, y, lane, rows);
    }
    tl_stamp(kTlGateUpMq, tl_slot + 2u + (s < 4u ? s : 4u));
  };

  // Round s computes buf[s % 2] after requesting round s + 1 (no load inside
  // a branch, so each round waits for its own tile only).
  std::uint32_t s = 0;
  for (; s + 2u < rounds; s += 2u) {
    load_tile(s + 1u, buf[1]);
    round(s, buf[0]);
    load_tile(s + 2u, buf[0]);
    round(s + 1u, buf[1]);
  }
  if (s + 1u < rounds) {
    load_tile(s + 1u, buf[1]);
    round(s, buf[0]);
    round(s + 1u, buf[1]);
  } else {
    round(s, buf[0]);
  }
  tl_stamp(kTlGateUpMq, tl_slot + 7u);
}

// Whether mvq_kernel takes a matvec: a unit layout, whole 16-row tiles and
// whole 512-column panels, at most 16 of them.
inline bool mvq_fits(int fmt, std::uint32_t rows, std::uint32_t cols) {
  return fmt_is_units(fmt) && rows > 0u && rows % kMqRows == 0u && cols % kMqPanel == 0u && cols > 0u &&
         cols / kMqPanel <= kMqMaxWaves;
}

template <int FMT, class Epi>
inline int mvq_resident(std::uint32_t threads) {
  static int cache[kMqMaxWaves + 1] = {};
  const std::uint32_t wv = threads / 64u;
  if (wv == 0u || wv > kMqMaxWaves) return 0;
  if (cache[wv] == 0) {
    int r = 0;
    if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&r, reinterpret_cast<const void*>(&mvq_kernel<FMT, Epi>),
                                                     static_cast<int>(threads), 0) != hipSuccess ||
        r <= 0)
      return 0;
    cache[wv] = r;
  }
  return cache[wv];
}

template <int FMT, class Epi>
inline hipError_t launch_mvq_fmt(const QTensor& w, const XQ& xq, std::uint32_t rows, const Epi& epi,
                                 hipStream_t stream) {
  if (!mvq_fits(FMT, rows, w.cols)) return hipErrorInvalidValue;
  // the kernel addresses the tensor with 32-bit byte offsets
  if (static_cast<std::uint64_t>(rows) * (w.cols / 256u) * FmtBytes<FMT>::payload > 0xFFFFFFFFull)
    return hipErrorInvalidValue;
  const std::uint32_t panels = w.cols / kMqPanel, tiles = rows / kMqRows;
  const int per_cu = mvq_resident<FMT, Epi>(64u * panels);
  const std::uint32_t slots = static_cast<std::uint32_t>(per_cu > 0 ? per_cu : 1) * static_cast<std::uint32_t>(num_cus());
  const std::uint32_t grid = tiles < slots ? tiles : slots;
  hipLaunchKernelGGL((mvq_kernel<FMT, Epi>), dim3(grid), dim3(64u * panels), 0, stream, w, xq, rows, epi);
  return hipGetLastError();
}

template <class Epi>
inline hipError_t launch_mvq(int fmt, const QTensor& w, const XQ& xq, std::uint32_t rows, const Epi& epi,
                             hipStream_t stream) {
  switch (fmt) {
    case RTXLLM_FMT_IQ2S_UNITS: return launch_mvq_fmt<RTXLLM_FMT_IQ2S_UNITS>(w, xq, rows, epi, stream);
    case RTXLLM_FMT_IQ3S_UNITS: return launch_mvq_fmt<RTXLLM_FMT_IQ3S_UNITS>(w, xq, rows, epi, stream);
    default: return hipErrorInvalidValue;
  }
}

}  // namespace rtxllm
