// Batch-1 dequant-matvec kernels y = W x for the GGUF resident-pack layouts.
//
// Work split: a workgroup owns R consecutive rows; its lanes stride over the
// row's 32-weight "units" (Q4_K/Q5_K: 16 payload bytes = one half of a 64-value
// group, IQ2_S/IQ3_S: one 32-value sub-block), so each lane loads the unit's 32
// activations once and reuses them for all R rows. Per-unit scales are factored
// out of the inner product: Q4_K/Q5_K accumulate S*sum(q*x) - M*sum(x), the IQ
// formats scale*sum(+-grid*x). Lane partials are reduced across the wave and
// then across the workgroup's waves in LDS, so the summation order is fixed and
// results are deterministic.
#pragma once

#include "common.h"
#include "iq_grids.h"

namespace rtxllm {

struct QTensor {
  const std::uint8_t* payload;  // raw blocks, or the Q4_K split payload stream
  const std::uint8_t* meta;     // Q4_K split metadata stream, else unused
  std::uint32_t rows;
  std::uint32_t cols;
};

// Side effects of the reference's *_decode launchers, applied by the thread that
// finishes a row (decode_kernels.cu:1600-1606): kv[(row*page_words +
// (token+row) % page_words) % kv_words] = y[row] for row < active_pages.
struct KvSideWrite {
  float* kv;
  const std::uint32_t* token;
  std::uint32_t kv_words;
  std::uint32_t page_words;
  std::uint32_t active_pages;
};

__device__ __forceinline__ void kv_side_write(const KvSideWrite& e, std::uint32_t row, float value) {
  if (e.kv != nullptr && e.token != nullptr && row < e.active_pages && e.kv_words > 0u && e.page_words > 0u) {
    const std::size_t base = static_cast<std::size_t>(row) * e.page_words;
    const std::size_t off = (e.token[0] + row) % e.page_words;
    e.kv[(base + off) % e.kv_words] = value;
  }
}

static __constant__ std::uint16_t kIq2sGridDev[1024] = {RTXLLM_IQ2S_GRID_VALUES};
static __constant__ std::uint32_t kIq3sGridDev[512] = {RTXLLM_IQ3S_GRID_VALUES};

// ---- K-quant units ---------------------------------------------------------

// Scale/min products of the two sub-blocks 2g and 2g+1 covered by a Q4_K/Q5_K
// unit, from the 16-byte native head (d, dmin, 12 packed scale bytes).
__device__ __forceinline__ void kq_head_pairs(uint4 head, std::uint32_t g, float& s0, float& m0, float& s1,
                                              float& m1) {
  const float d = f16_bits_to_f32(head.x & 0xFFFFu);
  const float dmin = f16_bits_to_f32(head.x >> 16);
  std::uint32_t sc0, mn0, sc1, mn1;
  scale_min_k4(static_cast<int>(2u * g), head.y, head.z, head.w, sc0, mn0);
  scale_min_k4(static_cast<int>(2u * g + 1u), head.y, head.z, head.w, sc1, mn1);
  s0 = d * static_cast<float>(sc0);
  m0 = dmin * static_cast<float>(mn0);
  s1 = d * static_cast<float>(sc1);
  m1 = dmin * static_cast<float>(mn1);
}

template <int FMT>
__device__ __forceinline__ void q4k_unit_meta(const QTensor& w, std::size_t blk, std::uint32_t g, float& s0,
                                              float& m0, float& s1, float& m1) {
  if constexpr (FMT == RTXLLM_FMT_Q4K_RAW) {
    kq_head_pairs(ld_u128(w.payload + blk * 144u), g, s0, m0, s1, m1);
  } else if constexpr (FMT == RTXLLM_FMT_Q4K_SPLIT_NATIVE) {
    kq_head_pairs(ld_u128(w.meta + blk * 16u), g, s0, m0, s1, m1);
  } else if constexpr (FMT == RTXLLM_FMT_Q4K_SPLIT_PREDECODED || FMT == RTXLLM_FMT_Q4K_RAW_PREDECODED) {
    const float4 p = *reinterpret_cast<const float4*>(w.meta + blk * 64u + g * 16u);
    s0 = p.x;
    m0 = p.y;
    s1 = p.z;
    m1 = p.w;
  } else if constexpr (FMT == RTXLLM_FMT_Q4K_SPLIT_HALF) {
    const uint2 p = *reinterpret_cast<const uint2*>(w.meta + blk * 32u + g * 8u);
    s0 = f16_bits_to_f32(p.x & 0xFFFFu);
    m0 = f16_bits_to_f32(p.x >> 16);
    s1 = f16_bits_to_f32(p.y & 0xFFFFu);
    m1 = f16_bits_to_f32(p.y >> 16);
  } else {  // split-compact: f16 d, f16 dmin, u8 sc[8], u8 m[8]
    const std::uint8_t* m = w.meta + blk * 20u;
    const std::uint32_t dd = ld_u32(m);
    const std::uint32_t sc = ld_u16(m + 4u + 2u * g);
    const std::uint32_t mn = ld_u16(m + 12u + 2u * g);
    const float d = f16_bits_to_f32(dd & 0xFFFFu);
    const float dmin = f16_bits_to_f32(dd >> 16);
    s0 = d * static_cast<float>(sc & 0xFFu);
    s1 = d * static_cast<float>(sc >> 8);
    m0 = dmin * static_cast<float>(mn & 0xFFu);
    m1 = dmin * static_cast<float>(mn >> 8);
  }
}

template <int FMT>
__device__ __forceinline__ uint4 q4k_unit_payload(const QTensor& w, std::size_t blk, std::uint32_t k) {
  if constexpr (FMT == RTXLLM_FMT_Q4K_RAW || FMT == RTXLLM_FMT_Q4K_RAW_PREDECODED)
    return ld_u128(w.payload + blk * 144u + 16u + 16u * k);
  else return ld_u128(w.payload + blk * 128u + 16u * k);
}

// sum_j lo_nibble(byte j) * xl[j] and sum_j hi_nibble(byte j) * xh[j].
__device__ __forceinline__ void nibble_dots(const std::uint32_t q[4], const float xl[16], const float xh[16],
                                            float& dl, float& dh) {
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const std::uint32_t lo = q[i] & 0x0F0F0F0Fu;
    const std::uint32_t hi = (q[i] >> 4) & 0x0F0F0F0Fu;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      dl = fmaf(static_cast<float>((lo >> (8 * j)) & 0xFFu), xl[4 * i + j], dl);
      dh = fmaf(static_cast<float>((hi >> (8 * j)) & 0xFFu), xh[4 * i + j], dh);
    }
  }
}

// Q5_K: the 5th bit of value (group g, half, byte j) is bit (2g + half) of qh[16h + j].
__device__ __forceinline__ void q5k_dots(const std::uint32_t q[4], const std::uint32_t qh[4], std::uint32_t g,
                                         const float xl[16], const float xh[16], float& dl, float& dh) {
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const std::uint32_t bl = (qh[i] >> (2u * g)) & 0x01010101u;
    const std::uint32_t bh = (qh[i] >> (2u * g + 1u)) & 0x01010101u;
    const std::uint32_t lo = (q[i] & 0x0F0F0F0Fu) | (bl << 4);
    const std::uint32_t hi = ((q[i] >> 4) & 0x0F0F0F0Fu) | (bh << 4);
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      dl = fmaf(static_cast<float>((lo >> (8 * j)) & 0xFFu), xl[4 * i + j], dl);
      dh = fmaf(static_cast<float>((hi >> (8 * j)) & 0xFFu), xh[4 * i + j], dh);
    }
  }
}

template <int FMT>
__device__ __forceinline__ float kq_unit(const QTensor& w, std::size_t blk, std::uint32_t k, const float xl[16],
                                         const float xh[16], float xsl, float xsh) {
  const std::uint32_t g = k >> 1;
  float s0, m0, s1, m1, dl = 0.0f, dh = 0.0f;
  if constexpr (FMT == RTXLLM_FMT_Q5K) {
    const std::uint8_t* b = w.payload + blk * 176u;
    kq_head_pairs(ld_u128(b), g, s0, m0, s1, m1);
    const uint4 qv = ld_u128(b + 48u + 16u * k);
    const uint4 hv = ld_u128(b + 16u + 16u * (k & 1u));
    const std::uint32_t q[4] = {qv.x, qv.y, qv.z, qv.w};
    const std::uint32_t qh[4] = {hv.x, hv.y, hv.z, hv.w};
    q5k_dots(q, qh, g, xl, xh, dl, dh);
  } else {
    q4k_unit_meta<FMT>(w, blk, g, s0, m0, s1, m1);
    const uint4 qv = q4k_unit_payload<FMT>(w, blk, k);
    const std::uint32_t q[4] = {qv.x, qv.y, qv.z, qv.w};
    nibble_dots(q, xl, xh, dl, dh);
  }
  return (s0 * dl - m0 * xsl) + (s1 * dh - m1 * xsh);
}

// ---- IQ units --------------------------------------------------------------

// Four bytes starting at a 2-byte aligned address.
__device__ __forceinline__ std::uint32_t ld_u32_a2(const std::uint8_t* p) { return ld_u16(p) | (ld_u16(p + 2) << 16); }

__device__ __forceinline__ float iq2s_unit(const QTensor& w, std::size_t blk, std::uint32_t k, const float xv[32]) {
  const std::uint8_t* b = w.payload + blk * 82u;
  const float d = f16_bits_to_f32(ld_u16(b));
  const std::uint32_t qs = ld_u32_a2(b + 2u + 4u * k);
  const std::uint32_t sg = ld_u32_a2(b + 34u + 4u * k);
  const std::uint32_t qh = ld_u8(b + 66u + k);
  const std::uint32_t sc = ld_u8(b + 74u + k);
  float dots[4];
#pragma unroll
  for (int grp = 0; grp < 4; ++grp) {
    const std::uint32_t idx = ((qs >> (8 * grp)) & 0xFFu) | ((qh << (8 - 2 * grp)) & 0x300u);
    const std::uint32_t word = kIq2sGridDev[idx];
    const std::uint32_t sb = sg >> (8 * grp);
    float dd = 0.0f;
#pragma unroll
    for (int l = 0; l < 8; ++l) {
      const float mag = static_cast<float>(2u * ((word >> (2 * l)) & 3u) + 1u);
      dd = fmaf(((sb >> l) & 1u) ? -mag : mag, xv[8 * grp + l], dd);
    }
    dots[grp] = dd;
  }
  const float slo = d * (0.5f + static_cast<float>(sc & 0x0Fu)) * 0.25f;
  const float shi = d * (0.5f + static_cast<float>(sc >> 4)) * 0.25f;
  return slo * (dots[0] + dots[1]) + shi * (dots[2] + dots[3]);
}

__device__ __forceinline__ float iq3s_unit(const QTensor& w, std::size_t blk, std::uint32_t k, const float xv[32]) {
  const std::uint8_t* b = w.payload + blk * 110u;
  const float d = f16_bits_to_f32(ld_u16(b));
  const std::uint32_t qs0 = ld_u32_a2(b + 2u + 8u * k);
  const std::uint32_t qs1 = ld_u32_a2(b + 6u + 8u * k);
  const std::uint32_t qh = ld_u8(b + 66u + k);
  const std::uint32_t sg = ld_u32_a2(b + 74u + 4u * k);
  const std::uint32_t scb = ld_u8(b + 106u + (k >> 1));
  float dot = 0.0f;
#pragma unroll
  for (int grp = 0; grp < 4; ++grp) {
    const std::uint32_t sb = sg >> (8 * grp);
#pragma unroll
    for (int pair = 0; pair < 2; ++pair) {
      const int sel = 2 * grp + pair;  // 0..7 within the unit
      const std::uint32_t qb = ((sel < 4 ? qs0 : qs1) >> (8 * (sel & 3))) & 0xFFu;
      const std::uint32_t idx = qb | (((qh >> sel) & 1u) << 8);
      const std::uint32_t word = kIq3sGridDev[idx];
#pragma unroll
      for (int gl = 0; gl < 4; ++gl) {
        const float mag = static_cast<float>((word >> (8 * gl)) & 0xFFu);
        dot = fmaf(((sb >> (4 * pair + gl)) & 1u) ? -mag : mag, xv[8 * grp + 4 * pair + gl], dot);
      }
    }
  }
  const std::uint32_t nib = (k & 1u) ? (scb >> 4) : (scb & 0x0Fu);
  return d * static_cast<float>(1u + 2u * nib) * dot;
}

// ---- the kernel ------------------------------------------------------------

template <int FMT>
struct UnitTraits {
  static constexpr bool kIq = (FMT == RTXLLM_FMT_IQ2S || FMT == RTXLLM_FMT_IQ3S);
};

// Workgroup: R rows x (blockDim.x / 64) waves; lanes stride over units.
template <int FMT, int R>
__global__ __launch_bounds__(512) void matvec_b1_kernel(QTensor w, const float* __restrict__ x,
                                                        float* __restrict__ y, std::uint32_t row_count,
                                                        KvSideWrite side) {
  __shared__ float red[8][R];
  const std::uint32_t row0 = blockIdx.x * R;
  const std::uint32_t bpr = w.cols >> 8;
  const std::uint32_t units = bpr * 8u;
  float acc[R];
#pragma unroll
  for (int r = 0; r < R; ++r) acc[r] = 0.0f;

  for (std::uint32_t u = threadIdx.x; u < units; u += blockDim.x) {
    const std::uint32_t b = u >> 3, k = u & 7u;
    if constexpr (UnitTraits<FMT>::kIq) {
      float xv[32];
      const float4* xp = reinterpret_cast<const float4*>(x + 256u * b + 32u * k);
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        const float4 t = xp[i];
        xv[4 * i] = t.x;
        xv[4 * i + 1] = t.y;
        xv[4 * i + 2] = t.z;
        xv[4 * i + 3] = t.w;
      }
#pragma unroll
      for (int r = 0; r < R; ++r) {
        const std::uint32_t row = row0 + r;
        if (row < row_count) {
          const std::size_t blk = static_cast<std::size_t>(row) * bpr + b;
          if constexpr (FMT == RTXLLM_FMT_IQ2S) acc[r] += iq2s_unit(w, blk, k, xv);
          else acc[r] += iq3s_unit(w, blk, k, xv);
        }
      }
    } else {
      const std::uint32_t g = k >> 1, h = k & 1u;
      float xl[16], xh[16];
      const float4* xpl = reinterpret_cast<const float4*>(x + 256u * b + 64u * g + 16u * h);
      const float4* xph = reinterpret_cast<const float4*>(x + 256u * b + 64u * g + 32u + 16u * h);
      float xsl = 0.0f, xsh = 0.0f;
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const float4 a = xpl[i], c = xph[i];
        xl[4 * i] = a.x;
        xl[4 * i + 1] = a.y;
        xl[4 * i + 2] = a.z;
        xl[4 * i + 3] = a.w;
        xh[4 * i] = c.x;
        xh[4 * i + 1] = c.y;
        xh[4 * i + 2] = c.z;
        xh[4 * i + 3] = c.w;
        xsl += (a.x + a.y) + (a.z + a.w);
        xsh += (c.x + c.y) + (c.z + c.w);
      }
#pragma unroll
      for (int r = 0; r < R; ++r) {
        const std::uint32_t row = row0 + r;
        if (row < row_count) {
          const std::size_t blk = static_cast<std::size_t>(row) * bpr + b;
          acc[r] += kq_unit<FMT>(w, blk, k, xl, xh, xsl, xsh);
        }
      }
    }
  }

  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6, nw = blockDim.x >> 6;
#pragma unroll
  for (int r = 0; r < R; ++r) {
    const float s = wave_sum(acc[r]);
    if (lane == 0) red[wave][r] = s;
  }
  __syncthreads();
  if (threadIdx.x < R) {
    const std::uint32_t row = row0 + threadIdx.x;
    if (row < row_count) {
      float s = red[0][threadIdx.x];
      for (int i = 1; i < nw; ++i) s += red[i][threadIdx.x];
      y[row] = s;
      kv_side_write(side, row, s);
    }
  }
}

}  // namespace rtxllm
