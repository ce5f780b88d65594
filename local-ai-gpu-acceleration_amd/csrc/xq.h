// Activation staging for the integer-dot matvec kernels.
//
// The matvec kernels multiply small integer weight codes (Q4_K/Q5_K quants,
// signed IQ grid magnitudes) with the activation through v_dot4_i32_i8. For
// that the fp32 activation is staged once per 16-value group as fixed point:
// X_j = rint(x_j * K / max|x|) with K = 127 * 256 = 32512, split into two int8
// digits X_j = 256 H_j + L_j (H in [-127, 127], L in [-128, 127]), with the
// group scale s = max|x| / K, so that x_j ~= s * X_j (a step of 3.1e-5 of the
// group maximum: 15 bits, finer than fp16's 11-bit mantissa). The integer dot
// products are exact; only the staging rounds.
// Every producer (the staging kernel, the kernels' self-staging path, fused
// epilogues) implements this one rule, so all paths see identical digits.
//
// HBM layout of a staged vector of `cols` values (cols % 256 == 0), one
// allocation of xq_bytes(cols):
//   [0, cols)               int8 H digits
//   [cols, 2 cols)          int8 L digits
//   [2 cols, 2 cols + G*4)  f32 group scale s, G = cols / 16
//   [.., + G*4)             f32 group sum s * sum_j X_j
#pragma once

#include "common.h"

namespace rtxllm {

constexpr int kXGroup = 16;
constexpr int kXQLimit = 32512;  // 127 * 256
constexpr float kXQLimitF = 32512.0f;

// X -> (H, L) with X = 256 H + L, |X| <= kXQLimit.
__host__ __device__ inline void xq_digits(int X, int& H, int& L) {
  H = (X + 128) >> 8;
  L = X - 256 * H;
}

// One staged group in a lane's registers: digit j in byte (j & 3) of word j >> 2.
struct XG {
  std::uint32_t h[4];
  std::uint32_t l[4];
  float s;
  float sum;
};

struct XQ {
  const std::int8_t* h;
  const std::int8_t* l;
  const float* s;
  const float* sum;
};

struct XQOut {
  std::int8_t* h;
  std::int8_t* l;
  float* s;
  float* sum;
};

__host__ __device__ inline std::size_t xq_bytes(std::uint32_t cols) {
  return 2u * static_cast<std::size_t>(cols) + 8u * static_cast<std::size_t>(cols / kXGroup);
}

__host__ __device__ inline XQ xq_view(const void* base, std::uint32_t cols) {
  const std::int8_t* b = static_cast<const std::int8_t*>(base);
  const float* s = reinterpret_cast<const float*>(b + 2u * static_cast<std::size_t>(cols));
  return XQ{b, b + cols, s, s + cols / kXGroup};
}

__host__ __device__ inline XQOut xq_out(void* base, std::uint32_t cols) {
  std::int8_t* b = static_cast<std::int8_t*>(base);
  float* s = reinterpret_cast<float*>(b + 2u * static_cast<std::size_t>(cols));
  return XQOut{b, b + cols, s, s + cols / kXGroup};
}

__device__ __forceinline__ void xg_zero(XG& g) {
#pragma unroll
  for (int i = 0; i < 4; ++i) g.h[i] = g.l[i] = 0u;
  g.s = 0.0f;
  g.sum = 0.0f;
}

// Stage 16 values. Non-finite inputs stage as zero digits (their scale is kept,
// so an infinite maximum still poisons the products, as fp32 would).
// The digits come from Y = X + 128 as int16 (|X| <= 32512): H is Y's high byte
// (floor((X + 128) / 256)) and L = X - 256 H its low byte minus 128 (the low
// byte xor 0x80), so two int16 packs and two byte permutes give four values'
// digit words; the group sum is 256 sum H + sum L, from two dot products.
__device__ __forceinline__ void quant16(const float v[16], XG& g) {
  typedef short short2_t __attribute__((ext_vector_type(2)));
  float m = 0.0f;
#pragma unroll
  for (int j = 0; j < 16; ++j) m = fmaxf(m, fabsf(v[j]));
  const float inv = m > 0.0f ? kXQLimitF / m : 0.0f;
  g.s = m / kXQLimitF;
  int hsum = 0, lsum = 0;
#pragma unroll
  for (int w = 0; w < 4; ++w) {
    int X[4];
#pragma unroll
    for (int b = 0; b < 4; ++b) {
      const int x = static_cast<int>(rintf(v[4 * w + b] * inv));
      X[b] = x > kXQLimit ? kXQLimit : (x < -kXQLimit ? -kXQLimit : x);
    }
    const short2_t bias = {128, 128};
    const short2_t y01 = __builtin_amdgcn_cvt_pk_i16(X[0], X[1]) + bias;
    const short2_t y23 = __builtin_amdgcn_cvt_pk_i16(X[2], X[3]) + bias;
    const std::uint32_t u01 = __builtin_bit_cast(std::uint32_t, y01), u23 = __builtin_bit_cast(std::uint32_t, y23);
    // byte i of the result: selector byte i, 0-3 = bytes of the second source, 4-7 of the first
    g.h[w] = __builtin_amdgcn_perm(u23, u01, 0x07050301u);
    g.l[w] = __builtin_amdgcn_perm(u23, u01, 0x06040200u) ^ 0x80808080u;
    hsum = __builtin_amdgcn_sdot4(static_cast<int>(g.h[w]), 0x01010101, hsum, false);
    lsum = __builtin_amdgcn_sdot4(static_cast<int>(g.l[w]), 0x01010101, lsum, false);
  }
  g.sum = g.s * static_cast<float>(256 * hsum + lsum);
}

__device__ __forceinline__ void xg_load(const XQ& x, std::uint32_t group, XG& g) {
  const uint4 h = *reinterpret_cast<const uint4*>(x.h + kXGroup * group);
  const uint4 l = *reinterpret_cast<const uint4*>(x.l + kXGroup * group);
  g.h[0] = h.x, g.h[1] = h.y, g.h[2] = h.z, g.h[3] = h.w;
  g.l[0] = l.x, g.l[1] = l.y, g.l[2] = l.z, g.l[3] = l.w;
  g.s = x.s[group];
  g.sum = x.sum[group];
}

// Stage group `group` of an fp32 vector (optionally times an elementwise weight).
__device__ __forceinline__ void xg_stage(const float* __restrict__ x, const float* __restrict__ mul,
                                         std::uint32_t group, XG& g) {
  float v[16];
  const float4* p = reinterpret_cast<const float4*>(x + kXGroup * group);
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const float4 t = p[i];
    v[4 * i] = t.x, v[4 * i + 1] = t.y, v[4 * i + 2] = t.z, v[4 * i + 3] = t.w;
  }
  if (mul != nullptr) {
    const float4* q = reinterpret_cast<const float4*>(mul + kXGroup * group);
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const float4 t = q[i];
      v[4 * i] *= t.x, v[4 * i + 1] *= t.y, v[4 * i + 2] *= t.z, v[4 * i + 3] *= t.w;
    }
  }
  quant16(v, g);
}

__device__ __forceinline__ void xg_store(const XQOut& x, std::uint32_t group, const XG& g) {
  *reinterpret_cast<uint4*>(x.h + kXGroup * group) = make_uint4(g.h[0], g.h[1], g.h[2], g.h[3]);
  *reinterpret_cast<uint4*>(x.l + kXGroup * group) = make_uint4(g.l[0], g.l[1], g.l[2], g.l[3]);
  x.s[group] = g.s;
  x.sum[group] = g.sum;
}

// sum_j w_j X_j = 256 sum w H + sum w L, exact in int32 for int8 weights
// (|result| <= 16 * 128 * 32640 < 2^27); one shift-add.
__device__ __forceinline__ int dot_digits(int ah, int al) {
  return static_cast<int>((static_cast<std::uint32_t>(ah) << 8) + static_cast<std::uint32_t>(al));
}

// a . b over four int8 lanes, starting a chain from 0: the three-operand
// encoding with an inline zero accumulator (the two-operand accumulate form
// would need the zero moved into its destination first).
__device__ __forceinline__ int sdot4_0(std::uint32_t a, std::uint32_t b) {
  int r;
  asm("v_dot4_i32_i8 %0, %1, %2, 0" : "=v"(r) : "v"(a), "v"(b));
  return r;
}

// The dot of 16 int8 weights (4 words) with a staged group.
__device__ __forceinline__ int dot16(const std::uint32_t w[4], const XG& x) {
  int ah = sdot4_0(w[0], x.h[0]), al = sdot4_0(w[0], x.l[0]);
#pragma unroll
  for (int i = 1; i < 4; ++i) {
    ah = __builtin_amdgcn_sdot4(static_cast<int>(w[i]), static_cast<int>(x.h[i]), ah, false);
    al = __builtin_amdgcn_sdot4(static_cast<int>(w[i]), static_cast<int>(x.l[i]), al, false);
  }
  return dot_digits(ah, al);
}

}  // namespace rtxllm
