// Activation staging for the integer-dot matvec kernels.
//
// The matvec kernels multiply small integer weight codes (Q4_K/Q5_K quants,
// signed IQ grid magnitudes) with the activation through v_dot4_i32_i8. For
// that the fp32 activation is staged once per 16-value group as block fixed
// point with a power-of-two scale: with m = max|x| = f 2^e (f in [0.5, 1)),
// s = 2^(e - 22) and X_j = rint(x_j 2^(22 - e)), so |X_j| <= 2^22 and x_j ~= s
// X_j with an error of at most s / 2 <= 2^-22 m (the power-of-two scaling is
// exact, so X_j is x_j rounded once). X_j is held as three int8 digits X_j =
// 65536 H_j + 256 M_j + L_j (H in [-64, 64], M and L in [-128, 127]). The
// integer dot products with the weight codes are exact; only the staging
// rounds, by less than an fp32 product accumulated over a row does (a
// 4096-column row's fp32 sequential sum carries ~2^-24 n / 2 of its terms'
// size; the staging ~2^-23 sqrt(n)).
// A group holding a NaN gets s = NaN and zero digits, so every product it
// enters is NaN (as in fp32); a group whose maximum is infinite gets s = inf
// and zero digits (its products become NaN, where fp32 gives +-inf or NaN).
// Every producer (the staging kernel, the kernels' self-staging path, fused
// epilogues) implements this one rule, so all paths see identical digits.
//
// HBM layout of a staged vector of `cols` values (cols % 256 == 0), one
// allocation of xq_bytes(cols):
//   [0, cols)               int8 H digits
//   [cols, 2 cols)          int8 M digits
//   [2 cols, 3 cols)        int8 L digits
//   [3 cols, 3 cols + G*4)  f32 group scale s, G = cols / 16
//   [.., + G*4)             f32 group sum s * sum_j X_j
#pragma once

#include "common.h"

namespace rtxllm {

constexpr int kXGroup = 16;
constexpr int kXQBits = 22;  // |X| <= 2^22
// X + kXQBias = 65536 H + 256 (M + 128) + (L + 128): the digits are bytes of it.
constexpr int kXQBias = 128 * 256 + 128;

// X -> (H, M, L) with X = 65536 H + 256 M + L, |X| <= 2^22.
__host__ __device__ inline void xq_digits(int X, int& H, int& M, int& L) {
  const int Y = X + kXQBias;
  L = (Y & 0xFF) - 128;
  M = ((Y >> 8) & 0xFF) - 128;
  H = Y >> 16;
}

// The scale of a group from its maximum magnitude m (NaN ignored) and whether
// it holds a NaN: s and the shift 22 - e with which X = rint(ldexp(x, shift));
// finite is false for a NaN or infinite group (all digits zero).
struct XScale {
  float s;
  int shift;
  bool finite;
};

__device__ __forceinline__ XScale xq_scale(float m, bool nan) {
  XScale r;
  r.finite = !nan && m <= 3.40282347e38f;
  const int e = (r.finite && m > 0.0f) ? __builtin_amdgcn_frexp_expf(m) : 0;
  r.shift = kXQBits - e;
  r.s = nan ? __builtin_nanf("") : (!r.finite ? __builtin_inff() : (m > 0.0f ? __builtin_amdgcn_ldexpf(1.0f, e - kXQBits) : 0.0f));
  return r;
}

__device__ __forceinline__ int xq_fixed(float x, const XScale& sc) {
  return sc.finite ? static_cast<int>(rintf(__builtin_amdgcn_ldexpf(x, sc.shift))) : 0;
}

// One staged group in a lane's registers: digit j in byte (j & 3) of word j >> 2.
struct XG {
  std::uint32_t h[4];
  std::uint32_t m[4];
  std::uint32_t l[4];
  float s;
  float sum;
};

struct XQ {
  const std::int8_t* h;
  const std::int8_t* m;
  const std::int8_t* l;
  const float* s;
  const float* sum;
};

struct XQOut {
  std::int8_t* h;
  std::int8_t* m;
  std::int8_t* l;
  float* s;
  float* sum;
};

__host__ __device__ constexpr std::size_t xq_bytes(std::uint32_t cols) {
  return 3u * static_cast<std::size_t>(cols) + 8u * static_cast<std::size_t>(cols / kXGroup);
}

__host__ __device__ inline XQ xq_view(const void* base, std::uint32_t cols) {
  const std::int8_t* b = static_cast<const std::int8_t*>(base);
  const std::size_t c = cols;
  const float* s = reinterpret_cast<const float*>(b + 3u * c);
  return XQ{b, b + c, b + 2u * c, s, s + cols / kXGroup};
}

__host__ __device__ inline XQOut xq_out(void* base, std::uint32_t cols) {
  std::int8_t* b = static_cast<std::int8_t*>(base);
  const std::size_t c = cols;
  float* s = reinterpret_cast<float*>(b + 3u * c);
  return XQOut{b, b + c, b + 2u * c, s, s + cols / kXGroup};
}

// Stage 16 values (the rule above). The digit words come from Y = X + kXQBias:
// byte 0 of Y is L + 128, byte 1 is M + 128 and byte 2 is H (as int8), so byte
// permutes gather four values' digits into a word (the bias is undone by
// flipping bit 7 of L and M).
__device__ __forceinline__ void quant16(const float v[16], XG& g) {
  float m = 0.0f;
  bool nan = false;
#pragma unroll
  for (int j = 0; j < 16; j += 2) nan = nan || __builtin_isunordered(v[j], v[j + 1]);
#pragma unroll
  for (int j = 0; j < 16; ++j) m = fmaxf(m, fabsf(v[j]));
  const XScale sc = xq_scale(m, nan);
  g.s = sc.s;
  int total = 0;
#pragma unroll
  for (int w = 0; w < 4; ++w) {
    std::uint32_t Y[4];
#pragma unroll
    for (int b = 0; b < 4; ++b) {
      const int X = xq_fixed(v[4 * w + b], sc);
      total += X;
      Y[b] = static_cast<std::uint32_t>(X + kXQBias);
    }
    // byte i of the result: selector byte i, 0-3 = bytes of the second source, 4-7 of the first
    const std::uint32_t p01 = __builtin_amdgcn_perm(Y[1], Y[0], 0x05010400u);  // Y0.b0 Y1.b0 Y0.b1 Y1.b1
    const std::uint32_t p23 = __builtin_amdgcn_perm(Y[3], Y[2], 0x05010400u);
    const std::uint32_t q01 = __builtin_amdgcn_perm(Y[1], Y[0], 0x06020602u);  // Y0.b2 Y1.b2
    const std::uint32_t q23 = __builtin_amdgcn_perm(Y[3], Y[2], 0x06020602u);
    g.l[w] = __builtin_amdgcn_perm(p23, p01, 0x05040100u) ^ 0x80808080u;
    g.m[w] = __builtin_amdgcn_perm(p23, p01, 0x07060302u) ^ 0x80808080u;
    g.h[w] = __builtin_amdgcn_perm(q23, q01, 0x05040100u);
  }
  g.sum = g.s * static_cast<float>(total);
}

__device__ __forceinline__ void xg_load(const XQ& x, std::uint32_t group, XG& g) {
  const uint4 h = *reinterpret_cast<const uint4*>(x.h + kXGroup * group);
  const uint4 m = *reinterpret_cast<const uint4*>(x.m + kXGroup * group);
  const uint4 l = *reinterpret_cast<const uint4*>(x.l + kXGroup * group);
  g.h[0] = h.x, g.h[1] = h.y, g.h[2] = h.z, g.h[3] = h.w;
  g.m[0] = m.x, g.m[1] = m.y, g.m[2] = m.z, g.m[3] = m.w;
  g.l[0] = l.x, g.l[1] = l.y, g.l[2] = l.z, g.l[3] = l.w;
  g.s = x.s[group];
  g.sum = x.sum[group];
}

// Stage group `group` of an fp32 vector (optionally times an elementwise weight).
// ALIGNED: x (and mul) are 16-byte aligned, so the group is read as four
// float4; otherwise as sixteen floats.
template <bool ALIGNED = true>
__device__ __forceinline__ void xg_stage(const float* __restrict__ x, const float* __restrict__ mul,
                                         std::uint32_t group, XG& g) {
  float v[16];
  if constexpr (ALIGNED) {
    const float4* p = reinterpret_cast<const float4*>(x + kXGroup * group);
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const float4 t = p[i];
      v[4 * i] = t.x, v[4 * i + 1] = t.y, v[4 * i + 2] = t.z, v[4 * i + 3] = t.w;
    }
  } else {
#pragma unroll
    for (int i = 0; i < 16; ++i) v[i] = x[kXGroup * group + i];
  }
  if (mul != nullptr) {
    if constexpr (ALIGNED) {
      const float4* q = reinterpret_cast<const float4*>(mul + kXGroup * group);
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const float4 t = q[i];
        v[4 * i] *= t.x, v[4 * i + 1] *= t.y, v[4 * i + 2] *= t.z, v[4 * i + 3] *= t.w;
      }
    } else {
#pragma unroll
      for (int i = 0; i < 16; ++i) v[i] *= mul[kXGroup * group + i];
    }
  }
  quant16(v, g);
}

// xg_stage without the multiplier, in two steps: the group's sixteen floats as
// one vector value (xg_read), then the quant16 rule (xg_quant), so that a
// caller can issue other loads between them. The same digits as xg_stage.
typedef float f32x16 __attribute__((ext_vector_type(16)));
template <bool ALIGNED = true>
__device__ __forceinline__ f32x16 xg_read(const float* __restrict__ x, std::uint32_t group) {
  f32x16 v;
  if constexpr (ALIGNED) {
    const float4* p = reinterpret_cast<const float4*>(x + kXGroup * group);
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const float4 t = p[i];
      v[4 * i] = t.x, v[4 * i + 1] = t.y, v[4 * i + 2] = t.z, v[4 * i + 3] = t.w;
    }
  } else {
#pragma unroll
    for (int i = 0; i < 16; ++i) v[i] = x[kXGroup * group + i];
  }
  return v;
}
__device__ __forceinline__ void xg_quant(const f32x16& v, XG& g) {
  float a[16];
#pragma unroll
  for (int i = 0; i < 16; ++i) a[i] = v[i];
  quant16(a, g);
}

__device__ __forceinline__ void xg_store(const XQOut& x, std::uint32_t group, const XG& g) {
  *reinterpret_cast<uint4*>(x.h + kXGroup * group) = make_uint4(g.h[0], g.h[1], g.h[2], g.h[3]);
  *reinterpret_cast<uint4*>(x.m + kXGroup * group) = make_uint4(g.m[0], g.m[1], g.m[2], g.m[3]);
  *reinterpret_cast<uint4*>(x.l + kXGroup * group) = make_uint4(g.l[0], g.l[1], g.l[2], g.l[3]);
  x.s[group] = g.s;
  x.sum[group] = g.sum;
}

// The dot of 16 int8 weights (4 words) with a staged group: sum_j w_j X_j =
// 65536 sum w H + 256 sum w M + sum w L, exact in int32 for weight codes |w| <=
// 31 (|result| <= 16 * 31 * 2^22 < 2^31). One chain of dot4 accumulations:
// the H sums from 0, then the M sums from that shifted by 8, then the L sums
// from that shifted by 8, i.e. ((sum w H) 256 + sum w M) 256 + sum w L; the
// shifts and adds may wrap in between without changing the result. All of it
// goes through the builtin, so the compiler sees each dot instruction (a
// dot's result read by a different VALU opcode needs three wait states,
// which its hazard pass inserts only for instructions it can see).
__device__ __forceinline__ int dot16(const std::uint32_t w[4], const XG& x) {
  int a = __builtin_amdgcn_sdot4(static_cast<int>(w[0]), static_cast<int>(x.h[0]), 0, false);
#pragma unroll
  for (int i = 1; i < 4; ++i) a = __builtin_amdgcn_sdot4(static_cast<int>(w[i]), static_cast<int>(x.h[i]), a, false);
  a = static_cast<int>(static_cast<std::uint32_t>(a) << 8);
#pragma unroll
  for (int i = 0; i < 4; ++i) a = __builtin_amdgcn_sdot4(static_cast<int>(w[i]), static_cast<int>(x.m[i]), a, false);
  a = static_cast<int>(static_cast<std::uint32_t>(a) << 8);
#pragma unroll
  for (int i = 0; i < 4; ++i) a = __builtin_amdgcn_sdot4(static_cast<int>(w[i]), static_cast<int>(x.l[i]), a, false);
  return a;
}

}  // namespace rtxllm
