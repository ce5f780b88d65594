// Batched (up to 8 activation vectors) dequant-matvec on the matrix cores:
// Y[s][r] = sum_c W[r][c] X[s][c] for s < batch, W in a GGUF pack.
//
// Operands of v_mfma_f32_16x16x32_f16 (lane layouts checked on gfx950):
//   A (16 rows x 32 k):  lane l holds A[l % 16][8 (l / 16) + i], i < 8;
//   B (32 k x 16 cols):  lane l holds B[8 (l / 16) + i][l % 16];
//   C (16 x 16, fp32):   lane l holds C[4 (l / 16) + i][l % 16], i < 4.
// The k order inside one instruction is free as long as A and B agree. Lane
// q = l / 16 of a 256-value block takes values [64 q, 64 q + 64), eight per
// instruction (instruction j: values 64 q + 8 j .. + 8), so each lane reads its
// weight fields as a few contiguous runs.
//
// * A: the weight codes times their sub-block scale integer, in fp16. These
//   products are small integers (IQ2_S |mag (2n+1)| <= 217, IQ3_S <= 465, Q4_K
//   q sc <= 945, Q5_K <= 1953), exact in fp16. K-quant mins go through a second
//   product with A = the sub-block's m (<= 63).
// * B: column n = 2 s + h holds sequence s's activation as two fp16 halves
//   (h = 0: hi = fp16(x'), h = 1: lo = fp16(x' - hi)), x' = x 2^-e_s with a
//   per-sequence power of two that puts max |x'| in [0.5, 1): ~22 bits of x.
// * C accumulates one 256-value block exactly-rounded in fp32 (every A*B
//   product is exact); per block the rows' fp16 super-block scale d (and dmin)
//   multiply it into the fp32 result.
//
// A wave owns a panel of 512 columns (two blocks) for the whole launch, its 16
// B operands (64 VGPRs) loaded once; a workgroup holds up to 8 panels (one wave
// each) and loops over 16-row tiles, combining the panels' partial sums in LDS.
// Matrices wider than 8 panels split into panel groups whose partial results a
// second kernel adds.
#pragma once

#include <type_traits>

#include "mv.cuh"
#include "x16.h"

namespace rtxllm {

typedef _Float16 half8 __attribute__((ext_vector_type(8)));
typedef float f32x4 __attribute__((ext_vector_type(4)));

// 512-column panels measured faster than 256-column ones in 16-wave workgroups
// (the latter halve B's registers, 4 waves per SIMD instead of 3, but add
// partials and barrier waits: the batch-8 step lost 6 %).
constexpr std::uint32_t kPanel = 512;                 // columns per wave
constexpr int kPanelBlocks = kPanel / 256;            // 256-value blocks per panel
constexpr std::uint32_t kMaxPanels = 4096 / kPanel;   // waves per workgroup (4096 columns)

constexpr bool fmt_mm_supported(int f) {
  return f == RTXLLM_FMT_IQ2S || f == RTXLLM_FMT_IQ3S || f == RTXLLM_FMT_Q5K || f == RTXLLM_FMT_Q4K_RAW ||
         f == RTXLLM_FMT_Q4K_SPLIT_NATIVE;
}

// ---- LDS tables: int8 codebooks and sign masks ------------------------------------------

// grid2b: IQ2_S entry -> its 8 magnitude bytes 2 l + 1, each ^ 0x80; grid3b: IQ3_S
// entry -> 4 magnitude bytes ^ 0x80; sign: sign byte -> (M0, M1), byte j of M
// 0xFF when value j is negative. As in the batch-1 decode, (g ^ M) | 0x01010101
// signs the odd magnitudes in one v_bitop3; with the stored ^ 0x80 each byte
// comes out as 128 + w, the biased form mm_biased_pair turns into fp16.
struct MmLds2 {
  uint2 grid2b[1024];
  uint2 sign[256];
};
struct MmLds3 {
  std::uint32_t grid3b[512];
  uint2 sign[256];
};
template <int FMT>
using MmLds = typename std::conditional<FMT == RTXLLM_FMT_IQ2S, MmLds2, MmLds3>::type;

constexpr IqImage<2560> mm2_image() {
  IqImage<2560> im{};
  for (std::uint32_t i = 0; i < 1024u; ++i) {
    const std::uint32_t w = kIq2sGridSrc[i];
    std::uint32_t lo = 0u, hi = 0u;
    for (int j = 0; j < 4; ++j) {
      lo |= ((2u * ((w >> (2 * j)) & 3u) + 1u) ^ 0x80u) << (8 * j);
      hi |= ((2u * ((w >> (2 * j + 8)) & 3u) + 1u) ^ 0x80u) << (8 * j);
    }
    im.w[2 * i] = lo;
    im.w[2 * i + 1] = hi;
  }
  iq_image_signs(im, 2048);
  return im;
}
constexpr IqImage<1024> mm3_image() {
  IqImage<1024> im{};
  for (std::uint32_t i = 0; i < 512u; ++i) im.w[i] = kIq3sGridSrc[i] ^ 0x80808080u;
  iq_image_signs(im, 512);
  return im;
}
static_assert(sizeof(IqImage<2560>) == sizeof(MmLds2) && sizeof(IqImage<1024>) == sizeof(MmLds3), "mm images");
__device__ const IqImage<2560> kMm2Image = mm2_image();
__device__ const IqImage<1024> kMm3Image = mm3_image();

template <int FMT>
__device__ __forceinline__ MmLds<FMT>& mm_lds() {
  __shared__ MmLds<FMT> t;
  return t;
}

// The codebook fill of the batch kernels: lds_grid_issue / lds_grid_commit,
// sized for workgroups of eight waves (one 16-byte piece per thread).
template <int FMT>
using MmGridStage = LdsGridStage<MmLds<FMT>, 512u>;
template <int FMT>
__device__ __forceinline__ const void* mm_image() {
  return FMT == RTXLLM_FMT_IQ2S ? static_cast<const void*>(&kMm2Image) : static_cast<const void*>(&kMm3Image);
}

// ---- per-lane block fields --------------------------------------------------------

// Lane q's fields of one 256-value block (values [64 q, 64 q + 64)).
struct MmRaw {
  std::uint32_t a[8];  // IQ2_S: qs[0..1] signs[2..3]; IQ3_S: qs[0..3] signs[4..5]; K: quants (32 B)
  std::uint32_t b[8];  // Q5_K: qh (32 B)
  std::uint32_t h[4];  // K: the 16 B head (d, dmin, scales)
  // IQ: d, the qh pair, the scale pair (IQ2_S) or byte (IQ3_S), kept at their
  // loaded width so their zero extension happens where they are used
  std::uint16_t s[3];
  std::uint8_t s8;
};

template <int FMT>
__device__ __forceinline__ void mm_load(Rsrc rp, Rsrc rm, std::uint32_t vp, std::uint32_t vm, std::uint32_t sp,
                                        std::uint32_t sm, std::uint32_t blk, std::uint32_t q, MmRaw& r) {
  constexpr int P = load_policy<FMT>();
  if constexpr (FMT == RTXLLM_FMT_IQ2S) {
    const std::uint32_t o = vp + blk * 82u;
    const u32x2 qs = bld_u64<P>(rp, o + 2u + 8u * q, sp);
    const u32x2 sg = bld_u64<P>(rp, o + 34u + 8u * q, sp);
    r.a[0] = qs.x, r.a[1] = qs.y, r.a[2] = sg.x, r.a[3] = sg.y;
    r.s[0] = bld_u16<P>(rp, o, sp);
    r.s[1] = bld_u16<P>(rp, o + 66u + 2u * q, sp);
    r.s[2] = bld_u16<P>(rp, o + 74u + 2u * q, sp);
  } else if constexpr (FMT == RTXLLM_FMT_IQ3S) {
    const std::uint32_t o = vp + blk * 110u;
    const u32x2 q0 = bld_u64<P>(rp, o + 2u + 16u * q, sp);
    const u32x2 q1 = bld_u64<P>(rp, o + 10u + 16u * q, sp);
    const u32x2 sg = bld_u64<P>(rp, o + 74u + 8u * q, sp);
    r.a[0] = q0.x, r.a[1] = q0.y, r.a[2] = q1.x, r.a[3] = q1.y, r.a[4] = sg.x, r.a[5] = sg.y;
    r.s[0] = bld_u16<P>(rp, o, sp);
    r.s[1] = bld_u16<P>(rp, o + 66u + 2u * q, sp);
    r.s8 = bld_u8<P>(rp, o + 106u + q, sp);
  } else {
    std::uint32_t qo, ho;
    Rsrc hr = rp;
    std::uint32_t hs = sp;
    if constexpr (FMT == RTXLLM_FMT_Q5K) {
      qo = vp + blk * 176u + 48u + 32u * q, ho = vp + blk * 176u;
      const u32x4 h0 = bld_u128<P>(rp, ho + 16u, sp);
      const u32x4 h1 = bld_u128<P>(rp, ho + 32u, sp);
      r.b[0] = h0.x, r.b[1] = h0.y, r.b[2] = h0.z, r.b[3] = h0.w;
      r.b[4] = h1.x, r.b[5] = h1.y, r.b[6] = h1.z, r.b[7] = h1.w;
    } else if constexpr (FMT == RTXLLM_FMT_Q4K_RAW) {
      qo = vp + blk * 144u + 16u + 32u * q, ho = vp + blk * 144u;
    } else {  // split-native: 128 B payload, 16 B head in the metadata stream
      qo = vp + blk * 128u + 32u * q, ho = vm + blk * 16u;
      hr = rm, hs = sm;
    }
    const u32x4 a0 = bld_u128<P>(rp, qo, sp);
    const u32x4 a1 = bld_u128<P>(rp, qo + 16u, sp);
    r.a[0] = a0.x, r.a[1] = a0.y, r.a[2] = a0.z, r.a[3] = a0.w;
    r.a[4] = a1.x, r.a[5] = a1.y, r.a[6] = a1.z, r.a[7] = a1.w;
    const u32x4 hh = bld_u128<P>(hr, ho, hs);
    r.h[0] = hh.x, r.h[1] = hh.y, r.h[2] = hh.z, r.h[3] = hh.w;
  }
}

__device__ __forceinline__ half8 as_half8(const uint4& u) { return __builtin_bit_cast(half8, u); }

// Two fp16 values fma(v, f, -1024 f) of two fp16 halves v = 1024 + c: c f in
// one rounding.
__device__ __forceinline__ std::uint32_t code_pair_times(std::uint32_t halves, _Float16 f) {
  typedef _Float16 half2 __attribute__((ext_vector_type(2)));
  const half2 v = __builtin_bit_cast(half2, halves);
  const half2 ff = {f, f};
  const half2 c = {static_cast<_Float16>(-1024.0f) * f, static_cast<_Float16>(-1024.0f) * f};
  return __builtin_bit_cast(std::uint32_t, __builtin_elementwise_fma(v, ff, c));
}

// Two fp16 products w m from bytes b0, b1 of `biased` (selector 0x04010400) or
// b2, b3 (0x04030402), each byte 128 + w: the halves (0x64 << 8 | byte) are
// 1152 + w, and fma(1152 + w, m, -1152 m) = w m in one rounding (exact: |w m|
// < 2048, and 1152 m = 2^7 * 9 m is an fp16 integer for m < 228).
__device__ __forceinline__ std::uint32_t mm_biased_pair(std::uint32_t biased, std::uint32_t sel, _Float16 m) {
  typedef _Float16 half2 __attribute__((ext_vector_type(2)));
  const half2 v = __builtin_bit_cast(half2, __builtin_amdgcn_perm(0x64646464u, biased, sel));
  const half2 mm = {m, m};
  const half2 c = {static_cast<_Float16>(-1152.0f) * m, static_cast<_Float16>(-1152.0f) * m};
  return __builtin_bit_cast(std::uint32_t, __builtin_elementwise_fma(v, mm, c));
}

// A operand of instruction j (values 64 q + 8 j .. + 8 of the block).
template <int FMT>
__device__ __forceinline__ half8 mm_decode(const MmRaw& r, const MmLds<FMT>* t, int j, std::uint32_t q,
                                           half8& amin) {
  if constexpr (FMT == RTXLLM_FMT_IQ2S) {
    // grid index qs[j] | (qh >> 2 (j & 3) & 3) << 8: the qh byte's four 2-bit
    // fields spread one per byte, and one v_perm lays the index pair (j, j ^ 1)
    // into the two 16-bit halves (both computed once per word / pair)
    const std::uint32_t qh = (std::uint32_t{r.s[1]} >> (8 * (j >> 2))) & 0xFFu;  // qh of sub-block 2 q + j / 4
    const std::uint32_t s6 = (qh << 6) | qh;
    const std::uint32_t hb = ((s6 << 12) | s6) & 0x03030303u;
    const std::uint32_t ip = __builtin_amdgcn_perm(hb, r.a[j >> 2], (j & 2) ? 0x07030602u : 0x05010400u);
    const std::uint32_t idx = (j & 1) ? ip >> 16 : ip & 0xFFFFu;
    const std::uint32_t sgb = (r.a[2 + (j >> 2)] >> (8 * (j & 3))) & 0xFFu;
    const uint2 g = t->grid2b[idx];
    const uint2 sm = t->sign[sgb];
    const std::uint32_t nib = ((std::uint32_t{r.s[2]} >> (8 * (j >> 2))) >> (4 * ((j & 3) >> 1))) & 15u;
    const _Float16 m = static_cast<_Float16>(static_cast<std::uint16_t>(2u * nib + 1u));  // one v_cvt_f16_u16
    const std::uint32_t b0 = (g.x ^ sm.x) | 0x01010101u, b1 = (g.y ^ sm.y) | 0x01010101u;
    return as_half8(make_uint4(mm_biased_pair(b0, 0x04010400u, m), mm_biased_pair(b0, 0x04030402u, m),
                               mm_biased_pair(b1, 0x04010400u, m), mm_biased_pair(b1, 0x04030402u, m)));
  } else if constexpr (FMT == RTXLLM_FMT_IQ3S) {
    const std::uint32_t sub = static_cast<std::uint32_t>(j >> 2);          // 32-value sub-block 2 q + sub
    const std::uint32_t qh = (std::uint32_t{r.s[1]} >> (8 * sub)) & 0xFFu;
    const int sel0 = 2 * (j & 3), sel1 = sel0 + 1;                         // qs bytes of this group
    const std::uint32_t w16 = r.a[(2 * j) >> 2] >> (8 * ((2 * j) & 3));    // qs[2 j], qs[2 j + 1]
    const std::uint32_t i0 = (w16 & 0xFFu) | (((qh >> sel0) & 1u) << 8);
    const std::uint32_t i1 = ((w16 >> 8) & 0xFFu) | (((qh >> sel1) & 1u) << 8);
    const std::uint32_t sgb = (r.a[4 + (j >> 2)] >> (8 * (j & 3))) & 0xFFu;
    const std::uint32_t g0 = t->grid3b[i0], g1 = t->grid3b[i1];
    const uint2 sm = t->sign[sgb];
    const std::uint32_t nib = (std::uint32_t{r.s8} >> (4u * sub)) & 15u;
    const _Float16 m = static_cast<_Float16>(static_cast<std::uint16_t>(2u * nib + 1u));  // one v_cvt_f16_u16
    const std::uint32_t b0 = (g0 ^ sm.x) | 0x01010101u, b1 = (g1 ^ sm.y) | 0x01010101u;
    return as_half8(make_uint4(mm_biased_pair(b0, 0x04010400u, m), mm_biased_pair(b0, 0x04030402u, m),
                               mm_biased_pair(b1, 0x04010400u, m), mm_biased_pair(b1, 0x04030402u, m)));
  } else {
    // K-quants: j < 4 low nibbles of bytes 8 j .. + 8 of the lane's 32 (sub-block
    // 2 q), j >= 4 high nibbles of bytes 8 (j - 4) .. (sub-block 2 q + 1).
    const int hi = j >> 2, w = 2 * (j & 3);
    const std::uint32_t sc03 = r.h[1] & 0x3F3F3F3Fu;
    const std::uint32_t m03 = r.h[2] & 0x3F3F3F3Fu;
    const std::uint32_t sc47 = (r.h[3] & 0x0F0F0F0Fu) | ((r.h[1] >> 2) & 0x30303030u);
    const std::uint32_t m47 = ((r.h[3] >> 4) & 0x0F0F0F0Fu) | ((r.h[2] >> 2) & 0x30303030u);
    const std::uint32_t pair = 2u * q + static_cast<std::uint32_t>(hi);   // sub-block 0..7
    const std::uint32_t scw = pair < 4u ? sc03 : sc47, mw = pair < 4u ? m03 : m47;
    const std::uint32_t sc = (scw >> (8u * (pair & 3u))) & 0xFFu, mn = (mw >> (8u * (pair & 3u))) & 0xFFu;
    const _Float16 scf = static_cast<_Float16>(static_cast<float>(sc));
    const _Float16 mf = static_cast<_Float16>(static_cast<float>(mn));
    amin = half8{mf, mf, mf, mf, mf, mf, mf, mf};
    // Each code byte stays in place, masked to its nibble: the low nibble n
    // (j < 4), or the high one as 16 n (j >= 4). v_perm pairs two such bytes
    // with a high byte 0x64 into fp16 halves 1024 + n (+ 16 h for Q5_K: the
    // qh bit at bit 4), or 1024 + 16 n (+ 256 h: the qh bit at bit 0 of the
    // high byte). fma(half, f, -1024 f) with f = sc, or sc / 16 for the
    // high nibbles, is then (n + 16 h) sc in one rounding (exact: < 2048, and
    // sc / 16 and 1024 f are fp16-exact for sc < 64).
    const _Float16 f = hi ? scf * static_cast<_Float16>(0.0625f) : scf;
    std::uint32_t out[4];
#pragma unroll
    for (int k = 0; k < 2; ++k) {
      std::uint32_t codes = r.a[w + k] & (hi ? 0xF0F0F0F0u : 0x0F0F0F0Fu);
      std::uint32_t top = 0x64646464u;
      if constexpr (FMT == RTXLLM_FMT_Q5K) {
        // bit `pair` of each qh byte, rotated to bit 4 (low nibbles) or bit 0
        // (high nibbles, into the 0x64 byte) of the same byte
        if (hi)
          top |= __builtin_rotateright32(r.b[w + k], pair) & 0x01010101u;
        else
          codes |= __builtin_rotateright32(r.b[w + k], (pair + 28u) & 31u) & 0x10101010u;
      }
      out[2 * k] = code_pair_times(__builtin_amdgcn_perm(top, codes, 0x05010400u), f);      // bytes 0, 1
      out[2 * k + 1] = code_pair_times(__builtin_amdgcn_perm(top, codes, 0x07030602u), f);  // bytes 2, 3
    }
    return as_half8(make_uint4(out[0], out[1], out[2], out[3]));
  }
}

// d (and dmin) of the block for the lane's row, as fp32.
// (IQ2_S: d (0.5 + n) / 4 = d / 8 * (2 n + 1), the 2 n + 1 being in A.)
template <int FMT>
__device__ __forceinline__ void mm_block_scale(const MmRaw& r, float& d, float& dmin) {
  if constexpr (fmt_is_iq(FMT)) {
    d = h2f(r.s[0]);
    if constexpr (FMT == RTXLLM_FMT_IQ2S) d *= 0.125f;
    dmin = 0.0f;
  } else {
    d = h2f(r.h[0]);
    dmin = h2f(r.h[0] >> 16);
  }
}

// ---- the kernel ----------------------------------------------------------------------

// f(integral_constant<int, I>) for I = 0 .. N - 1, unrolled at compile time.
template <int N, int I = 0, class F>
__device__ __forceinline__ void static_for(F&& f) {
  if constexpr (I < N) {
    f(std::integral_constant<int, I>{});
    static_for<N, I + 1>(f);
  }
}

// Depth of the per-wave ring of block loads in flight (units issued ahead of
// the one being computed = depth - 1); the wider the lane's fields, the shallower.
template <int FMT>
constexpr int mm_ring() {
  return FMT == RTXLLM_FMT_Q5K ? 2 : (fmt_is_iq(FMT) ? 4 : 3);
}

// Plain output: out[pg][s][row] (pg = panel group = blockIdx.y, row stride
// `stride`): y itself with one panel group, else the groups' partial sums.
struct MmStore {
  static constexpr int tl_region(int fmt) { return fmt_is_iq(fmt) ? kTlMmO : kTlMmDown; }
  float* out;
  std::uint32_t stride, batch;
  __device__ __forceinline__ void init(std::uint32_t) {}
  __device__ __forceinline__ void operator()(std::uint32_t row, std::uint32_t s, float v, float) const {
    out[(static_cast<std::size_t>(blockIdx.y) * batch + s) * stride + row] = v;
  }
  __device__ __forceinline__ void finish(std::uint32_t, std::uint32_t, std::uint32_t) {}
};

// Grid: x = workgroups over 16-row tiles (persistent: workgroup g takes tiles
// g, g + gridDim.x, ...), y = panel group of blockDim.x / 64 panels. Each
// finished y[s][row] (s < batch) goes to the epilogue: epi.init(s) once per
// thread (a thread only ever sees one sequence), epi(row, s, y, y of row ^ 1),
// and epi.finish(wave, lane, waves) after the last tile. Epilogues other than
// MmStore need a single panel group.
// SELF: x16 is instead the fp32 activation [batch][cols], staged by each wave
// for its own panel with the plain staging rule (block exponent from the
// block's max |x|, hi / lo fp16 halves), so no staging launch precedes it.
template <int FMT, class Epi, bool SELF = false>
__global__ __launch_bounds__(64 * kMaxPanels) void mm_kernel(QTensor w, const void* __restrict__ x16,
                                                             std::uint32_t batch, Epi epi) {
  // per-panel partial C of a tile, double buffered by tile parity
  __shared__ float red[2][kMaxPanels][256];
  const std::uint32_t lane = threadIdx.x & 63u;
  const std::uint32_t wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  constexpr int kTlR = TlRegionOf<Epi>::value(FMT);
  const std::uint32_t tl_slot = ((blockIdx.y * gridDim.x + blockIdx.x) * kMaxPanels + wave) * 16u;
  tl_stamp(kTlR, tl_slot);
  // read once, in an SGPR: a later read of the workgroup size is a vector load,
  // and its wait would also wait for the ring's loads in flight
  const std::uint32_t nw = __builtin_amdgcn_readfirstlane(blockDim.x >> 6);
  const std::uint32_t panel = blockIdx.y * nw + wave;  // the launcher makes nw divide the panel count
  const std::uint32_t cols = w.cols, rows = w.rows, bpr = cols >> 8;
  const std::uint32_t q = lane >> 4, r16 = lane & 15u;
  const std::uint32_t tiles = (rows + 15u) >> 4;
  const std::uint32_t nb = cols >> 8;  // 256-value blocks per row

  // The codebook image is the first load of the wave: the barrier after its
  // LDS fill then waits for it alone (the wait counters complete in issue
  // order), not for the B operands and weights behind it.
  const MmLds<FMT>* tables = nullptr;
  MmGridStage<FMT> grid_stage;
  if constexpr (fmt_is_iq(FMT)) {
    tables = &mm_lds<FMT>();
    lds_grid_issue(grid_stage, mm_image<FMT>(), threadIdx.x, blockDim.x);
  }

  // Tile epilogue: thread t takes C elements t, t + blockDim.x, ... < 256;
  // element (lane l = e / 4, i = e % 4) is row 4 (l / 16) + i, column
  // n = l % 16 = 2 s + hi/lo. blockDim.x being a multiple of 64, n and s are
  // the same for all of a thread's elements; t_post is the sequence's RMSNorm
  // scale (1 for a plainly staged input).
  const std::uint32_t t_n = (threadIdx.x >> 2) & 15u, t_s = t_n >> 1;
  const bool t_store = (t_n & 1u) == 0u && t_s < batch;
  // Its inputs (eps and the sequence's per-block sums of squares from the
  // staged tail) are read first and added once the weight loads are issued:
  // a value used right away would make the wave wait for every load before
  // it, here the B operands. Held as one vector value (no array the compiler
  // could move to memory); inputs wider than 16 blocks add the rest later.
  typedef float f32x16 __attribute__((ext_vector_type(16)));
  f32x16 t_ssv = {};
  float t_eps = -1.0f;
  if constexpr (!SELF) {
    const X16Tail tail = x16_tail(x16, cols);
    t_eps = *tail.eps;
#pragma unroll
    for (int b = 0; b < 16; ++b) {
      const std::uint32_t bb = static_cast<std::uint32_t>(b) < nb ? static_cast<std::uint32_t>(b) : nb - 1u;
      t_ssv[b] = tail.ss[t_s * nb + bb];
    }
  }

  // B operands of the panel: its blocks x 8 instructions, 1 KB of whole lanes each.
  // The lane's C column is n = lane % 16 = 2 s + hi/lo: its products of block
  // b of the panel carry that sequence's block exponent, 2^e[s][b].
  constexpr int PB = kPanelBlocks;
  uint4 B[PB][8];
  float fb[PB];
  if constexpr (SELF) {
    // lane (q, n = 2 s + h) holds values 256 kb + 64 q + 8 j + i of sequence s
    // in instruction j of block kb; the 4 lanes of a column (q = 0..3) cover
    // the block, so its max is two exchanges away
    const std::uint32_t n = lane & 15u, s = n >> 1;
    const bool ok = s < batch;
    const float* xr = static_cast<const float*>(x16) + static_cast<std::size_t>(ok ? s : 0u) * cols +
                      256u * (PB * panel) + 64u * q;
#pragma unroll
    for (int b = 0; b < PB; ++b) {
      float v[64];
#pragma unroll
      for (int j = 0; j < 16; ++j) {
        const float4 t = reinterpret_cast<const float4*>(xr + 256u * b)[j];
        v[4 * j] = ok ? t.x : 0.0f, v[4 * j + 1] = ok ? t.y : 0.0f;
        v[4 * j + 2] = ok ? t.z : 0.0f, v[4 * j + 3] = ok ? t.w : 0.0f;
      }
      float m = 0.0f;
#pragma unroll
      for (int i = 0; i < 64; ++i) m = fmaxf(m, fabsf(v[i]));
      m = fmaxf(m, __shfl_xor(m, 16, 64));
      m = fmaxf(m, __shfl_xor(m, 32, 64));
      int e = 0;
      if (m > 0.0f && m <= 3.0e38f) frexpf(m, &e);  // m = f 2^e, f in [0.5, 1)
      fb[b] = ldexpf(1.0f, e);
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        half8 h;
#pragma unroll
        for (int i = 0; i < 8; ++i) {
          const float t = ldexpf(v[8 * j + i], -e);
          const _Float16 hi = static_cast<_Float16>(t);
          h[i] = (n & 1u) ? static_cast<_Float16>(t - static_cast<float>(hi)) : hi;
        }
        B[b][j] = __builtin_bit_cast(uint4, h);
      }
    }
  } else {
    // block 0's operands here; the later blocks' go out after the ring's
    // first weight loads, so the first unit waits for block 0 and its weights
    // only
    const uint4* xb = reinterpret_cast<const uint4*>(x16) + PB * panel * 8u * 64u + lane;
#pragma unroll
    for (int j = 0; j < 8; ++j) B[0][j] = xb[j * 64u];
    const X16Tail tail = x16_tail(x16, cols);
#pragma unroll
    for (int b = 0; b < PB; ++b) fb[b] = ldexpf(1.0f, tail.e[((lane & 15u) >> 1) * nb + PB * panel + b]);
  }

  epi.init(t_s);

  const std::uint32_t prow = bpr * FmtBytes<FMT>::payload, mrow = bpr * FmtBytes<FMT>::meta;
  const Rsrc rsp = make_rsrc(w.payload, rows * prow);
  const Rsrc rsm = make_rsrc(FmtBytes<FMT>::meta > 0u ? w.meta : w.payload, rows * mrow);

  // (tile, block) units of this wave in order: unit u -> tile blockIdx.x +
  // (u / PB) * gridDim.x, block PB panel + u % PB. Loads past the workgroup's
  // last unit re-read that unit (no branch around the loads, so the waits on
  // the ring stay exact counts).
  const std::uint32_t rounds = blockIdx.x < tiles ? (tiles - blockIdx.x + gridDim.x - 1u) / gridDim.x : 0u;
  const std::uint32_t units = PB * rounds;
  auto load_unit = [&](std::uint32_t u, MmRaw& raw) {
    u = u < units ? u : units - 1u;
    const std::uint32_t row0 = __builtin_amdgcn_readfirstlane((blockIdx.x + (u / PB) * gridDim.x) * 16u);
    // the tile's first row in the uniform offset, the lane's row within the
    // tile (clamped to the last row) in the per-lane offset
    const std::uint32_t r = min(r16, rows - 1u - row0);
    mm_load<FMT>(rsp, rsm, r * prow, r * mrow, row0 * prow, row0 * mrow, PB * panel + (u % PB), q, raw);
  };
  if (units == 0u) {  // whole workgroup: no barrier is left waiting
    epi.finish(wave, lane, nw);
    tl_stamp(kTlR, tl_slot + 15u);
    return;
  }
  constexpr int NB = mm_ring<FMT>();
  MmRaw ring[NB];
#pragma unroll
  for (int j = 0; j < NB - 1; ++j) load_unit(static_cast<std::uint32_t>(j), ring[j]);
  if constexpr (!SELF) {
    __builtin_amdgcn_sched_barrier(0);  // the ring's loads ahead of the later blocks' operands
    const uint4* xb = reinterpret_cast<const uint4*>(x16) + PB * panel * 8u * 64u + lane;
#pragma unroll
    for (int b = 1; b < PB; ++b)
#pragma unroll
      for (int j = 0; j < 8; ++j) B[b][j] = xb[(8u * b + j) * 64u];
    __builtin_amdgcn_sched_barrier(0);
  }
  if constexpr (fmt_is_iq(FMT))
    lds_grid_commit(mm_lds<FMT>(), grid_stage, mm_image<FMT>(), threadIdx.x, blockDim.x);
  tl_stamp(kTlR, tl_slot + 1u);
  float t_post = 1.0f;
  if constexpr (!SELF) {
    if (t_eps >= 0.0f) {
      float ss = 0.0f;  // in block order
#pragma unroll
      for (int b = 0; b < 16; ++b) ss += static_cast<std::uint32_t>(b) < nb ? t_ssv[b] : 0.0f;
      const X16Tail tail = x16_tail(x16, cols);
      for (std::uint32_t b = 16; b < nb; ++b) ss += tail.ss[t_s * nb + b];
      t_post = 1.0f / sqrtf(ss / static_cast<float>(cols) + t_eps);
    }
  }

  tl_stamp(kTlR, tl_slot + 2u);
  f32x4 acc = {0.0f, 0.0f, 0.0f, 0.0f};
  auto finish_unit = [&](std::uint32_t u, const MmRaw& raw) {
    const int b = static_cast<int>(u % PB);
    f32x4 c = {0.0f, 0.0f, 0.0f, 0.0f}, cm = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      half8 amin;
      const half8 a = mm_decode<FMT>(raw, tables, j, q, amin);
      c = __builtin_amdgcn_mfma_f32_16x16x32_f16(a, as_half8(B[b][j]), c, 0, 0, 0);
      if constexpr (!fmt_is_iq(FMT)) cm = __builtin_amdgcn_mfma_f32_16x16x32_f16(amin, as_half8(B[b][j]), cm, 0, 0, 0);
    }
    // the C rows of this lane are 4 (l / 16) + i; their scales live in the
    // lanes that loaded those rows (lane = row, q = 0); the block exponent of
    // the lane's column is a power of two (exact)
    float d, dmin;
    mm_block_scale<FMT>(raw, d, dmin);
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int src = static_cast<int>(4u * q) + i;
      const float di = __shfl(d, src, 64) * fb[b];
      acc[i] = __builtin_fmaf(c[i], di, acc[i]);
      if constexpr (!fmt_is_iq(FMT)) acc[i] = __builtin_fmaf(-cm[i], __shfl(dmin, src, 64) * fb[b], acc[i]);
    }
  };
  // tile done: every panel's partial to LDS, one barrier, then each of the 256
  // C elements summed over the panels and hi + lo of a sequence written.
  auto tile_end = [&](std::uint32_t round) {
    float* const mine = red[round & 1u][wave];
#pragma unroll
    for (int i = 0; i < 4; ++i) mine[4u * lane + static_cast<std::uint32_t>(i)] = acc[i];
    acc = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
    __syncthreads();
    for (std::uint32_t e = threadIdx.x; e < 256u; e += 64u * nw) {  // whole waves
      float v = 0.0f;
      for (std::uint32_t k = 0; k < nw; ++k) v += red[round & 1u][k][e];
      const float tot = v + __shfl_xor(v, 4, 64);  // column n ^ 1 is lane l ^ 1 = element e ^ 4
      const float y = tot * t_post;
      const float partner = __shfl_xor(y, 1, 64);  // row ^ 1 is element e ^ 1
      const std::uint32_t row = (blockIdx.x + round * gridDim.x) * 16u + 4u * (e >> 6) + (e & 3u);
      if (t_store && row < rows) epi(row, t_s, y, partner);
    }
    tl_stamp(kTlR, tl_slot + 3u + (round < 11u ? round : 11u));
  };

  // unit u sits in ring slot u % NB; PERIOD units bring both the slot and the
  // block within the panel back. The main loop's body runs whole (no exit
  // inside it, so the waits on the ring stay exact counts); the tail runs what
  // is left.
  constexpr int PERIOD = NB % PB == 0 ? NB : PB * NB;
  auto step = [&](std::uint32_t u, auto jc) {
    constexpr int j = decltype(jc)::value;
    load_unit(u + NB - 1u, ring[(j + NB - 1) % NB]);
    __builtin_amdgcn_sched_barrier(0);  // the prefetch is issued before this unit's work
    finish_unit(u, ring[j % NB]);
    if constexpr (j % PB == PB - 1) tile_end(u / PB);
  };
  std::uint32_t u0 = 0;
  for (; u0 + PERIOD <= units; u0 += PERIOD)
    static_for<PERIOD>([&](auto jc) { step(u0 + decltype(jc)::value, jc); });
  static_for<PERIOD>([&](auto jc) {
    if (u0 + decltype(jc)::value < units) step(u0 + decltype(jc)::value, jc);
  });
  epi.finish(wave, lane, nw);
  tl_stamp(kTlR, tl_slot + 15u);
}

// y[s][r] = sum over panel groups of partial[pg][s][r].
__global__ void mm_reduce_kernel(const float* __restrict__ partial, std::uint32_t groups, std::uint32_t n,
                                 float* __restrict__ y) {
  const std::uint32_t i = blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= n) return;
  float s = 0.0f;
  for (std::uint32_t g = 0; g < groups; ++g) s += partial[static_cast<std::size_t>(g) * n + i];
  y[i] = s;
}

}  // namespace rtxllm
