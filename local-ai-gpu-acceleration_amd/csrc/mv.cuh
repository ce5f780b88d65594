// Batch-1 dequant-matvec core for the GGUF resident-pack layouts (gfx950).
//
// Work split. A row of `cols` values is cut into 32-value units (Q4_K/Q5_K: 16
// payload bytes = one half of a 64-value group; IQ2_S/IQ3_S: one 32-value
// sub-block). Lane `lane` of a wave owns units lane, lane + 64, ... of its
// column slice for the whole launch and keeps their staged activation digits
// in registers (two 16-value groups per unit), so x is read once per wave and
// never again. Waves then sweep tiles of TILE consecutive rows: for each row
// every lane loads only its own units' bytes (16-byte nontemporal loads for
// the K-quants, coalesced across the 64 lanes) and accumulates
//   Q4_K/Q5_K:  S_sub * (s_x * sum(q * X)) - M_sub * sum(x_hat)
//   IQ2_S/3_S:  scale_sub * s_x * sum(+-grid * X)
// with the integer sums from v_dot4_i32_i8 on int8 weight codes and the three
// int8 activation digits of the 22-bit staged x (xq.h). Per-row partial sums of a tile are folded across the 64
// lanes by a butterfly transpose-reduce, which leaves row r of the tile in
// lanes [r * 64/TILE, (r+1) * 64/TILE); wide rows (cols > 4096) split their
// columns over KS waves of one workgroup and add the KS partials through LDS.
// The epilogue functor receives the finished tile and writes y (plus any fused
// work). Summation order is fixed, so results are deterministic run to run.
#pragma once

#include <type_traits>
#include <utility>

#include "common.h"
#include "iq_grids.h"
#include "timeline.h"
#include "xq.h"

namespace rtxllm {

typedef unsigned u32x4 __attribute__((ext_vector_type(4)));
typedef unsigned u32x2 __attribute__((ext_vector_type(2)));
typedef unsigned u32x3 __attribute__((ext_vector_type(3)));

struct QTensor {
  const std::uint8_t* payload;  // raw blocks, or the Q4_K split payload stream
  const std::uint8_t* meta;     // Q4_K split metadata stream, else unused
  std::uint32_t rows;
  std::uint32_t cols;
};

// Activation source: staged digits, or fp32 x staged by each wave itself
// (read as float4 when x is 16-byte aligned, else value by value).
struct XSrc {
  XQ xq;
  const float* x;
  std::uint32_t x_aligned;
};

inline XSrc staged_src(const XQ& xq) { return XSrc{xq, nullptr, 1u}; }
inline XSrc self_src(const float* x) {
  return XSrc{XQ{}, x, (reinterpret_cast<std::uintptr_t>(x) % 16u) == 0u ? 1u : 0u};
}


// Weight streams are read through buffer resources: the row's byte offset is a
// scalar (soffset), the lane's field offset a fixed VGPR (voffset), so a load
// costs no address arithmetic, and the hardware range check (num_records = the
// stream's size) turns any access past the end into a zero. Fields at 2-byte
// aligned offsets are read with one unaligned dword / dwordx2 load (gfx950 runs
// in unaligned access mode). Cache policy per format (measured at the 8B
// shapes): the Q4_K streams, one 16 B run of quants per lane, are read
// nontemporal; the IQ and Q5_K blocks are read as several small fields of the
// same cache lines, which only the L1 turns into one L2 request per line, so
// those loads keep the default policy.
typedef __amdgpu_buffer_rsrc_t Rsrc;
constexpr bool fmt_is_iq(int f) {
  return f == RTXLLM_FMT_IQ2S || f == RTXLLM_FMT_IQ3S || f == RTXLLM_FMT_IQ2S_UNITS || f == RTXLLM_FMT_IQ3S_UNITS;
}
// IQ2_S values in either layout (same codebooks, same arithmetic); the rest
// of the IQ formats are IQ3_S.
constexpr bool fmt_is_iq2s(int f) { return f == RTXLLM_FMT_IQ2S || f == RTXLLM_FMT_IQ2S_UNITS; }
constexpr bool fmt_is_units(int f) { return f == RTXLLM_FMT_IQ2S_UNITS || f == RTXLLM_FMT_IQ3S_UNITS; }
template <int FMT>
constexpr int load_policy() {
  return (fmt_is_iq(FMT) || FMT == RTXLLM_FMT_Q5K) ? 0 : 2;  // 2 = nt
}

__device__ __forceinline__ Rsrc make_rsrc(const void* p, std::uint32_t bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(p), 0, static_cast<int>(bytes), 0x00020000);
}
template <int P>
__device__ __forceinline__ std::uint32_t bld_u8(Rsrc r, std::uint32_t voff, std::uint32_t soff) {
  return __builtin_amdgcn_raw_buffer_load_b8(r, voff, soff, P);
}
template <int P>
__device__ __forceinline__ std::uint32_t bld_u16(Rsrc r, std::uint32_t voff, std::uint32_t soff) {
  return __builtin_amdgcn_raw_buffer_load_b16(r, voff, soff, P);
}
template <int P>
__device__ __forceinline__ std::uint32_t bld_u32(Rsrc r, std::uint32_t voff, std::uint32_t soff) {
  return __builtin_amdgcn_raw_buffer_load_b32(r, voff, soff, P);
}
template <int P>
__device__ __forceinline__ u32x2 bld_u64(Rsrc r, std::uint32_t voff, std::uint32_t soff) {
  return __builtin_amdgcn_raw_buffer_load_b64(r, voff, soff, P);
}
template <int P>
__device__ __forceinline__ u32x4 bld_u128(Rsrc r, std::uint32_t voff, std::uint32_t soff) {
  return __builtin_amdgcn_raw_buffer_load_b128(r, voff, soff, P);
}

constexpr bool fmt_is_raw_q4k(int f) { return f == RTXLLM_FMT_Q4K_RAW || f == RTXLLM_FMT_Q4K_RAW_PREDECODED; }

// ---- LDS codebooks for the IQ formats ---------------------------------------
// Codebooks as read by the bit-exact dequant path.
static __constant__ std::uint16_t kIq2sGridDev[1024] = {RTXLLM_IQ2S_GRID_VALUES};
static __constant__ std::uint32_t kIq3sGridDev[512] = {RTXLLM_IQ3S_GRID_VALUES};

// LDS codebooks of the IQ formats. grid2: IQ2_S entry -> its eight magnitude
// bytes 2 l + 1; grid3: IQ3_S entry -> four magnitude bytes; sign: sign byte ->
// (M0, M1), where byte j of M is 0xFF when value j is negative. Every magnitude
// is odd, so a signed int8 word is (magnitude ^ M) | 0x01010101 (one v_bitop3):
// a byte with M = 0 keeps its odd magnitude, and ~mag = -mag - 1 is even, so
// or-ing in its low bit gives -mag.
struct IqLds2 {
  uint2 grid2[1024];
  uint2 sign[256];
};
struct IqLds3 {
  std::uint32_t grid3[512];
  uint2 sign[256];
};
constexpr std::uint32_t kIqLowBits = 0x01010101u;
template <int FMT>
using IqLds = typename std::conditional<fmt_is_iq2s(FMT), IqLds2, IqLds3>::type;

// The same tables as device-global images, built at compile time, in the LDS
// layout: a workgroup copies the grid part with direct global -> LDS loads and
// computes the sign part (iq_sign_mask, checked against the image below).
template <std::size_t N>
struct IqImage {
  std::uint32_t w[N];
};
constexpr std::uint16_t kIq2sGridSrc[1024] = {RTXLLM_IQ2S_GRID_VALUES};
constexpr std::uint32_t kIq3sGridSrc[512] = {RTXLLM_IQ3S_GRID_VALUES};

template <std::size_t N>
constexpr void iq_image_signs(IqImage<N>& im, std::size_t at) {
  for (std::uint32_t i = 0; i < 256u; ++i) {
    std::uint32_t m0 = 0u, m1 = 0u;
    for (int j = 0; j < 4; ++j) {
      m0 |= ((i >> j) & 1u) ? (0xFFu << (8 * j)) : 0u;
      m1 |= ((i >> (j + 4)) & 1u) ? (0xFFu << (8 * j)) : 0u;
    }
    im.w[at + 2 * i] = m0;
    im.w[at + 2 * i + 1] = m1;
  }
}
constexpr IqImage<2560> iq2s_image() {
  IqImage<2560> im{};
  for (std::uint32_t i = 0; i < 1024u; ++i) {
    const std::uint32_t w = kIq2sGridSrc[i];
    std::uint32_t lo = 0u, hi = 0u;
    for (int j = 0; j < 4; ++j) {
      lo |= (2u * ((w >> (2 * j)) & 3u) + 1u) << (8 * j);
      hi |= (2u * ((w >> (2 * j + 8)) & 3u) + 1u) << (8 * j);
    }
    im.w[2 * i] = lo;
    im.w[2 * i + 1] = hi;
  }
  iq_image_signs(im, 2048);
  return im;
}
constexpr IqImage<1024> iq3s_image() {
  IqImage<1024> im{};
  for (std::uint32_t i = 0; i < 512u; ++i) im.w[i] = kIq3sGridSrc[i];
  iq_image_signs(im, 512);
  return im;
}
static_assert(sizeof(IqImage<2560>) == sizeof(IqLds2) && sizeof(IqImage<1024>) == sizeof(IqLds3), "image layout");

// Sign mask of a nibble n: bit j of n spread to bit 8 j by two shift-ors (no
// two copies of n meet in a kept bit), masked, times 0xFF.
constexpr std::uint32_t iq_sign_mask(std::uint32_t n) {
  const std::uint32_t t7 = n | (n << 7);
  const std::uint32_t b = (t7 | (t7 << 14)) & 0x01010101u;
  return (b << 8) - b;
}
constexpr bool iq_sign_masks_match() {
  const IqImage<1024> im = iq3s_image();
  for (std::uint32_t i = 0; i < 256u; ++i)
    if (im.w[512 + 2 * i] != iq_sign_mask(i & 15u) || im.w[512 + 2 * i + 1] != iq_sign_mask(i >> 4)) return false;
  return true;
}
static_assert(iq_sign_masks_match(), "computed sign table");
__device__ const IqImage<2560> kIq2sImage = iq2s_image();
__device__ const IqImage<1024> kIq3sImage = iq3s_image();

// The workgroup's codebook copy (only IQ instantiations reference it).
template <int FMT>
__device__ __forceinline__ IqLds<FMT>& iq_lds() {
  __shared__ IqLds<FMT> t;
  return t;
}

// Filling a workgroup's codebook table T (a grid part, then sign[256]), in two
// steps around the rest of the prologue's loads:
//  * lds_grid_issue loads the grid part of the image into registers, 16 B per
//    thread per step for NT threads (a thread whose step falls past the grid
//    re-reads the last piece), first among the wave's loads;
//  * lds_grid_commit, after the activation and first-tile loads are issued,
//    writes the pieces to LDS (smaller workgroups add the rest piece by
//    piece), computes the sign table (which keeps 2 KB per workgroup off the
//    L2) and meets the workgroup's other waves at the barrier.
// The compiler counts these plain loads exactly, so the writes wait for the
// grid loads only, and the barrier for the LDS writes: the activation and the
// first tile stay in flight through it, and the first round starts on the rows
// that have arrived. After a direct-to-LDS copy the barrier would wait for
// every outstanding load (the compiler cannot tell the copy's completion from
// the later loads'). The writes carry no branch (a load would move into it): a
// re-read last piece is stored again, the same bytes to the same place.
template <class T, std::uint32_t NT>
struct LdsGridStage {
  static constexpr std::uint32_t kUnits = (sizeof(T) - 256u * sizeof(uint2)) / 16u;  // 16-byte pieces
  static constexpr std::uint32_t kPer = (kUnits + NT - 1u) / NT;
  uint4 v[kPer];
};
template <class T, std::uint32_t NT>
__device__ __forceinline__ void lds_grid_issue(LdsGridStage<T, NT>& g, const void* image, std::uint32_t tid,
                                               std::uint32_t nt) {
  constexpr std::uint32_t U = LdsGridStage<T, NT>::kUnits;
  const uint4* src = static_cast<const uint4*>(image);
#pragma unroll
  for (std::uint32_t j = 0; j < LdsGridStage<T, NT>::kPer; ++j) {
    const std::uint32_t c = tid + j * nt;
    g.v[j] = src[c < U ? c : U - 1u];
  }
  __builtin_amdgcn_sched_barrier(0);  // issued here, ahead of the later loads
}
template <class T, std::uint32_t NT>
__device__ __forceinline__ void lds_grid_commit(T& t, const LdsGridStage<T, NT>& g, const void* image,
                                                std::uint32_t tid, std::uint32_t nt) {
  constexpr std::uint32_t U = LdsGridStage<T, NT>::kUnits;
  constexpr std::uint32_t P = LdsGridStage<T, NT>::kPer;
  uint4* dst = reinterpret_cast<uint4*>(&t);
#pragma unroll
  for (std::uint32_t j = 0; j < P; ++j) {
    const std::uint32_t c = tid + j * nt;
    dst[c < U ? c : U - 1u] = g.v[j];
  }
  const uint4* src = static_cast<const uint4*>(image);
  for (std::uint32_t c = tid + P * nt; c < U; c += nt) dst[c] = src[c];  // workgroups under NT threads
  for (std::uint32_t e = tid; e < 256u; e += nt) t.sign[e] = make_uint2(iq_sign_mask(e & 15u), iq_sign_mask(e >> 4));
  __syncthreads();
}
template <int FMT>
using IqGridStage = LdsGridStage<IqLds<FMT>, 128u>;
template <int FMT>
__device__ __forceinline__ const void* iq_image() {
  return fmt_is_iq2s(FMT) ? static_cast<const void*>(&kIq2sImage) : static_cast<const void*>(&kIq3sImage);
}

// ---- per-format unit load + compute ------------------------------------------

// Hardware fp16 -> fp32 (exact for every finite and infinite input; a NaN stays
// a NaN). The bit-exact dequant path keeps the reference's NaN rule instead.
__device__ __forceinline__ float h2f(std::uint32_t bits) {
  return static_cast<float>(__builtin_bit_cast(_Float16, static_cast<unsigned short>(bits & 0xFFFFu)));
}

// Byte offsets, relative to the start of a row, of the fields lane's unit
// (block b, unit k) reads; fixed for the whole launch. Rows are addressed by a
// wave-uniform base pointer, so every load is (uniform base + lane offset).
// The byte choice of kq_head_scales for a lane's 64-value group g (fixed for
// the launch): a v_perm selector for head words 1-2 and one for word 3, the
// shift and the mask of the word 1-2 bytes.
struct KqHeadSel {
  std::uint32_t sel12, sel3, sh, mask;
};

struct UnitOff {
  std::uint32_t o[5];
  std::uint32_t g;      // K-quants: 64-value group k >> 1
  KqHeadSel hs;         // K-quants with the native head
};

template <int FMT>
struct FmtBytes {
  // Bytes per block in the payload stream and the metadata stream.
  static constexpr std::uint32_t payload = FMT == RTXLLM_FMT_Q5K ? 176u
                                           : fmt_is_iq2s(FMT) ? 82u
                                           : FMT == RTXLLM_FMT_IQ3S ? 110u
                                           : FMT == RTXLLM_FMT_IQ3S_UNITS ? 114u
                                           : fmt_is_raw_q4k(FMT) ? 144u : 128u;
  static constexpr std::uint32_t meta = FMT == RTXLLM_FMT_Q4K_SPLIT_PREDECODED || FMT == RTXLLM_FMT_Q4K_RAW_PREDECODED ? 64u
                                        : FMT == RTXLLM_FMT_Q4K_SPLIT_HALF ? 32u
                                        : FMT == RTXLLM_FMT_Q4K_SPLIT_COMPACT ? 20u
                                        : FMT == RTXLLM_FMT_Q4K_SPLIT_NATIVE ? 16u : 0u;
};

// Byte i (GGUF order: d, qs[32], signs[32], qh[8], scales[8]) of block b of an
// IQ2S_UNITS tensor of nb blocks.
__host__ __device__ inline std::size_t iq2s_units_offset(std::size_t b, std::uint32_t i, std::size_t nb) {
  if (i < 2u) return 80u * nb + 2u * b + i;                             // d
  if (i < 34u) return 64u * b + 8u * ((i - 2u) >> 2) + ((i - 2u) & 3u);  // qs
  if (i < 66u) return 64u * b + 8u * ((i - 34u) >> 2) + 4u + ((i - 34u) & 3u);  // signs
  if (i < 74u) return 64u * nb + 16u * b + 2u * (i - 66u);              // qh
  return 64u * nb + 16u * b + 2u * (i - 74u) + 1u;                      // scales
}

// Byte i (GGUF order: d, qs[64], qh[8], signs[32], scales[4]) of block b of an
// IQ3S_UNITS tensor of nb blocks (a scale byte: its copy in the even unit).
__host__ __device__ inline std::size_t iq3s_units_offset(std::size_t b, std::uint32_t i, std::size_t nb) {
  if (i < 2u) return 112u * nb + 2u * b + i;                              // d
  if (i < 66u) return 96u * b + 12u * ((i - 2u) >> 3) + ((i - 2u) & 7u);  // qs
  if (i < 74u) return 96u * nb + 16u * b + 2u * (i - 66u);                // qh
  if (i < 106u) return 96u * b + 12u * ((i - 74u) >> 2) + 8u + ((i - 74u) & 3u);  // signs
  return 96u * nb + 16u * b + 4u * (i - 106u) + 1u;                       // scales (unit 2j)
}

// nb: blocks in the tensor (where the unit layouts' field streams start); the
// unit-layout offsets are relative to the row's first block.
template <int FMT>
__device__ __forceinline__ UnitOff unit_offsets(std::uint32_t b, std::uint32_t k, std::uint32_t nb) {
  UnitOff u{};
  const std::uint32_t pb = b * FmtBytes<FMT>::payload, mb = b * FmtBytes<FMT>::meta, g = k >> 1;
  u.g = g;
  // sub-blocks 2g, 2g + 1: bytes i, i + 1 (i = 2 (g & 1)) of head words 1-3
  const std::uint32_t i2 = 0x02020202u * (g & 1u);
  u.hs.sel12 = 0x05040100u + i2;                         // (w1 byte i, i + 1, w2 byte i, i + 1)
  u.hs.sel3 = g < 2u ? 0x0C0C0C0Cu : 0x01000100u + i2;  // zeros / (w3 byte i, i + 1, i, i + 1)
  u.hs.sh = g < 2u ? 0u : 2u;
  u.hs.mask = g < 2u ? 0x3F3F3F3Fu : 0x30303030u;
  // opaque to the compiler: from the two constants it would learn that bits
  // 6-7 of each scale byte are zero and turn the byte-to-float conversions
  // (v_cvt_f32_ubyte1-3, one instruction each) into bit-field extracts first
  asm("" : "+v"(u.hs.mask));
  if constexpr (FMT == RTXLLM_FMT_IQ2S_UNITS) {
    u.o[0] = 64u * b + 8u * k;             // qs, signs of the unit
    u.o[1] = 64u * nb + 16u * b + 2u * k;  // qh, scales of the unit
    u.o[2] = 80u * nb + 2u * b;            // d
  } else if constexpr (FMT == RTXLLM_FMT_IQ3S_UNITS) {
    u.o[0] = 96u * b + 12u * k;            // qs (8 B), signs (4 B) of the unit
    u.o[1] = 96u * nb + 16u * b + 2u * k;  // qh, scale byte of the unit
    u.o[2] = 112u * nb + 2u * b;           // d
  } else if constexpr (fmt_is_iq2s(FMT)) {
    u.o[0] = pb;                 // d
    u.o[1] = pb + 2u + 4u * k;   // qs (grid low bytes)
    u.o[2] = pb + 34u + 4u * k;  // sign bytes
    u.o[3] = pb + 66u + k;       // qh
    u.o[4] = pb + 74u + k;       // scale nibbles
  } else if constexpr (FMT == RTXLLM_FMT_IQ3S) {
    u.o[0] = pb;                   // d
    u.o[1] = pb + 2u + 8u * k;     // qs (8 grid low bytes)
    u.o[2] = pb + 74u + 4u * k;    // sign bytes
    u.o[3] = pb + 66u + k;         // qh
    u.o[4] = pb + 106u + (k >> 1); // scale nibbles
  } else if constexpr (FMT == RTXLLM_FMT_Q5K) {
    u.o[0] = pb + 48u + 16u * k;          // qs
    u.o[1] = pb;                          // head
    u.o[2] = pb + 16u + 16u * (k & 1u);   // qh
  } else {
    u.o[0] = pb + (fmt_is_raw_q4k(FMT) ? 16u : 0u) + 16u * k;  // payload quants
    if constexpr (FMT == RTXLLM_FMT_Q4K_RAW) u.o[1] = pb;
    else if constexpr (FMT == RTXLLM_FMT_Q4K_SPLIT_NATIVE) u.o[1] = mb;
    else if constexpr (FMT == RTXLLM_FMT_Q4K_SPLIT_PREDECODED || FMT == RTXLLM_FMT_Q4K_RAW_PREDECODED)
      u.o[1] = mb + 16u * g;
    else if constexpr (FMT == RTXLLM_FMT_Q4K_SPLIT_HALF) u.o[1] = mb + 8u * g;
    else {  // split-compact
      u.o[1] = mb;
      u.o[2] = mb + 4u + 2u * g;
      u.o[3] = mb + 12u + 2u * g;
    }
  }
  return u;
}

// Bytes of one (row, unit) kept in registers between the load and compute phases.
struct UnitRaw {
  std::uint32_t a[4];  // K-quants: payload quants; IQ2_S: qs, signs; IQ3_S: qs0, qs1, signs
  std::uint32_t b[4];  // K-quants: native head / metadata
  std::uint32_t c[4];  // Q5_K: qh bytes; IQ: d, qh, scale byte
};

// Value groups (16-value staging groups) covered by unit k of block b.
template <int FMT>
__device__ __forceinline__ void unit_groups(std::uint32_t b, std::uint32_t k, std::uint32_t& g0, std::uint32_t& g1) {
  if constexpr (fmt_is_iq(FMT)) {
    g0 = 16u * b + 2u * k;
    g1 = g0 + 1u;
  } else {
    const std::uint32_t g = k >> 1, h = k & 1u;
    g0 = 16u * b + 4u * g + h;  // low nibbles: values 64g + 16h + [0, 16)
    g1 = g0 + 2u;               // high nibbles: values 64g + 32 + 16h + [0, 16)
  }
}

// rp / rm: this row's start in the payload / metadata stream (wave-uniform);
// unit layouts: sp = blocks before this row.
template <int FMT>
__device__ __forceinline__ void unit_load(Rsrc rp, Rsrc rm, std::uint32_t sp, std::uint32_t sm, const UnitOff& u,
                                          UnitRaw& r) {
  constexpr int P = load_policy<FMT>();
  if constexpr (FMT == RTXLLM_FMT_Q5K) {
    const u32x4 q = bld_u128<P>(rp, u.o[0], sp);
    const u32x4 h = bld_u128<P>(rp, u.o[1], sp);
    const u32x4 qh = bld_u128<P>(rp, u.o[2], sp);
    r.a[0] = q.x, r.a[1] = q.y, r.a[2] = q.z, r.a[3] = q.w;
    r.b[0] = h.x, r.b[1] = h.y, r.b[2] = h.z, r.b[3] = h.w;
    r.c[0] = qh.x, r.c[1] = qh.y, r.c[2] = qh.z, r.c[3] = qh.w;
  } else if constexpr (FMT == RTXLLM_FMT_IQ2S_UNITS) {
    const u32x2 q = bld_u64<P>(rp, u.o[0], 64u * sp);
    r.a[0] = q.x, r.a[1] = q.y;
    r.c[1] = bld_u16<P>(rp, u.o[1], 16u * sp);  // qh | scale << 8, kept in one register
    r.c[0] = bld_u16<P>(rp, u.o[2], 2u * sp);
  } else if constexpr (FMT == RTXLLM_FMT_IQ3S_UNITS) {
    const u32x3 q = __builtin_amdgcn_raw_buffer_load_b96(rp, u.o[0], 96u * sp, P);
    r.a[0] = q.x, r.a[1] = q.y, r.a[2] = q.z;
    r.c[1] = bld_u16<P>(rp, u.o[1], 16u * sp);  // qh | scale << 8
    r.c[0] = bld_u16<P>(rp, u.o[2], 2u * sp);
  } else if constexpr (fmt_is_iq2s(FMT)) {
    r.c[0] = bld_u16<P>(rp, u.o[0], sp);
    r.a[0] = bld_u32<P>(rp, u.o[1], sp);
    r.a[1] = bld_u32<P>(rp, u.o[2], sp);
    r.c[1] = bld_u8<P>(rp, u.o[3], sp);
    r.c[2] = bld_u8<P>(rp, u.o[4], sp);
  } else if constexpr (FMT == RTXLLM_FMT_IQ3S) {
    r.c[0] = bld_u16<P>(rp, u.o[0], sp);
    const u32x2 q = bld_u64<P>(rp, u.o[1], sp);
    r.a[0] = q.x, r.a[1] = q.y;
    r.a[2] = bld_u32<P>(rp, u.o[2], sp);
    r.c[1] = bld_u8<P>(rp, u.o[3], sp);
    r.c[2] = bld_u8<P>(rp, u.o[4], sp);
  } else {
    const u32x4 q = bld_u128<P>(rp, u.o[0], sp);
    r.a[0] = q.x, r.a[1] = q.y, r.a[2] = q.z, r.a[3] = q.w;
    if constexpr (FMT == RTXLLM_FMT_Q4K_RAW) {
      const u32x4 h = bld_u128<P>(rp, u.o[1], sp);
      r.b[0] = h.x, r.b[1] = h.y, r.b[2] = h.z, r.b[3] = h.w;
    } else if constexpr (FMT == RTXLLM_FMT_Q4K_SPLIT_NATIVE || FMT == RTXLLM_FMT_Q4K_SPLIT_PREDECODED ||
                         FMT == RTXLLM_FMT_Q4K_RAW_PREDECODED) {
      const u32x4 h = bld_u128<P>(rm, u.o[1], sm);
      r.b[0] = h.x, r.b[1] = h.y, r.b[2] = h.z, r.b[3] = h.w;
    } else if constexpr (FMT == RTXLLM_FMT_Q4K_SPLIT_HALF) {
      const u32x2 h = bld_u64<P>(rm, u.o[1], sm);
      r.b[0] = h.x, r.b[1] = h.y;
    } else {  // split-compact: f16 d, f16 dmin, u8 sc[8], u8 m[8]
      r.b[0] = bld_u32<P>(rm, u.o[1], sm);
      r.b[1] = bld_u16<P>(rm, u.o[2], sm);
      r.b[2] = bld_u16<P>(rm, u.o[3], sm);
    }
  }
}

// The 6-bit scales and mins of sub-blocks j = 2g, 2g + 1 from the native
// 16-byte head (d, dmin, 12 packed scale/min bytes q), as get_scale_min_k4
// unpacks them, in one word: bytes (sc_2g, sc_2g+1, m_2g, m_2g+1). With i = 2
// (g & 1) and head words w1 = q[0..3], w2 = q[4..7], w3 = q[8..11]:
//  * g < 2: sc_j = q[j] & 63, m_j = q[j + 4] & 63 (bytes i, i + 1 of w1, w2);
//  * g >= 2: sc_j = (q[j + 4] & 15) | (q[j - 4] >> 6) << 4, m_j = q[j + 4] >> 4
//    | (q[j] >> 6) << 4: the low / high nibbles of w3 bytes i, i + 1 under the
//    top two bits of w1 / w2 bytes i, i + 1.
// One perm gathers the w1 / w2 bytes and one the w3 bytes (zeros for g < 2)
// by the lane's fixed selectors, so no lane unpacks bytes it does not use.
__device__ __forceinline__ std::uint32_t kq_head_scales(const std::uint32_t h[4], const KqHeadSel& s) {
  const std::uint32_t w12 = (__builtin_amdgcn_perm(h[2], h[1], s.sel12) >> s.sh) & s.mask;
  const std::uint32_t w3 = __builtin_amdgcn_perm(h[3], h[3], s.sel3);
  return w12 | (w3 & 0x00000F0Fu) | ((w3 >> 4) & 0x0F0F0000u);
}

// The IQ scale byte: beside qh in one 16-bit field in the unit layouts, its
// own byte in the GGUF layouts. (qh bits above bit 7 never reach an index.)
template <int FMT>
__device__ __forceinline__ std::uint32_t iq_scale_byte(const UnitRaw& r) {
  if constexpr (fmt_is_units(FMT)) return r.c[1] >> 8;
  else return r.c[2];
}

// IQ units in two phases, so the LDS lookups of one row can be in flight while
// the previous row's dot products run: unit_lookup issues the codebook and
// sign-table reads and applies the signs; unit_dot_iq multiplies the signed
// int8 words with the activation digits.
struct IqWords {
  std::uint32_t w[8];  // signed int8 weights, 4 per word, in value order
};

template <int FMT>
__device__ __forceinline__ void unit_lookup(const UnitRaw& r, const IqLds<FMT>* t, IqWords& q) {
  if constexpr (fmt_is_iq2s(FMT)) {
    // the high index bits of group g, (qh >> 2 g) & 3, one per byte of hb:
    // qh | qh << 6 | qh << 12 | qh << 18 puts them at bits 8 g (ors, no carries)
    const std::uint32_t qh = r.c[1] & 0xFFu;
    const std::uint32_t s6 = (qh << 6) | qh;
    const std::uint32_t hb = ((s6 << 12) | s6) & 0x03030303u;
#pragma unroll
    for (int grp = 0; grp < 4; ++grp) {
      // index = qs byte | high bits << 8: bytes grp of (qs, hb) into bytes 0, 1
      const std::uint32_t idx = __builtin_amdgcn_perm(hb, r.a[0], 0x0C0C0400u + 0x101u * static_cast<std::uint32_t>(grp));
      const uint2 gm = t->grid2[idx];
      const uint2 sm = t->sign[(r.a[1] >> (8 * grp)) & 0xFFu];
      q.w[2 * grp] = (gm.x ^ sm.x) | kIqLowBits;
      q.w[2 * grp + 1] = (gm.y ^ sm.y) | kIqLowBits;
    }
  } else {
    // the high index bit of value group j, (qh >> j) & 1, one per byte of
    // (hb0: j < 4, hb1: j >= 4): qh | qh << 7 | qh << 14 | qh << 21 (ors)
    const std::uint32_t qh = r.c[1] & 0xFFu;
    const std::uint32_t s7 = (qh << 7) | qh;
    const std::uint32_t s14 = (s7 << 14) | s7;
    const std::uint32_t hb0 = s14 & 0x01010101u, hb1 = (s14 >> 4) & 0x01010101u;
#pragma unroll
    for (int grp = 0; grp < 4; ++grp) {
      const uint2 sm = t->sign[(r.a[2] >> (8 * grp)) & 0xFFu];
#pragma unroll
      for (int pair = 0; pair < 2; ++pair) {
        const int sel = 2 * grp + pair;
        const std::uint32_t idx = __builtin_amdgcn_perm(sel < 4 ? hb0 : hb1, r.a[sel >> 2],
                                                        0x0C0C0400u + 0x101u * static_cast<std::uint32_t>(sel & 3));
        q.w[sel] = (t->grid3[idx] ^ (pair ? sm.y : sm.x)) | kIqLowBits;
      }
    }
  }
}

// Per-lane scale factors of an IQ unit's two 16-value halves, fixed for the
// launch: IQ2_S sub-scale (0.5 + n) / 4 folded with the activation scale as
// n * a + b (a = s / 4, b = s / 8); IQ3_S takes the scale nibble's shift.
struct IqLaneScale {
  float a0, b0, a1, b1;
  std::uint32_t nib_shift;
};

template <int FMT>
__device__ __forceinline__ IqLaneScale iq_lane_scale(std::uint32_t k, const XG& x0, const XG& x1) {
  IqLaneScale ls;
  ls.a0 = 0.25f * x0.s, ls.b0 = 0.125f * x0.s;
  ls.a1 = 0.25f * x1.s, ls.b1 = 0.125f * x1.s;
  ls.nib_shift = (k & 1u) ? 4u : 0u;
  return ls;
}

template <int FMT>
__device__ __forceinline__ float unit_dot_iq(const UnitRaw& r, const XG& x0, const XG& x1, const IqLaneScale& ls,
                                             const IqWords& q) {
  const float d = h2f(r.c[0]);
  const float D0 = static_cast<float>(dot16(q.w, x0));
  const float D1 = static_cast<float>(dot16(q.w + 4, x1));
  if constexpr (fmt_is_iq2s(FMT)) {
    // d * (0.5 + n) / 4 * s = d * (n * s / 4 + s / 8)
    const std::uint32_t sc = iq_scale_byte<FMT>(r);
    const float f0 = __builtin_fmaf(static_cast<float>(sc & 15u), ls.a0, ls.b0);
    const float f1 = __builtin_fmaf(static_cast<float>(sc >> 4), ls.a1, ls.b1);
    return d * __builtin_fmaf(f1, D1, f0 * D0);
  } else {
    // d * (1 + 2 n) for the whole unit
    const float m = __builtin_fmaf(static_cast<float>((iq_scale_byte<FMT>(r) >> ls.nib_shift) & 15u), 2.0f, 1.0f);
    return (d * m) * __builtin_fmaf(x1.s, D1, x0.s * D0);
  }
}

// K-quant unit: weight codes, scales and the dot with the staged activation.
template <int FMT>
__device__ __forceinline__ float unit_compute(const UnitRaw& r, const UnitOff& u, std::uint32_t k, const XG& x0,
                                              const XG& x1) {
  {
    const std::uint32_t g = u.g;
    std::uint32_t lo[4], hi[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      lo[i] = r.a[i] & 0x0F0F0F0Fu;
      hi[i] = (r.a[i] >> 4) & 0x0F0F0F0Fu;
      if constexpr (FMT == RTXLLM_FMT_Q5K) {
        // bit 2 g (low nibbles) / 2 g + 1 (high nibbles) of each qh byte,
        // rotated to bit 4 of the same byte: one funnel shift and one and-or
        lo[i] |= __builtin_rotateright32(r.c[i], (2u * g + 28u) & 31u) & 0x10101010u;
        hi[i] |= __builtin_rotateright32(r.c[i], (2u * g + 29u) & 31u) & 0x10101010u;
      }
    }
    const float c0 = static_cast<float>(dot16(lo, x0));
    const float c1 = static_cast<float>(dot16(hi, x1));
    if constexpr (FMT == RTXLLM_FMT_Q4K_RAW || FMT == RTXLLM_FMT_Q4K_SPLIT_NATIVE || FMT == RTXLLM_FMT_Q5K) {
      // d (sc0 s0 c0 + sc1 s1 c1) - dmin (m0 sum0 + m1 sum1): the group scales
      // s are powers of two, so sc s is exact
      const std::uint32_t sm = kq_head_scales(r.b, u.hs);
      const float d = h2f(r.b[0]), dmin = h2f(r.b[0] >> 16);
      const float p = __builtin_fmaf(static_cast<float>((sm >> 8) & 0xFFu) * x1.s, c1,
                                     (static_cast<float>(sm & 0xFFu) * x0.s) * c0);
      const float q = __builtin_fmaf(static_cast<float>(sm >> 24), x1.sum,
                                     static_cast<float>((sm >> 16) & 0xFFu) * x0.sum);
      return __builtin_fmaf(-dmin, q, d * p);
    }
    float s0, m0, s1, m1;
    if constexpr (FMT == RTXLLM_FMT_Q4K_SPLIT_PREDECODED || FMT == RTXLLM_FMT_Q4K_RAW_PREDECODED) {
      s0 = __uint_as_float(r.b[0]), m0 = __uint_as_float(r.b[1]);
      s1 = __uint_as_float(r.b[2]), m1 = __uint_as_float(r.b[3]);
    } else if constexpr (FMT == RTXLLM_FMT_Q4K_SPLIT_HALF) {
      s0 = h2f(r.b[0]), m0 = h2f(r.b[0] >> 16);
      s1 = h2f(r.b[1]), m1 = h2f(r.b[1] >> 16);
    } else {  // split-compact
      const float d = h2f(r.b[0]), dmin = h2f(r.b[0] >> 16);
      s0 = d * static_cast<float>(r.b[1] & 0xFFu), s1 = d * static_cast<float>(r.b[1] >> 8);
      m0 = dmin * static_cast<float>(r.b[2] & 0xFFu), m1 = dmin * static_cast<float>(r.b[2] >> 8);
    }
    return ((s0 * x0.s) * c0 - m0 * x0.sum) + ((s1 * x1.s) * c1 - m1 * x1.sum);
  }
}

// ---- tile reduction -----------------------------------------------------------

template <int CTRL>
__device__ __forceinline__ float dpp(float v) {
  return __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), CTRL, 0xF, 0xF, false));
}
constexpr int kDppQuadXor1 = 0xB1;        // quad_perm [1,0,3,2]
constexpr int kDppQuadXor2 = 0x4E;        // quad_perm [2,3,0,1]
constexpr int kDppRowHalfMirror = 0x141;  // lane i -> 7 - i within 8
constexpr int kDppRowRor8 = 0x128;
constexpr int kDppRowRor4 = 0x124;
constexpr int kDppRowRor2 = 0x122;
constexpr int kDppRowRor1 = 0x121;

// acc[j] holds lane partials of row j (T in {4, 8, 16}); afterwards every lane
// of [r * 64/T, (r+1) * 64/T) holds the full sum of row r. Each halving step
// keeps one half of the live rows per lane group and adds the partner's
// partial of that half: lane bit 5 via permlane32_swap, bit 4 via
// permlane16_swap, bit 3 via DPP row_ror:8 and bit 2 via row_half_mirror;
// the lanes left sharing a row are then summed with DPP (8 VALU ops at T = 4).
template <int T>
__device__ __forceinline__ float tile_reduce(float (&acc)[T], std::uint32_t lane) {
  static_assert(T == 4 || T == 8 || T == 16, "tile of 4, 8 or 16 rows");
#pragma unroll
  for (int j = 0; j < T / 2; ++j) {
    float a = acc[j], b = acc[j + T / 2];
    permlane32_swap(a, b);
    acc[j] = a + b;
  }
#pragma unroll
  for (int j = 0; j < T / 4; ++j) {
    float a = acc[j], b = acc[j + T / 4];
    permlane16_swap(a, b);
    acc[j] = a + b;
  }
  if constexpr (T == 4) {
    float v = acc[0];
    v += dpp<kDppRowRor8>(v);
    v += dpp<kDppRowRor4>(v);
    v += dpp<kDppRowRor2>(v);
    v += dpp<kDppRowRor1>(v);
    return v;
  } else {
    const bool b3 = (lane & 8u) != 0u;
#pragma unroll
    for (int j = 0; j < T / 8; ++j) {
      const float keep = b3 ? acc[j + T / 8] : acc[j];
      const float send = b3 ? acc[j] : acc[j + T / 8];
      acc[j] = keep + dpp<kDppRowRor8>(send);
    }
    float v = acc[0];
    if constexpr (T == 16) {
      const bool b2 = (lane & 4u) != 0u;
      const float keep = b2 ? acc[1] : acc[0];
      const float send = b2 ? acc[0] : acc[1];
      v = keep + dpp<kDppRowHalfMirror>(send);
    } else {
      v += dpp<kDppRowHalfMirror>(v);
    }
    v += dpp<kDppQuadXor2>(v);
    v += dpp<kDppQuadXor1>(v);
    return v;
  }
}

// ---- the kernel -------------------------------------------------------------

constexpr int kMaxKs = 8;  // waves per workgroup unless the epilogue declares kWaves

// Rows per epilogue group: epilogues that declare kGroupRows (a multiple of
// their tile) receive the results of kGroupRows consecutive rows at once.
template <class E, class = void>
struct EpiGroupRows {
  static constexpr std::uint32_t value = 0;
};
template <class E>
struct EpiGroupRows<E, std::void_t<decltype(E::kGroupRows)>> {
  static constexpr std::uint32_t value = E::kGroupRows;
};

// Epilogues with a ready(lane) member get that call once the prologue's loads
// have been waited for (init(lane) issues their own loads first, ready uses
// them), so an epilogue's set-up costs no round trip of its own.
template <class E, class = void>
struct EpiHasReady {
  static constexpr bool value = false;
};
template <class E>
struct EpiHasReady<E, std::void_t<decltype(std::declval<E&>().ready(0u))>> {
  static constexpr bool value = true;
};

// Epilogues that declare kFinish get epi.finish(slot, lane) from each row
// group's epilogue wave after its last tile; slot = blockIdx.x * nrg + rg is
// unique per row group (< gridDim.x * nrg).
template <class E, class = void>
struct EpiHasFinish {
  static constexpr bool value = false;
};
template <class E>
struct EpiHasFinish<E, std::void_t<decltype(E::kFinish)>> {
  static constexpr bool value = E::kFinish;
};

// Plain epilogues that declare kWaves (> kMaxKs) run in workgroups of up to
// kWaves waves whose row groups do not wait for each other: the column-split
// waves of one row group hand over their partials through LDS counters
// (pair_publish / pair_wait) instead of a workgroup barrier, so one workgroup
// can hold many row groups without running them in lockstep.
template <class E, class = void>
struct EpiWaves {
  static constexpr std::uint32_t value = kMaxKs;
};
template <class E>
struct EpiWaves<E, std::void_t<decltype(E::kWaves)>> {
  static constexpr std::uint32_t value = E::kWaves;
};

// Epilogues that declare kShareX read a staged x of at most kShareXCols
// columns (the launcher's guarantee) from one LDS copy per workgroup, made in
// the prologue, instead of every wave loading its own slice: the CU's load
// path then carries the activation once per workgroup.
constexpr std::uint32_t kShareXCols = 4096;
template <class E, class = void>
struct EpiShareX {
  static constexpr bool value = false;
};
template <class E>
struct EpiShareX<E, std::void_t<decltype(E::kShareX)>> {
  static constexpr bool value = E::kShareX;
};

// A wave waits until the LDS counter reaches `target`, sleeping between reads,
// for at most `limit` reads, and returns whether the counter got there. The
// counters only grow and each is advanced by a wave of the same workgroup that
// runs the same rounds, so the wait ends; the limit (kPairSpinLimit, ~10^6
// sleeps) only bounds a wave's time if that ever failed, and the kernel then
// reports it (PairWait::status) instead of passing a stale partial on
// silently. Counter updates go to LDS in the wave's program order, after the
// data they announce (the empty asm statements keep the compiler from moving
// LDS accesses across them).
constexpr std::uint32_t kPairSpinLimit = 1u << 20;
__device__ __forceinline__ bool pair_wait(const std::uint32_t* counter, std::uint32_t target, std::uint32_t limit) {
  asm volatile("" ::: "memory");
  bool reached = false;
  for (std::uint32_t i = 0; i < limit; ++i) {
    const std::uint32_t c = __builtin_amdgcn_readfirstlane(
        __hip_atomic_load(counter, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP));
    if (c >= target) {
      reached = true;
      break;
    }
    __builtin_amdgcn_s_sleep(1);
  }
  asm volatile("" ::: "memory");
  return reached;
}

// Status bit set when a bounded wait of a kernel ran out: that launch's
// results are not valid.
constexpr std::uint32_t kStatusWaitTimeout = 2u;

// What an epilogue with the pairwise hand-over (kWaves) carries as `wait`:
// the status word that gets kStatusWaitTimeout if any wave's wait ran out
// (null: not reported), the wait limit (kPairSpinLimit) and a bias added to
// every wait target (0; a host-side test sets it to make every wait run out
// after `limit` reads, so that the report can be checked while each wave
// still finishes its rounds).
struct PairWait {
  std::uint32_t* status = nullptr;
  std::uint32_t limit = kPairSpinLimit;
  std::uint32_t bias = 0u;
};
__device__ __forceinline__ void pair_publish(std::uint32_t* counter, std::uint32_t value) {
  asm volatile("" ::: "memory");
  __hip_atomic_store(counter, value, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
  asm volatile("" ::: "memory");
}

// UPL units (32 columns each) per lane; a row's `cols / 32` units are split over
// ks waves of one workgroup, which also holds nrg row groups (blockDim.x = 64 *
// ks * nrg, ks * nrg <= 8, or <= kWaves for epilogues that declare it). Each
// row group loads the next tile's rows before it computes the current one.
// Tile schedule:
//  * plain epilogues: row group rg of workgroup b handles tiles b + G * (rg +
//    nrg * j), j = 0, 1, ... (G = gridDim.x), so tiles spread evenly over the
//    CUs; the epilogue wave of the row group gets each tile's results;
//  * grouped epilogues (kGroupRows = GR): workgroup b owns the GR-row groups
//    b + G j; the GR / TILE tiles of a group are spread over the nrg row groups
//    and R = GR / (TILE nrg) consecutive rounds (the host picks nrg dividing
//    GR / TILE). Results collect in LDS, and after the group's last round wave 0
//    hands all GR of them to epi.group(), inside the workgroup: no other
//    workgroup's results are needed, so no device-wide synchronisation.
template <int FMT, int UPL, int TILE, bool SELF, class Epi>
__global__ __launch_bounds__(64 * EpiWaves<Epi>::value) void mv_kernel(QTensor w, XSrc xs, std::uint32_t rows,
                                                                      std::uint32_t ks, Epi epi_arg) {
  static_assert(Epi::kTile == TILE, "epilogue tile");
  constexpr int kTlR = TlRegionOf<Epi>::value(FMT);
  const std::uint32_t tl_slot = (blockIdx.x * EpiWaves<Epi>::value + (threadIdx.x >> 6)) * 2u;
  tl_stamp(kTlR, tl_slot);
  constexpr std::uint32_t GR = EpiGroupRows<Epi>::value;
  static_assert(GR % TILE == 0u, "epilogue group of whole tiles");
  constexpr std::uint32_t TG = GR > 0u ? GR / TILE : 1u;  // tiles per group
  constexpr std::uint32_t WMAX = EpiWaves<Epi>::value;
  constexpr bool kPair = WMAX > static_cast<std::uint32_t>(kMaxKs);
  static_assert(!kPair || GR == 0u, "pairwise hand-over for plain epilogues");
  constexpr bool kShareX = EpiShareX<Epi>::value && !SELF;
  Epi epi = epi_arg;
  // Column-split partials, one slot per wave, double buffered by round parity
  // so a fast wave cannot overwrite a slot another wave still reads.
  __shared__ float part[2][WMAX][TILE];
  // Pairwise hand-over: ready[w] = rounds wave w has published, taken[w] =
  // rounds the row group's epilogue wave w has consumed.
  __shared__ std::uint32_t ready[kPair ? WMAX : 1u], taken[kPair ? WMAX : 1u];
  // The workgroup's copy of the staged x (kShareX), in its global layout.
  constexpr std::uint32_t kXPieces = kShareX ? static_cast<std::uint32_t>(xq_bytes(kShareXCols) / 16u) : 1u;
  __shared__ uint4 xshare[kXPieces];
  // Grouped epilogues: a group's results, double buffered by group parity.
  __shared__ float gbuf[2][GR > 0u ? GR : 1u];
  const std::uint32_t lane = threadIdx.x & 63u;
  // Wave-uniform values live in SGPRs: row bases become scalar and every load
  // is (scalar row base + per-lane offset).
  const std::uint32_t wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const std::uint32_t kw = wave % ks, rg = wave / ks, nrg = (blockDim.x >> 6) / ks;
  const std::uint32_t units = w.cols >> 5, bpr = w.cols >> 8;

  std::uint32_t uk[UPL], ub[UPL];
  bool uvalid[UPL];
  UnitOff off[UPL];
#pragma unroll
  for (int i = 0; i < UPL; ++i) {
    std::uint32_t u = (kw * UPL + i) * 64u + lane;
    uvalid[i] = u < units;
    u = uvalid[i] ? u : units - 1u;
    ub[i] = u >> 3;
    uk[i] = u & 7u;
    off[i] = unit_offsets<FMT>(ub[i], uk[i], rows * bpr);
  }

  // Row strides and stream sizes in bytes (the host keeps every stream under
  // 4 GiB).
  const std::uint32_t prow = bpr * FmtBytes<FMT>::payload, mrow = bpr * FmtBytes<FMT>::meta;
  const Rsrc rsp = make_rsrc(w.payload, rows * prow);
  const Rsrc rsm = make_rsrc(FmtBytes<FMT>::meta > 0u ? w.meta : w.payload, rows * mrow);
  const std::uint32_t tiles = (rows + TILE - 1) / TILE;
  const std::uint32_t per_round = gridDim.x * nrg;
  // grouped: rounds per group R = TG / nrg (a power of two), R = 1 << rshift
  const std::uint32_t rshift = GR > 0u ? static_cast<std::uint32_t>(__builtin_ctz(TG / nrg)) : 0u;
  const std::uint32_t groups = (tiles + TG - 1u) / TG;
  const std::uint32_t rounds = GR > 0u ? ((groups + gridDim.x - 1u) / gridDim.x) << rshift
                                       : (tiles + per_round - 1) / per_round;
  // tile of round s (>= tiles once s >= rounds)
  auto tile_of = [&](std::uint32_t s) -> std::uint32_t {
    if constexpr (GR > 0u) {
      const std::uint32_t group = blockIdx.x + (s >> rshift) * gridDim.x;
      return group * TG + ((s & ((1u << rshift) - 1u)) * nrg + rg);
    } else {
      return s * per_round + rg * gridDim.x + blockIdx.x;
    }
  };

  // Loads a tile's rows (clamped to the last row). Called only where the tile
  // is needed and never inside a branch: the compiler's wait counts then see
  // one straight sequence per round, so computing tile s waits only for tile
  // s's loads while tile s + 1's stay in flight (after a conditional load block
  // it waits for both).
  auto load_tile = [&](std::uint32_t t, UnitRaw (&raw)[TILE][UPL]) {
    // t is wave-uniform; saying so keeps the row bases in SGPRs in every round
    t = __builtin_amdgcn_readfirstlane(t);
#pragma unroll
    for (int rr = 0; rr < TILE; ++rr) {
      std::uint32_t row = t * TILE + rr;
      row = row < rows ? row : rows - 1u;
#pragma unroll
      for (int i = 0; i < UPL; ++i)
        unit_load<FMT>(rsp, rsm, fmt_is_units(FMT) ? row * bpr : row * prow, row * mrow, off[i], raw[rr][i]);
    }
  };

  // Prologue, ordered so that loads complete in issue order: the epilogue's
  // set-up loads, the codebook grid (into registers), the staged activation,
  // then the first tile's weights; the codebook commit waits for the grid
  // loads only and leaves the activation and the weights in flight.
  epi.init(lane);
  IqLds<FMT>* tables = nullptr;
  LdsGridStage<IqLds<FMT>, kPair ? 64u * WMAX : 128u> grid_stage;
  if constexpr (fmt_is_iq(FMT)) {
    tables = &iq_lds<FMT>();
    lds_grid_issue(grid_stage, iq_image<FMT>(), threadIdx.x, blockDim.x);
  }
  // shared x: 16-byte pieces of the staged buffer, loaded here, written to LDS
  // with the codebook (a thread past the buffer re-reads its last piece)
  constexpr std::uint32_t kXPer = (kXPieces + 64u * WMAX - 1u) / (64u * WMAX);
  const std::uint32_t xpieces = kShareX ? static_cast<std::uint32_t>(xq_bytes(w.cols) / 16u) : 1u;
  uint4 xreg[kXPer];
  if constexpr (kShareX) {
    const uint4* src = reinterpret_cast<const uint4*>(xs.xq.h);
#pragma unroll
    for (std::uint32_t j = 0; j < kXPer; ++j) {
      const std::uint32_t c = threadIdx.x + j * blockDim.x;
      xreg[j] = src[c < xpieces ? c : xpieces - 1u];
    }
    __builtin_amdgcn_sched_barrier(0);
  }
  // Self-staging reads its fp32 groups here and converts them after the first
  // tile's loads are issued: converting at once would make the first tile's
  // request wait for these loads.
  XG x0[UPL], x1[UPL];
  f32x16 xf0[UPL], xf1[UPL];
#pragma unroll
  for (int i = 0; i < UPL; ++i) {
    std::uint32_t g0, g1;
    unit_groups<FMT>(ub[i], uk[i], g0, g1);
    if constexpr (SELF) {
      if (xs.x_aligned != 0u) {
        xf0[i] = xg_read<true>(xs.x, g0);
        xf1[i] = xg_read<true>(xs.x, g1);
      } else {
        xf0[i] = xg_read<false>(xs.x, g0);
        xf1[i] = xg_read<false>(xs.x, g1);
      }
    } else if constexpr (!kShareX) {
      xg_load(xs.xq, g0, x0[i]);
      xg_load(xs.xq, g1, x1[i]);
    }
  }
  // Two tile buffers: tile s + 1 is requested before tile s is computed, so
  // each row group keeps one tile of weights in flight.
  UnitRaw buf[2][TILE][UPL];
  load_tile(tile_of(0u), buf[0]);
  if constexpr (SELF) {
    __builtin_amdgcn_sched_barrier(0);  // every load of the first tile issued before the conversion
#pragma unroll
    for (int i = 0; i < UPL; ++i) {
      xg_quant(xf0[i], x0[i]);
      xg_quant(xf1[i], x1[i]);
    }
    tl_stamp(kTlR >= 0 ? kTlSelfStaged : -1, tl_slot / 2u);
  }
  if constexpr (kPair) {
    ready[wave] = 0u;
    taken[wave] = 0u;
  }
  if constexpr (kShareX) {
#pragma unroll
    for (std::uint32_t j = 0; j < kXPer; ++j) {
      const std::uint32_t c = threadIdx.x + j * blockDim.x;
      xshare[c < xpieces ? c : xpieces - 1u] = xreg[j];  // no branch, as for the codebook
    }
    for (std::uint32_t c = threadIdx.x + kXPer * blockDim.x; c < xpieces; c += blockDim.x)
      xshare[c] = reinterpret_cast<const uint4*>(xs.xq.h)[c];
  }
  if constexpr (fmt_is_iq(FMT)) lds_grid_commit(*tables, grid_stage, iq_image<FMT>(), threadIdx.x, blockDim.x);
  else if constexpr (kPair || kShareX) __syncthreads();
  if constexpr (kShareX) {
    // the staged layout (h, m, l: cols bytes each; s, sum: cols / 16 floats)
    const std::uint8_t* xb = reinterpret_cast<const std::uint8_t*>(xshare);
    const std::uint32_t c = w.cols;
    const XQ xl{reinterpret_cast<const std::int8_t*>(xb), reinterpret_cast<const std::int8_t*>(xb + c),
                reinterpret_cast<const std::int8_t*>(xb + 2u * c), reinterpret_cast<const float*>(xb + 3u * c),
                reinterpret_cast<const float*>(xb + 3u * c) + c / kXGroup};
#pragma unroll
    for (int i = 0; i < UPL; ++i) {
      std::uint32_t g0, g1;
      unit_groups<FMT>(ub[i], uk[i], g0, g1);
      xg_load(xl, g0, x0[i]);
      xg_load(xl, g1, x1[i]);
    }
  }
  if constexpr (EpiHasReady<Epi>::value) epi.ready(lane);
  IqLaneScale ls[UPL];
  if constexpr (fmt_is_iq(FMT)) {
#pragma unroll
    for (int i = 0; i < UPL; ++i) ls[i] = iq_lane_scale<FMT>(uk[i], x0[i], x1[i]);
  }

  bool late = false;  // a pairwise wait of this wave ran out (wave-uniform)
  auto finish_tile = [&](std::uint32_t sj, std::uint32_t t, std::uint32_t parity, std::uint32_t gpar,
                         const UnitRaw (&raw)[TILE][UPL]) {
    // Every wave of the workgroup runs the same rounds, so the barrier below is
    // uniform; waves without a tile this round still take part in it (and in
    // the pairwise hand-over: every round is published and consumed).
    const bool active = t < tiles;
    float acc[TILE];
#pragma unroll
    for (int rr = 0; rr < TILE; ++rr) acc[rr] = 0.0f;
    if (active) {
      // a lane past the row's last unit computes a clamped copy and adds 0
      if constexpr (fmt_is_iq(FMT)) {
        // row rr + 1's codebook lookups are issued before row rr's dot products
        IqWords q[2][UPL];
#pragma unroll
        for (int i = 0; i < UPL; ++i) unit_lookup<FMT>(raw[0][i], tables, q[0][i]);
#pragma unroll
        for (int rr = 0; rr < TILE; ++rr) {
          if (rr + 1 < TILE) {
#pragma unroll
            for (int i = 0; i < UPL; ++i) unit_lookup<FMT>(raw[rr + 1][i], tables, q[(rr + 1) & 1][i]);
          }
#pragma unroll
          for (int i = 0; i < UPL; ++i) {
            const float v = unit_dot_iq<FMT>(raw[rr][i], x0[i], x1[i], ls[i], q[rr & 1][i]);
            acc[rr] += uvalid[i] ? v : 0.0f;
          }
        }
      } else {
#pragma unroll
        for (int rr = 0; rr < TILE; ++rr) {
#pragma unroll
          for (int i = 0; i < UPL; ++i) {
            const float v = unit_compute<FMT>(raw[rr][i], off[i], uk[i], x0[i], x1[i]);
            acc[rr] += uvalid[i] ? v : 0.0f;
          }
        }
      }
    }
    float v = tile_reduce<TILE>(acc, lane);
    constexpr std::uint32_t spread = 64u / TILE;
    const std::uint32_t r = lane / spread;
    if (ks > 1u) {
      if constexpr (kPair) {
        // round sj: the non-epilogue waves write slot parity once the
        // epilogue wave has consumed round sj - 2 (the slot's last use), then
        // announce it; the epilogue wave adds the row group's slots in wave
        // order once all are announced (the same sum as below)
        const std::uint32_t w0 = wave - kw;
        if (kw != 0u) {
          if (sj >= 2u) late |= !pair_wait(&taken[w0], sj - 1u + epi.wait.bias, epi.wait.limit);
          if ((lane % spread) == 0u) part[parity][wave][r] = v;
          pair_publish(&ready[wave], sj + 1u);
          return;
        }
        for (std::uint32_t k = 1; k < ks; ++k)
          late |= !pair_wait(&ready[wave + k], sj + 1u + epi.wait.bias, epi.wait.limit);
        for (std::uint32_t k = 1; k < ks; ++k) v += part[parity][wave + k][r];
        pair_publish(&taken[wave], sj + 1u);
      } else {
        if ((lane % spread) == 0u) part[parity][wave][r] = v;
        __syncthreads();
        if (kw != 0u) return;
        v = part[parity][wave][r];
        for (std::uint32_t k = 1; k < ks; ++k) v += part[parity][wave + k][r];
      }
    }
    if constexpr (GR > 0u) {
      if (active && (lane % spread) == 0u) gbuf[gpar][(t % TG) * TILE + r] = v;
    } else {
      if (active) epi(t * TILE, v, lane, rows);
    }
  };
  // After round s: a grouped epilogue's group is complete when s is its last
  // round. The condition is uniform over the workgroup, so is the barrier.
  auto group_end = [&](std::uint32_t s) {
    if constexpr (GR > 0u) {
      if ((s & ((1u << rshift) - 1u)) != (1u << rshift) - 1u) return;
      const std::uint32_t group = blockIdx.x + (s >> rshift) * gridDim.x;
      if (group >= groups) return;
      __syncthreads();
      if (wave == 0u) epi.group(group * GR, gbuf[(s >> rshift) & 1u], lane, rows);
    }
  };

  // Round s computes buf[s % 2] after requesting round s + 1 into the other
  // buffer; the loop runs round pairs while a later round exists, and the last
  // one or two rounds follow without a request past the end. rounds is uniform
  // over the workgroup (and >= 1), so are the branches.
  // Wave priority by progress (plain epilogues): a SIMD issues for its oldest
  // wave first, so with a static tile split the workgroups dispatched first
  // finish early and the last ones run on at low occupancy. Each round sets the
  // priority from the fraction of the row group's tiles already done (3 for
  // the first quarter, ..., 0 for the last), so waves that fell behind are
  // issued first and the row groups of a CU finish together.
  const std::uint32_t first = rg * gridDim.x + blockIdx.x;
  const std::uint32_t active_rounds = first < tiles ? (tiles - first + per_round - 1u) / per_round : 1u;
  auto round = [&](std::uint32_t sj, const UnitRaw (&raw)[TILE][UPL]) {
    if constexpr (GR == 0u) {
      switch ((4u * sj) / active_rounds) {
        case 0: __builtin_amdgcn_s_setprio(3); break;
        case 1: __builtin_amdgcn_s_setprio(2); break;
        case 2: __builtin_amdgcn_s_setprio(1); break;
        default: __builtin_amdgcn_s_setprio(0); break;
      }
    }
    finish_tile(sj, tile_of(sj), sj & 1u, (sj >> rshift) & 1u, raw);
    group_end(sj);
  };
  std::uint32_t s = 0;
  for (; s + 2u < rounds; s += 2u) {
    load_tile(tile_of(s + 1u), buf[1]);
    round(s, buf[0]);
    load_tile(tile_of(s + 2u), buf[0]);
    round(s + 1u, buf[1]);
  }
  if (s + 1u < rounds) {
    load_tile(tile_of(s + 1u), buf[1]);
    round(s, buf[0]);
    round(s + 1u, buf[1]);
  } else {
    round(s, buf[0]);
  }
  if constexpr (EpiHasFinish<Epi>::value) {
    if (kw == 0u) epi.finish(blockIdx.x * nrg + rg, lane);
  }
  if constexpr (kPair) {
    if (late && lane == 0u && epi.wait.status != nullptr)
      __hip_atomic_fetch_or(epi.wait.status, kStatusWaitTimeout, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  }
  tl_stamp(kTlR, tl_slot + 1u);
}

// ---- epilogues ---------------------------------------------------------------

// Row r of the tile is in lanes [r * 64/T, (r+1) * 64/T); epilogues write from the
// first lane of each range.
template <int TILE>
struct EpiStore {
  static constexpr int kTile = TILE;
  float* y;
  __device__ __forceinline__ void init(std::uint32_t) {}
  __device__ __forceinline__ void operator()(std::uint32_t row0, float v, std::uint32_t lane,
                                             std::uint32_t rows) const {
    constexpr std::uint32_t spread = 64u / TILE;
    const std::uint32_t row = row0 + lane / spread;
    if ((lane % spread) == 0u && row < rows) y[row] = v;
  }
};

// The reference's decode side effect (decode_kernels.cu:1600-1606): kv[(row *
// page_words + (token + row) % page_words) % kv_words] = y[row] for row <
// active_pages.
template <int TILE>
struct EpiDecode {
  static constexpr int kTile = TILE;
  float* y;
  float* kv;
  const std::uint32_t* token;
  std::uint32_t kv_words, page_words, active_pages;
  __device__ __forceinline__ void init(std::uint32_t) {}
  __device__ __forceinline__ void operator()(std::uint32_t row0, float v, std::uint32_t lane,
                                             std::uint32_t rows) const {
    constexpr std::uint32_t spread = 64u / TILE;
    const std::uint32_t row = row0 + lane / spread;
    if ((lane % spread) != 0u || row >= rows) return;
    y[row] = v;
    if (kv != nullptr && row < active_pages && kv_words > 0u && page_words > 0u) {
      const std::size_t base = static_cast<std::size_t>(row) * page_words;
      const std::size_t off = (token[0] + row) % page_words;
      kv[(base + off) % kv_words] = v;
    }
  }
};

}  // namespace rtxllm
