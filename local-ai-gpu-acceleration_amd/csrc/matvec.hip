// Batch-1 matvec and dequant entry points (C-ABI) for the GGUF resident packs.
#include "rtxllm/decode_kernels.h"

#include "internal.h"
#include "mv.cuh"

namespace rtxllm {
namespace {

constexpr int kTile = 4;

[[maybe_unused]] int num_cus() {
  static int cached = 0;
  if (cached == 0) {
    int dev = 0, n = 0;
    if (hipGetDevice(&dev) == hipSuccess &&
        hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) == hipSuccess && n > 0)
      cached = n;
    else
      cached = 256;
  }
  return cached;
}

// Launch geometry of mv_kernel, from a sweep on MI355X at the 8B shapes: one
// unit (32 columns) per lane for rows of up to 16384 columns (two beyond),
// ks = ceil(units / 64) waves per row, nrg = 4 / ks row groups per workgroup
// (at least 1), and one 4-row tile per row group: many small workgroups keep
// enough loads in flight and the dispatcher's tail short.
struct MvGeom {
  int upl;
  unsigned ks, nrg, grid;
};

bool mv_geom(int fmt, std::uint32_t rows, std::uint32_t cols, int tile, MvGeom& g) {
  (void)fmt;
  const std::uint32_t units = cols / 32u;
  g.upl = units > 512u ? 2 : 1;
  g.ks = (units + 64u * g.upl - 1u) / (64u * g.upl);
  if (g.ks > static_cast<unsigned>(kMaxKs)) return false;
  g.nrg = g.ks >= 4u ? 1u : 4u / g.ks;
  const std::uint32_t tiles = (rows + tile - 1) / tile;
  const std::uint32_t grid = (tiles + g.nrg - 1) / g.nrg;
  g.grid = grid < 1u ? 1u : (grid > 1048576u ? 1048576u : grid);
  return true;
}

template <int FMT, bool SELF, class Epi>
hipError_t launch_mv_fmt(const QTensor& w, const XSrc& xs, std::uint32_t row_count, const Epi& epi,
                         hipStream_t stream) {
  MvGeom g;
  if (!mv_geom(FMT, row_count, w.cols, kTile, g)) return hipErrorInvalidValue;
  const dim3 grid(g.grid), block(64u * g.ks * g.nrg);
  if (g.upl == 2) {
    hipLaunchKernelGGL((mv_kernel<FMT, 2, kTile, SELF, Epi>), grid, block, 0, stream, w, xs, row_count, g.ks, epi);
  } else {
    hipLaunchKernelGGL((mv_kernel<FMT, 1, kTile, SELF, Epi>), grid, block, 0, stream, w, xs, row_count, g.ks, epi);
  }
  return hipGetLastError();
}

template <bool SELF, class Epi>
hipError_t launch_mv(int fmt, const QTensor& w, const XSrc& xs, std::uint32_t row_count, const Epi& epi,
                     hipStream_t stream) {
  switch (fmt) {
    case RTXLLM_FMT_Q4K_RAW: return launch_mv_fmt<RTXLLM_FMT_Q4K_RAW, SELF>(w, xs, row_count, epi, stream);
    case RTXLLM_FMT_Q4K_SPLIT_PREDECODED:
      return launch_mv_fmt<RTXLLM_FMT_Q4K_SPLIT_PREDECODED, SELF>(w, xs, row_count, epi, stream);
    case RTXLLM_FMT_Q4K_SPLIT_HALF:
      return launch_mv_fmt<RTXLLM_FMT_Q4K_SPLIT_HALF, SELF>(w, xs, row_count, epi, stream);
    case RTXLLM_FMT_Q4K_SPLIT_COMPACT:
      return launch_mv_fmt<RTXLLM_FMT_Q4K_SPLIT_COMPACT, SELF>(w, xs, row_count, epi, stream);
    case RTXLLM_FMT_Q4K_SPLIT_NATIVE:
      return launch_mv_fmt<RTXLLM_FMT_Q4K_SPLIT_NATIVE, SELF>(w, xs, row_count, epi, stream);
    case RTXLLM_FMT_Q5K: return launch_mv_fmt<RTXLLM_FMT_Q5K, SELF>(w, xs, row_count, epi, stream);
    case RTXLLM_FMT_IQ2S: return launch_mv_fmt<RTXLLM_FMT_IQ2S, SELF>(w, xs, row_count, epi, stream);
    case RTXLLM_FMT_IQ3S: return launch_mv_fmt<RTXLLM_FMT_IQ3S, SELF>(w, xs, row_count, epi, stream);
    case RTXLLM_FMT_Q4K_RAW_PREDECODED:
      return launch_mv_fmt<RTXLLM_FMT_Q4K_RAW_PREDECODED, SELF>(w, xs, row_count, epi, stream);
    default: return hipErrorInvalidValue;
  }
}

bool needs_meta(int fmt) { return rtxllm_format_meta_bytes(fmt) != 0u; }

bool aligned(const void* p, std::uintptr_t a) { return (reinterpret_cast<std::uintptr_t>(p) % a) == 0u; }

// The kernels issue 16-byte loads of x, of 16-byte aligned block fields and of
// the Q4_K metadata records; reject pointers that break those alignments.
bool pointers_ok(int fmt, const void* payload, const void* meta, const void* x) {
  if (x != nullptr && !aligned(x, 16)) return false;
  const bool iq = fmt == RTXLLM_FMT_IQ2S || fmt == RTXLLM_FMT_IQ3S;
  if (!aligned(payload, iq ? 2 : 16)) return false;
  if (needs_meta(fmt)) {
    const std::uintptr_t ma = fmt == RTXLLM_FMT_Q4K_SPLIT_HALF ? 8 : fmt == RTXLLM_FMT_Q4K_SPLIT_COMPACT ? 4 : 16;
    if (!aligned(meta, ma)) return false;
  }
  return true;
}

// ---- bit-exact dequant -----------------------------------------------------

#pragma clang fp contract(off)
// Value v of a block, with the reference's expression order (main.cpp:1133-1259).
template <int FMT>
__device__ float dequant_value(const std::uint8_t* p, const std::uint8_t* m, std::uint32_t v) {
  if constexpr (FMT == RTXLLM_FMT_Q5K) {
    const float d = f16_bits_to_f32(ld_u16(p));
    const float dmin = f16_bits_to_f32(ld_u16(p + 2));
    const std::uint32_t g = v >> 6, lane = v & 31u, high = (v & 63u) >= 32u;
    std::uint32_t sc, mn;
    scale_min_k4(static_cast<int>(2u * g + high), ld_u32(p + 4), ld_u32(p + 8), ld_u32(p + 12), sc, mn);
    const std::uint32_t packed = p[48u + 32u * g + lane];
    const std::uint32_t low = high ? (packed >> 4) : (packed & 15u);
    const std::uint32_t quant = low + (((p[16u + lane] >> (2u * g + high)) & 1u) ? 16u : 0u);
    return d * static_cast<float>(sc) * static_cast<float>(quant) - dmin * static_cast<float>(mn);
  } else if constexpr (FMT == RTXLLM_FMT_IQ2S) {
    const std::uint32_t ib32 = v >> 5, grp = (v & 31u) >> 3, lane = v & 7u;
    const float d = f16_bits_to_f32(ld_u16(p));
    const std::uint32_t go = ib32 * 4u + grp;
    const std::uint32_t idx = p[2u + go] | ((static_cast<std::uint32_t>(p[66u + ib32]) << (8u - 2u * grp)) & 0x300u);
    const std::uint32_t grid = 2u * ((kIq2sGridDev[idx] >> (2u * lane)) & 3u) + 1u;
    const std::uint32_t sb = p[74u + ib32];
    const std::uint32_t nib = grp < 2u ? (sb & 15u) : (sb >> 4);
    const float scale = d * (0.5f + static_cast<float>(nib)) * 0.25f;
    const bool neg = (p[34u + go] >> lane) & 1u;
    return scale * static_cast<float>(grid) * (neg ? -1.0f : 1.0f);
  } else if constexpr (FMT == RTXLLM_FMT_IQ3S) {
    const std::uint32_t ib32 = v >> 5, grp = (v & 31u) >> 3, lane = v & 7u, pair = lane >> 2, gl = lane & 3u;
    const float d = f16_bits_to_f32(ld_u16(p));
    const std::uint32_t sel = ib32 * 8u + grp * 2u + pair;
    const std::uint32_t hb = (p[66u + ib32] >> (2u * grp + pair)) & 1u;
    const std::uint32_t idx = p[2u + sel] | (hb << 8);
    const std::uint32_t grid = (kIq3sGridDev[idx] >> (8u * gl)) & 0xFFu;
    const std::uint32_t sb = p[106u + (ib32 >> 1)];
    const std::uint32_t nib = (ib32 & 1u) == 0u ? (sb & 15u) : (sb >> 4);
    const float scale = d * static_cast<float>(1u + 2u * nib);
    const bool neg = (p[74u + ib32 * 4u + grp] >> lane) & 1u;
    return scale * static_cast<float>(grid) * (neg ? -1.0f : 1.0f);
  } else {
    const std::uint32_t g = v >> 6, lane = v & 31u, high = (v & 63u) >= 32u, pair = 2u * g + high;
    const std::uint8_t* qs = (FMT == RTXLLM_FMT_Q4K_RAW || FMT == RTXLLM_FMT_Q4K_RAW_PREDECODED) ? p + 16 : p;
    const std::uint32_t packed = qs[32u * g + lane];
    const float quant = static_cast<float>(high ? (packed >> 4) : (packed & 15u));
    if constexpr (FMT == RTXLLM_FMT_Q4K_SPLIT_PREDECODED || FMT == RTXLLM_FMT_Q4K_RAW_PREDECODED) {
      const float* pm = reinterpret_cast<const float*>(m) + 2u * pair;
      return pm[0] * quant - pm[1];
    } else if constexpr (FMT == RTXLLM_FMT_Q4K_SPLIT_HALF) {
      return f16_bits_to_f32(ld_u16(m + 4u * pair)) * quant - f16_bits_to_f32(ld_u16(m + 4u * pair + 2u));
    } else if constexpr (FMT == RTXLLM_FMT_Q4K_SPLIT_COMPACT) {
      const float d = f16_bits_to_f32(ld_u16(m));
      const float dmin = f16_bits_to_f32(ld_u16(m + 2));
      return d * static_cast<float>(m[4u + pair]) * quant - dmin * static_cast<float>(m[12u + pair]);
    } else {  // native head: split-native metadata or the raw block itself
      const std::uint8_t* h = (FMT == RTXLLM_FMT_Q4K_RAW) ? p : m;
      const float d = f16_bits_to_f32(ld_u16(h));
      const float dmin = f16_bits_to_f32(ld_u16(h + 2));
      std::uint32_t sc, mn;
      scale_min_k4(static_cast<int>(pair), ld_u32(h + 4), ld_u32(h + 8), ld_u32(h + 12), sc, mn);
      return d * static_cast<float>(sc) * quant - dmin * static_cast<float>(mn);
    }
  }
}
#pragma clang fp contract(on)

// One workgroup of 256 threads per block; thread v writes value v.
template <int FMT>
__global__ __launch_bounds__(256) void dequant_kernel(const std::uint8_t* __restrict__ payload,
                                                      const std::uint8_t* __restrict__ meta, std::uint32_t cols,
                                                      float* __restrict__ out) {
  const std::size_t blk = blockIdx.x;
  const std::uint32_t bpr = cols >> 8;
  const std::size_t row = blk / bpr, b = blk % bpr;
  const std::uint8_t* p = payload + blk * rtxllm_format_payload_bytes(FMT);
  const std::uint8_t* m = meta ? meta + blk * rtxllm_format_meta_bytes(FMT) : nullptr;
  out[row * cols + b * 256u + threadIdx.x] = dequant_value<FMT>(p, m, threadIdx.x);
}

template <int FMT>
hipError_t launch_dequant_fmt(const std::uint8_t* payload, const std::uint8_t* meta, std::uint32_t rows,
                              std::uint32_t cols, float* out, hipStream_t stream) {
  const std::size_t blocks = static_cast<std::size_t>(rows) * (cols / 256u);
  hipLaunchKernelGGL(dequant_kernel<FMT>, dim3(static_cast<unsigned>(blocks)), dim3(256), 0, stream, payload,
                     meta, cols, out);
  return hipGetLastError();
}

bool shape_ok(std::uint32_t rows, std::uint32_t cols) { return rows != 0u && cols != 0u && (cols % 256u) == 0u; }

// Matvec + KV side-write + decode-chain token update (the reference's
// *_decode launchers, decode_kernels.cu:4032-4072, 4473-4607).
hipError_t decode_call(int fmt, const std::uint8_t* payload, const std::uint8_t* meta, const float* x, float* y,
                       float* kv, std::uint32_t* token, std::uint32_t rows, std::uint32_t cols,
                       std::uint32_t launched_rows, std::uint32_t kv_words, std::uint32_t page_words,
                       std::uint32_t active_pages, hipStream_t stream) {
  if (!shape_ok(rows, cols) || launched_rows == 0u || payload == nullptr || x == nullptr || y == nullptr ||
      token == nullptr || (needs_meta(fmt) && meta == nullptr) || !pointers_ok(fmt, payload, meta, x))
    return hipErrorInvalidValue;
  const QTensor w{payload, meta, rows, cols};
  const EpiDecode<kTile> epi{y, kv, token, kv_words, page_words, active_pages};
  const hipError_t st = launch_mv<true>(fmt, w, XSrc{XQ{}, x}, launched_rows, epi, stream);
  if (st != hipSuccess) return st;
  return launch_argmax_token(y, token, launched_rows, 0, 32000u, 0u, stream);
}

}  // namespace
}  // namespace rtxllm

using namespace rtxllm;

extern "C" hipError_t rtxllm_dequant_f32(int format, const std::uint8_t* payload, const std::uint8_t* meta,
                                         std::uint32_t rows, std::uint32_t cols, float* out, hipStream_t stream) {
  if (!shape_ok(rows, cols) || payload == nullptr || out == nullptr || (needs_meta(format) && meta == nullptr) ||
      !pointers_ok(format, payload, meta, nullptr))
    return hipErrorInvalidValue;
  switch (format) {
    case RTXLLM_FMT_Q4K_RAW: return launch_dequant_fmt<RTXLLM_FMT_Q4K_RAW>(payload, meta, rows, cols, out, stream);
    case RTXLLM_FMT_Q4K_SPLIT_PREDECODED:
      return launch_dequant_fmt<RTXLLM_FMT_Q4K_SPLIT_PREDECODED>(payload, meta, rows, cols, out, stream);
    case RTXLLM_FMT_Q4K_SPLIT_HALF:
      return launch_dequant_fmt<RTXLLM_FMT_Q4K_SPLIT_HALF>(payload, meta, rows, cols, out, stream);
    case RTXLLM_FMT_Q4K_SPLIT_COMPACT:
      return launch_dequant_fmt<RTXLLM_FMT_Q4K_SPLIT_COMPACT>(payload, meta, rows, cols, out, stream);
    case RTXLLM_FMT_Q4K_SPLIT_NATIVE:
      return launch_dequant_fmt<RTXLLM_FMT_Q4K_SPLIT_NATIVE>(payload, meta, rows, cols, out, stream);
    case RTXLLM_FMT_Q5K: return launch_dequant_fmt<RTXLLM_FMT_Q5K>(payload, meta, rows, cols, out, stream);
    case RTXLLM_FMT_IQ2S: return launch_dequant_fmt<RTXLLM_FMT_IQ2S>(payload, meta, rows, cols, out, stream);
    case RTXLLM_FMT_IQ3S: return launch_dequant_fmt<RTXLLM_FMT_IQ3S>(payload, meta, rows, cols, out, stream);
    case RTXLLM_FMT_Q4K_RAW_PREDECODED:
      return launch_dequant_fmt<RTXLLM_FMT_Q4K_RAW_PREDECODED>(payload, meta, rows, cols, out, stream);
    default: return hipErrorInvalidValue;
  }
}

extern "C" hipError_t rtxllm_matvec(int format, const std::uint8_t* payload, const std::uint8_t* meta,
                                    const float* x, float* y, std::uint32_t rows, std::uint32_t cols,
                                    hipStream_t stream) {
  if (!shape_ok(rows, cols) || payload == nullptr || x == nullptr || y == nullptr ||
      (needs_meta(format) && meta == nullptr) || !pointers_ok(format, payload, meta, x))
    return hipErrorInvalidValue;
  const QTensor w{payload, meta, rows, cols};
  return launch_mv<true>(format, w, XSrc{XQ{}, x}, rows, EpiStore<kTile>{y}, stream);
}

extern "C" std::size_t rtxllm_xq_bytes(std::uint32_t cols) { return xq_bytes(cols); }

extern "C" hipError_t rtxllm_matvec_xq(int format, const std::uint8_t* payload, const std::uint8_t* meta,
                                       const void* xq, float* y, std::uint32_t rows, std::uint32_t cols,
                                       hipStream_t stream) {
  if (!shape_ok(rows, cols) || payload == nullptr || xq == nullptr || y == nullptr ||
      (needs_meta(format) && meta == nullptr) || !pointers_ok(format, payload, meta, xq))
    return hipErrorInvalidValue;
  const QTensor w{payload, meta, rows, cols};
  return launch_mv<false>(format, w, XSrc{xq_view(xq, cols), nullptr}, rows, EpiStore<kTile>{y}, stream);
}

// ---- reference-named matvec launchers --------------------------------------

#define RTXLLM_Q4K_RAW_ALIAS(name)                                                                               \
  extern "C" hipError_t name(const std::uint8_t* q4k_blocks, const float* activation, float* logits, float* kv, \
                             std::uint32_t* token, std::uint32_t rows, std::uint32_t cols,                      \
                             std::uint32_t kv_words, std::uint32_t page_words, std::uint32_t active_pages,      \
                             hipStream_t stream) {                                                              \
    return decode_call(RTXLLM_FMT_Q4K_RAW, q4k_blocks, nullptr, activation, logits, kv, token, rows, cols, rows, \
                       kv_words, page_words, active_pages, stream);                                             \
  }

RTXLLM_Q4K_RAW_ALIAS(rtxllm_launch_q4k_matvec_decode)
RTXLLM_Q4K_RAW_ALIAS(rtxllm_launch_q4k_matvec_decode_shared)
RTXLLM_Q4K_RAW_ALIAS(rtxllm_launch_q4k_matvec_decode_warp)
RTXLLM_Q4K_RAW_ALIAS(rtxllm_launch_q4k_matvec_decode_warp_broadcast)
RTXLLM_Q4K_RAW_ALIAS(rtxllm_launch_q4k_matvec_decode_warp_broadcast_vec4)
RTXLLM_Q4K_RAW_ALIAS(rtxllm_launch_q4k_matvec_decode_warp_broadcast_vec4x2)
RTXLLM_Q4K_RAW_ALIAS(rtxllm_launch_q4k_matvec_decode_warp_broadcast_vec4x4)

extern "C" hipError_t rtxllm_launch_q4k_matvec_decode_predecoded_vec4x4(
    const std::uint8_t* q4k_blocks, const float* q4k_scale_min_pairs, const float* activation, float* logits,
    float* kv, std::uint32_t* token, std::uint32_t rows, std::uint32_t cols, std::uint32_t kv_words,
    std::uint32_t page_words, std::uint32_t active_pages, hipStream_t stream) {
  return decode_call(RTXLLM_FMT_Q4K_RAW_PREDECODED, q4k_blocks,
                     reinterpret_cast<const std::uint8_t*>(q4k_scale_min_pairs), activation, logits, kv, token,
                     rows, cols, rows, kv_words, page_words, active_pages, stream);
}

extern "C" hipError_t rtxllm_launch_q4k_matvec_decode_split_predecoded_vec4x4(
    const std::uint8_t* q4k_payload, const float* q4k_scale_min_pairs, const float* activation, float* logits,
    float* kv, std::uint32_t* token, std::uint32_t rows, std::uint32_t cols, std::uint32_t kv_words,
    std::uint32_t page_words, std::uint32_t active_pages, hipStream_t stream) {
  return decode_call(RTXLLM_FMT_Q4K_SPLIT_PREDECODED, q4k_payload,
                     reinterpret_cast<const std::uint8_t*>(q4k_scale_min_pairs), activation, logits, kv, token,
                     rows, cols, rows, kv_words, page_words, active_pages, stream);
}

extern "C" hipError_t rtxllm_launch_q4k_matvec_decode_split_half_vec4x4(
    const std::uint8_t* q4k_payload, const std::uint16_t* q4k_scale_min_half_pairs, const float* activation,
    float* logits, float* kv, std::uint32_t* token, std::uint32_t rows, std::uint32_t cols,
    std::uint32_t kv_words, std::uint32_t page_words, std::uint32_t active_pages, hipStream_t stream) {
  return decode_call(RTXLLM_FMT_Q4K_SPLIT_HALF, q4k_payload,
                     reinterpret_cast<const std::uint8_t*>(q4k_scale_min_half_pairs), activation, logits, kv,
                     token, rows, cols, rows, kv_words, page_words, active_pages, stream);
}

extern "C" hipError_t rtxllm_launch_q4k_matvec_decode_split_compact_vec4x4(
    const std::uint8_t* q4k_payload, const std::uint8_t* q4k_compact_meta, const float* activation, float* logits,
    float* kv, std::uint32_t* token, std::uint32_t rows, std::uint32_t cols, std::uint32_t kv_words,
    std::uint32_t page_words, std::uint32_t active_pages, hipStream_t stream) {
  return decode_call(RTXLLM_FMT_Q4K_SPLIT_COMPACT, q4k_payload, q4k_compact_meta, activation, logits, kv, token,
                     rows, cols, rows, kv_words, page_words, active_pages, stream);
}

extern "C" hipError_t rtxllm_launch_q4k_matvec_decode_split_native_vec4x4(
    const std::uint8_t* q4k_payload, const std::uint8_t* q4k_native_meta, const float* activation, float* logits,
    float* kv, std::uint32_t* token, std::uint32_t rows, std::uint32_t cols, std::uint32_t kv_words,
    std::uint32_t page_words, std::uint32_t active_pages, hipStream_t stream) {
  return decode_call(RTXLLM_FMT_Q4K_SPLIT_NATIVE, q4k_payload, q4k_native_meta, activation, logits, kv, token,
                     rows, cols, rows, kv_words, page_words, active_pages, stream);
}

static std::uint32_t clip_rows(std::uint32_t rows, std::uint32_t rows_limit) {
  return rows_limit < rows ? rows_limit : rows;
}

extern "C" hipError_t rtxllm_launch_q5k_matvec_decode_probe(
    const std::uint8_t* q5k_blocks, const float* activation, float* logits, float* kv, std::uint32_t* token,
    std::uint32_t rows, std::uint32_t cols, std::uint32_t rows_limit, std::uint32_t kv_words,
    std::uint32_t page_words, std::uint32_t active_pages, hipStream_t stream) {
  return decode_call(RTXLLM_FMT_Q5K, q5k_blocks, nullptr, activation, logits, kv, token, rows, cols,
                     clip_rows(rows, rows_limit), kv_words, page_words, active_pages, stream);
}

extern "C" hipError_t rtxllm_launch_iq2s_matvec_decode_probe(
    const std::uint8_t* iq2s_blocks, const float* activation, float* logits, float* kv, std::uint32_t* token,
    std::uint32_t rows, std::uint32_t cols, std::uint32_t rows_limit, std::uint32_t kv_words,
    std::uint32_t page_words, std::uint32_t active_pages, hipStream_t stream) {
  return decode_call(RTXLLM_FMT_IQ2S, iq2s_blocks, nullptr, activation, logits, kv, token, rows, cols,
                     clip_rows(rows, rows_limit), kv_words, page_words, active_pages, stream);
}

extern "C" hipError_t rtxllm_launch_iq3s_matvec_decode_probe(
    const std::uint8_t* iq3s_blocks, const float* activation, float* logits, float* kv, std::uint32_t* token,
    std::uint32_t rows, std::uint32_t cols, std::uint32_t rows_limit, std::uint32_t kv_words,
    std::uint32_t page_words, std::uint32_t active_pages, hipStream_t stream) {
  return decode_call(RTXLLM_FMT_IQ3S, iq3s_blocks, nullptr, activation, logits, kv, token, rows, cols,
                     clip_rows(rows, rows_limit), kv_words, page_words, active_pages, stream);
}

// decode_kernels.cu:4074-4093: matvec over min(rows, rows_limit) rows, no side effects.
extern "C" hipError_t rtxllm_launch_iq2s_matvec_probe(const std::uint8_t* iq2s_blocks, const float* activation,
                                                      float* logits, std::uint32_t rows, std::uint32_t cols,
                                                      std::uint32_t rows_limit, hipStream_t stream) {
  if (!shape_ok(rows, cols) || rows_limit == 0u || iq2s_blocks == nullptr || activation == nullptr ||
      logits == nullptr || !pointers_ok(RTXLLM_FMT_IQ2S, iq2s_blocks, nullptr, activation))
    return hipErrorInvalidValue;
  const QTensor w{iq2s_blocks, nullptr, rows, cols};
  return launch_mv<true>(RTXLLM_FMT_IQ2S, w, XSrc{XQ{}, activation}, clip_rows(rows, rows_limit),
                         EpiStore<kTile>{logits}, stream);
}
