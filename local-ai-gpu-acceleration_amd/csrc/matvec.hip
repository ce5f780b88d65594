// Batch-1 matvec and dequant entry points (C-ABI) for the GGUF resident packs.
#include "rtxllm/decode_kernels.h"

#include "rtxllm/testing.h"

#include "internal.h"
#include "dequant.cuh"
#include "layer.h"
#include "mv_launch.cuh"
#include "mvq.cuh"

static_assert(rtxllm::kPairSpinLimit == (1u << 20), "launch_gate_up's default wait limit");
static_assert(rtxllm::kStatusWaitTimeout == RTXLLM_STATUS_WAIT_TIMEOUT, "status bit of the C-ABI");

namespace rtxllm {
namespace {

constexpr int kTile = 4;

bool needs_meta(int fmt) { return rtxllm_format_meta_bytes(fmt) != 0u; }

bool aligned(const void* p, std::uintptr_t a) { return (reinterpret_cast<std::uintptr_t>(p) % a) == 0u; }

bool shape_ok(std::uint32_t rows, std::uint32_t cols) { return rows != 0u && cols != 0u && (cols % 256u) == 0u; }

// The kernels issue 16-byte loads of 16-byte aligned block fields and of the
// Q4_K metadata records; reject weight pointers that break those alignments.
// An fp32 activation may have any 4-byte alignment (the kernels stage a
// misaligned one value by value); a staged activation is 16-byte aligned.
bool pointers_ok(int fmt, const void* payload, const void* meta, const void* x, bool staged = false) {
  if (x != nullptr && !aligned(x, staged ? 16 : 4)) return false;
  const bool iq = fmt == RTXLLM_FMT_IQ2S || fmt == RTXLLM_FMT_IQ3S;  // IQ2S_UNITS: 16 (8-byte field loads)
  if (!aligned(payload, iq ? 2 : 16)) return false;
  if (needs_meta(fmt)) {
    const std::uintptr_t ma = fmt == RTXLLM_FMT_Q4K_SPLIT_HALF ? 8 : fmt == RTXLLM_FMT_Q4K_SPLIT_COMPACT ? 4 : 16;
    if (!aligned(meta, ma)) return false;
  }
  return true;
}

// ---- bit-exact dequant -----------------------------------------------------


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

// Unit layouts: the workgroup gathers its block's bytes back into the GGUF
// order in LDS, then dequantises them exactly as the GGUF format.
template <int FMT>
__global__ __launch_bounds__(256) void dequant_units_kernel(const std::uint8_t* __restrict__ payload,
                                                            std::uint32_t cols, std::size_t nb,
                                                            float* __restrict__ out) {
  constexpr bool k2 = FMT == RTXLLM_FMT_IQ2S_UNITS;
  constexpr std::uint32_t kRaw = k2 ? 82u : 110u;
  __shared__ std::uint8_t blk[112];
  const std::size_t b = blockIdx.x;
  const std::uint32_t bpr = cols >> 8, i = threadIdx.x;
  if (i < kRaw) blk[i] = payload[k2 ? iq2s_units_offset(b, i, nb) : iq3s_units_offset(b, i, nb)];
  __syncthreads();
  out[(b / bpr) * cols + (b % bpr) * 256u + i] =
      dequant_value<k2 ? RTXLLM_FMT_IQ2S : RTXLLM_FMT_IQ3S>(blk, nullptr, i);
}

// One thread per block: GGUF IQ2_S / IQ3_S bytes -> the unit layout (IQ3_S:
// each scale byte also goes to the odd unit of its pair).
template <int FMT>
__global__ __launch_bounds__(256) void units_pack_kernel(const std::uint8_t* __restrict__ raw, std::size_t nb,
                                                         std::uint8_t* __restrict__ out) {
  constexpr bool k2 = FMT == RTXLLM_FMT_IQ2S_UNITS;
  constexpr std::uint32_t kRaw = k2 ? 82u : 110u;
  const std::size_t b = static_cast<std::size_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  if (b >= nb) return;
  const std::uint8_t* src = raw + kRaw * b;
  for (std::uint32_t i = 0; i < kRaw; ++i) {
    const std::size_t o = k2 ? iq2s_units_offset(b, i, nb) : iq3s_units_offset(b, i, nb);
    out[o] = src[i];
    if (!k2 && i >= 106u) out[o + 2u] = src[i];  // (qh, scale) pair of unit 2j + 1
  }
}

template <int FMT>
hipError_t launch_units_pack(const std::uint8_t* raw, std::uint32_t rows, std::uint32_t cols, std::uint8_t* out,
                             hipStream_t stream) {
  if (!shape_ok(rows, cols) || raw == nullptr || out == nullptr || !aligned(out, 16)) return hipErrorInvalidValue;
  const std::size_t nb = static_cast<std::size_t>(rows) * (cols / 256u);
  if (nb * rtxllm_format_payload_bytes(FMT) > 0xFFFFFFFFull) return hipErrorInvalidValue;
  hipLaunchKernelGGL(units_pack_kernel<FMT>, dim3(static_cast<unsigned>((nb + 255u) / 256u)), dim3(256), 0, stream,
                     raw, nb, out);
  return hipGetLastError();
}

template <int FMT>
hipError_t launch_dequant_fmt(const std::uint8_t* payload, const std::uint8_t* meta, std::uint32_t rows,
                              std::uint32_t cols, float* out, hipStream_t stream) {
  const std::size_t blocks = static_cast<std::size_t>(rows) * (cols / 256u);
  hipLaunchKernelGGL(dequant_kernel<FMT>, dim3(static_cast<unsigned>(blocks)), dim3(256), 0, stream, payload,
                     meta, cols, out);
  return hipGetLastError();
}

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
  const hipError_t st = launch_mv<true>(fmt, w, self_src(x), launched_rows, epi, stream);
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
    case RTXLLM_FMT_IQ2S_UNITS:
    case RTXLLM_FMT_IQ3S_UNITS: {
      const std::size_t nb = static_cast<std::size_t>(rows) * (cols / 256u);
      if (format == RTXLLM_FMT_IQ2S_UNITS)
        hipLaunchKernelGGL(dequant_units_kernel<RTXLLM_FMT_IQ2S_UNITS>, dim3(static_cast<unsigned>(nb)), dim3(256), 0,
                           stream, payload, cols, nb, out);
      else
        hipLaunchKernelGGL(dequant_units_kernel<RTXLLM_FMT_IQ3S_UNITS>, dim3(static_cast<unsigned>(nb)), dim3(256), 0,
                           stream, payload, cols, nb, out);
      return hipGetLastError();
    }
    case RTXLLM_FMT_Q4K_RAW_PREDECODED:
      return launch_dequant_fmt<RTXLLM_FMT_Q4K_RAW_PREDECODED>(payload, meta, rows, cols, out, stream);
    default: return hipErrorInvalidValue;
  }
}

extern "C" hipError_t rtxllm_iq2s_units_pack(const std::uint8_t* raw, std::uint32_t rows, std::uint32_t cols,
                                             std::uint8_t* out, hipStream_t stream) {
  return launch_units_pack<RTXLLM_FMT_IQ2S_UNITS>(raw, rows, cols, out, stream);
}

extern "C" hipError_t rtxllm_iq3s_units_pack(const std::uint8_t* raw, std::uint32_t rows, std::uint32_t cols,
                                             std::uint8_t* out, hipStream_t stream) {
  return launch_units_pack<RTXLLM_FMT_IQ3S_UNITS>(raw, rows, cols, out, stream);
}

extern "C" hipError_t rtxllm_matvec(int format, const std::uint8_t* payload, const std::uint8_t* meta,
                                    const float* x, float* y, std::uint32_t rows, std::uint32_t cols,
                                    hipStream_t stream) {
  if (!shape_ok(rows, cols) || payload == nullptr || x == nullptr || y == nullptr ||
      (needs_meta(format) && meta == nullptr) || !pointers_ok(format, payload, meta, x))
    return hipErrorInvalidValue;
  const QTensor w{payload, meta, rows, cols};
  return launch_mv<true>(format, w, self_src(x), rows, EpiStore<kTile>{y}, stream);
}

extern "C" std::size_t rtxllm_xq_bytes(std::uint32_t cols) { return xq_bytes(cols); }

extern "C" hipError_t rtxllm_matvec_xq(int format, const std::uint8_t* payload, const std::uint8_t* meta,
                                       const void* xq, float* y, std::uint32_t rows, std::uint32_t cols,
                                       hipStream_t stream) {
  if (!shape_ok(rows, cols) || payload == nullptr || xq == nullptr || y == nullptr ||
      (needs_meta(format) && meta == nullptr) || !pointers_ok(format, payload, meta, xq, true))
    return hipErrorInvalidValue;
  const QTensor w{payload, meta, rows, cols};
  return launch_mv<false>(format, w, staged_src(xq_view(xq, cols)), rows, EpiStore<kTile>{y}, stream);
}

extern "C" hipError_t rtxllm_matvec_xq_mfma(int format, const std::uint8_t* payload, const void* xq, float* y,
                                            std::uint32_t rows, std::uint32_t cols, hipStream_t stream) {
  if (!mvq_fits(format, rows, cols) || payload == nullptr || xq == nullptr || y == nullptr ||
      !pointers_ok(format, payload, nullptr, xq, true))
    return hipErrorInvalidValue;
  const QTensor w{payload, nullptr, rows, cols};
  return launch_mvq(format, w, xq_view(xq, cols), rows, EpiStore<kTile>{y}, stream);
}

namespace {
hipError_t gate_up_call(int format, const std::uint8_t* payload, const std::uint8_t* meta, const void* xq,
                        const float* sumsq, std::uint32_t nslots, float eps, float* act, std::uint32_t rows,
                        std::uint32_t cols, std::uint32_t* status, hipStream_t stream, std::uint32_t wait_limit,
                        std::uint32_t wait_bias) {
  if (!shape_ok(rows, cols) || (rows % 4u) != 0u || payload == nullptr || xq == nullptr || sumsq == nullptr ||
      nslots == 0u || act == nullptr || (needs_meta(format) && meta == nullptr) ||
      !pointers_ok(format, payload, meta, xq, true) || wait_limit == 0u)
    return hipErrorInvalidValue;
  const NormIn in{xq, sumsq, nslots, cols, eps};
  return launch_gate_up(format, payload, meta, rows, cols, in, act, status, stream, wait_limit, wait_bias);
}
}  // namespace

extern "C" hipError_t rtxllm_gate_up_silu(int format, const std::uint8_t* payload, const std::uint8_t* meta,
                                          const void* xq, const float* sumsq, std::uint32_t nslots, float eps,
                                          float* act, std::uint32_t rows, std::uint32_t cols, std::uint32_t* status,
                                          hipStream_t stream) {
  return gate_up_call(format, payload, meta, xq, sumsq, nslots, eps, act, rows, cols, status, stream,
                      kPairSpinLimit, 0u);
}

extern "C" hipError_t rtxllm_test_gate_up_silu_waits(int format, const std::uint8_t* payload,
                                                     const std::uint8_t* meta, const void* xq, const float* sumsq,
                                                     std::uint32_t nslots, float eps, float* act, std::uint32_t rows,
                                                     std::uint32_t cols, std::uint32_t* status,
                                                     std::uint32_t wait_limit, std::uint32_t wait_bias,
                                                     hipStream_t stream) {
  return gate_up_call(format, payload, meta, xq, sumsq, nslots, eps, act, rows, cols, status, stream, wait_limit,
                      wait_bias);
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
  return launch_mv<true>(RTXLLM_FMT_IQ2S, w, self_src(activation), clip_rows(rows, rows_limit),
                         EpiStore<kTile>{logits}, stream);
}
