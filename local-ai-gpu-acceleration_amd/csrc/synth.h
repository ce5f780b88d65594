/* Seeded synthetic inputs for the decode hot path: quant packs, activations,
 * norm weights and fp16 KV contents.
 *
 * The generator is splitmix64 used as a counter-based stream: output k of stream
 * s is mix(s + (k + 1) * golden), so any byte range of a pack can be produced
 * independently and in parallel, and C, C++ and Python produce the same bytes.
 * Header-only C so the host library and test tools compile the same code.
 *
 * Field distributions follow the workload definitions: quant bytes uniform
 * (nibbles, 6-bit scales/mins, grid indices, sign bits and 4-bit sub-block
 * scales all come out uniform because every field is a whole bit range of a
 * uniform byte), fp16 d/dmin = fp16_rne(U[lo, hi]), x ~ N(0, 1) by Box-Muller.
 */
#ifndef RTXLLM_SYNTH_H
#define RTXLLM_SYNTH_H

#include <math.h>
#include <stddef.h>
#include <stdint.h>
#include <string.h>

#if defined(__HIPCC__)
#define RTXLLM_SYNTH_INLINE static inline __host__ __device__
#else
#define RTXLLM_SYNTH_INLINE static inline
#endif

RTXLLM_SYNTH_INLINE uint64_t rtxllm_splitmix64_at(uint64_t stream, uint64_t k) {
  uint64_t z = stream + (k + 1u) * 0x9E3779B97F4A7C15ull;
  z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
  z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
  return z ^ (z >> 31);
}

/* Stream id of sub-stream `tag` of a tensor seeded with `seed`. */
RTXLLM_SYNTH_INLINE uint64_t rtxllm_synth_stream(uint64_t seed, uint64_t tag) {
  return rtxllm_splitmix64_at(seed ^ 0xD1B54A32D192ED03ull, tag);
}

/* Uniform double in [0, 1) with 53 random bits. */
RTXLLM_SYNTH_INLINE double rtxllm_synth_unit(uint64_t stream, uint64_t k) {
  return (double)(rtxllm_splitmix64_at(stream, k) >> 11) * (1.0 / 9007199254740992.0);
}

/* fp32 -> IEEE binary16 bits, round to nearest, ties to even (numpy.float16 and
 * Python struct '<e' semantics). Overflow gives +-inf, NaN gives a quiet NaN. */
RTXLLM_SYNTH_INLINE uint16_t rtxllm_f32_to_f16_rne(float value) {
  uint32_t bits;
  memcpy(&bits, &value, 4);
  const uint32_t sign = (bits >> 16) & 0x8000u;
  const uint32_t abs_bits = bits & 0x7FFFFFFFu;
  if (abs_bits > 0x7F800000u) return (uint16_t)(sign | 0x7E00u);
  if (abs_bits >= 0x477FF000u) return (uint16_t)(sign | 0x7C00u); /* >= 65520 rounds to inf */
  if (abs_bits < 0x38800000u) {                                     /* below 2^-14: subnormal */
    if (abs_bits < 0x33000000u) return (uint16_t)sign;              /* < 2^-25 rounds to 0 */
    const uint32_t exp = abs_bits >> 23;
    const uint32_t mant = (abs_bits & 0x7FFFFFu) | 0x800000u;
    const uint32_t shift = 126u - exp; /* 14 + 23 - 10 - (exp - 127) ... in [14, 24] */
    uint32_t half = mant >> shift;
    const uint32_t rem = mant & ((1u << shift) - 1u);
    const uint32_t halfway = 1u << (shift - 1u);
    if (rem > halfway || (rem == halfway && (half & 1u))) half += 1u;
    return (uint16_t)(sign | half);
  }
  uint32_t half = ((abs_bits >> 13) - (112u << 10));
  const uint32_t rem = abs_bits & 0x1FFFu;
  if (rem > 0x1000u || (rem == 0x1000u && (half & 1u))) half += 1u;
  return (uint16_t)(sign | half);
}

/* Fill n bytes with stream `stream` (byte i = byte (i & 7) of output i >> 3). */
RTXLLM_SYNTH_INLINE void rtxllm_synth_bytes(uint64_t stream, uint8_t* out, size_t begin, size_t n) {
  for (size_t i = 0; i < n; ++i) {
    const size_t g = begin + i;
    out[i] = (uint8_t)(rtxllm_splitmix64_at(stream, g >> 3) >> (8u * (unsigned)(g & 7u)));
  }
}

/* Standard normal sample k of a stream (Box-Muller, cosine branch). */
RTXLLM_SYNTH_INLINE float rtxllm_synth_normal(uint64_t stream, uint64_t k) {
  const double u1 = 1.0 - rtxllm_synth_unit(stream, 2u * k); /* (0, 1] */
  const double u2 = rtxllm_synth_unit(stream, 2u * k + 1u);
  return (float)(sqrt(-2.0 * log(u1)) * cos(6.283185307179586 * u2));
}

/* fp16 bits of U[lo, hi], sample k of a stream. */
RTXLLM_SYNTH_INLINE uint16_t rtxllm_synth_f16_uniform(uint64_t stream, uint64_t k, float lo, float hi) {
  const double u = rtxllm_synth_unit(stream, k);
  return rtxllm_f32_to_f16_rne((float)(lo + u * (hi - lo)));
}

/* Quant formats of the resident packs. Raw GGUF blocks except the Q4_K split
 * layouts, whose 128-byte nibble payload and per-block metadata live in two
 * separate streams, and IQ2S_UNITS: the same bytes as IQ2_S, regrouped over a
 * tensor of N blocks (row-major) so that each 32-value unit k of block b reads
 * three aligned fields: [0, 64 N) 8 B per unit (qs[4k..4k+3], signs[4k..4k+3])
 * at 64 b + 8 k; [64 N, 80 N) 2 B per unit (qh[k], scales[k]) at 16 b + 2 k;
 * [80 N, 82 N) the block's fp16 d at 2 b. IQ3S_UNITS likewise for IQ3_S (d, qs[64],
 * qh[8], signs[32], scales[4]): [0, 96 N) 12 B per unit (qs[8k..8k+7],
 * signs[4k..4k+3]) at 96 b + 12 k; [96 N, 112 N) (qh[k], scales[k / 2]) at
 * 16 b + 2 k (each scale byte twice); [112 N, 114 N) d at 2 b. */
enum rtxllm_format {
  RTXLLM_FMT_Q4K_RAW = 0,             /* 144 B GGUF block */
  RTXLLM_FMT_Q4K_SPLIT_PREDECODED = 1, /* 128 B payload + 8 x (f32 S, f32 M) */
  RTXLLM_FMT_Q4K_SPLIT_HALF = 2,       /* 128 B payload + 8 x (f16 S, f16 M) */
  RTXLLM_FMT_Q4K_SPLIT_COMPACT = 3,    /* 128 B payload + f16 d, f16 dmin, u8 sc[8], u8 m[8] */
  RTXLLM_FMT_Q4K_SPLIT_NATIVE = 4,     /* 128 B payload + the original 16 B head */
  RTXLLM_FMT_Q5K = 5,                  /* 176 B GGUF block */
  RTXLLM_FMT_IQ2S = 6,                 /* 82 B GGUF block */
  RTXLLM_FMT_IQ3S = 7,                 /* 110 B GGUF block */
  RTXLLM_FMT_Q4K_RAW_PREDECODED = 8,   /* 144 B GGUF block (quants) + 8 x (f32 S, f32 M) */
  RTXLLM_FMT_IQ2S_UNITS = 9,           /* IQ2_S blocks regrouped per 32-value unit (see below) */
  RTXLLM_FMT_IQ3S_UNITS = 10,          /* IQ3_S blocks regrouped per 32-value unit, 114 B per block */
  RTXLLM_FMT_COUNT = 11
};

RTXLLM_SYNTH_INLINE uint32_t rtxllm_format_payload_bytes(int fmt) {
  switch (fmt) {
    case RTXLLM_FMT_Q4K_RAW:
    case RTXLLM_FMT_Q4K_RAW_PREDECODED: return 144u;
    case RTXLLM_FMT_Q4K_SPLIT_PREDECODED:
    case RTXLLM_FMT_Q4K_SPLIT_HALF:
    case RTXLLM_FMT_Q4K_SPLIT_COMPACT:
    case RTXLLM_FMT_Q4K_SPLIT_NATIVE: return 128u;
    case RTXLLM_FMT_Q5K: return 176u;
    case RTXLLM_FMT_IQ2S:
    case RTXLLM_FMT_IQ2S_UNITS: return 82u;
    case RTXLLM_FMT_IQ3S: return 110u;
    case RTXLLM_FMT_IQ3S_UNITS: return 114u;
    default: return 0u;
  }
}

RTXLLM_SYNTH_INLINE uint32_t rtxllm_format_meta_bytes(int fmt) {
  switch (fmt) {
    case RTXLLM_FMT_Q4K_SPLIT_PREDECODED:
    case RTXLLM_FMT_Q4K_RAW_PREDECODED: return 64u;
    case RTXLLM_FMT_Q4K_SPLIT_HALF: return 32u;
    case RTXLLM_FMT_Q4K_SPLIT_COMPACT: return 20u;
    case RTXLLM_FMT_Q4K_SPLIT_NATIVE: return 16u;
    default: return 0u;
  }
}

/* GGUF block bytes of the source format (the roofline's algorithmic bytes). */
RTXLLM_SYNTH_INLINE uint32_t rtxllm_format_gguf_block_bytes(int fmt) {
  if (fmt <= RTXLLM_FMT_Q4K_SPLIT_NATIVE || fmt == RTXLLM_FMT_Q4K_RAW_PREDECODED) return 144u;
  return rtxllm_format_payload_bytes(fmt);
}

/* Raw GGUF blocks [first_block, first_block + n_blocks) of a synthetic tensor in
 * format q4k_raw / q5k / iq2s / iq3s: uniform bytes with fp16 d (and dmin) fields
 * replaced by fp16_rne(U[d_lo, d_hi]). */
RTXLLM_SYNTH_INLINE void rtxllm_synth_raw_blocks(int fmt, uint64_t seed, size_t first_block,
                                                 size_t n_blocks, float d_lo, float d_hi,
                                                 uint8_t* out) {
  const uint32_t bb = rtxllm_format_payload_bytes(fmt);
  const uint64_t s_bytes = rtxllm_synth_stream(seed, 1u);
  const uint64_t s_d = rtxllm_synth_stream(seed, 2u);
  const int has_dmin = (fmt == RTXLLM_FMT_Q4K_RAW || fmt == RTXLLM_FMT_Q5K);
  rtxllm_synth_bytes(s_bytes, out, first_block * (size_t)bb, n_blocks * (size_t)bb);
  for (size_t j = 0; j < n_blocks; ++j) {
    uint8_t* blk = out + j * bb;
    const uint64_t b = first_block + j;
    const uint16_t d = rtxllm_synth_f16_uniform(s_d, 2u * b, d_lo, d_hi);
    blk[0] = (uint8_t)(d & 0xFFu);
    blk[1] = (uint8_t)(d >> 8);
    if (has_dmin) {
      const uint16_t dm = rtxllm_synth_f16_uniform(s_d, 2u * b + 1u, d_lo, d_hi);
      blk[2] = (uint8_t)(dm & 0xFFu);
      blk[3] = (uint8_t)(dm >> 8);
    }
  }
}

#endif
