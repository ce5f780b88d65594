/* CPU oracle for the decode hot path -- TEST INFRASTRUCTURE ONLY (see rtxllm_oracle.h).
 *
 * Compiled with gcc -O2 -ffp-contract=off and no fast-math, so every float
 * expression rounds exactly as written, matching the reference gate's scalar
 * x86-64 code (no FMA contraction). Reference citations are file:line in the
 * reference repository.
 */
#include "rtxllm_oracle.h"

#include <float.h>
#include <math.h>
#include <pthread.h>
#include <stdlib.h>
#include <string.h>

#include "iq_grids.h"

static const uint16_t kIq2sGrid[1024] = {RTXLLM_IQ2S_GRID_VALUES};
static const uint32_t kIq3sGrid[512] = {RTXLLM_IQ3S_GRID_VALUES};

const uint16_t* orc_iq2s_grid(void) { return kIq2sGrid; }
const uint32_t* orc_iq3s_grid(void) { return kIq3sGrid; }

static uint16_t rd16(const uint8_t* p) { return (uint16_t)(p[0] | ((uint16_t)p[1] << 8)); }

static float rdf32(const uint8_t* p) {
  float v;
  memcpy(&v, p, 4);
  return v;
}

/* main.cpp:1086-1098: sign * ldexp(1 + mant/1024, exp - 15); subnormals
 * sign * ldexp(mant, -24); inf kept; any NaN -> +quiet NaN. */
float orc_fp16_to_f32(uint16_t bits) {
  const float sign = (bits & 0x8000u) ? -1.0f : 1.0f;
  const int e = (int)((bits >> 10) & 0x1Fu);
  const int mant = (int)(bits & 0x3FFu);
  if (e == 0) return mant == 0 ? sign * 0.0f : sign * ldexpf((float)mant, -24);
  if (e == 31) return mant == 0 ? sign * INFINITY : NAN;
  return sign * ldexpf(1.0f + (float)mant / 1024.0f, e - 15);
}

/* Python struct.pack('<e') (round half to even); tools/bench/q4k_resident_pack.py:47-48. */
uint16_t orc_f32_to_fp16_rne(float value) {
  if (isnan(value)) return (uint16_t)(signbit(value) ? 0xFE00u : 0x7E00u);
  const double a = fabs((double)value);
  const uint16_t sign = signbit(value) ? 0x8000u : 0u;
  if (a >= 65520.0) return (uint16_t)(sign | 0x7C00u);
  /* Find the binade and scale so the fp16 ulp becomes 1, then round with rint
   * (the default rounding mode is nearest-even). */
  if (a < 6.103515625e-05) { /* subnormal range: ulp = 2^-24 */
    const double q = rint(a * 16777216.0);
    return (uint16_t)(sign | (uint16_t)q);
  }
  int e;
  frexp(a, &e); /* a = f * 2^e, f in [0.5, 1) -> exponent of leading bit is e-1 */
  const double ulp = ldexp(1.0, e - 1 - 10);
  double q = rint(a / ulp); /* in [1024, 2048] */
  int ebits = e - 1 + 15;
  if (q >= 2048.0) {
    q /= 2.0;
    ebits += 1;
  }
  if (ebits >= 31) return (uint16_t)(sign | 0x7C00u);
  return (uint16_t)(sign | (uint16_t)(ebits << 10) | (uint16_t)((uint32_t)q - 1024u));
}

/* main.cpp:1100-1114 (ggml get_scale_min_k4). */
void orc_scale_min_k4(int index, const uint8_t* packed, uint8_t* scale, uint8_t* min_value) {
  if (index < 4) {
    *scale = (uint8_t)(packed[index] & 63u);
    *min_value = (uint8_t)(packed[index + 4] & 63u);
    return;
  }
  *scale = (uint8_t)((packed[index + 4] & 0x0Fu) | ((packed[index - 4] >> 6) << 4));
  *min_value = (uint8_t)((packed[index + 4] >> 4) | ((packed[index] >> 6) << 4));
}

uint32_t orc_payload_bytes(int fmt) {
  switch (fmt) {
    case ORC_Q4K_RAW: return 144u;
    case ORC_Q4K_SPLIT_PREDECODED:
    case ORC_Q4K_SPLIT_HALF:
    case ORC_Q4K_SPLIT_COMPACT:
    case ORC_Q4K_SPLIT_NATIVE: return 128u;
    case ORC_Q5K: return 176u;
    case ORC_IQ2S: return 82u;
    case ORC_IQ3S: return 110u;
    default: return 0u;
  }
}

/* main.cpp:1116-1131 and q4k_resident_pack.py:91-97. */
uint32_t orc_meta_bytes(int fmt) {
  switch (fmt) {
    case ORC_Q4K_SPLIT_PREDECODED: return 64u;
    case ORC_Q4K_SPLIT_HALF: return 32u;
    case ORC_Q4K_SPLIT_COMPACT: return 20u;
    case ORC_Q4K_SPLIT_NATIVE: return 16u;
    default: return 0u;
  }
}

/* main.cpp:1133-1171 (split layouts); the raw 144 B block is the native head
 * followed by the payload (decode_kernels.cu:1946-1953, fused runner main.cpp:871-909). */
static float q4k_value(int fmt, const uint8_t* payload, const uint8_t* meta, uint32_t v) {
  const uint32_t group64 = v >> 6;
  const uint32_t within64 = v & 63u;
  const uint32_t lane = within64 & 31u;
  const int high = within64 >= 32u;
  const uint32_t pair = group64 * 2u + (high ? 1u : 0u);
  const uint8_t packed = payload[group64 * 32u + lane];
  const float quant = (float)(high ? (packed >> 4) : (packed & 0x0Fu));
  switch (fmt) {
    case ORC_Q4K_SPLIT_PREDECODED: {
      const uint8_t* pm = meta + pair * 8u;
      return rdf32(pm) * quant - rdf32(pm + 4);
    }
    case ORC_Q4K_SPLIT_HALF: {
      const uint8_t* pm = meta + pair * 4u;
      return orc_fp16_to_f32(rd16(pm)) * quant - orc_fp16_to_f32(rd16(pm + 2));
    }
    case ORC_Q4K_SPLIT_COMPACT: {
      const float d = orc_fp16_to_f32(rd16(meta));
      const float dmin = orc_fp16_to_f32(rd16(meta + 2));
      return d * (float)meta[4u + pair] * quant - dmin * (float)meta[12u + pair];
    }
    default: { /* native head (split-native, raw) */
      const float d = orc_fp16_to_f32(rd16(meta));
      const float dmin = orc_fp16_to_f32(rd16(meta + 2));
      uint8_t sc, m;
      orc_scale_min_k4((int)pair, meta + 4, &sc, &m);
      return d * (float)sc * quant - dmin * (float)m;
    }
  }
}

/* main.cpp:1231-1259. */
static float q5k_value(const uint8_t* block, uint32_t v) {
  const float d = orc_fp16_to_f32(rd16(block));
  const float dmin = orc_fp16_to_f32(rd16(block + 2));
  const uint8_t* scales = block + 4;
  const uint8_t* qh = block + 16;
  const uint8_t* qs = block + 48;
  const uint32_t group64 = v >> 6;
  const uint32_t within64 = v & 63u;
  const uint32_t lane = within64 & 31u;
  const int high = within64 >= 32u;
  uint8_t sc, m;
  orc_scale_min_k4((int)(group64 * 2u + (high ? 1u : 0u)), scales, &sc, &m);
  const uint8_t packed = qs[group64 * 32u + lane];
  const uint8_t low = high ? (uint8_t)(packed >> 4) : (uint8_t)(packed & 0x0Fu);
  const uint8_t mask = (uint8_t)((high ? 2u : 1u) << (group64 * 2u));
  const uint8_t quant = (uint8_t)(low + ((qh[lane] & mask) ? 16u : 0u));
  return d * (float)sc * (float)quant - dmin * (float)m;
}

/* main.cpp:1173-1194. */
static float iq2s_value(const uint8_t* block, uint32_t v) {
  const uint32_t ib32 = v >> 5;
  const uint32_t within32 = v & 31u;
  const uint32_t group = within32 >> 3;
  const uint32_t lane = within32 & 7u;
  const float d = orc_fp16_to_f32(rd16(block));
  const uint8_t* qs = block + 2;
  const uint8_t* qh = block + 66;
  const uint8_t* scales = block + 74;
  const uint32_t go = ib32 * 4u + group;
  const uint32_t idx = qs[go] | (((uint32_t)qh[ib32] << (8u - 2u * group)) & 0x300u);
  const uint32_t grid = 2u * ((kIq2sGrid[idx] >> (2u * lane)) & 3u) + 1u;
  const uint32_t nib = group < 2u ? (scales[ib32] & 0x0Fu) : (uint32_t)(scales[ib32] >> 4);
  const float scale = d * (0.5f + (float)nib) * 0.25f;
  const int neg = (qs[32u + go] & (1u << lane)) != 0u;
  return scale * (float)grid * (neg ? -1.0f : 1.0f);
}

/* main.cpp:1196-1221. */
static float iq3s_value(const uint8_t* block, uint32_t v) {
  const uint32_t ib32 = v >> 5;
  const uint32_t within32 = v & 31u;
  const uint32_t group = within32 >> 3;
  const uint32_t lane = within32 & 7u;
  const uint32_t pair = lane >> 2;
  const uint32_t grid_lane = lane & 3u;
  const float d = orc_fp16_to_f32(rd16(block));
  const uint8_t* qs = block + 2;
  const uint8_t* qh = block + 66;
  const uint8_t* signs = block + 74;
  const uint8_t* scales = block + 106;
  const uint32_t sel = ib32 * 8u + group * 2u + pair;
  const uint32_t hb = ((uint32_t)qh[ib32] >> (2u * group + pair)) & 1u;
  const uint32_t idx = qs[sel] | (hb << 8);
  const uint32_t grid = (kIq3sGrid[idx] >> (8u * grid_lane)) & 0xFFu;
  const uint32_t nib = (ib32 & 1u) == 0u ? (scales[ib32 >> 1] & 0x0Fu) : (uint32_t)(scales[ib32 >> 1] >> 4);
  const float scale = d * (float)(1u + 2u * nib);
  const int neg = (signs[ib32 * 4u + group] & (1u << lane)) != 0u;
  return scale * (float)grid * (neg ? -1.0f : 1.0f);
}

float orc_dequant_value(int fmt, const uint8_t* payload_block, const uint8_t* meta_block, uint32_t v) {
  switch (fmt) {
    case ORC_Q4K_RAW: return q4k_value(ORC_Q4K_SPLIT_NATIVE, payload_block + 16, payload_block, v);
    case ORC_Q4K_SPLIT_PREDECODED:
    case ORC_Q4K_SPLIT_HALF:
    case ORC_Q4K_SPLIT_COMPACT:
    case ORC_Q4K_SPLIT_NATIVE: return q4k_value(fmt, payload_block, meta_block, v);
    case ORC_Q5K: return q5k_value(payload_block, v);
    case ORC_IQ2S: return iq2s_value(payload_block, v);
    case ORC_IQ3S: return iq3s_value(payload_block, v);
    default: return NAN;
  }
}

static const uint8_t* blk_ptr(const uint8_t* base, uint32_t bytes, size_t index) {
  return base ? base + index * (size_t)bytes : NULL;
}

void orc_dequant(int fmt, const uint8_t* payload, const uint8_t* meta, uint32_t rows, uint32_t cols,
                 float* out) {
  const uint32_t bpr = cols / 256u;
  const uint32_t pb = orc_payload_bytes(fmt), mb = orc_meta_bytes(fmt);
  for (uint32_t r = 0; r < rows; ++r)
    for (uint32_t b = 0; b < bpr; ++b) {
      const size_t bi = (size_t)r * bpr + b;
      const uint8_t* p = blk_ptr(payload, pb, bi);
      const uint8_t* m = blk_ptr(meta, mb, bi);
      for (uint32_t v = 0; v < 256u; ++v) out[(size_t)r * cols + b * 256u + v] = orc_dequant_value(fmt, p, m, v);
    }
}

/* ---- threaded row loops ------------------------------------------------- */

typedef struct {
  int fmt;
  const uint8_t *payload, *meta;
  const float* x;
  uint32_t cols, r0, r1;
  float* y32;
  double* y64;
} mv_job;

/* main.cpp:1266-1309: per row, blocks in order, values in order, acc += w * x. */
static void* mv_worker(void* arg) {
  const mv_job* j = (const mv_job*)arg;
  const uint32_t bpr = j->cols / 256u;
  const uint32_t pb = orc_payload_bytes(j->fmt), mb = orc_meta_bytes(j->fmt);
  for (uint32_t r = j->r0; r < j->r1; ++r) {
    float acc = 0.0f;
    double acc64 = 0.0;
    for (uint32_t b = 0; b < bpr; ++b) {
      const size_t bi = (size_t)r * bpr + b;
      const uint8_t* p = blk_ptr(j->payload, pb, bi);
      const uint8_t* m = blk_ptr(j->meta, mb, bi);
      const float* xb = j->x + (size_t)b * 256u;
      if (j->y32) {
        for (uint32_t v = 0; v < 256u; ++v) acc += orc_dequant_value(j->fmt, p, m, v) * xb[v];
      } else {
        for (uint32_t v = 0; v < 256u; ++v) acc64 += (double)orc_dequant_value(j->fmt, p, m, v) * (double)xb[v];
      }
    }
    if (j->y32) j->y32[r] = acc;
    else j->y64[r] = acc64;
  }
  return NULL;
}

static void run_rows(int fmt, const uint8_t* payload, const uint8_t* meta, const float* x, uint32_t rows,
                     uint32_t cols, float* y32, double* y64, int nthreads) {
  if (nthreads < 1) nthreads = 1;
  if ((uint32_t)nthreads > rows) nthreads = rows ? (int)rows : 1;
  mv_job jobs[256];
  pthread_t th[256];
  if (nthreads > 256) nthreads = 256;
  for (int t = 0; t < nthreads; ++t) {
    jobs[t].fmt = fmt;
    jobs[t].payload = payload;
    jobs[t].meta = meta;
    jobs[t].x = x;
    jobs[t].cols = cols;
    jobs[t].r0 = (uint32_t)((uint64_t)rows * t / nthreads);
    jobs[t].r1 = (uint32_t)((uint64_t)rows * (t + 1) / nthreads);
    jobs[t].y32 = y32;
    jobs[t].y64 = y64;
  }
  if (nthreads == 1) {
    mv_worker(&jobs[0]);
    return;
  }
  for (int t = 0; t < nthreads; ++t) pthread_create(&th[t], NULL, mv_worker, &jobs[t]);
  for (int t = 0; t < nthreads; ++t) pthread_join(th[t], NULL);
}

void orc_matvec_f32(int fmt, const uint8_t* payload, const uint8_t* meta, const float* x, uint32_t rows,
                    uint32_t cols, float* y, int nthreads) {
  run_rows(fmt, payload, meta, x, rows, cols, y, NULL, nthreads);
}

void orc_matvec_f64(int fmt, const uint8_t* payload, const uint8_t* meta, const float* x, uint32_t rows,
                    uint32_t cols, double* y, int nthreads) {
  run_rows(fmt, payload, meta, x, rows, cols, NULL, y, nthreads);
}

/* q4k_resident_pack.py:100-145: payload = bytes 16..143 of each block; metadata
 * per policy (predecoded: f32 (d*sc, dmin*m) x 8; half: the same products as fp16
 * RNE; compact: raw d, dmin + unpacked sc[8], m[8]; native: bytes 0..15). The
 * products d*sc and dmin*m have at most 17 significant bits, so computing them in
 * float (here) or double (the Python packer) gives the same value. */
void orc_q4k_split(int fmt, const uint8_t* raw, size_t n_blocks, uint8_t* payload, uint8_t* meta) {
  const uint32_t mb = orc_meta_bytes(fmt);
  for (size_t b = 0; b < n_blocks; ++b) {
    const uint8_t* blk = raw + b * 144u;
    memcpy(payload + b * 128u, blk + 16, 128);
    uint8_t* m = meta + b * mb;
    if (fmt == ORC_Q4K_SPLIT_NATIVE) {
      memcpy(m, blk, 16);
      continue;
    }
    if (fmt == ORC_Q4K_SPLIT_COMPACT) {
      memcpy(m, blk, 4);
      for (int i = 0; i < 8; ++i) orc_scale_min_k4(i, blk + 4, &m[4 + i], &m[12 + i]);
      continue;
    }
    const float d = orc_fp16_to_f32(rd16(blk));
    const float dmin = orc_fp16_to_f32(rd16(blk + 2));
    for (int i = 0; i < 8; ++i) {
      uint8_t sc, mn;
      orc_scale_min_k4(i, blk + 4, &sc, &mn);
      const float s = d * (float)sc;
      const float mm = dmin * (float)mn;
      if (fmt == ORC_Q4K_SPLIT_PREDECODED) {
        memcpy(m + i * 8, &s, 4);
        memcpy(m + i * 8 + 4, &mm, 4);
      } else {
        const uint16_t hs = orc_f32_to_fp16_rne(s), hm = orc_f32_to_fp16_rne(mm);
        m[i * 4 + 0] = (uint8_t)(hs & 0xFF);
        m[i * 4 + 1] = (uint8_t)(hs >> 8);
        m[i * 4 + 2] = (uint8_t)(hm & 0xFF);
        m[i * 4 + 3] = (uint8_t)(hm >> 8);
      }
    }
  }
}

void orc_stage_activation(const float* x, const float* weight, uint32_t cols, int8_t* h, int8_t* m, int8_t* l,
                          float* scale, float* sum) {
  for (uint32_t g = 0; g < cols / 16u; ++g) {
    float v[16];
    float mx = 0.0f;
    int nan = 0;
    for (int j = 0; j < 16; ++j) {
      v[j] = weight ? x[16u * g + j] * weight[16u * g + j] : x[16u * g + j];
      const float a = fabsf(v[j]);
      if (isnan(v[j])) nan = 1;
      else if (a > mx) mx = a;
    }
    /* s = 2^(e - 22) with mx = f 2^e, f in [0.5, 1); X = rint(v 2^(22 - e)) */
    const int finite = !nan && mx <= FLT_MAX;
    int e = 0;
    if (finite && mx > 0.0f) (void)frexpf(mx, &e);
    scale[g] = nan ? NAN : (!finite ? INFINITY : (mx > 0.0f ? ldexpf(1.0f, e - 22) : 0.0f));
    int total = 0;
    for (int j = 0; j < 16; ++j) {
      const int X = finite ? (int)rintf(ldexpf(v[j], 22 - e)) : 0; /* |X| <= 2^22 */
      /* balanced base-256 digits: L, M in [-128, 127], X = 65536 H + 256 M + L */
      const int L = X - 256 * (int)floor((X + 128) / 256.0);
      const int X1 = (X - L) / 256;
      const int M = X1 - 256 * (int)floor((X1 + 128) / 256.0);
      h[16u * g + j] = (int8_t)((X1 - M) / 256);
      m[16u * g + j] = (int8_t)M;
      l[16u * g + j] = (int8_t)L;
      total += X;
    }
    sum[g] = scale[g] * (float)total;
  }
}

typedef struct {
  int fmt;
  const uint8_t *payload, *meta;
  const int8_t *h, *m, *l;
  const float* scale;
  uint32_t cols, r0, r1;
  double* y;
} st_job;

static void* st_worker(void* arg) {
  const st_job* j = (const st_job*)arg;
  const uint32_t bpr = j->cols / 256u;
  const uint32_t pb = orc_payload_bytes(j->fmt), mb = orc_meta_bytes(j->fmt);
  for (uint32_t r = j->r0; r < j->r1; ++r) {
    double acc = 0.0;
    for (uint32_t b = 0; b < bpr; ++b) {
      const size_t bi = (size_t)r * bpr + b;
      const uint8_t* p = blk_ptr(j->payload, pb, bi);
      const uint8_t* mt = blk_ptr(j->meta, mb, bi);
      for (uint32_t v = 0; v < 256u; ++v) {
        const uint32_t c = b * 256u + v;
        const double X = 65536.0 * j->h[c] + 256.0 * j->m[c] + j->l[c];
        acc += (double)orc_dequant_value(j->fmt, p, mt, v) * ((double)j->scale[c / 16u] * X);
      }
    }
    j->y[r] = acc;
  }
  return NULL;
}

void orc_matvec_staged_f64(int fmt, const uint8_t* payload, const uint8_t* meta, const int8_t* h, const int8_t* m,
                           const int8_t* l, const float* scale, uint32_t rows, uint32_t cols, double* y,
                           int nthreads) {
  if (nthreads < 1) nthreads = 1;
  if (nthreads > 64) nthreads = 64;
  if ((uint32_t)nthreads > rows) nthreads = rows ? (int)rows : 1;
  st_job jobs[64];
  pthread_t th[64];
  for (int t = 0; t < nthreads; ++t) {
    st_job jb = {fmt, payload, meta, h, m, l, scale, cols, (uint32_t)((uint64_t)rows * t / nthreads),
                 (uint32_t)((uint64_t)rows * (t + 1) / nthreads), y};
    jobs[t] = jb;
  }
  if (nthreads == 1) {
    st_worker(&jobs[0]);
    return;
  }
  for (int t = 0; t < nthreads; ++t) pthread_create(&th[t], NULL, st_worker, &jobs[t]);
  for (int t = 0; t < nthreads; ++t) pthread_join(th[t], NULL);
}

/* main.cpp:1311-1322 and decode_kernels.cu:2993-3031. */
uint32_t orc_argmax(const float* y, uint32_t n) {
  float best = -FLT_MAX;
  uint32_t bi = 0;
  for (uint32_t r = 0; r < n; ++r) {
    const float v = y[r];
    if (v > best || (v == best && r < bi)) {
      best = v;
      bi = r;
    }
  }
  return bi;
}

/* main.cpp:1324-1341. */
void orc_kv_side_write(const float* y, uint32_t rows, float* kv, uint32_t kv_words, uint32_t page_words,
                       uint32_t active_pages, uint32_t token) {
  if (kv_words == 0u || page_words == 0u) return;
  const uint32_t active = rows < active_pages ? rows : active_pages;
  for (uint32_t r = 0; r < active; ++r) {
    const size_t base = (size_t)r * page_words;
    const size_t off = (token + r) % page_words;
    kv[(base + off) % kv_words] = y[r];
  }
}

/* main.cpp:1363-1382: inv = 1/sqrt(sum(y^2)/rows + eps), float sequential sum. */
static float inv_rms(const float* y, uint32_t n, float eps) {
  float s = 0.0f;
  for (uint32_t i = 0; i < n; ++i) s += y[i] * y[i];
  const float mean = s / (float)n;
  return 1.0f / sqrtf(mean + eps);
}

static float silu_f(float v) {
  const float sig = 1.0f / (1.0f + expf(-v));
  return v * sig;
}

void orc_rmsnorm_feedback(const float* logits, uint32_t rows, float* act, uint32_t cols, float eps) {
  if (rows == 0u) return;
  const float inv = inv_rms(logits, rows, eps);
  for (uint32_t c = 0; c < cols; ++c) act[c] = logits[c % rows] * inv;
}

/* main.cpp:1384-1405. */
void orc_silu_rmsnorm_feedback(const float* logits, uint32_t rows, float* act, uint32_t cols, float eps) {
  if (rows == 0u) return;
  const float inv = inv_rms(logits, rows, eps);
  for (uint32_t c = 0; c < cols; ++c) act[c] = silu_f(logits[c % rows] * inv);
}

/* main.cpp:1407-1433. */
void orc_rmsnorm_feedback_with_silu_cache(const float* logits, uint32_t rows, float* act, float* silu_cache,
                                          uint32_t cols, float eps) {
  if (rows == 0u) return;
  const float inv = inv_rms(logits, rows, eps);
  for (uint32_t c = 0; c < cols; ++c) {
    const float n = logits[c % rows] * inv;
    act[c] = n;
    silu_cache[c] = silu_f(n);
  }
}

/* main.cpp:1435-1457. */
void orc_gated_silu_rmsnorm_feedback(const float* logits, uint32_t rows, const float* silu_cache,
                                     uint32_t cache_cols, float* act, uint32_t cols, float eps) {
  if (rows == 0u || cache_cols == 0u) return;
  const float inv = inv_rms(logits, rows, eps);
  for (uint32_t c = 0; c < cols; ++c) act[c] = silu_cache[c % cache_cols] * (logits[c % rows] * inv);
}

/* main.cpp:1459-1488. */
void orc_rmsnorm_cache(const float* logits, uint32_t rows, float* cache, uint32_t cache_cols, float eps,
                       int apply_silu, int accumulate) {
  if (rows == 0u) return;
  const float inv = inv_rms(logits, rows, eps);
  for (uint32_t c = 0; c < cache_cols; ++c) {
    float v = logits[c % rows] * inv;
    if (apply_silu) v = silu_f(v);
    cache[c] = accumulate ? cache[c] + v : v;
  }
}

/* decode_kernels.cu:263-289 (no CPU twin in one piece: main.cpp:1459-1503 does
 * the up-cache update then the gated product). */
void orc_rmsnorm_cache_and_gated_product(const float* logits, uint32_t rows, const float* gate, float* up,
                                         float* act, uint32_t cache_cols, uint32_t out_cols, float eps,
                                         int accumulate) {
  if (rows == 0u || cache_cols == 0u) return;
  const float inv = inv_rms(logits, rows, eps);
  for (uint32_t c = 0; c < out_cols; ++c) {
    const float v = logits[c % rows] * inv;
    const float u = accumulate ? up[c] + v : v;
    up[c] = u;
    act[c] = gate[c] * u;
  }
}

/* main.cpp:1744-1758 (pair rotation; the angle is supplied by the caller). */
void orc_rope_rotate_pair(float e, float o, float angle, float* out_e, float* out_o) {
  const float s = sinf(angle), c = cosf(angle);
  *out_e = e * c - o * s;
  *out_o = e * s + o * c;
}

/* ---- Llama-layer math (textbook; no counterpart in the reference) ---------- */

void orc_rmsnorm_weighted(const float* x, const float* w, uint32_t n, float eps, float* out) {
  const float inv = inv_rms(x, n, eps);
  for (uint32_t i = 0; i < n; ++i) out[i] = (x[i] * inv) * w[i];
}

/* inv_freq[i] = theta^(-2i/head_dim), computed in double and rounded once. */
void orc_rope_inv_freq(uint32_t head_dim, double theta, float* inv_freq) {
  for (uint32_t i = 0; i < head_dim / 2u; ++i) inv_freq[i] = (float)pow(theta, -2.0 * (double)i / (double)head_dim);
}

/* Adjacent pairs (2i, 2i+1) of each head rotated by angle pos * inv_freq[i]. */
void orc_rope(float* vec, uint32_t n_heads, uint32_t head_dim, const float* inv_freq, uint32_t pos) {
  for (uint32_t h = 0; h < n_heads; ++h)
    for (uint32_t i = 0; i < head_dim / 2u; ++i) {
      float* p = vec + (size_t)h * head_dim + 2u * i;
      const float angle = (float)pos * inv_freq[i];
      orc_rope_rotate_pair(p[0], p[1], angle, &p[0], &p[1]);
    }
}

void orc_silu_mul(const float* gate, const float* up, uint32_t n, float* out) {
  for (uint32_t i = 0; i < n; ++i) out[i] = silu_f(gate[i]) * up[i];
}

void orc_embed_q5k(const uint8_t* table, uint32_t cols, uint32_t token, float* out) {
  const uint32_t bpr = cols / 256u;
  for (uint32_t c = 0; c < cols; ++c) {
    const uint8_t* blk = table + ((size_t)token * bpr + c / 256u) * 176u;
    out[c] = q5k_value(blk, c & 255u);
  }
}

static size_t kv_index(const orc_kv_cache* kv, uint32_t pos, uint32_t head) {
  const uint32_t page = (uint32_t)kv->block_table[pos / kv->page_size];
  const uint32_t slot = pos % kv->page_size;
  return (((size_t)page * kv->n_kv_heads + head) * kv->page_size + slot) * kv->head_dim;
}

void orc_kv_append(const orc_kv_cache* kv, uint32_t pos, const float* k, const float* v) {
  for (uint32_t h = 0; h < kv->n_kv_heads; ++h) {
    const size_t base = kv_index(kv, pos, h);
    for (uint32_t d = 0; d < kv->head_dim; ++d) {
      kv->k_pages[base + d] = orc_f32_to_fp16_rne(k[h * kv->head_dim + d]);
      kv->v_pages[base + d] = orc_f32_to_fp16_rne(v[h * kv->head_dim + d]);
    }
  }
}

/* Causal decode attention of one query over positions 0..pos; query head h reads
 * KV head h / (n_heads / n_kv_heads); scale 1/sqrt(head_dim); softmax with the
 * max subtracted. */
void orc_attention_decode(const orc_kv_cache* kv, const float* q, uint32_t n_heads, uint32_t pos, float* out) {
  const uint32_t hd = kv->head_dim;
  const uint32_t group = n_heads / kv->n_kv_heads;
  const float scale = 1.0f / sqrtf((float)hd);
  float* scores = (float*)malloc(sizeof(float) * (pos + 1u));
  float* acc = (float*)malloc(sizeof(float) * hd);
  for (uint32_t h = 0; h < n_heads; ++h) {
    const uint32_t kvh = h / group;
    const float* qh = q + (size_t)h * hd;
    float m = -INFINITY;
    for (uint32_t t = 0; t <= pos; ++t) {
      const uint16_t* kr = kv->k_pages + kv_index(kv, t, kvh);
      float s = 0.0f;
      for (uint32_t d = 0; d < hd; ++d) s += qh[d] * orc_fp16_to_f32(kr[d]);
      s *= scale;
      scores[t] = s;
      if (s > m) m = s;
    }
    float l = 0.0f;
    for (uint32_t d = 0; d < hd; ++d) acc[d] = 0.0f;
    for (uint32_t t = 0; t <= pos; ++t) {
      const float p = expf(scores[t] - m);
      l += p;
      const uint16_t* vr = kv->v_pages + kv_index(kv, t, kvh);
      for (uint32_t d = 0; d < hd; ++d) acc[d] += p * orc_fp16_to_f32(vr[d]);
    }
    for (uint32_t d = 0; d < hd; ++d) out[(size_t)h * hd + d] = acc[d] / l;
  }
  free(scores);
  free(acc);
}

static void layer_forward(const orc_layer_weights* w, const orc_layer_shape* s, orc_kv_cache* kv, uint32_t pos,
                          float* h, int nthreads, int append) {
  const uint32_t H = s->hidden, qd = s->n_heads * s->head_dim, kvd = s->n_kv_heads * s->head_dim;
  float* xn = (float*)malloc(sizeof(float) * (H > s->ffn ? H : s->ffn));
  float* q = (float*)malloc(sizeof(float) * qd);
  float* k = (float*)malloc(sizeof(float) * kvd);
  float* v = (float*)malloc(sizeof(float) * kvd);
  float* att = (float*)malloc(sizeof(float) * qd);
  float* o = (float*)malloc(sizeof(float) * H);
  float* g = (float*)malloc(sizeof(float) * s->ffn);
  float* u = (float*)malloc(sizeof(float) * s->ffn);

  orc_rmsnorm_weighted(h, w->attn_norm, H, s->eps, xn);
  orc_matvec_f32(w->fmt_q, w->wq, w->wq_meta, xn, qd, H, q, nthreads);
  orc_matvec_f32(w->fmt_k, w->wk, w->wk_meta, xn, kvd, H, k, nthreads);
  orc_matvec_f32(w->fmt_v, w->wv, w->wv_meta, xn, kvd, H, v, nthreads);
  orc_rope(q, s->n_heads, s->head_dim, s->inv_freq, pos);
  orc_rope(k, s->n_kv_heads, s->head_dim, s->inv_freq, pos);
  if (append) orc_kv_append(kv, pos, k, v);
  orc_attention_decode(kv, q, s->n_heads, pos, att);
  orc_matvec_f32(w->fmt_o, w->wo, w->wo_meta, att, H, qd, o, nthreads);
  for (uint32_t i = 0; i < H; ++i) h[i] += o[i];

  orc_rmsnorm_weighted(h, w->ffn_norm, H, s->eps, xn);
  orc_matvec_f32(w->fmt_gate, w->wgate, w->wgate_meta, xn, s->ffn, H, g, nthreads);
  orc_matvec_f32(w->fmt_up, w->wup, w->wup_meta, xn, s->ffn, H, u, nthreads);
  orc_silu_mul(g, u, s->ffn, g);
  orc_matvec_f32(w->fmt_down, w->wdown, w->wdown_meta, g, H, s->ffn, o, nthreads);
  for (uint32_t i = 0; i < H; ++i) h[i] += o[i];

  free(xn);
  free(q);
  free(k);
  free(v);
  free(att);
  free(o);
  free(g);
  free(u);
}

void orc_layer_forward(const orc_layer_weights* w, const orc_layer_shape* s, orc_kv_cache* kv, uint32_t pos,
                       float* h, int nthreads) {
  layer_forward(w, s, kv, pos, h, nthreads, 1);
}

void orc_layer_forward_given_kv(const orc_layer_weights* w, const orc_layer_shape* s, orc_kv_cache* kv,
                                uint32_t pos, float* h, int nthreads) {
  layer_forward(w, s, kv, pos, h, nthreads, 0);
}
