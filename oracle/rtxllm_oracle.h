/* CPU oracle for the decode hot path -- TEST INFRASTRUCTURE ONLY.
 *
 * A plain-C restatement of the reference runtime's CPU reference gate
 * (runtime/apps/mixed_sequence_benchmark_runner/main.cpp:1075-1503 and the
 * probes' reference paths), plus textbook restatements of the Llama-layer math
 * the reference does not contain (weighted RMSNorm, RoPE with a theta schedule,
 * SiLU-gate multiply, GQA attention over a paged fp16 KV cache, Q5_K embedding
 * gather). Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg
 * may load it, and only as the checker / the timed CPU baseline. The product
 * never calls it.
 *
 * Pinning status per function is listed in oracle/README.md.
 */
#ifndef RTXLLM_ORACLE_H
#define RTXLLM_ORACLE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Formats: same numbering as the product's enum rtxllm_format. */
enum {
  ORC_Q4K_RAW = 0,
  ORC_Q4K_SPLIT_PREDECODED = 1,
  ORC_Q4K_SPLIT_HALF = 2,
  ORC_Q4K_SPLIT_COMPACT = 3,
  ORC_Q4K_SPLIT_NATIVE = 4,
  ORC_Q5K = 5,
  ORC_IQ2S = 6,
  ORC_IQ3S = 7
};

float orc_fp16_to_f32(uint16_t bits);
uint16_t orc_f32_to_fp16_rne(float value);
void orc_scale_min_k4(int index, const uint8_t* packed, uint8_t* scale, uint8_t* min_value);
const uint16_t* orc_iq2s_grid(void);
const uint32_t* orc_iq3s_grid(void);

uint32_t orc_payload_bytes(int fmt);
uint32_t orc_meta_bytes(int fmt);

/* Value v (0..255) of block `block` of a tensor. For split layouts payload points
 * at the 128 B payload block and meta at its metadata; otherwise meta is unused. */
float orc_dequant_value(int fmt, const uint8_t* payload_block, const uint8_t* meta_block, uint32_t v);

/* Full tensor dequant to fp32 [rows][cols]. */
void orc_dequant(int fmt, const uint8_t* payload, const uint8_t* meta, uint32_t rows, uint32_t cols,
                 float* out);

/* y = W x; fp32, sequential accumulation over columns per row, as the reference
 * gate does. nthreads > 1 splits rows across threads (bit-identical output). */
void orc_matvec_f32(int fmt, const uint8_t* payload, const uint8_t* meta, const float* x,
                    uint32_t rows, uint32_t cols, float* y, int nthreads);
/* Same product accumulated in double (closed-form check). */
void orc_matvec_f64(int fmt, const uint8_t* payload, const uint8_t* meta, const float* x,
                    uint32_t rows, uint32_t cols, double* y, int nthreads);

/* Q4_K resident-pack split: raw 144 B blocks -> 128 B payload + metadata of fmt. */
void orc_q4k_split(int fmt, const uint8_t* raw_blocks, size_t n_blocks, uint8_t* payload,
                   uint8_t* meta);

/* Activation staging of the product's integer-dot matvec (its own design, no
 * reference counterpart): per 16-value group, m = max|v| (NaN ignored) = f 2^e
 * with f in [0.5, 1), s = 2^(e - 22), X = rint(v 2^(22 - e)) (|X| <= 2^22),
 * digits X = 65536 H + 256 M + L with M, L in [-128, 127], sum = s * sum(X).
 * A group holding a NaN gets s = NaN, one with an infinite maximum s = inf,
 * both zero digits; an all-zero group s = 0. v = x * weight when weight is
 * non-null. */
void orc_stage_activation(const float* x, const float* weight, uint32_t cols, int8_t* h, int8_t* m, int8_t* l,
                          float* scale, float* sum);
/* y = W x_hat with x_hat = s * X (the staged activation), accumulated in double. */
void orc_matvec_staged_f64(int fmt, const uint8_t* payload, const uint8_t* meta, const int8_t* h,
                           const int8_t* m, const int8_t* l, const float* scale, uint32_t rows, uint32_t cols,
                           double* y, int nthreads);

/* Greedy token: lowest index among the maxima; start (-FLT_MAX, 0). */
uint32_t orc_argmax(const float* y, uint32_t n);
/* KV side-write of the *_decode launchers. */
void orc_kv_side_write(const float* y, uint32_t rows, float* kv, uint32_t kv_words,
                       uint32_t page_words, uint32_t active_pages, uint32_t token);

/* Feedback family of the reference runner (unweighted RMSNorm over rows logits). */
void orc_rmsnorm_feedback(const float* logits, uint32_t rows, float* act, uint32_t cols, float eps);
void orc_silu_rmsnorm_feedback(const float* logits, uint32_t rows, float* act, uint32_t cols,
                               float eps);
void orc_rmsnorm_feedback_with_silu_cache(const float* logits, uint32_t rows, float* act,
                                          float* silu_cache, uint32_t cols, float eps);
void orc_gated_silu_rmsnorm_feedback(const float* logits, uint32_t rows, const float* silu_cache,
                                     uint32_t cache_cols, float* act, uint32_t cols, float eps);
void orc_rmsnorm_cache(const float* logits, uint32_t rows, float* cache, uint32_t cache_cols,
                       float eps, int apply_silu, int accumulate);
void orc_rmsnorm_cache_and_gated_product(const float* logits, uint32_t rows, const float* gate,
                                         float* up, float* act, uint32_t cache_cols,
                                         uint32_t out_cols, float eps, int accumulate);
void orc_rope_rotate_pair(float e, float o, float angle, float* out_e, float* out_o);

/* Llama-layer math. */
void orc_rmsnorm_weighted(const float* x, const float* w, uint32_t n, float eps, float* out);
void orc_rope_inv_freq(uint32_t head_dim, double theta, float* inv_freq);
void orc_rope(float* vec, uint32_t n_heads, uint32_t head_dim, const float* inv_freq, uint32_t pos);
void orc_silu_mul(const float* gate, const float* up, uint32_t n, float* out);
void orc_embed_q5k(const uint8_t* table, uint32_t cols, uint32_t token, float* out);

/* Paged fp16 KV cache: page p holds k (and v) as [n_kv_heads][page_size][head_dim].
 * block_table maps logical page -> physical page. */
typedef struct {
  uint16_t* k_pages;
  uint16_t* v_pages;
  const int32_t* block_table;
  uint32_t page_size;
  uint32_t n_kv_heads;
  uint32_t head_dim;
} orc_kv_cache;

void orc_kv_append(const orc_kv_cache* kv, uint32_t pos, const float* k, const float* v);
void orc_attention_decode(const orc_kv_cache* kv, const float* q, uint32_t n_heads, uint32_t pos,
                          float* out);

/* One decoder layer on hidden state h (in place), batch 1, at position pos. */
typedef struct {
  int fmt_q, fmt_k, fmt_v, fmt_o, fmt_gate, fmt_up, fmt_down;
  const uint8_t *wq, *wq_meta, *wk, *wk_meta, *wv, *wv_meta, *wo, *wo_meta;
  const uint8_t *wgate, *wgate_meta, *wup, *wup_meta, *wdown, *wdown_meta;
  const float* attn_norm;
  const float* ffn_norm;
} orc_layer_weights;

typedef struct {
  uint32_t hidden, n_heads, n_kv_heads, head_dim, ffn;
  float eps;
  const float* inv_freq;
} orc_layer_shape;

void orc_layer_forward(const orc_layer_weights* w, const orc_layer_shape* s, orc_kv_cache* kv,
                       uint32_t pos, float* h, int nthreads);
/* The same layer with the cache taken as given: the K / V of position pos are
 * already in it (no append), so a caller can run the layer on exactly the
 * cache state another implementation wrote (its own fp16 rounding of k and v). */
void orc_layer_forward_given_kv(const orc_layer_weights* w, const orc_layer_shape* s, orc_kv_cache* kv,
                                uint32_t pos, float* h, int nthreads);

#ifdef __cplusplus
}
#endif

#endif
