/* C-ABI of the MI355X Llama decode runner (batch 1, or 2..8 sequences): one
 * resident VRAM arena holding every layer's packs, the fp16 paged KV cache and
 * the workspace; one decode step = embedding gather, per layer {fused qkv
 * matvec + RoPE + KV append, split-context GQA attention, o matvec + residual
 * + ffn-norm staging, fused gate/up matvec + SiLU-gate, down matvec + residual
 * + next-norm staging}, final norm + LM head + greedy argmax; replayable as one
 * hipGraph. A batch step runs every sequence through the same weights once,
 * on the matrix cores (each sequence with its own token, position and KV
 * pages).
 *
 * No counterpart in the reference: its layer-slice runner
 * (runtime/apps/mixed_sequence_benchmark_runner/main.cpp:3136-5818) drives
 * synthetic stages of one Qwen3.6 layer; this runner keeps its structure
 * (arena upload, launch sequence, graph capture, replay with the token read
 * back) for a real Llama decode step. All entry points return hipSuccess or a
 * hipError_t; hipErrorInvalidValue for rejected configurations. */
#ifndef RTXLLM_LLAMA_H
#define RTXLLM_LLAMA_H

#include <hip/hip_runtime_api.h>
#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef struct {
  uint32_t hidden;     /* model width, % 256 == 0, <= 16384 */
  uint32_t n_heads;    /* query heads of 128 dims */
  uint32_t n_kv_heads; /* kv heads (n_heads % n_kv_heads == 0, group <= 8) */
  uint32_t ffn;        /* FFN width, % 256 == 0 */
  uint32_t vocab;
  uint32_t n_layers;
  uint32_t max_ctx;    /* KV positions per sequence, % page_size == 0 */
  uint32_t page_size;  /* positions per KV page */
  float rope_theta;
  float rms_eps;
  int fmt_qkv;         /* formats (enum rtxllm_format) of the stacked q|k|v, o, */
  int fmt_o;           /* interleaved gate/up, down and LM-head tensors; the */
  int fmt_gate_up;     /* embedding table is Q5_K */
  int fmt_down;
  int fmt_lm_head;
  uint32_t batch;      /* sequences per step, 0 or 1: batch 1; 2..8: the batch
                          step (hidden % 512 == 0 and <= 4096, n_heads % 4 == 0,
                          ffn % 512 == 0) */
} rtxllm_llama_config;

typedef struct rtxllm_llama rtxllm_llama;

/* Allocate the arena on the current device (one hipMalloc) and set up the
 * RoPE table, identity KV block tables, token = 0, pos = 0. Strict admission
 * first (include/rtxllm/admission.h): hipErrorOutOfMemory when weights + KV
 * + workspace + graph memory exceed the device's free bytes. */
hipError_t rtxllm_llama_create(const rtxllm_llama_config* cfg, rtxllm_llama** out);

/* The admission decision rtxllm_llama_create would make, without allocating:
 * *admitted = 1 or 0, the bytes the model needs and the device bytes it is
 * measured against (free bytes less guard_bytes: the reference runner's
 * --wddm-guard-mib, runtime/core/scheduler/admission.h:10-65), and the decision's reason
 * (at most reason_len bytes with the NUL). hipErrorInvalidValue for a config
 * create refuses. */
hipError_t rtxllm_llama_admission(const rtxllm_llama_config* cfg, size_t guard_bytes, int* admitted,
                                  size_t* required_bytes, size_t* usable_bytes, char* reason, size_t reason_len);
void rtxllm_llama_destroy(rtxllm_llama* m);

/* Device pointer (and size) of a named region, or NULL. Per layer: "qkv",
 * "qkv_meta", "o", "o_meta", "gate_up", "gate_up_meta", "down", "down_meta"
 * (meta regions exist for Q4_K split layouts only), "attn_norm", "ffn_norm",
 * "k_cache", "v_cache" (fp16 [pages][n_kv][page_size][128]), "block_table"
 * (int32 [max_ctx / page_size]). Global (layer ignored): "embed", "lm_head",
 * "lm_head_meta", "out_norm", "h", "q", "att", "act", "logits", "token", "pos",
 * "status",
 * and the work buffers "xq" / "xq_att" (staged activations), "sumsq",
 * "attn_partials", "argkeys", "inv_freq", "rope" ((cos, sin) of every
 * position's rotary angles, float2 [max_ctx][64]); with batch > 1 also "x16" (staged
 * batch activation) and "mm_work" (matvec outputs before the residual).
 * "q" holds the rotated query as the attention's operand: per sequence and kv
 * head 4096 bytes of fp16 hi / lo pairs of q / sqrt(128) (matrix-core order).
 * With batch B > 1 the per-sequence regions hold B rows, sequence s at row s:
 * h [B][hidden], q, att [B][n_heads*128], act [B][ffn], logits [B][vocab],
 * token / pos [B]; the KV caches hold B * max_ctx / page_size pages and
 * block_table is [B][max_ctx / page_size] (initially sequence s owns pages
 * [s * max_ctx / page_size, (s + 1) * max_ctx / page_size)).
 * Row layouts: qkv = q rows (n_heads*128) | k rows | v rows; gate_up rows
 * interleaved (2i = gate_i, 2i+1 = up_i).
 * At batch 1 every IQ2_S / IQ3_S layer tensor (qkv, o, gate_up, down) also has
 * "<role>_units" per layer: its weights regrouped into the IQ2S_UNITS /
 * IQ3S_UNITS layout (rtxllm_iq2s_units_pack, rtxllm_iq3s_units_pack), which its
 * matvec reads. The runner rebuilds a layer's copy before its next launch after
 * rtxllm_llama_upload of that layer's tensor, rtxllm_llama_load_packs or
 * rtxllm_llama_synth_weights; after writing a tensor through a region pointer,
 * call rtxllm_llama_weights_changed. */
void* rtxllm_llama_region(rtxllm_llama* m, const char* name, uint32_t layer, size_t* bytes);
/* The weights were written through region pointers: rebuild the derived unit
 * copies before the next launch (no counterpart in the reference). */
void rtxllm_llama_weights_changed(rtxllm_llama* m);

/* Synchronous host <-> region copies (setup and inspection; not capture-safe):
 * `bytes` at byte `offset` of the region. hipErrorInvalidValue if out of range,
 * and for an upload to "pos" (or "token") of a value >= max_ctx (>= vocab):
 * a position must have a KV slot, a token an embedding row. */
hipError_t rtxllm_llama_upload(rtxllm_llama* m, const char* name, uint32_t layer, size_t offset, const void* src,
                               size_t bytes);
hipError_t rtxllm_llama_download(rtxllm_llama* m, const char* name, uint32_t layer, size_t offset, void* dst,
                                 size_t bytes);

/* Fill every weight tensor with the seeded synthetic generator (on the device,
 * bit-identical to rtxllm_synth_raw_blocks): tensor seed = seed + 4096 *
 * (layer + 1) + role (qkv 1, o 2, gate_up 3, down 4), embed seed + 5, LM head
 * seed + 6; d, dmin = fp16(U[1e-4, 2e-3]). Norm weights and the KV cache are
 * left to the caller. Q4_K split layouts other than split-native are refused. */
hipError_t rtxllm_llama_synth_weights(rtxllm_llama* m, uint64_t seed, hipStream_t stream);

/* Fill every weight tensor from resident packs: the Q4_K manifest and the
 * raw-block (IQ2_S / IQ3_S / Q5_K) manifest of the pack producers
 * (tools/bench/q4k_resident_pack.py, iq_resident_pack.py schema; either may be
 * null), pack paths relative to payload_root unless absolute. Tensors by GGUF
 * name: blk.<l>.attn_q / attn_k / attn_v (stacked into "qkv"), attn_output,
 * ffn_gate / ffn_up (interleaved into "gate_up"), ffn_down, token_embd and
 * output (".weight"). Each must be in the configured format (a Q4_K split
 * layout's pack policy must match it; raw Q4_K comes from blocks_path) with
 * the model's shape, and every file's size and byte-sum checksum must match
 * its manifest. hipErrorInvalidValue with the reason in err otherwise; every
 * tensor is read and checked before the first upload, so a refused pack set
 * leaves the model's weights as they were. */
hipError_t rtxllm_llama_load_packs(rtxllm_llama* m, const char* q4k_manifest, const char* iq_manifest,
                                   const char* payload_root, char* err, size_t err_len);

/* rtxllm_llama_load_packs over any number of manifests (count entries), each
 * read by the loader its "path" field names: the reference producers write one
 * manifest per producer (q4k_resident_pack, iq_resident_pack,
 * q5k_resident_pack), as does rtxllm_gguf_pack (rtxllm/pack_producer.h). A
 * tensor in two manifests is refused; the rest as rtxllm_llama_load_packs. */
hipError_t rtxllm_llama_load_pack_set(rtxllm_llama* m, const char* const* manifests, uint32_t count,
                                      const char* payload_root, char* err, size_t err_len);

/* The admission check made at create: bytes the model needs (weights, KV,
 * workspace, graph), the device bytes it was admitted against, and the arena
 * size. */
hipError_t rtxllm_llama_memory(const rtxllm_llama* m, size_t* required_bytes, size_t* usable_bytes,
                               size_t* arena_bytes);

enum { RTXLLM_LLAMA_EMBED = 1, RTXLLM_LLAMA_HEAD = 2 };

/* Layers [first, last) at position *pos (per sequence: pos[s]). flags & EMBED:
 * h = embed[*token], else h is taken as is. flags & HEAD: final norm, LM head,
 * token = argmax, pos += 1. */
hipError_t rtxllm_llama_forward(rtxllm_llama* m, uint32_t first, uint32_t last, int flags, hipStream_t stream);
/* One full decode step: forward(0, n_layers, EMBED | HEAD). */
hipError_t rtxllm_llama_step(rtxllm_llama* m, hipStream_t stream);
/* Capture one decode step into the model's hipGraph / replay it. */
hipError_t rtxllm_llama_graph_capture(rtxllm_llama* m, hipStream_t stream);
hipError_t rtxllm_llama_graph_replay(rtxllm_llama* m, hipStream_t stream);
/* Context-bucketed step graphs (the reference's graph buckets keyed by query
 * length, cuda_graph_bucket.h:70-177, and the runner's bucket replay,
 * main.cpp:4838-4869): a step graph whose attention launches cover only the
 * first `span` positions (rounded up to whole 128-position chunks), so a short
 * context does not pay for max_ctx. Capture admits the bucket's graph memory
 * strictly (hipErrorOutOfMemory); capturing a span again replaces its graph.
 * Replay is valid while every sequence's position is below span. span_for
 * returns the smallest captured span above `position` (0: none); graph_bytes
 * the graph-memory plan over every captured graph. */
hipError_t rtxllm_llama_graph_capture_span(rtxllm_llama* m, uint32_t span, hipStream_t stream);
hipError_t rtxllm_llama_graph_replay_span(rtxllm_llama* m, uint32_t span, hipStream_t stream);
uint32_t rtxllm_llama_graph_span_for(const rtxllm_llama* m, uint32_t position);
size_t rtxllm_llama_graph_bytes(const rtxllm_llama* m);
/* One stage of the step alone, on the current state, for per-stage timing (the
 * reference runner's per-phase replay timing, main.cpp:4838-4869): stage 0
 * embedding gather + staging, 1 qkv of `layer`, 2 attention of `layer`, 3 o,
 * 4 gate/up, 5 down, 6 LM head + argmax. */
hipError_t rtxllm_llama_launch_stage(rtxllm_llama* m, uint32_t layer, int stage, hipStream_t stream);
/* Kernel launches per decode step. */
uint32_t rtxllm_llama_launches_per_step(const rtxllm_llama* m);

/* Per-sequence status words (region "status", uint32 [batch], 0 at create).
 * RTXLLM_LLAMA_STATUS_CONTEXT_FULL: a step ran while the sequence's position
 * was max_ctx (its KV cache full): that step had no slot for its token, so it
 * left the sequence's token and position as they were (the sequence halts at
 * max_ctx instead of decoding past the context end).
 * RTXLLM_LLAMA_STATUS_WAIT_TIMEOUT (word 0): a bounded in-kernel wait of the
 * batch-1 gate/up matvec ran out (its column-split waves hand partials over
 * through LDS counters when a K-quant gate/up has hidden <= 4096), so that
 * step's results are not valid. The bits stay set until cleared.
 * rtxllm_llama_status copies the batch's words to host memory and waits for
 * the stream; rtxllm_llama_clear_status zeroes them (both synchronous, not
 * capture-safe). */
enum { RTXLLM_LLAMA_STATUS_CONTEXT_FULL = 1, RTXLLM_LLAMA_STATUS_WAIT_TIMEOUT = 2 };
hipError_t rtxllm_llama_status(rtxllm_llama* m, uint32_t* status, hipStream_t stream);
hipError_t rtxllm_llama_clear_status(rtxllm_llama* m, hipStream_t stream);

#ifdef __cplusplus
}
#endif

#endif
