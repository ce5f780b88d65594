// Host-side interface of the Llama decode-layer kernels (layer.hip), used by the
// decode runner (model.cpp). All pointers are device pointers; every launcher
// is asynchronous on `stream` and capture-safe.
#pragma once

#include <hip/hip_runtime.h>

#include <cstddef>
#include <cstdint>

namespace rtxllm {

// fp16 paged KV cache of one layer: page p (physical) holds K (and V) as
// [n_kv_heads][page_size][head_dim]; block_table maps logical page -> physical.
struct KvLayer {
  std::uint16_t* k;
  std::uint16_t* v;
  const std::int32_t* block_table;
  std::uint32_t page_size;
  std::uint32_t n_kv;
  std::uint32_t capacity;  // positions; a position >= capacity is never read or written
};

// RMSNorm input of a fused matvec: the staged vector holds h * w (16-value
// groups), and the matvec multiplies its row sums by 1 / sqrt(sum(h^2) / n +
// eps), sum(h^2) being the sum of `nslots` partials written by the producer.
struct NormIn {
  const void* xq;
  const float* sumsq;
  std::uint32_t nslots;
  std::uint32_t n;
  float eps;
};

constexpr std::uint32_t kHeadDim = 128;
// The attention's query operand ("q16"): per sequence and kv head, the rotated
// query heads of the kv head scaled by 1 / sqrt(head_dim) as fp16 hi / lo
// pairs in matrix-core operand order, kQ16BytesPerKv bytes (zero where a kv
// head has fewer than 8 query heads; the qkv launchers never write there).
constexpr std::uint32_t kQ16BytesPerKv = 4096;

// h = dequant(embed[*token]) (Q5_K row, bit-exact; table null: h as is), then
// xq = stage(h * wnorm), sumsq[0] = sum(h^2), sumsq[1, nslots) = 0.
// cols % 256 == 0, cols <= 16384; a token >= vocab reads row vocab - 1.
hipError_t launch_embed_q5k(const std::uint8_t* table, std::uint32_t cols, std::uint32_t vocab,
                            const std::uint32_t* token, float* h, const float* wnorm, void* xq, float* sumsq,
                            std::uint32_t nslots, hipStream_t stream);

// qkv = Wqkv * rmsnorm(h) (q_rows + 2 kv_rows rows, q | k | v), then RoPE
// (adjacent pairs) on q and k at position *pos, q -> q_out (q16), k and v ->
// fp16 KV cache slot *pos. rope[p * head_dim / 2 + i] = (cos, sin) of the angle
// of pair i at position p < rope_positions (rope_table()).
hipError_t launch_qkv(int fmt, const std::uint8_t* payload, const std::uint8_t* meta, std::uint32_t cols,
                      const NormIn& in, std::uint32_t q_rows, std::uint32_t kv_rows, const float2* rope,
                      std::uint32_t rope_positions, const std::uint32_t* pos, void* q_out, const KvLayer& kv,
                      hipStream_t stream);

// GQA decode attention over positions [0, *pos] of the paged cache: split over
// context chunks (partials) then combined into att[n_heads * head_dim], which
// is also staged (16-value groups) into xq_att for the o projection. The launch
// covers positions [0, span) (span <= kv.capacity, its chunks only): the
// position must be below span, positions at or beyond it are not attended.
hipError_t launch_attention(const void* q, const KvLayer& kv, std::uint32_t n_heads, const std::uint32_t* pos,
                            std::uint32_t span, float* partials, float* att, void* xq_att, hipStream_t stream);
// Per sequence partial-record floats of a launch over `span` positions (the
// batch needs batch times as many).
std::size_t attention_partials_floats(std::uint32_t n_heads, std::uint32_t n_kv, std::uint32_t span);
// The same for `batch` sequences: sequence s has q16 n_kv * kQ16BytesPerKv
// bytes on, block-table row s (table_stride entries, >= capacity /
// page_size), position pos[s], and writes att[s]; xq_att must be null when
// batch > 1. x16_att (batch <= 8, xq_att null): att of every sequence is also
// staged there for the batched o projection (the launch_stage_batch rule;
// sequences >= batch zero), in the same launch as the combine.
hipError_t launch_attention_batch(const void* q, const KvLayer& kv, std::uint32_t n_heads, const std::uint32_t* pos,
                                  std::uint32_t span, std::uint32_t batch, std::uint32_t table_stride,
                                  float* partials, float* att, void* xq_att, void* x16_att, hipStream_t stream);

// h += W x (rows % 16 == 0), x either the staged input xq_in or the fp32 x_in
// (staged by each wave itself; exactly one of the two non-null); then xq_next =
// stage(h * w_next), sumsq_next[t] = sum of h^2 over rows [16 t, 16 t + 16).
hipError_t launch_residual(int fmt, const std::uint8_t* payload, const std::uint8_t* meta, std::uint32_t rows,
                           std::uint32_t cols, const void* xq_in, const float* x_in, float* h, const float* w_next,
                           void* xq_next, float* sumsq_next, hipStream_t stream);

// Rows interleaved gate / up (row 2i = gate_i, row 2i + 1 = up_i), x =
// rmsnorm(h): act[i] = silu(gate_i) * up_i. Kernel: the int8 matrix cores for
// the IQ unit layouts on whole 16-row tiles and 512-column panels; else the
// dot-product matvec, for cols <= 4096 in one 16-wave workgroup per CU whose
// column-split waves hand partials over through bounded LDS waits: a wait that
// ran out ORs kStatusWaitTimeout into *status (status may be null).
// wait_limit / wait_bias: reads per wait and a bias on its target (production:
// kPairSpinLimit and 0; a test forces the timeout with a bias no wave reaches).
hipError_t launch_gate_up(int fmt, const std::uint8_t* payload, const std::uint8_t* meta, std::uint32_t rows,
                          std::uint32_t cols, const NormIn& in, float* act, std::uint32_t* status,
                          hipStream_t stream, std::uint32_t wait_limit = 1u << 20, std::uint32_t wait_bias = 0u);

// logits = W rmsnorm(h), and per row group of the launch the best argmax key
// (ordered(logit) << 32 | ~row: greedy argmax, lowest index on ties, NaN never
// wins) in keys[0, *key_count); logits_key_slots() is that count (the launch
// fails if it exceeds key_capacity).
std::uint32_t logits_key_slots(int fmt, std::uint32_t rows, std::uint32_t cols);
hipError_t launch_logits(int fmt, const std::uint8_t* payload, const std::uint8_t* meta, std::uint32_t rows,
                         std::uint32_t cols, const NormIn& in, float* logits, unsigned long long* keys,
                         std::uint32_t key_capacity, std::uint32_t* key_count, hipStream_t stream);

// Status bit of a sequence whose step ran at a position >= the KV capacity.
// (Bit 2, kStatusWaitTimeout of mv.cuh: a bounded in-kernel wait ran out.)
constexpr std::uint32_t kStatusContextFull = 1u;

// token[0] = argmax over keys[0, count) (0 if every logit was NaN); *pos +=
// advance; but when *pos >= capacity (the step had no KV slot) token and pos
// stay and *status |= kStatusContextFull (status may be null).
hipError_t launch_argmax_finalize(const unsigned long long* keys, std::uint32_t count, std::uint32_t* token,
                                  std::uint32_t* pos, std::uint32_t advance, std::uint32_t capacity,
                                  std::uint32_t* status, hipStream_t stream);
// The same per sequence s < batch over keys[s * key_stride, + count): token[s],
// pos[s], status[s].
hipError_t launch_argmax_finalize_batch(const unsigned long long* keys, std::uint32_t key_stride,
                                        std::uint32_t count, std::uint32_t batch, std::uint32_t* token,
                                        std::uint32_t* pos, std::uint32_t advance, std::uint32_t capacity,
                                        std::uint32_t* status, hipStream_t stream);

// ---- batch (2..8 sequences) step, on the matrix cores (batch.hip) ------------
// x16: a staged batch activation (rtxllm_x16_bytes); columns of sequences >=
// batch are never written by these launchers.

// h[s] = embed ? Q5_K row token[s] : h[s] (+ sum over g of res[g][s], res being
// [groups][batch][cols], when non-null); then x16 = stage(rmsnorm(h[s]) * w).
hipError_t launch_rms_stage_batch(float* h, const float* res, std::uint32_t groups, const std::uint8_t* embed,
                                  const std::uint32_t* token, std::uint32_t vocab, const float* w, float eps,
                                  std::uint32_t cols, std::uint32_t batch, void* x16, hipStream_t stream);
// x16 = stage(x[s]) for x [batch][cols].
hipError_t launch_stage_batch(const float* x, std::uint32_t batch, std::uint32_t cols, void* x16,
                              hipStream_t stream);
// Panel groups of a batched matvec (1: the output is y itself) and the
// partial-sum workspace it needs (0 with one group).
std::uint32_t mm_panel_groups(int fmt, std::uint32_t rows, std::uint32_t cols);
std::size_t mm_batch_workspace_bytes(int fmt, std::uint32_t rows, std::uint32_t cols);
// out[g][s][row] = panel group g's part of (W x_s)[row] (out = y with one group).
hipError_t launch_mm_batch(int fmt, const std::uint8_t* payload, const std::uint8_t* meta, std::uint32_t rows,
                           std::uint32_t cols, const void* x16, std::uint32_t batch, float* out, hipStream_t stream);
// The same with the activation given as fp32 x [batch][cols] (16-byte aligned):
// each wave stages its own panel (the plain x16 rule), so no staging launch is
// needed between the producer of x and this matvec.
hipError_t launch_mm_batch_self(int fmt, const std::uint8_t* payload, const std::uint8_t* meta, std::uint32_t rows,
                                std::uint32_t cols, const float* x, std::uint32_t batch, float* out,
                                hipStream_t stream);
// qkv of every sequence with the batch-1 qkv epilogue's RoPE and KV append at
// pos[s], the KV block table of sequence s being row s (table_stride entries).
hipError_t launch_mm_qkv_batch(int fmt, const std::uint8_t* payload, const std::uint8_t* meta, std::uint32_t cols,
                               const void* x16, std::uint32_t batch, std::uint32_t q_rows, std::uint32_t kv_rows,
                               const float2* rope, std::uint32_t rope_positions, const std::uint32_t* pos,
                               void* q_out, const KvLayer& kv, std::uint32_t table_stride, hipStream_t stream);
// Interleaved gate / up rows: act[s][i] = silu(gate_i) * up_i (act [batch][rows / 2]).
hipError_t launch_mm_gate_up_batch(int fmt, const std::uint8_t* payload, const std::uint8_t* meta,
                                   std::uint32_t rows, std::uint32_t cols, const void* x16, std::uint32_t batch,
                                   float* act, hipStream_t stream);
// logits[s][rows] and per sequence mm_logits_key_slots() argmax keys at
// keys[s * key_stride] (key_stride >= that count), for launch_argmax_finalize_batch.
std::uint32_t mm_logits_key_slots(int fmt, std::uint32_t rows, std::uint32_t cols);
hipError_t launch_mm_logits_batch(int fmt, const std::uint8_t* payload, const std::uint8_t* meta, std::uint32_t rows,
                                  std::uint32_t cols, const void* x16, std::uint32_t batch, float* logits,
                                  unsigned long long* keys, std::uint32_t key_stride, std::uint32_t* key_count,
                                  hipStream_t stream);

// Device-side synthetic packs, bit-identical to the host generator
// (rtxllm_synth_raw_blocks): raw blocks of format 0/5/6/7, or the Q4_K
// split-native pair (payload + 16 B heads) of synthetic raw Q4_K blocks.
hipError_t launch_synth_raw(int fmt, std::uint64_t seed, std::size_t n_blocks, float d_lo, float d_hi,
                            std::uint8_t* out, hipStream_t stream);
hipError_t launch_synth_q4k_native(std::uint64_t seed, std::size_t n_blocks, float d_lo, float d_hi,
                                   std::uint8_t* payload, std::uint8_t* meta, hipStream_t stream);

}  // namespace rtxllm
