/* C-ABI of the MI355X (gfx950) decode hot path.
 *
 * Drop-in for the reference's runtime/kernels/decode/decode_kernels.h: the
 * rtxllm_launch_* entry points below keep the reference's names, argument order
 * and meaning, with hipError_t / hipStream_t in place of the CUDA types. Every
 * pointer argument is a device pointer into caller-owned memory; no entry point
 * allocates, frees, copies or synchronises, so all are hipGraph-capturable.
 * Each returns hipGetLastError() after its launches, or hipErrorInvalidValue
 * for rejected arguments before launching anything.
 *
 * The rtxllm_* entry points without "launch" in their names have no
 * counterpart in the reference; they carry the math of a real Llama decode step
 * (pure y = W x on an fp32 or a staged activation, batched matvecs, weighted
 * RMSNorm, RoPE with a theta schedule, SiLU-gate multiply, Q5_K embedding
 * gather, GQA attention over a paged fp16 KV cache, greedy argmax) and the
 * host-side pack helpers. The decode runner of rtxllm/llama.h fuses the same
 * math into its matvec epilogues.
 *
 * Activation precision of every batch-1 matvec (the reference-named launchers
 * included): the kernels multiply the weight codes with the fp32 activation
 * through exact integer dot products after staging x per 16-value group as
 * 22-bit block fixed point (see rtxllm_stage_activation): each value is
 * rounded once, to a multiple of s = 2^(e - 22) where max|x| of its group is in
 * [2^(e-1), 2^e), so its error is at most 2^-23 of the group maximum. A
 * 4096-column product then stays closer to the exact (float64) result than
 * the reference's fp32 sequential accumulation (main.cpp:1261-1309) does, also
 * for groups with outliers. A NaN activation makes its group's scale NaN, so
 * the outputs become NaN as in fp32; an infinite one makes them NaN where fp32
 * gives +-inf or NaN.
 *
 * Pointer alignment: activation pointers (x, activation) may have any 4-byte
 * alignment. Weight streams must be aligned as the kernels' vector loads need
 * them (the reference's vec4x4 kernels likewise read 16-byte float4 of x and
 * 4-byte words of the payload, decode_kernels.cu:2893-2991): Q4_K payloads and
 * predecoded / native metadata, Q5_K blocks and the IQ2S_UNITS / IQ3S_UNITS
 * layouts 16 bytes, split-half metadata 8, split-compact metadata 4, IQ2_S /
 * IQ3_S blocks 2. A misaligned weight pointer is refused with
 * hipErrorInvalidValue. The staged buffers (xq, x16) and workspaces are 16-byte
 * aligned (256 for the attention workspace).
 *
 * Pack layouts (all row-major, rows x (cols / 256) blocks, cols % 256 == 0):
 *   Q4_K raw 144 B, Q5_K 176 B, IQ2_S 82 B, IQ3_S 110 B GGUF blocks;
 *   Q4_K split: 128 B payload stream + metadata stream of 64 B (predecoded,
 *   8 x f32 (d*sc, dmin*m)), 32 B (half, the same as fp16), 20 B (compact:
 *   f16 d, f16 dmin, u8 sc[8], u8 m[8]) or 16 B (native: the GGUF head).
 */
#ifndef RTXLLM_DECODE_KERNELS_H
#define RTXLLM_DECODE_KERNELS_H

#include <hip/hip_runtime_api.h>
#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ===== Reference-named entry points =====================================
 * Feedback family: decode_kernels.h:38-101. act[c] is computed from
 * logits[c % rows] normalised by inv_rms = rsqrt(mean(logits^2) + epsilon). */

/* decode_kernels.h:38-44: activation[c] = logits[c % rows] * inv_rms. */
hipError_t rtxllm_launch_rmsnorm_feedback(const float* logits, float* activation, uint32_t rows, uint32_t cols,
                                          float epsilon, hipStream_t stream);

/* decode_kernels.h:46-52: activation[c] = silu(logits[c % rows] * inv_rms). */
hipError_t rtxllm_launch_silu_rmsnorm_feedback(const float* logits, float* activation, uint32_t rows,
                                               uint32_t cols, float epsilon, hipStream_t stream);

/* decode_kernels.h:54-61: activation[c] = n, silu_cache[c] = silu(n). */
hipError_t rtxllm_launch_rmsnorm_feedback_with_silu_cache(const float* logits, float* activation,
                                                          float* silu_cache, uint32_t rows, uint32_t cols,
                                                          float epsilon, hipStream_t stream);

/* decode_kernels.h:63-71: activation[c] = silu_cache[c % cache_cols] * n. */
hipError_t rtxllm_launch_gated_silu_rmsnorm_feedback(const float* logits, const float* silu_cache,
                                                     float* activation, uint32_t rows, uint32_t cache_cols,
                                                     uint32_t cols, float epsilon, hipStream_t stream);

/* decode_kernels.h:73-80: silu_cache[c] (+)= silu(n). cache_cols == 0 -> InvalidValue. */
hipError_t rtxllm_launch_rmsnorm_silu_cache(const float* logits, float* silu_cache, uint32_t rows,
                                            uint32_t cache_cols, float epsilon, uint32_t accumulate,
                                            hipStream_t stream);

/* decode_kernels.h:82-89: cache[c] (+)= n. cache_cols == 0 -> InvalidValue. */
hipError_t rtxllm_launch_rmsnorm_cache(const float* logits, float* cache, uint32_t rows, uint32_t cache_cols,
                                       float epsilon, uint32_t accumulate, hipStream_t stream);

/* decode_kernels.h:91-101: up_cache[c] (+)= n; activation[c] = gate_cache[c] * up_cache[c]. */
hipError_t rtxllm_launch_rmsnorm_cache_and_gated_product(const float* logits, const float* gate_cache,
                                                         float* up_cache, float* activation, uint32_t rows,
                                                         uint32_t cache_cols, uint32_t output_cols,
                                                         float epsilon, uint32_t accumulate,
                                                         hipStream_t stream);

/* decode_kernels.h:319-325: token[0] = (argmax(logits[0:rows]) + token_offset) % vocab_size;
 * ties -> lowest index. Null pointers or zero rows / vocab -> InvalidValue. */
hipError_t rtxllm_launch_output_token_sample(const float* logits, uint32_t* token, uint32_t rows,
                                             uint32_t vocab_size, uint32_t token_offset, hipStream_t stream);

/* Matvec + decode side effects. Each *_decode* call runs y = W x over the
 * launched rows, the KV side-write kv[(r*page_words + (token+r) % page_words) %
 * kv_words] = y[r] for r < active_pages, then token = (argmax(y) + token + 1) %
 * 32000. IQ/Q5_K calls clip to min(rows, rows_limit) rows. */

/* decode_kernels.h:345-357. */
hipError_t rtxllm_launch_q5k_matvec_decode_probe(const uint8_t* q5k_blocks, const float* activation,
                                                 float* logits, float* kv, uint32_t* token, uint32_t rows,
                                                 uint32_t cols, uint32_t rows_limit, uint32_t kv_words,
                                                 uint32_t page_words, uint32_t active_pages,
                                                 hipStream_t stream);

/* decode_kernels.h:359-366: matvec only (no KV, no token). */
hipError_t rtxllm_launch_iq2s_matvec_probe(const uint8_t* iq2s_blocks, const float* activation, float* logits,
                                           uint32_t rows, uint32_t cols, uint32_t rows_limit,
                                           hipStream_t stream);

/* decode_kernels.h:368-380. */
hipError_t rtxllm_launch_iq2s_matvec_decode_probe(const uint8_t* iq2s_blocks, const float* activation,
                                                  float* logits, float* kv, uint32_t* token, uint32_t rows,
                                                  uint32_t cols, uint32_t rows_limit, uint32_t kv_words,
                                                  uint32_t page_words, uint32_t active_pages,
                                                  hipStream_t stream);

/* decode_kernels.h:382-394. */
hipError_t rtxllm_launch_iq3s_matvec_decode_probe(const uint8_t* iq3s_blocks, const float* activation,
                                                  float* logits, float* kv, uint32_t* token, uint32_t rows,
                                                  uint32_t cols, uint32_t rows_limit, uint32_t kv_words,
                                                  uint32_t page_words, uint32_t active_pages,
                                                  hipStream_t stream);

/* decode_kernels.h:424-513: Q4_K on raw 144 B blocks. The reference's variants
 * (direct, shared, warp, warp_broadcast, _vec4, _vec4x2, _vec4x4) are CUDA
 * implementation choices of one operation; all map to the one gfx950 kernel. */
hipError_t rtxllm_launch_q4k_matvec_decode(const uint8_t* q4k_blocks, const float* activation, float* logits,
                                           float* kv, uint32_t* token, uint32_t rows, uint32_t cols,
                                           uint32_t kv_words, uint32_t page_words, uint32_t active_pages,
                                           hipStream_t stream);
hipError_t rtxllm_launch_q4k_matvec_decode_shared(const uint8_t* q4k_blocks, const float* activation,
                                                  float* logits, float* kv, uint32_t* token, uint32_t rows,
                                                  uint32_t cols, uint32_t kv_words, uint32_t page_words,
                                                  uint32_t active_pages, hipStream_t stream);
hipError_t rtxllm_launch_q4k_matvec_decode_warp(const uint8_t* q4k_blocks, const float* activation,
                                                float* logits, float* kv, uint32_t* token, uint32_t rows,
                                                uint32_t cols, uint32_t kv_words, uint32_t page_words,
                                                uint32_t active_pages, hipStream_t stream);
hipError_t rtxllm_launch_q4k_matvec_decode_warp_broadcast(const uint8_t* q4k_blocks, const float* activation,
                                                          float* logits, float* kv, uint32_t* token,
                                                          uint32_t rows, uint32_t cols, uint32_t kv_words,
                                                          uint32_t page_words, uint32_t active_pages,
                                                          hipStream_t stream);
hipError_t rtxllm_launch_q4k_matvec_decode_warp_broadcast_vec4(const uint8_t* q4k_blocks,
                                                               const float* activation, float* logits,
                                                               float* kv, uint32_t* token, uint32_t rows,
                                                               uint32_t cols, uint32_t kv_words,
                                                               uint32_t page_words, uint32_t active_pages,
                                                               hipStream_t stream);
hipError_t rtxllm_launch_q4k_matvec_decode_warp_broadcast_vec4x2(const uint8_t* q4k_blocks,
                                                                 const float* activation, float* logits,
                                                                 float* kv, uint32_t* token, uint32_t rows,
                                                                 uint32_t cols, uint32_t kv_words,
                                                                 uint32_t page_words, uint32_t active_pages,
                                                                 hipStream_t stream);
hipError_t rtxllm_launch_q4k_matvec_decode_warp_broadcast_vec4x4(const uint8_t* q4k_blocks,
                                                                 const float* activation, float* logits,
                                                                 float* kv, uint32_t* token, uint32_t rows,
                                                                 uint32_t cols, uint32_t kv_words,
                                                                 uint32_t page_words, uint32_t active_pages,
                                                                 hipStream_t stream);

/* decode_kernels.h:515-527: raw 144 B blocks for the quants, predecoded f32
 * (d*sc, dmin*m) pairs (8 per block) for the scales. */
hipError_t rtxllm_launch_q4k_matvec_decode_predecoded_vec4x4(const uint8_t* q4k_blocks,
                                                             const float* q4k_scale_min_pairs,
                                                             const float* activation, float* logits, float* kv,
                                                             uint32_t* token, uint32_t rows, uint32_t cols,
                                                             uint32_t kv_words, uint32_t page_words,
                                                             uint32_t active_pages, hipStream_t stream);

/* decode_kernels.h:529-583: Q4_K split resident layouts. */
hipError_t rtxllm_launch_q4k_matvec_decode_split_predecoded_vec4x4(const uint8_t* q4k_payload,
                                                                   const float* q4k_scale_min_pairs,
                                                                   const float* activation, float* logits,
                                                                   float* kv, uint32_t* token, uint32_t rows,
                                                                   uint32_t cols, uint32_t kv_words,
                                                                   uint32_t page_words, uint32_t active_pages,
                                                                   hipStream_t stream);
hipError_t rtxllm_launch_q4k_matvec_decode_split_half_vec4x4(const uint8_t* q4k_payload,
                                                             const uint16_t* q4k_scale_min_half_pairs,
                                                             const float* activation, float* logits, float* kv,
                                                             uint32_t* token, uint32_t rows, uint32_t cols,
                                                             uint32_t kv_words, uint32_t page_words,
                                                             uint32_t active_pages, hipStream_t stream);
hipError_t rtxllm_launch_q4k_matvec_decode_split_compact_vec4x4(const uint8_t* q4k_payload,
                                                                const uint8_t* q4k_compact_meta,
                                                                const float* activation, float* logits,
                                                                float* kv, uint32_t* token, uint32_t rows,
                                                                uint32_t cols, uint32_t kv_words,
                                                                uint32_t page_words, uint32_t active_pages,
                                                                hipStream_t stream);
hipError_t rtxllm_launch_q4k_matvec_decode_split_native_vec4x4(const uint8_t* q4k_payload,
                                                               const uint8_t* q4k_native_meta,
                                                               const float* activation, float* logits,
                                                               float* kv, uint32_t* token, uint32_t rows,
                                                               uint32_t cols, uint32_t kv_words,
                                                               uint32_t page_words, uint32_t active_pages,
                                                               hipStream_t stream);

/* ===== New entry points (no reference counterpart) ======================= */

/* Format ids (payload / metadata layouts): 0 Q4_K raw, 1 split-predecoded,
 * 2 split-half, 3 split-compact, 4 split-native, 5 Q5_K, 6 IQ2_S, 7 IQ3_S,
 * 8 Q4_K raw + predecoded pairs. meta is null except for 1-4 and 8. */

/* Dequantise to fp32 [rows][cols], bit-exact with the reference's per-element
 * formulas (main.cpp:1133-1259). */
hipError_t rtxllm_dequant_f32(int format, const uint8_t* payload, const uint8_t* meta, uint32_t rows,
                              uint32_t cols, float* out, hipStream_t stream);

/* y[rows] = W x (batch 1), no side effects. x is fp32; each wave stages the
 * columns it owns itself (the rtxllm_stage_activation rule). */
hipError_t rtxllm_matvec(int format, const uint8_t* payload, const uint8_t* meta, const float* x, float* y,
                         uint32_t rows, uint32_t cols, hipStream_t stream);

/* Staged activation ("xq"): x is cut into 16-value groups. For a group with
 * maximum magnitude m = f 2^e (f in [0.5, 1)) the scale is s = 2^(e - 22) and
 * each value is held as X_j = rint(x_j 2^(22 - e)) (|X_j| <= 2^22, so x_j =
 * s X_j up to s / 2), split into three int8 digits X_j = 65536 H_j + 256 M_j +
 * L_j (H in [-64, 64], M and L in [-128, 127]), plus the group scale s and the
 * group sum s * sum(X). A group holding a NaN has s = NaN, one whose maximum
 * is infinite s = inf (all digits 0); an all-zero group s = 0. Layout of one
 * buffer of rtxllm_xq_bytes(cols) bytes (16-byte aligned): H[cols], M[cols],
 * L[cols] (int8), s[cols/16], sum[cols/16] (f32). The matvec kernels multiply
 * the weight codes with the digits through exact integer dot products. */
size_t rtxllm_xq_bytes(uint32_t cols);
/* xq = stage(x * weight) (weight may be null: stage x). cols % 256 == 0. */
hipError_t rtxllm_stage_activation(const float* x, const float* weight, uint32_t cols, void* xq,
                                   hipStream_t stream);
/* y[rows] = W x_hat for a staged x (the layer pipeline's matvec). */
hipError_t rtxllm_matvec_xq(int format, const uint8_t* payload, const uint8_t* meta, const void* xq, float* y,
                            uint32_t rows, uint32_t cols, hipStream_t stream);
/* The same on the int8 matrix cores (v_mfma_i32_16x16x64_i8 over 16-row
 * tiles, one wave per 512-column panel), the kernel of the decode runner's
 * batch-1 gate/up: IQ unit layouts only (formats 9, 10), rows % 16 == 0,
 * cols % 512 == 0, cols <= 8192. Each 16-value group's integer dot is the
 * exact one rtxllm_matvec_xq forms; the scaled group results are added in
 * another order, so y agrees with rtxllm_matvec_xq to fp32 rounding, not bit
 * for bit. */
hipError_t rtxllm_matvec_xq_mfma(int format, const uint8_t* payload, const void* xq, float* y, uint32_t rows,
                                 uint32_t cols, hipStream_t stream);

/* The decode runner's fused gate/up stage. W [rows][cols] holds the gate and
 * up rows interleaved (row 2i = gate_i, row 2i + 1 = up_i); with (g, u) =
 * W x_hat for the staged xq and the RMSNorm scale s = 1 / sqrt(sum(sumsq[0 ..
 * nslots)) / cols + eps) from the producer's partial sums of squares,
 * act[i] = silu(s g_i) (s u_i), silu(v) = v / (1 + exp(-v)) (main.cpp:
 * 1435-1503 for silu). Kernels: the matrix cores for the IQ unit layouts at
 * rtxllm_matvec_xq_mfma's shapes; otherwise the dot-product matvec, for cols
 * <= 4096 in one 16-wave workgroup per CU whose column-split waves hand their
 * partials over through bounded LDS waits. A wait that ran out ORs
 * RTXLLM_STATUS_WAIT_TIMEOUT into *status (status may be null) and act is
 * then not valid. rows % 4 == 0. */
#define RTXLLM_STATUS_WAIT_TIMEOUT 2u
hipError_t rtxllm_gate_up_silu(int format, const uint8_t* payload, const uint8_t* meta, const void* xq,
                               const float* sumsq, uint32_t nslots, float eps, float* act, uint32_t rows,
                               uint32_t cols, uint32_t* status, hipStream_t stream);

/* Batched matvec on the matrix cores: y[s][rows] = W x_s for s < batch <= 8
 * (the batch-8 decode variant). Formats: 0 Q4_K raw, 4 Q4_K split-native,
 * 5 Q5_K, 6 IQ2_S, 7 IQ3_S; cols % 512 == 0.
 * Staged batch activation ("x16"), rtxllm_x16_bytes(cols) bytes: 16 fp16
 * columns X[n] of cols values, X[2 s] = hi, X[2 s + 1] = lo of x' = x_s
 * 2^-e[s][b] over each block b of 256 values (hi = fp16(x'), lo = fp16(x' -
 * hi), e[s][b] the power of two putting the block's max |x'| in [0.5, 1)),
 * stored in the matrix cores' operand order: the fp16 at ((b * 8 + j) * 64 +
 * l) * 8 + i is X[l % 16][256 b + 64 (l / 16) + 8 j + i]; then int32
 * e[8][cols / 256], float ss[8][cols / 256], float eps (rtxllm_stage_batch
 * writes eps = -1; the decode runner's RMSNorm staging writes eps >= 0 with
 * the blocks' sums of squares in ss, and the matvec then scales each y[s] by
 * 1 / sqrt(sum(ss[s]) / cols + eps)). The weight codes times their sub-block scale
 * integers are exact in fp16, so each product is exact and only the ~22-bit
 * hi/lo split and the fp32 accumulation round. Matrices wider than 4096
 * columns need a workspace of rtxllm_matvec_batch_workspace() bytes (0: none). */
size_t rtxllm_x16_bytes(uint32_t cols);
hipError_t rtxllm_stage_batch(const float* x /* [batch][cols] */, uint32_t batch, uint32_t cols, void* x16,
                              hipStream_t stream);
size_t rtxllm_matvec_batch_workspace(int format, uint32_t rows, uint32_t cols);
hipError_t rtxllm_matvec_batch(int format, const uint8_t* payload, const uint8_t* meta, const void* x16,
                               float* y /* [batch][rows] */, uint32_t rows, uint32_t cols, uint32_t batch,
                               void* workspace, size_t workspace_bytes, hipStream_t stream);
/* The same without a workspace argument, for callers that cannot allocate
 * (code under graph capture, tight serving loops, harnesses that forbid
 * hipMalloc); no counterpart in the reference. The panel groups' partial sums
 * go to a scratch array of RTXLLM_NOALLOC_SCRATCH_BYTES that the library
 * holds on every GPU it runs on until the process ends; its address is looked
 * up on the first call on each device. Calls whose 4 * batch * rows * panel
 * groups bytes exceed it are refused with hipErrorInvalidValue (matrices of
 * at most 4096 columns have one panel group and need none). Every call on a
 * GPU shares that GPU's array, so calls that overlap on one GPU (other
 * streams, other host threads) race; calls in one stream are ordered. Nothing
 * is allocated, freed or cleared: each call writes every partial sum it reads. */
#define RTXLLM_NOALLOC_SCRATCH_BYTES (8u << 20)
hipError_t rtxllm_matvec_batch_noalloc(int format, const uint8_t* payload, const uint8_t* meta, const void* x16,
                                       float* y /* [batch][rows] */, uint32_t rows, uint32_t cols, uint32_t batch,
                                       hipStream_t stream);
/* The same from the fp32 activation x [batch][cols] (16-byte aligned): every
 * wave stages its own 512 columns with the rtxllm_stage_batch rule, so the
 * result equals rtxllm_stage_batch + rtxllm_matvec_batch bit for bit without
 * the staging launch (the batch decode step's down projection). */
hipError_t rtxllm_matvec_batch_f32(int format, const uint8_t* payload, const uint8_t* meta, const float* x,
                                   float* y /* [batch][rows] */, uint32_t rows, uint32_t cols, uint32_t batch,
                                   void* workspace, size_t workspace_bytes, hipStream_t stream);

/* ---- Llama layer math (no counterpart in the reference; its stages are
 * composed from separate launchers the same way, decode_kernels.h:38-101,
 * 319-325, main.cpp:4073-4279). All asynchronous on `stream`. ---- */

/* out[r] = (x[r] * inv_rms) * weight (weight null: no weight), inv_rms = 1 /
 * sqrt(sum(x[r]^2) / n + eps), for count vectors x [count][n] (in place
 * allowed). */
hipError_t rtxllm_rmsnorm_w(const float* x, const float* weight, uint32_t n, uint32_t count, float eps,
                            float* out, hipStream_t stream);

/* In place on vec [count][n_heads][head_dim] (8-byte aligned): each adjacent
 * pair (2i, 2i+1) of every head of vector r rotated by the angle pos[r] *
 * theta^(-2i / head_dim) (pos a device array of count positions):
 * (e, o) -> (e cos - o sin, e sin + o cos). head_dim even. */
hipError_t rtxllm_rope_theta(float* vec, uint32_t n_heads, uint32_t head_dim, float theta, const uint32_t* pos,
                             uint32_t count, hipStream_t stream);

/* out[i] = silu(gate[i]) * up[i], silu(v) = v / (1 + exp(-v)) (in place allowed). */
hipError_t rtxllm_silu_mul(const float* gate, const float* up, size_t n, float* out, hipStream_t stream);

/* out[t][cols] = the Q5_K row tokens[t] of table [vocab][cols / 256 blocks]
 * dequantised (bit-exact with the reference's Q5_K formula, main.cpp:1231-1259),
 * for count device token ids; a token >= vocab gives a row of NaN. table
 * 4-byte aligned. */
hipError_t rtxllm_embed_gather_q5k(const uint8_t* table, uint32_t vocab, uint32_t cols, const uint32_t* tokens,
                                   uint32_t count, float* out, hipStream_t stream);

/* GQA decode attention of count queries (head_dim 128): q [count][n_heads][128]
 * fp32; query head h reads kv head h / (n_heads / n_kv_heads) (group 1, 2, 4
 * or 8); K and V fp16 caches of pages [page][n_kv_heads][page_size][128]
 * (16-byte aligned); query r attends positions 0..pos[r] (pos a device array,
 * pos[r] < capacity) through block-table row r (table_stride entries apart,
 * capacity / page_size entries used: logical page -> physical page); scores
 * scaled by 1 / sqrt(128), softmax with the maximum subtracted; out [count]
 * [n_heads][128] fp32. workspace: rtxllm_attn_decode_workspace() bytes. */
size_t rtxllm_attn_decode_workspace(uint32_t n_heads, uint32_t n_kv_heads, uint32_t capacity, uint32_t count);
hipError_t rtxllm_attn_decode_gqa_f16(const float* q, const uint16_t* k_cache, const uint16_t* v_cache,
                                      const int32_t* block_table, uint32_t table_stride, uint32_t n_heads,
                                      uint32_t n_kv_heads, uint32_t page_size, uint32_t capacity,
                                      const uint32_t* pos, uint32_t count, float* out, void* workspace,
                                      size_t workspace_bytes, hipStream_t stream);

/* index[r] = argmax of x [count][n] row r: the lowest index among equal maxima;
 * the scan starts from (-FLT_MAX, 0) as the reference's (decode_kernels.cu:
 * 2993-3031), so a NaN never wins and a row with nothing above -FLT_MAX gives 0. */
hipError_t rtxllm_argmax(const float* x, uint32_t n, uint32_t count, uint32_t* index, hipStream_t stream);

/* GGUF IQ2_S blocks (format 6) of a rows x cols tensor -> the same bytes in the
 * IQ2S_UNITS layout (format 9), device to device: per 32-value unit k of block b
 * of N blocks, qs[4k..4k+3] and signs[4k..4k+3] at 64 b + 8 k, (qh[k],
 * scales[k]) at 64 N + 16 b + 2 k, and the block's d at 80 N + 2 b. A matvec
 * then reads three aligned fields per unit instead of five. No counterpart in
 * the reference (its IQ packs keep the GGUF blocks, iq_resident_pack.py:115-147);
 * the decode runner keeps a unit copy of IQ2_S gate/up weights at batch 1. out
 * is 16-byte aligned and rows * cols / 256 * 82 bytes. */
hipError_t rtxllm_iq2s_units_pack(const uint8_t* raw, uint32_t rows, uint32_t cols, uint8_t* out,
                                  hipStream_t stream);
/* The same for GGUF IQ3_S blocks (format 7) -> IQ3S_UNITS (format 10, 114 B per
 * block): per unit k of block b, qs[8k..8k+7] and signs[4k..4k+3] at 96 b +
 * 12 k, (qh[k], scales[k / 2]) at 96 N + 16 b + 2 k, d at 112 N + 2 b. A unit
 * then reads three aligned fields instead of five, for 4 more bytes per block
 * (each scale byte is stored for both units that share it). The runner keeps
 * unit copies of IQ3_S qkv and o weights at batch 1. */
hipError_t rtxllm_iq3s_units_pack(const uint8_t* raw, uint32_t rows, uint32_t cols, uint8_t* out,
                                  hipStream_t stream);

/* Host-side helpers (no device work). */
uint32_t rtxllm_format_payload_block_bytes(int format);
uint32_t rtxllm_format_meta_block_bytes(int format);
/* Split raw Q4_K blocks into a payload stream and format-`format` metadata
 * (tools/bench/q4k_resident_pack.py:100-145). Host memory. Returns 0 or -1. */
int rtxllm_q4k_split_pack(int format, const uint8_t* raw_blocks, size_t n_blocks, uint8_t* payload,
                          uint8_t* meta);
/* Seeded synthetic raw blocks (format 0, 5, 6, 7) into host memory, d/dmin =
 * fp16(U[d_lo, d_hi]); threads <= 0 picks the hardware concurrency. */
int rtxllm_synth_raw_blocks(int format, uint64_t seed, size_t n_blocks, float d_lo, float d_hi,
                            uint8_t* out, int threads);
/* Seeded N(mean, std^2) fp32 values, or fp16 bits of them. */
int rtxllm_synth_normal_f32(uint64_t seed, size_t n, float mean, float stddev, float* out, int threads);
int rtxllm_synth_normal_f16(uint64_t seed, size_t n, float mean, float stddev, uint16_t* out, int threads);

#ifdef __cplusplus
}
#endif

#endif
