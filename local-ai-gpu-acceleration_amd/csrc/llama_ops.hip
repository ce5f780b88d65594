// Standalone C-ABI entry points for the Llama layer math that the decode runner
// otherwise fuses into its matvec epilogues: weighted RMSNorm, rotary embedding
// with a theta schedule, SiLU-gate multiply, the Q5_K embedding gather, GQA
// decode attention over a paged fp16 KV cache and greedy argmax. Each is one or
// two kernel launches on the caller's stream with caller-owned device memory
// (no allocation, no synchronisation: capture-safe).
//
// The reference runtime composes its per-stage math from separate launchers
// (rtxllm_launch_rmsnorm_feedback / output_token_sample etc.,
// runtime/kernels/decode/decode_kernels.h:38-101, 319-325, called per stage
// from launch_feedback, mixed_sequence_benchmark_runner/main.cpp:4073-4279);
// these entry points are the Llama-layer counterparts of that style. Formulas:
// weighted RMSNorm (x * inv_rms) * w with inv_rms = 1 / sqrt(mean(x^2) + eps)
// (main.cpp:1363-1382 plus the weight), rotary pairs (e c - o s, e s + o c)
// (decode_kernels.cu:327-343) at angle pos * theta^(-2i/d), silu(v) = v / (1 +
// exp(-v)) (main.cpp:1435-1503), Q5_K dequant (main.cpp:1231-1259), argmax with
// the lowest index among maxima (decode_kernels.cu:2993-3031).
#include <cfloat>

#include "dequant.cuh"
#include "layer.h"
#include "layer_common.cuh"
#include "rtxllm/decode_kernels.h"

namespace rtxllm {
namespace {

constexpr std::uint32_t kOpThreads = 256;

__device__ float block_sum256(float v, float* sh) {
  v = wave_sum(v);
  const std::uint32_t lane = threadIdx.x & 63u, wave = threadIdx.x >> 6;
  if (lane == 0u) sh[wave] = v;
  __syncthreads();
  const float s = (sh[0] + sh[1]) + (sh[2] + sh[3]);
  __syncthreads();
  return s;
}

// One workgroup per vector r of x [count][n].
__global__ __launch_bounds__(kOpThreads) void rmsnorm_w_kernel(const float* __restrict__ x, const float* __restrict__ w,
                                                               std::uint32_t n, float eps, float* __restrict__ out) {
  __shared__ float sh[kOpThreads / 64];
  const std::size_t base = static_cast<std::size_t>(blockIdx.x) * n;
  float s = 0.0f;
  for (std::uint32_t i = threadIdx.x; i < n; i += kOpThreads) {
    const float v = x[base + i];
    s = fmaf(v, v, s);
  }
  const float inv = 1.0f / sqrtf(block_sum256(s, sh) / static_cast<float>(n) + eps);
  for (std::uint32_t i = threadIdx.x; i < n; i += kOpThreads) {
    const float v = x[base + i] * inv;
    out[base + i] = w != nullptr ? v * w[i] : v;
  }
}

// One thread per rotary pair (vector r = blockIdx.y, pair p of n_heads *
// head_dim / 2); inv_freq = theta^(-2i/d) in double, rounded once, and the
// angle (float)pos * inv_freq in fp32, as the textbook rotary is evaluated;
// (cos, sin) of that fp32 angle in double, each rounded once.
__global__ __launch_bounds__(kOpThreads) void rope_theta_kernel(float* __restrict__ vec, std::uint32_t pairs,
                                                                std::uint32_t head_dim, double theta,
                                                                const std::uint32_t* __restrict__ pos) {
  const std::uint32_t p = blockIdx.x * kOpThreads + threadIdx.x;
  if (p >= pairs) return;
  const std::uint32_t r = blockIdx.y, i = p % (head_dim / 2u);
  const float inv_freq = static_cast<float>(pow(theta, -2.0 * static_cast<double>(i) / static_cast<double>(head_dim)));
  const float angle = static_cast<float>(pos[r]) * inv_freq;
  const float c = static_cast<float>(cos(static_cast<double>(angle)));
  const float s = static_cast<float>(sin(static_cast<double>(angle)));
  float2* v = reinterpret_cast<float2*>(vec + static_cast<std::size_t>(r) * 2u * pairs) + p;
  const float2 eo = *v;
  *v = make_float2(eo.x * c - eo.y * s, eo.x * s + eo.y * c);
}

__global__ __launch_bounds__(kOpThreads) void silu_mul_kernel(const float* __restrict__ gate, const float* __restrict__ up,
                                                              std::size_t n, float* __restrict__ out) {
  const std::size_t i = static_cast<std::size_t>(blockIdx.x) * kOpThreads + threadIdx.x;
  if (i < n) out[i] = silu(gate[i]) * up[i];
}

// Workgroup (block b of the row, token t): 256 threads, one value each.
__global__ __launch_bounds__(256) void embed_gather_q5k_kernel(const std::uint8_t* __restrict__ table,
                                                               std::uint32_t vocab, std::uint32_t cols,
                                                               const std::uint32_t* __restrict__ tokens,
                                                               float* __restrict__ out) {
  const std::uint32_t b = blockIdx.x, t = blockIdx.y, bpr = cols / 256u;
  const std::uint32_t tok = tokens[t];
  float* o = out + static_cast<std::size_t>(t) * cols + 256u * b + threadIdx.x;
  if (tok >= vocab) {  // no such row: a loud NaN row instead of a silent clamp
    *o = __builtin_nanf("");
    return;
  }
  const std::uint8_t* blk = table + (static_cast<std::size_t>(tok) * bpr + b) * 176u;
  *o = dequant_value<RTXLLM_FMT_Q5K>(blk, nullptr, threadIdx.x);
}

// fp32 queries q [count][n_heads][128] -> the attention's query operand (q16):
// one thread per fp16 slot of the operand image of one vector (n_kv * 2048
// slots; slot = ((g * 4 + j) * 64 + l) * 8 + i holds dim 32 (l / 16) + 8 j + i
// of column n = l % 16 = 2 h + part of kv head g, zero for h >= group).
__global__ __launch_bounds__(kOpThreads) void q16_stage_kernel(const float* __restrict__ q, std::uint32_t n_kv,
                                                               std::uint32_t group, _Float16* __restrict__ q16) {
  const std::uint32_t slots = n_kv * (kQ16PerKv);
  const std::uint32_t idx = blockIdx.x * kOpThreads + threadIdx.x;
  if (idx >= slots) return;
  const std::uint32_t r = blockIdx.y;
  const std::uint32_t i = idx & 7u, l = (idx >> 3) & 63u, j = (idx >> 9) & 3u, g = idx >> 11;
  const std::uint32_t d = 32u * (l >> 4) + 8u * j + i, n = l & 15u, h = n >> 1, part = n & 1u;
  _Float16 v = static_cast<_Float16>(0.0f);
  if (h < group) {
    const float x = q[(static_cast<std::size_t>(r) * n_kv * group + g * group + h) * kHeadDim + d] *
                    0.08838834764831845f;  // 1 / sqrt(128)
    const _Float16 hi = static_cast<_Float16>(x);
    v = part == 0u ? hi : static_cast<_Float16>(x - static_cast<float>(hi));
  }
  q16[static_cast<std::size_t>(r) * slots + idx] = v;
}

// One workgroup per vector: the reference's argmax scan (start (-FLT_MAX, 0),
// strictly greater wins, equal values keep the lower index; NaN never wins).
__global__ __launch_bounds__(1024) void argmax_rows_kernel(const float* __restrict__ x, std::uint32_t n,
                                                           std::uint32_t* __restrict__ index) {
  __shared__ float sv[16];
  __shared__ std::uint32_t si[16];
  auto better = [](float v, std::uint32_t i, float bv, std::uint32_t bi) { return v > bv || (v == bv && i < bi); };
  const float* row = x + static_cast<std::size_t>(blockIdx.x) * n;
  float bv = -FLT_MAX;
  std::uint32_t bi = 0u;
  for (std::uint32_t r = threadIdx.x; r < n; r += blockDim.x) {
    const float v = row[r];
    if (better(v, r, bv, bi)) bv = v, bi = r;
  }
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) {
    const float ov = __shfl_xor(bv, o, 64);
    const std::uint32_t oi = __shfl_xor(bi, o, 64);
    if (better(ov, oi, bv, bi)) bv = ov, bi = oi;
  }
  const std::uint32_t lane = threadIdx.x & 63u, wave = threadIdx.x >> 6;
  if (lane == 0u) sv[wave] = bv, si[wave] = bi;
  __syncthreads();
  if (threadIdx.x != 0u) return;
  for (std::uint32_t w = 1; w < blockDim.x / 64u; ++w)
    if (better(sv[w], si[w], bv, bi)) bv = sv[w], bi = si[w];
  index[blockIdx.x] = bi;
}

bool group_ok(std::uint32_t n_heads, std::uint32_t n_kv) {
  if (n_kv == 0u || n_heads == 0u || n_heads % n_kv != 0u) return false;
  const std::uint32_t g = n_heads / n_kv;
  return g == 1u || g == 2u || g == 4u || g == 8u;
}

std::size_t align256(std::size_t b) { return (b + 255u) & ~std::size_t{255}; }

}  // namespace
}  // namespace rtxllm

using namespace rtxllm;

extern "C" hipError_t rtxllm_rmsnorm_w(const float* x, const float* weight, uint32_t n, uint32_t count, float eps,
                                       float* out, hipStream_t stream) {
  if (x == nullptr || out == nullptr || n == 0u || count == 0u || count > 65535u * 1024u || !(eps >= 0.0f))
    return hipErrorInvalidValue;
  hipLaunchKernelGGL(rmsnorm_w_kernel, dim3(count), dim3(kOpThreads), 0, stream, x, weight, n, eps, out);
  return hipGetLastError();
}

extern "C" hipError_t rtxllm_rope_theta(float* vec, uint32_t n_heads, uint32_t head_dim, float theta,
                                        const uint32_t* pos, uint32_t count, hipStream_t stream) {
  if (vec == nullptr || pos == nullptr || n_heads == 0u || head_dim == 0u || (head_dim % 2u) != 0u || count == 0u ||
      count > 65535u || !(theta > 0.0f) || (reinterpret_cast<std::uintptr_t>(vec) % 8u) != 0u)
    return hipErrorInvalidValue;
  const std::uint64_t pairs = static_cast<std::uint64_t>(n_heads) * head_dim / 2u;
  if (pairs > 0xFFFFFFFFull / 2u) return hipErrorInvalidValue;
  const dim3 grid(static_cast<unsigned>((pairs + kOpThreads - 1u) / kOpThreads), count);
  hipLaunchKernelGGL(rope_theta_kernel, grid, dim3(kOpThreads), 0, stream, vec, static_cast<std::uint32_t>(pairs),
                     head_dim, static_cast<double>(theta), pos);
  return hipGetLastError();
}

extern "C" hipError_t rtxllm_silu_mul(const float* gate, const float* up, size_t n, float* out, hipStream_t stream) {
  if (gate == nullptr || up == nullptr || out == nullptr || n == 0u || n > (std::size_t{1} << 40))
    return hipErrorInvalidValue;
  hipLaunchKernelGGL(silu_mul_kernel, dim3(static_cast<unsigned>((n + kOpThreads - 1u) / kOpThreads)),
                     dim3(kOpThreads), 0, stream, gate, up, n, out);
  return hipGetLastError();
}

extern "C" hipError_t rtxllm_embed_gather_q5k(const uint8_t* table, uint32_t vocab, uint32_t cols,
                                              const uint32_t* tokens, uint32_t count, float* out,
                                              hipStream_t stream) {
  if (table == nullptr || tokens == nullptr || out == nullptr || vocab == 0u || cols == 0u || (cols % 256u) != 0u ||
      count == 0u || count > 65535u || (reinterpret_cast<std::uintptr_t>(table) % 4u) != 0u)
    return hipErrorInvalidValue;
  hipLaunchKernelGGL(embed_gather_q5k_kernel, dim3(cols / 256u, count), dim3(256), 0, stream, table, vocab, cols,
                     tokens, out);
  return hipGetLastError();
}

extern "C" size_t rtxllm_attn_decode_workspace(uint32_t n_heads, uint32_t n_kv_heads, uint32_t capacity,
                                               uint32_t count) {
  if (!group_ok(n_heads, n_kv_heads) || capacity == 0u || count == 0u) return 0u;
  return align256(static_cast<std::size_t>(count) * n_kv_heads * kQ16BytesPerKv) +
         4u * static_cast<std::size_t>(count) * attention_partials_floats(n_heads, n_kv_heads, capacity);
}

extern "C" hipError_t rtxllm_attn_decode_gqa_f16(const float* q, const uint16_t* k_cache, const uint16_t* v_cache,
                                                 const int32_t* block_table, uint32_t table_stride,
                                                 uint32_t n_heads, uint32_t n_kv_heads, uint32_t page_size,
                                                 uint32_t capacity, const uint32_t* pos, uint32_t count, float* out,
                                                 void* workspace, size_t workspace_bytes, hipStream_t stream) {
  if (q == nullptr || k_cache == nullptr || v_cache == nullptr || block_table == nullptr || pos == nullptr ||
      out == nullptr || workspace == nullptr || !group_ok(n_heads, n_kv_heads) || page_size == 0u ||
      capacity == 0u || capacity % page_size != 0u || count == 0u || count > 65535u ||
      (count > 1u && table_stride < capacity / page_size) ||
      (reinterpret_cast<std::uintptr_t>(k_cache) % 16u) != 0u || (reinterpret_cast<std::uintptr_t>(v_cache) % 16u) != 0u ||
      (reinterpret_cast<std::uintptr_t>(workspace) % 256u) != 0u)
    return hipErrorInvalidValue;
  const std::size_t need = rtxllm_attn_decode_workspace(n_heads, n_kv_heads, capacity, count);
  if (need == 0u || workspace_bytes < need) return hipErrorInvalidValue;
  auto* q16 = static_cast<_Float16*>(workspace);
  auto* partials = reinterpret_cast<float*>(static_cast<std::uint8_t*>(workspace) +
                                            align256(static_cast<std::size_t>(count) * n_kv_heads * kQ16BytesPerKv));
  const std::uint32_t slots = n_kv_heads * kQ16PerKv;
  hipLaunchKernelGGL(q16_stage_kernel, dim3((slots + kOpThreads - 1u) / kOpThreads, count), dim3(kOpThreads), 0, stream,
                     q, n_kv_heads, n_heads / n_kv_heads, q16);
  hipError_t st = hipGetLastError();
  if (st != hipSuccess) return st;
  KvLayer kv{};
  kv.k = const_cast<std::uint16_t*>(k_cache);
  kv.v = const_cast<std::uint16_t*>(v_cache);
  kv.block_table = block_table;
  kv.page_size = page_size;
  kv.n_kv = n_kv_heads;
  kv.capacity = capacity;
  return launch_attention_batch(q16, kv, n_heads, pos, capacity, count, table_stride, partials, out, nullptr, nullptr,
                                stream);
}

extern "C" hipError_t rtxllm_argmax(const float* x, uint32_t n, uint32_t count, uint32_t* index,
                                    hipStream_t stream) {
  if (x == nullptr || index == nullptr || n == 0u || count == 0u || count > 65535u * 1024u)
    return hipErrorInvalidValue;
  hipLaunchKernelGGL(argmax_rows_kernel, dim3(count), dim3(1024), 0, stream, x, n, index);
  return hipGetLastError();
}
