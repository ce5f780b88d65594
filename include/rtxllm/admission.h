/* Strict VRAM admission of a decode runner: required = weights + KV (cache
 * already held plus tokens x bytes per token) + workspace + DMA staging +
 * graph memory, against usable = free - guard.
 *
 * Keeps the interface of the reference's admission
 * (runtime/core/scheduler/admission.h:10-65, admission.cpp:26-98): the same
 * types, fields, decision rule and reasons. The guard defaults to 0 here: the
 * reference's 512 MiB is a Windows display-driver reserve, and a Linux ROCm
 * process has none. Header-only, host code, C++17. */
#ifndef RTXLLM_ADMISSION_H
#define RTXLLM_ADMISSION_H

#include <cstddef>
#include <limits>
#include <stdexcept>
#include <string>

namespace rtxllm {

enum class ResidencyPolicy { Strict, Balanced, Overflow };

struct MemoryBudget {
  std::size_t vram_free_bytes = 0;
  std::size_t wddm_guard_bytes = 0;  // bytes kept back from the free figure
};

struct RequestEstimate {
  std::size_t weight_bytes = 0;
  std::size_t prompt_tokens = 0;
  std::size_t max_new_tokens = 0;
  std::size_t kv_bytes_per_token = 0;
  std::size_t workspace_bytes = 0;
  std::size_t kv_cache_bytes = 0;
  std::size_t dma_bytes = 0;
  std::size_t graph_bytes = 0;
  std::size_t workspace_high_water_bytes = 0;
};

struct AdmissionBreakdown {
  std::size_t weight_bytes = 0;
  std::size_t prompt_tokens = 0;
  std::size_t max_new_tokens = 0;
  std::size_t token_count = 0;
  std::size_t kv_bytes_per_token = 0;
  std::size_t predicted_kv_bytes = 0;
  std::size_t kv_cache_bytes = 0;
  std::size_t total_kv_bytes = 0;
  std::size_t workspace_bytes = 0;
  std::size_t workspace_high_water_bytes = 0;
  std::size_t workspace_slack_bytes = 0;
  std::size_t dma_bytes = 0;
  std::size_t graph_bytes = 0;
  std::size_t required_bytes = 0;
  std::size_t vram_free_bytes = 0;
  std::size_t wddm_guard_bytes = 0;
  std::size_t usable_bytes = 0;
  std::size_t over_budget_bytes = 0;
};

struct AdmissionDecision {
  bool admit = false;
  bool host_spill_allowed = false;
  std::size_t required_bytes = 0;
  std::size_t usable_bytes = 0;
  AdmissionBreakdown breakdown;
  std::string reason;
};

namespace admission_detail {
inline std::size_t add(std::size_t a, std::size_t b) {
  if (a > std::numeric_limits<std::size_t>::max() - b) throw std::overflow_error("admission byte count overflow");
  return a + b;
}
inline std::size_t mul(std::size_t a, std::size_t b) {
  if (a != 0 && b > std::numeric_limits<std::size_t>::max() / a) throw std::overflow_error("admission byte count overflow");
  return a * b;
}
inline std::size_t sub0(std::size_t a, std::size_t b) { return a > b ? a - b : 0; }
}  // namespace admission_detail

// Admit when required <= usable; over budget, only the Overflow policy admits
// (with host spill allowed). Strict and Balanced reject with the figures.
inline AdmissionDecision decide_admission(ResidencyPolicy policy, const MemoryBudget& budget,
                                          const RequestEstimate& request) {
  using namespace admission_detail;
  AdmissionBreakdown b;
  b.weight_bytes = request.weight_bytes;
  b.prompt_tokens = request.prompt_tokens;
  b.max_new_tokens = request.max_new_tokens;
  b.token_count = add(request.prompt_tokens, request.max_new_tokens);
  b.kv_bytes_per_token = request.kv_bytes_per_token;
  b.predicted_kv_bytes = mul(b.token_count, request.kv_bytes_per_token);
  b.kv_cache_bytes = request.kv_cache_bytes;
  b.total_kv_bytes = add(b.predicted_kv_bytes, request.kv_cache_bytes);
  b.workspace_bytes = request.workspace_bytes;
  b.workspace_high_water_bytes = request.workspace_high_water_bytes;
  b.workspace_slack_bytes = sub0(request.workspace_bytes, request.workspace_high_water_bytes);
  b.dma_bytes = request.dma_bytes;
  b.graph_bytes = request.graph_bytes;
  b.vram_free_bytes = budget.vram_free_bytes;
  b.wddm_guard_bytes = budget.wddm_guard_bytes;
  b.usable_bytes = sub0(budget.vram_free_bytes, budget.wddm_guard_bytes);
  b.required_bytes = add(add(add(add(b.weight_bytes, b.total_kv_bytes), b.workspace_bytes), b.dma_bytes), b.graph_bytes);
  b.over_budget_bytes = sub0(b.required_bytes, b.usable_bytes);

  AdmissionDecision d;
  d.required_bytes = b.required_bytes;
  d.usable_bytes = b.usable_bytes;
  d.breakdown = b;
  if (b.required_bytes <= b.usable_bytes) {
    d.admit = true;
    d.reason = "fits strict VRAM budget";
  } else if (policy == ResidencyPolicy::Overflow) {
    d.admit = true;
    d.host_spill_allowed = true;
    d.reason = "requires explicit overflow policy";
  } else {
    d.reason = "rejected: required " + std::to_string(b.required_bytes) + " bytes, usable " +
               std::to_string(b.usable_bytes) + " bytes, over budget " + std::to_string(b.over_budget_bytes) +
               " bytes";
  }
  return d;
}

}  // namespace rtxllm

#endif
