/* Layer role plan of the layer-slice runner: which execution phase each
 * stage's weight role belongs to, the contiguous phase segments of a stage
 * list, their validation, and the kernel-count plan of one replay.
 *
 * Keeps the interface of the reference's role plan
 * (runtime/core/scheduler/layer_plan.h:10-80, layer_plan.cpp:27-198): the
 * same types, function names and argument meaning. Role ranks cover the
 * reference's roles (layer_plan.cpp:27-65) plus the Llama decoder roles of
 * GGUF (attn_q / attn_k / attn_v, their stacked attn_qkv, attn_output,
 * ffn_gate / ffn_up, the interleaved ffn_gate_up, ffn_down). The expected
 * phase order is attention -> ffn [-> ssm] [-> output]: the reference requires
 * the ssm phase of its hybrid model; a Llama layer has none, so here it is
 * expected only when present. Header-only, host code, C++17. */
#ifndef RTXLLM_LAYER_PLAN_H
#define RTXLLM_LAYER_PLAN_H

#include <cstddef>
#include <map>
#include <string>
#include <string_view>
#include <vector>

namespace rtxllm {

enum class LayerPhase { Attention, Ffn, Ssm, Output, Unknown };

struct LayerStageDescriptor {
  std::string_view role;
  bool layer_local = true;  // a role outside the layer (the LM head) is not ranked
};

struct LayerPhaseSegment {
  LayerPhase phase = LayerPhase::Unknown;
  std::size_t begin = 0;
  std::size_t count = 0;
};

struct LayerPlanValidation {
  bool passed = false;
  std::string message;
  std::vector<LayerPhase> expected_phases;
  std::vector<LayerPhase> observed_phases;
};

struct LayerPhaseExecution {
  LayerPhase phase = LayerPhase::Unknown;
  std::size_t begin = 0;
  std::size_t count = 0;
  std::size_t matvec_kernels_per_replay = 0;
  std::size_t activation_feedbacks_per_replay = 0;
  std::size_t total_kernels_per_replay = 0;
};

struct LayerExecutionPlan {
  std::vector<LayerPhaseExecution> phases;
  std::size_t stage_count = 0;
  std::size_t phase_count = 0;
  std::size_t matvec_kernels_per_replay = 0;
  std::size_t activation_feedbacks_per_replay = 0;
  std::size_t total_kernels_per_replay = 0;
};

inline const char* layer_phase_name(LayerPhase phase) {
  static const char* const kNames[] = {"attention", "ffn", "ssm", "output", "unknown"};
  return kNames[static_cast<int>(phase)];
}

namespace layer_plan_detail {
constexpr int kUnknownRank = 5000;
constexpr int kOutputRank = 10000;
struct RoleRank {
  const char* role;
  int rank;
};
// Order of the stages inside a layer. Reference roles keep their ranks; the
// Llama roles are placed around them in execution order.
constexpr RoleRank kRanks[] = {
    {"attn_gate.weight", 10},    {"attn_q.weight", 15},          {"attn_k.weight", 16},
    {"attn_v.weight", 17},       {"attn_qkv.weight", 20},        {"attn_output.weight", 25},
    {"ffn_gate_exps.weight", 30}, {"ffn_gate.weight", 35},       {"ffn_gate_shexp.weight", 40},
    {"ffn_gate_up.weight", 45},  {"ffn_up_exps.weight", 50},     {"ffn_up.weight", 55},
    {"ffn_up_shexp.weight", 60}, {"ffn_down_exps.weight", 70},   {"ffn_down.weight", 75},
    {"ffn_down_shexp.weight", 80}, {"ssm_alpha.weight", 90},     {"ssm_beta.weight", 100},
    {"ssm_out.weight", 110},
};
inline bool starts_with(std::string_view s, std::string_view prefix) {
  return s.size() >= prefix.size() && s.compare(0, prefix.size(), prefix) == 0;
}
}  // namespace layer_plan_detail

// Rank of a role inside a layer (5000 for a role the plan does not know, 10000
// for the LM head "output" / "output.weight").
inline int layer_role_rank(std::string_view role) {
  if (role == "output" || role == "output.weight") return layer_plan_detail::kOutputRank;
  for (const auto& r : layer_plan_detail::kRanks)
    if (role == r.role) return r.rank;
  return layer_plan_detail::kUnknownRank;
}

inline LayerPhase layer_phase_from_role(std::string_view role) {
  using layer_plan_detail::starts_with;
  if (role == "output" || role == "output.weight") return LayerPhase::Output;
  if (starts_with(role, "attn_")) return LayerPhase::Attention;
  if (starts_with(role, "ffn_")) return LayerPhase::Ffn;
  if (starts_with(role, "ssm_")) return LayerPhase::Ssm;
  return LayerPhase::Unknown;
}

inline std::size_t count_unknown_layer_roles(const std::vector<LayerStageDescriptor>& stages) {
  std::size_t n = 0;
  for (const auto& s : stages) n += (s.layer_local && layer_role_rank(s.role) == layer_plan_detail::kUnknownRank);
  return n;
}

inline std::size_t count_unknown_layer_phases(const std::vector<LayerStageDescriptor>& stages) {
  std::size_t n = 0;
  for (const auto& s : stages) n += layer_phase_from_role(s.role) == LayerPhase::Unknown;
  return n;
}

inline std::map<std::string, std::size_t> build_layer_phase_counts(const std::vector<LayerStageDescriptor>& stages) {
  std::map<std::string, std::size_t> counts;
  for (const auto& s : stages) ++counts[layer_phase_name(layer_phase_from_role(s.role))];
  return counts;
}

// Maximal runs of consecutive stages in one phase.
inline std::vector<LayerPhaseSegment> build_layer_phase_segments(const std::vector<LayerStageDescriptor>& stages) {
  std::vector<LayerPhaseSegment> out;
  for (std::size_t i = 0; i < stages.size(); ++i) {
    const LayerPhase p = layer_phase_from_role(stages[i].role);
    if (!out.empty() && out.back().phase == p)
      ++out.back().count;
    else
      out.push_back({p, i, 1});
  }
  return out;
}

// Passes iff every stage has a known role and phase and the segments are
// attention, ffn, then ssm if any stage is an ssm stage, then output if the
// last segment is the output.
inline LayerPlanValidation validate_layer_phase_plan(const std::vector<LayerStageDescriptor>& stages,
                                                     const std::vector<LayerPhaseSegment>& segments) {
  LayerPlanValidation v;
  v.expected_phases = {LayerPhase::Attention, LayerPhase::Ffn};
  bool has_ssm = false;
  for (const auto& s : stages) has_ssm = has_ssm || layer_phase_from_role(s.role) == LayerPhase::Ssm;
  if (has_ssm) v.expected_phases.push_back(LayerPhase::Ssm);
  if (!segments.empty() && segments.back().phase == LayerPhase::Output) v.expected_phases.push_back(LayerPhase::Output);
  for (const auto& seg : segments) v.observed_phases.push_back(seg.phase);
  auto fail = [&](const char* why) {
    v.message = why;
    return v;
  };
  if (stages.empty()) return fail("layer phase plan requires at least one stage");
  if (count_unknown_layer_roles(stages) != 0) return fail("layer phase plan contains unknown role-plan roles");
  if (count_unknown_layer_phases(stages) != 0) return fail("layer phase plan contains unknown execution phases");
  if (segments.size() != v.expected_phases.size()) return fail("layer phase plan segment count mismatch");
  for (std::size_t i = 0; i < segments.size(); ++i) {
    if (segments[i].phase != v.expected_phases[i]) return fail("layer phase plan phase order mismatch");
    if (segments[i].count == 0) return fail("layer phase plan contains an empty phase segment");
  }
  v.passed = true;
  v.message = "layer phase plan validated";
  return v;
}

// One matvec per stage, plus one activation feedback per stage when the
// stages are chained.
inline LayerExecutionPlan build_layer_execution_plan(const std::vector<LayerPhaseSegment>& segments,
                                                     bool chain_activation) {
  LayerExecutionPlan plan;
  plan.phase_count = segments.size();
  for (const auto& seg : segments) {
    LayerPhaseExecution e;
    e.phase = seg.phase;
    e.begin = seg.begin;
    e.count = seg.count;
    e.matvec_kernels_per_replay = seg.count;
    e.activation_feedbacks_per_replay = chain_activation ? seg.count : 0;
    e.total_kernels_per_replay = e.matvec_kernels_per_replay + e.activation_feedbacks_per_replay;
    plan.stage_count += e.count;
    plan.matvec_kernels_per_replay += e.matvec_kernels_per_replay;
    plan.activation_feedbacks_per_replay += e.activation_feedbacks_per_replay;
    plan.total_kernels_per_replay += e.total_kernels_per_replay;
    plan.phases.push_back(e);
  }
  return plan;
}

}  // namespace rtxllm

#endif
