/* Layer executor contract of the layer-slice runner: per-phase workspace
 * descriptors and their 256-B-aligned activation / logits slices plus named
 * auxiliary slices, binding to device pointers, the activation feedback
 * dataflow (stage i -> stage i + 1 mod n), workspace usage, and replay through
 * launch callbacks with counter validation.
 *
 * Keeps the interface of the reference's executor
 * (runtime/core/scheduler/layer_executor.h:18-1005): the same types, function
 * names, argument meaning and failure conditions (std::runtime_error). Spans
 * are std::vector references here (C++17). Header-only, host code. */
#ifndef RTXLLM_LAYER_EXECUTOR_H
#define RTXLLM_LAYER_EXECUTOR_H

#include <algorithm>
#include <cstddef>
#include <cstdint>
#include <limits>
#include <stdexcept>
#include <string>
#include <string_view>
#include <utility>
#include <vector>

#include "rtxllm/layer_plan.h"

namespace rtxllm {

struct LayerStageWorkspaceDescriptor {
  std::uint32_t rows = 0;  // output values of the stage's matvec
  std::uint32_t cols = 0;  // input values
};

struct LayerPhaseWorkspaceDescriptor {
  LayerPhase phase = LayerPhase::Unknown;
  std::size_t begin = 0;
  std::size_t count = 0;
  std::uint32_t max_rows = 0;
  std::uint32_t max_cols = 0;
  std::uint64_t logical_values_per_replay = 0;  // sum of rows * cols
};

struct LayerAuxWorkspaceDescriptor {
  std::string name;
  LayerPhase phase = LayerPhase::Unknown;
  std::uint32_t values = 0;
};

struct LayerExecutorWorkspacePlan {
  std::vector<LayerPhaseWorkspaceDescriptor> phases;
  std::uint32_t max_rows = 0;
  std::uint32_t max_cols = 0;
  std::uint64_t logical_values_per_replay = 0;
};

struct LayerPhaseWorkspaceAllocation {
  LayerPhase phase = LayerPhase::Unknown;
  std::size_t begin = 0;
  std::size_t count = 0;
  std::size_t activation_offset = 0;
  std::size_t activation_bytes = 0;
  std::size_t logits_offset = 0;
  std::size_t logits_bytes = 0;
  std::size_t total_bytes = 0;
};

struct LayerAuxWorkspaceAllocation {
  std::string name;
  LayerPhase phase = LayerPhase::Unknown;
  std::uint32_t values = 0;
  std::size_t offset = 0;
  std::size_t bytes = 0;
};

struct LayerExecutorWorkspaceAllocationPlan {
  std::vector<LayerPhaseWorkspaceAllocation> phases;
  std::vector<LayerAuxWorkspaceAllocation> auxiliaries;
  std::size_t activation_bytes = 0;
  std::size_t logits_bytes = 0;
  std::size_t phase_bytes = 0;
  std::size_t auxiliary_bytes = 0;
  std::size_t total_bytes = 0;
};

struct LayerPhaseWorkspaceRuntime {
  LayerPhase phase = LayerPhase::Unknown;
  std::size_t begin = 0;
  std::size_t count = 0;
  float* activation = nullptr;
  float* logits = nullptr;
  std::uint32_t max_rows = 0;
  std::uint32_t max_cols = 0;
  std::size_t activation_offset = 0;
  std::size_t activation_bytes = 0;
  std::size_t logits_offset = 0;
  std::size_t logits_bytes = 0;
  std::size_t total_bytes = 0;
};

struct LayerAuxWorkspaceRuntime {
  std::string name;
  LayerPhase phase = LayerPhase::Unknown;
  float* data = nullptr;
  std::uint32_t values = 0;
  std::size_t offset = 0;
  std::size_t bytes = 0;
};

struct LayerExecutorWorkspaceRuntime {
  std::vector<LayerPhaseWorkspaceRuntime> phases;
  std::vector<LayerAuxWorkspaceRuntime> auxiliaries;
  std::size_t activation_bytes = 0;
  std::size_t logits_bytes = 0;
  std::size_t phase_bytes = 0;
  std::size_t auxiliary_bytes = 0;
  std::size_t total_bytes = 0;
};

struct LayerPhaseWorkspaceUsage {
  LayerPhase phase = LayerPhase::Unknown;
  std::size_t begin = 0;
  std::size_t count = 0;
  std::size_t activation_high_water_bytes = 0;
  std::size_t logits_high_water_bytes = 0;
  std::size_t total_high_water_bytes = 0;
  std::size_t activation_slack_bytes = 0;
  std::size_t logits_slack_bytes = 0;
  std::size_t total_slack_bytes = 0;
};

struct LayerAuxWorkspaceUsage {
  std::string name;
  LayerPhase phase = LayerPhase::Unknown;
  std::size_t high_water_bytes = 0;
  std::size_t slack_bytes = 0;
};

struct LayerExecutorWorkspaceUsage {
  std::vector<LayerPhaseWorkspaceUsage> phases;
  std::vector<LayerAuxWorkspaceUsage> auxiliaries;
  std::size_t activation_high_water_bytes = 0;
  std::size_t logits_high_water_bytes = 0;
  std::size_t auxiliary_high_water_bytes = 0;
  std::size_t total_high_water_bytes = 0;
  std::size_t activation_slack_bytes = 0;
  std::size_t logits_slack_bytes = 0;
  std::size_t auxiliary_slack_bytes = 0;
  std::size_t total_slack_bytes = 0;
};

struct LayerActivationFeedbackEdge {
  std::size_t source_stage = 0;
  std::size_t target_stage = 0;
  std::size_t source_phase_index = 0;
  std::size_t target_phase_index = 0;
  LayerPhase source_phase = LayerPhase::Unknown;
  LayerPhase target_phase = LayerPhase::Unknown;
  std::uint32_t source_rows = 0;
  std::uint32_t target_cols = 0;
  std::uint32_t stage_id = 0;
  bool crosses_phase = false;
  bool wraps_to_first_stage = false;
};

struct LayerExecutorDataflowPlan {
  std::vector<LayerActivationFeedbackEdge> activation_feedback_edges;
  std::size_t phase_crossing_feedbacks = 0;
  std::size_t wrap_feedbacks = 0;
};

struct LayerReplayCounters {
  std::size_t phase_callbacks = 0;
  std::size_t attention_phase_callbacks = 0;
  std::size_t ffn_phase_callbacks = 0;
  std::size_t ssm_phase_callbacks = 0;
  std::size_t output_phase_callbacks = 0;
  std::size_t stage_callbacks = 0;
  std::size_t activation_feedback_callbacks = 0;
  std::size_t total_callbacks = 0;
};

namespace executor_detail {
[[noreturn]] inline void fail(const char* what) { throw std::runtime_error(what); }

inline std::size_t* phase_counter(LayerReplayCounters& c, LayerPhase p) {
  switch (p) {
    case LayerPhase::Attention: return &c.attention_phase_callbacks;
    case LayerPhase::Ffn: return &c.ffn_phase_callbacks;
    case LayerPhase::Ssm: return &c.ssm_phase_callbacks;
    case LayerPhase::Output: return &c.output_phase_callbacks;
    default: return nullptr;
  }
}

// Places consecutive slices, each starting at a multiple of the alignment.
struct Bump {
  std::size_t alignment, offset = 0;
  std::size_t take(std::size_t bytes);
};
}  // namespace executor_detail

inline std::size_t align_layer_workspace_bytes(std::size_t value, std::size_t alignment) {
  if (alignment == 0) executor_detail::fail("layer executor workspace alignment must be non-zero");
  const std::size_t r = value % alignment;
  return r == 0 ? value : value + (alignment - r);
}

inline std::size_t executor_detail::Bump::take(std::size_t bytes) {
  offset = align_layer_workspace_bytes(offset, alignment);
  const std::size_t at = offset;
  offset += bytes;
  return at;
}

inline std::size_t layer_workspace_logical_bytes(std::uint32_t values, std::size_t element_bytes) {
  if (element_bytes == 0) executor_detail::fail("layer executor workspace element size must be non-zero");
  if (values > std::numeric_limits<std::size_t>::max() / element_bytes)
    executor_detail::fail("layer executor workspace byte count overflow");
  return static_cast<std::size_t>(values) * element_bytes;
}

inline void note_layer_phase_callback(LayerReplayCounters& counters, LayerPhase phase) {
  std::size_t* c = executor_detail::phase_counter(counters, phase);
  if (c == nullptr) executor_detail::fail("layer executor cannot replay an unknown phase");
  ++*c;
}

inline void accumulate_layer_replay_counters(LayerReplayCounters& target, const LayerReplayCounters& source) {
  target.phase_callbacks += source.phase_callbacks;
  target.attention_phase_callbacks += source.attention_phase_callbacks;
  target.ffn_phase_callbacks += source.ffn_phase_callbacks;
  target.ssm_phase_callbacks += source.ssm_phase_callbacks;
  target.output_phase_callbacks += source.output_phase_callbacks;
  target.stage_callbacks += source.stage_callbacks;
  target.activation_feedback_callbacks += source.activation_feedback_callbacks;
  target.total_callbacks += source.total_callbacks;
}

inline void validate_layer_phase_execution_bounds(const LayerPhaseExecution& phase, std::size_t stage_count) {
  using executor_detail::fail;
  if (phase.count == 0) fail("layer executor phase contains no stages");
  if (phase.begin > stage_count || phase.count > stage_count - phase.begin)
    fail("layer executor phase exceeds stage count");
  if (phase.matvec_kernels_per_replay != phase.count) fail("layer executor phase matvec count mismatch");
  if (phase.activation_feedbacks_per_replay != 0 && phase.activation_feedbacks_per_replay != phase.count)
    fail("layer executor phase feedback count mismatch");
  if (phase.total_kernels_per_replay != phase.matvec_kernels_per_replay + phase.activation_feedbacks_per_replay)
    fail("layer executor phase total count mismatch");
}

inline void validate_layer_execution_plan_bounds(const LayerExecutionPlan& plan, std::size_t stage_count) {
  using executor_detail::fail;
  if (plan.stage_count != stage_count) fail("layer executor plan stage count mismatch");
  if (plan.phase_count != plan.phases.size()) fail("layer executor plan phase count mismatch");
  std::size_t mv = 0, fb = 0, tot = 0;
  for (const auto& p : plan.phases) {
    validate_layer_phase_execution_bounds(p, stage_count);
    mv += p.matvec_kernels_per_replay;
    fb += p.activation_feedbacks_per_replay;
    tot += p.total_kernels_per_replay;
  }
  if (mv != plan.matvec_kernels_per_replay || fb != plan.activation_feedbacks_per_replay ||
      tot != plan.total_kernels_per_replay)
    fail("layer executor plan kernel count mismatch");
}

// Per phase: the widest input and output of its stages and their total size.
inline LayerExecutorWorkspacePlan build_layer_executor_workspace_plan(
    const LayerExecutionPlan& plan, const std::vector<LayerStageWorkspaceDescriptor>& stages) {
  validate_layer_execution_plan_bounds(plan, stages.size());
  LayerExecutorWorkspacePlan ws;
  for (const auto& p : plan.phases) {
    LayerPhaseWorkspaceDescriptor d;
    d.phase = p.phase, d.begin = p.begin, d.count = p.count;
    for (std::size_t i = p.begin; i < p.begin + p.count; ++i) {
      const auto& s = stages[i];
      if (s.rows == 0 || s.cols == 0) executor_detail::fail("layer executor workspace contains an empty stage");
      d.max_rows = std::max(d.max_rows, s.rows);
      d.max_cols = std::max(d.max_cols, s.cols);
      d.logical_values_per_replay += static_cast<std::uint64_t>(s.rows) * s.cols;
    }
    ws.max_rows = std::max(ws.max_rows, d.max_rows);
    ws.max_cols = std::max(ws.max_cols, d.max_cols);
    ws.logical_values_per_replay += d.logical_values_per_replay;
    ws.phases.push_back(d);
  }
  return ws;
}

inline const LayerPhaseWorkspaceDescriptor& find_layer_workspace_phase_descriptor(
    const LayerExecutorWorkspacePlan& workspace, LayerPhase phase) {
  if (phase == LayerPhase::Unknown) executor_detail::fail("layer executor workspace lookup requires a known phase");
  for (const auto& d : workspace.phases)
    if (d.phase == phase) return d;
  executor_detail::fail("layer executor workspace phase is not present");
}

// Caches of a gated FFN (gate and / or up output), sized by the FFN phase's
// widest input.
inline std::vector<LayerAuxWorkspaceDescriptor> build_gated_ffn_aux_workspace_descriptors(
    const LayerExecutorWorkspacePlan& workspace, bool gate_cache, bool up_cache) {
  std::vector<LayerAuxWorkspaceDescriptor> out;
  if (!gate_cache && !up_cache) return out;
  const auto& ffn = find_layer_workspace_phase_descriptor(workspace, LayerPhase::Ffn);
  if (ffn.max_cols == 0) executor_detail::fail("gated FFN auxiliary workspace requires FFN columns");
  if (gate_cache) out.push_back({"ffn_gate_cache", LayerPhase::Ffn, ffn.max_cols});
  if (up_cache) out.push_back({"ffn_up_cache", LayerPhase::Ffn, ffn.max_cols});
  return out;
}

// Recurrent state (sized by the output phase's input) and scan scratch (the
// ssm phase's input) of a hybrid model's ssm phase.
inline std::vector<LayerAuxWorkspaceDescriptor> build_ssm_recurrent_aux_workspace_descriptors(
    const LayerExecutorWorkspacePlan& workspace, bool recurrent_state, bool scan_scratch = false) {
  std::vector<LayerAuxWorkspaceDescriptor> out;
  if (!recurrent_state && !scan_scratch) return out;
  const auto& ssm = find_layer_workspace_phase_descriptor(workspace, LayerPhase::Ssm);
  const auto& output = find_layer_workspace_phase_descriptor(workspace, LayerPhase::Output);
  if (recurrent_state && output.max_cols == 0) executor_detail::fail("SSM recurrent workspace requires output columns");
  if (scan_scratch && ssm.max_cols == 0) executor_detail::fail("SSM scan scratch workspace requires SSM columns");
  if (recurrent_state) out.push_back({"ssm_recurrent_state", LayerPhase::Ssm, output.max_cols});
  if (scan_scratch) out.push_back({"ssm_scan_scratch", LayerPhase::Ssm, ssm.max_cols});
  return out;
}

// Named scratch slices requested per phase (each phase must be in the plan).
inline std::vector<LayerAuxWorkspaceDescriptor> build_layer_phase_scratch_workspace_descriptors(
    const LayerExecutorWorkspacePlan& workspace, const std::vector<LayerAuxWorkspaceDescriptor>& scratch_requests) {
  using executor_detail::fail;
  for (const auto& r : scratch_requests) {
    if (r.name.empty()) fail("layer phase scratch workspace requires a name");
    if (r.phase == LayerPhase::Unknown) fail("layer phase scratch workspace requires a known phase");
    if (r.values == 0) fail("layer phase scratch workspace requires values");
    (void)find_layer_workspace_phase_descriptor(workspace, r.phase);
  }
  return scratch_requests;
}

// Arena layout: per phase an activation slice (max_cols values) and a logits
// slice (max_rows values), then the auxiliaries; every slice aligned.
inline LayerExecutorWorkspaceAllocationPlan build_layer_executor_workspace_allocation_plan(
    const LayerExecutorWorkspacePlan& workspace, const std::vector<LayerAuxWorkspaceDescriptor>& auxiliaries,
    std::size_t element_bytes, std::size_t alignment) {
  using executor_detail::fail;
  if (workspace.phases.empty()) fail("layer executor workspace allocation requires phases");
  if (element_bytes == 0) fail("layer executor workspace element size must be non-zero");
  LayerExecutorWorkspaceAllocationPlan a;
  executor_detail::Bump bump{alignment};
  for (const auto& d : workspace.phases) {
    if (d.phase == LayerPhase::Unknown) fail("layer executor workspace allocation has unknown phase");
    if (d.count == 0 || d.max_rows == 0 || d.max_cols == 0) fail("layer executor workspace allocation has empty phase");
    LayerPhaseWorkspaceAllocation p;
    p.phase = d.phase, p.begin = d.begin, p.count = d.count;
    p.activation_bytes = align_layer_workspace_bytes(std::size_t{d.max_cols} * element_bytes, alignment);
    p.activation_offset = bump.take(p.activation_bytes);
    p.logits_bytes = align_layer_workspace_bytes(std::size_t{d.max_rows} * element_bytes, alignment);
    p.logits_offset = bump.take(p.logits_bytes);
    p.total_bytes = p.activation_bytes + p.logits_bytes;
    a.activation_bytes += p.activation_bytes;
    a.logits_bytes += p.logits_bytes;
    a.phases.push_back(p);
  }
  a.phase_bytes = align_layer_workspace_bytes(bump.offset, alignment);
  bump.offset = a.phase_bytes;
  for (const auto& x : auxiliaries) {
    if (x.name.empty()) fail("layer executor auxiliary workspace requires a name");
    if (x.phase == LayerPhase::Unknown) fail("layer executor auxiliary workspace has unknown phase");
    if (x.values == 0) fail("layer executor auxiliary workspace is empty");
    for (const auto& e : a.auxiliaries)
      if (e.name == x.name) fail("layer executor auxiliary workspace name is duplicated");
    LayerAuxWorkspaceAllocation q;
    q.name = x.name, q.phase = x.phase, q.values = x.values;
    q.bytes = align_layer_workspace_bytes(std::size_t{x.values} * element_bytes, alignment);
    q.offset = bump.take(q.bytes);
    a.auxiliary_bytes += q.bytes;
    a.auxiliaries.push_back(std::move(q));
  }
  a.total_bytes = align_layer_workspace_bytes(bump.offset, alignment);
  return a;
}

inline LayerExecutorWorkspaceAllocationPlan build_layer_executor_workspace_allocation_plan(
    const LayerExecutorWorkspacePlan& workspace, std::size_t element_bytes, std::size_t alignment) {
  return build_layer_executor_workspace_allocation_plan(workspace, {}, element_bytes, alignment);
}

template <class Phases>
std::size_t layer_executor_phase_index_for_stage(const Phases& phases, std::size_t stage_index, const char* what) {
  for (std::size_t i = 0; i < phases.size(); ++i)
    if (stage_index >= phases[i].begin && stage_index < phases[i].begin + phases[i].count) return i;
  executor_detail::fail(what);
}

inline std::size_t find_layer_workspace_phase_index_for_stage(const LayerExecutorWorkspaceAllocationPlan& allocation,
                                                              std::size_t stage_index) {
  return layer_executor_phase_index_for_stage(allocation.phases, stage_index,
                                              "layer executor workspace does not cover stage");
}

// Device pointers of every slice, base + offset.
inline LayerExecutorWorkspaceRuntime bind_layer_executor_workspace_runtime(
    const LayerExecutorWorkspacePlan& workspace, const LayerExecutorWorkspaceAllocationPlan& allocation,
    void* workspace_base) {
  using executor_detail::fail;
  if (workspace.phases.size() != allocation.phases.size()) fail("layer executor workspace runtime phase count mismatch");
  if (allocation.total_bytes == 0) fail("layer executor workspace runtime requires bytes");
  if (workspace_base == nullptr) fail("layer executor workspace runtime base is null");
  auto* base = static_cast<std::uint8_t*>(workspace_base);
  auto inside = [&](std::size_t off, std::size_t bytes) { return off + bytes <= allocation.total_bytes; };
  LayerExecutorWorkspaceRuntime rt;
  rt.activation_bytes = allocation.activation_bytes;
  rt.logits_bytes = allocation.logits_bytes;
  rt.phase_bytes = allocation.phase_bytes;
  rt.auxiliary_bytes = allocation.auxiliary_bytes;
  rt.total_bytes = allocation.total_bytes;
  for (std::size_t i = 0; i < allocation.phases.size(); ++i) {
    const auto& d = workspace.phases[i];
    const auto& p = allocation.phases[i];
    if (d.phase != p.phase || d.begin != p.begin || d.count != p.count)
      fail("layer executor workspace runtime phase mismatch");
    if (p.activation_bytes == 0 || p.logits_bytes == 0) fail("layer executor workspace runtime has empty allocation");
    if (!inside(p.activation_offset, p.activation_bytes) || !inside(p.logits_offset, p.logits_bytes))
      fail("layer executor workspace runtime allocation exceeds arena");
    LayerPhaseWorkspaceRuntime r;
    r.phase = d.phase, r.begin = d.begin, r.count = d.count;
    r.activation = reinterpret_cast<float*>(base + p.activation_offset);
    r.logits = reinterpret_cast<float*>(base + p.logits_offset);
    r.max_rows = d.max_rows, r.max_cols = d.max_cols;
    r.activation_offset = p.activation_offset, r.activation_bytes = p.activation_bytes;
    r.logits_offset = p.logits_offset, r.logits_bytes = p.logits_bytes, r.total_bytes = p.total_bytes;
    rt.phases.push_back(r);
  }
  for (const auto& x : allocation.auxiliaries) {
    if (x.bytes == 0 || x.values == 0) fail("layer executor auxiliary runtime has empty allocation");
    if (!inside(x.offset, x.bytes)) fail("layer executor auxiliary runtime allocation exceeds arena");
    rt.auxiliaries.push_back({x.name, x.phase, reinterpret_cast<float*>(base + x.offset), x.values, x.offset, x.bytes});
  }
  return rt;
}

inline LayerAuxWorkspaceRuntime& find_layer_aux_workspace_runtime(LayerExecutorWorkspaceRuntime& runtime,
                                                                  std::string_view name) {
  for (auto& x : runtime.auxiliaries)
    if (x.name == name) return x;
  executor_detail::fail("layer executor auxiliary workspace is not present");
}

inline const LayerAuxWorkspaceRuntime& find_layer_aux_workspace_runtime(const LayerExecutorWorkspaceRuntime& runtime,
                                                                        std::string_view name) {
  for (const auto& x : runtime.auxiliaries)
    if (x.name == name) return x;
  executor_detail::fail("layer executor auxiliary workspace is not present");
}

inline std::size_t find_layer_workspace_runtime_phase_index_for_stage(const LayerExecutorWorkspaceRuntime& runtime,
                                                                      std::size_t stage_index) {
  return layer_executor_phase_index_for_stage(runtime.phases, stage_index,
                                              "layer executor workspace runtime does not cover stage");
}

// One feedback edge per stage of every chained phase: the stage's output
// feeds the next stage's input (the last stage feeds the first).
inline LayerExecutorDataflowPlan build_layer_executor_dataflow_plan(
    const LayerExecutionPlan& plan, const std::vector<LayerStageWorkspaceDescriptor>& stages,
    const LayerExecutorWorkspaceRuntime& runtime) {
  using executor_detail::fail;
  validate_layer_execution_plan_bounds(plan, stages.size());
  LayerExecutorDataflowPlan df;
  if (plan.activation_feedbacks_per_replay == 0) return df;
  if (runtime.phases.empty()) fail("layer executor dataflow requires runtime phases");
  for (const auto& p : plan.phases) {
    if (p.activation_feedbacks_per_replay == 0) continue;
    if (p.activation_feedbacks_per_replay != p.count) fail("layer executor dataflow feedback count mismatch");
    for (std::size_t src = p.begin; src < p.begin + p.count; ++src) {
      const std::size_t dst = (src + 1u) % stages.size();
      if (stages[src].rows == 0 || stages[dst].cols == 0) fail("layer executor dataflow contains an empty edge");
      LayerActivationFeedbackEdge e;
      e.source_stage = src, e.target_stage = dst;
      e.source_phase_index = find_layer_workspace_runtime_phase_index_for_stage(runtime, src);
      e.target_phase_index = find_layer_workspace_runtime_phase_index_for_stage(runtime, dst);
      e.source_phase = runtime.phases[e.source_phase_index].phase;
      e.target_phase = runtime.phases[e.target_phase_index].phase;
      e.source_rows = stages[src].rows, e.target_cols = stages[dst].cols;
      e.stage_id = static_cast<std::uint32_t>(src);
      e.crosses_phase = e.source_phase_index != e.target_phase_index;
      e.wraps_to_first_stage = dst == 0;
      df.phase_crossing_feedbacks += e.crosses_phase;
      df.wrap_feedbacks += e.wraps_to_first_stage;
      df.activation_feedback_edges.push_back(e);
    }
  }
  if (df.activation_feedback_edges.size() != plan.activation_feedbacks_per_replay)
    fail("layer executor dataflow edge count mismatch");
  return df;
}

inline const LayerActivationFeedbackEdge& find_layer_activation_feedback_edge(const LayerExecutorDataflowPlan& dataflow,
                                                                              std::size_t source_stage) {
  for (const auto& e : dataflow.activation_feedback_edges)
    if (e.source_stage == source_stage) return e;
  executor_detail::fail("layer executor dataflow does not cover source stage");
}

namespace executor_detail {
// High water = the logical bytes each slice must hold (max_cols / max_rows /
// values elements); slack = its allocation minus that. Shared by the plan and
// the bound runtime.
struct SliceView {
  LayerPhase phase;
  std::size_t begin, count;
  std::uint32_t max_rows, max_cols;
  std::size_t activation_bytes, logits_bytes, total_bytes;
};
inline LayerExecutorWorkspaceUsage measure(const std::vector<SliceView>& phases,
                                           const std::vector<LayerAuxWorkspaceAllocation>& aux,
                                           std::size_t arena_bytes, std::size_t element_bytes,
                                           const char* over_arena) {
  LayerExecutorWorkspaceUsage u;
  for (const auto& p : phases) {
    const std::size_t act = layer_workspace_logical_bytes(p.max_cols, element_bytes);
    const std::size_t lg = layer_workspace_logical_bytes(p.max_rows, element_bytes);
    if (act > p.activation_bytes || lg > p.logits_bytes) fail("layer executor workspace usage exceeds allocation");
    if (act + lg < act || act + lg > p.total_bytes) fail("layer executor workspace usage total exceeds allocation");
    LayerPhaseWorkspaceUsage q;
    q.phase = p.phase, q.begin = p.begin, q.count = p.count;
    q.activation_high_water_bytes = act, q.logits_high_water_bytes = lg, q.total_high_water_bytes = act + lg;
    q.activation_slack_bytes = p.activation_bytes - act;
    q.logits_slack_bytes = p.logits_bytes - lg;
    q.total_slack_bytes = p.total_bytes - (act + lg);
    u.activation_high_water_bytes += act;
    u.logits_high_water_bytes += lg;
    u.total_high_water_bytes += act + lg;
    u.activation_slack_bytes += q.activation_slack_bytes;
    u.logits_slack_bytes += q.logits_slack_bytes;
    u.phases.push_back(q);
  }
  for (const auto& x : aux) {
    if (x.phase == LayerPhase::Unknown) fail("layer executor auxiliary workspace usage has unknown phase");
    if (x.bytes == 0 || x.values == 0) fail("layer executor auxiliary workspace usage has empty allocation");
    const std::size_t hw = layer_workspace_logical_bytes(x.values, element_bytes);
    if (hw > x.bytes) fail("layer executor auxiliary workspace usage exceeds allocation");
    u.auxiliaries.push_back({x.name, x.phase, hw, x.bytes - hw});
    u.auxiliary_high_water_bytes += hw;
    u.auxiliary_slack_bytes += x.bytes - hw;
    u.total_high_water_bytes += hw;
  }
  if (u.total_high_water_bytes > arena_bytes) fail(over_arena);
  u.total_slack_bytes = arena_bytes - u.total_high_water_bytes;
  return u;
}
}  // namespace executor_detail

inline LayerExecutorWorkspaceUsage measure_layer_executor_workspace_usage(
    const LayerExecutorWorkspacePlan& workspace, const LayerExecutorWorkspaceAllocationPlan& allocation,
    std::size_t element_bytes) {
  using executor_detail::fail;
  if (workspace.phases.size() != allocation.phases.size()) fail("layer executor workspace usage phase count mismatch");
  if (allocation.phases.empty()) fail("layer executor workspace usage requires phases");
  std::vector<executor_detail::SliceView> v;
  for (std::size_t i = 0; i < allocation.phases.size(); ++i) {
    const auto& d = workspace.phases[i];
    const auto& p = allocation.phases[i];
    if (d.phase != p.phase || d.begin != p.begin || d.count != p.count)
      fail("layer executor workspace usage phase mismatch");
    if (p.activation_bytes == 0 || p.logits_bytes == 0) fail("layer executor workspace usage has empty allocation");
    v.push_back({d.phase, d.begin, d.count, d.max_rows, d.max_cols, p.activation_bytes, p.logits_bytes, p.total_bytes});
  }
  return executor_detail::measure(v, allocation.auxiliaries, allocation.total_bytes, element_bytes,
                                  "layer executor workspace usage exceeds allocation plan");
}

inline LayerExecutorWorkspaceUsage measure_layer_executor_workspace_usage(const LayerExecutorWorkspaceRuntime& runtime,
                                                                          std::size_t element_bytes) {
  using executor_detail::fail;
  if (runtime.phases.empty()) fail("layer executor workspace usage requires phases");
  std::vector<executor_detail::SliceView> v;
  for (const auto& p : runtime.phases) {
    if (p.phase == LayerPhase::Unknown) fail("layer executor workspace usage has unknown phase");
    if (p.activation == nullptr || p.logits == nullptr) fail("layer executor workspace usage has null runtime pointer");
    v.push_back({p.phase, p.begin, p.count, p.max_rows, p.max_cols, p.activation_bytes, p.logits_bytes, p.total_bytes});
  }
  std::vector<LayerAuxWorkspaceAllocation> aux;
  for (const auto& x : runtime.auxiliaries) {
    if (x.data == nullptr && x.phase != LayerPhase::Unknown)
      fail("layer executor auxiliary workspace usage has null runtime pointer");
    aux.push_back({x.name, x.phase, x.values, x.offset, x.bytes});
  }
  return executor_detail::measure(v, aux, runtime.total_bytes, element_bytes,
                                  "layer executor workspace usage exceeds runtime arena");
}

// The phase's stages in order: launch_stage(i), then launch_feedback(i) when
// the phase is chained.
template <typename LaunchStage, typename LaunchFeedback>
LayerReplayCounters replay_layer_phase(const LayerPhaseExecution& phase, std::size_t stage_count,
                                       LaunchStage&& launch_stage, LaunchFeedback&& launch_feedback) {
  validate_layer_phase_execution_bounds(phase, stage_count);
  LayerReplayCounters c;
  c.phase_callbacks = 1;
  note_layer_phase_callback(c, phase.phase);
  for (std::size_t i = phase.begin; i < phase.begin + phase.count; ++i) {
    launch_stage(i);
    ++c.stage_callbacks;
    if (phase.activation_feedbacks_per_replay != 0) {
      launch_feedback(i);
      ++c.activation_feedback_callbacks;
    }
  }
  c.total_callbacks = c.stage_callbacks + c.activation_feedback_callbacks;
  return c;
}

inline void validate_layer_phase_replay_counters(const LayerPhaseExecution& phase, const LayerReplayCounters& counters) {
  using executor_detail::fail;
  if (counters.phase_callbacks != 1) fail("layer executor phase callback count mismatch");
  if (counters.stage_callbacks != phase.count) fail("layer executor stage callback count mismatch");
  if (counters.activation_feedback_callbacks != phase.activation_feedbacks_per_replay)
    fail("layer executor feedback callback count mismatch");
  if (counters.total_callbacks != phase.total_kernels_per_replay) fail("layer executor total callback count mismatch");
  static const char* const kMismatch[] = {
      "layer executor attention phase callback mismatch", "layer executor ffn phase callback mismatch",
      "layer executor ssm phase callback mismatch", "layer executor output phase callback mismatch"};
  LayerReplayCounters probe = counters;
  const std::size_t* c = executor_detail::phase_counter(probe, phase.phase);
  if (c == nullptr) fail("layer executor cannot validate an unknown phase");
  if (*c != 1) fail(kMismatch[static_cast<int>(phase.phase)]);
}

template <typename LaunchStage, typename LaunchFeedback>
LayerReplayCounters replay_layer_execution_plan(const LayerExecutionPlan& plan, std::size_t stage_count,
                                                LaunchStage&& launch_stage, LaunchFeedback&& launch_feedback) {
  validate_layer_execution_plan_bounds(plan, stage_count);
  LayerReplayCounters total;
  for (const auto& p : plan.phases)
    accumulate_layer_replay_counters(total, replay_layer_phase(p, stage_count, launch_stage, launch_feedback));
  return total;
}

// One callback per phase (by kind), each returning that phase's counters,
// which must match the plan.
template <typename LaunchAttentionPhase, typename LaunchFfnPhase, typename LaunchSsmPhase, typename LaunchOutputPhase>
LayerReplayCounters replay_layer_execution_plan_by_phase(const LayerExecutionPlan& plan, std::size_t stage_count,
                                                         LaunchAttentionPhase&& launch_attention_phase,
                                                         LaunchFfnPhase&& launch_ffn_phase,
                                                         LaunchSsmPhase&& launch_ssm_phase,
                                                         LaunchOutputPhase&& launch_output_phase) {
  validate_layer_execution_plan_bounds(plan, stage_count);
  LayerReplayCounters total;
  for (const auto& p : plan.phases) {
    LayerReplayCounters c;
    switch (p.phase) {
      case LayerPhase::Attention: c = launch_attention_phase(p); break;
      case LayerPhase::Ffn: c = launch_ffn_phase(p); break;
      case LayerPhase::Ssm: c = launch_ssm_phase(p); break;
      case LayerPhase::Output: c = launch_output_phase(p); break;
      default: executor_detail::fail("layer executor cannot dispatch an unknown phase");
    }
    validate_layer_phase_replay_counters(p, c);
    accumulate_layer_replay_counters(total, c);
  }
  return total;
}

}  // namespace rtxllm

#endif
