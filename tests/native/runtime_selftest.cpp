// Self-test of the runner's host contracts (the layer role plan, the layer
// executor, admission, the tensor-pack manifest loaders), in the spirit of the
// reference's layer_plan_selftest (runtime/apps/layer_plan_selftest/main.cpp).
// Built with g++ from the headers and csrc/pack_manifest.cpp by
// tests/test_runtime_contracts.py; prints "runtime selftest: N cases passed".
#include <cstdio>
#include <cstdlib>
#include <filesystem>
#include <fstream>
#include <functional>
#include <string>
#include <vector>

#include <unistd.h>

#include "rtxllm/admission.h"
#include "rtxllm/layer_executor.h"
#include "rtxllm/layer_plan.h"
#include "rtxllm/pack_manifest.h"

using namespace rtxllm;

namespace {

int g_cases = 0, g_failed = 0;

#define CHECK(cond)                                                               \
  do {                                                                            \
    if (!(cond)) {                                                                \
      std::fprintf(stderr, "%s:%d: CHECK failed: %s\n", __FILE__, __LINE__, #cond); \
      throw std::logic_error("check");                                            \
    }                                                                             \
  } while (0)

// f() must throw std::runtime_error whose message contains `what`.
void expect_throw(const std::function<void()>& f, const std::string& what) {
  try {
    f();
  } catch (const std::runtime_error& e) {
    if (std::string(e.what()).find(what) == std::string::npos) {
      std::fprintf(stderr, "unexpected message: '%s' (wanted '%s')\n", e.what(), what.c_str());
      throw std::logic_error("message");
    }
    return;
  }
  std::fprintf(stderr, "no exception (wanted '%s')\n", what.c_str());
  throw std::logic_error("no throw");
}

void run(const char* name, const std::function<void()>& body) {
  ++g_cases;
  try {
    body();
  } catch (const std::exception& e) {
    ++g_failed;
    std::fprintf(stderr, "FAILED %s: %s\n", name, e.what());
  }
}

std::vector<LayerStageDescriptor> stages_of(const std::vector<const char*>& roles) {
  std::vector<LayerStageDescriptor> out;
  for (const char* r : roles) out.push_back({r, std::string(r) != "output.weight"});
  return out;
}

const std::vector<const char*> kLlama = {"attn_qkv.weight", "attn_output.weight", "ffn_gate_up.weight",
                                         "ffn_down.weight"};

std::filesystem::path g_dir;

std::filesystem::path write(const std::string& name, const std::string& text) {
  const auto p = g_dir / name;
  std::ofstream(p, std::ios::binary) << text;
  return p;
}

std::string q4k_record(const std::string& extra_or_override = "") {
  std::string r =
      R"({"name": "blk.3.ffn_down.weight", "dimensions": [512, 16], "rows": 16, "cols": 512, "block_count": 32,)"
      R"( "source_offset": 4096, "source_bytes": 4608, "source_checksum": 11, "policy": "split-native",)"
      R"( "metadata_format": "native16", "payload_path": "a.bin", "payload_bytes": 4096, "payload_checksum": 22,)"
      R"( "metadata_path": "b\/c.bin", "metadata_bytes": 512, "metadata_checksum": 33, "blocks_path": "",)"
      R"( "resident_bytes": 4608, "compression_ratio_vs_fp16": 3.55)";
  return r + extra_or_override + "}";
}

std::string iq_record(const std::string& layer = R"("layer": 2,)", const std::string& type = "IQ2_S",
                      const std::string& block_size = "256", const std::string& source_bytes = "2624") {
  return R"({"name": "blk.2.ffn_gate.weight", "type": ")" + type + R"(", )" + layer +
         R"( "role": "ffn_gate.weight", "dimensions": [512, 16], "element_count": 8192, "block_size": )" +
         block_size + R"(, "block_type_size": 82, "block_count": 32, "source_offset": 8704, "source_bytes": )" +
         source_bytes + R"(, "source_checksum": 7, "payload_path": "p.bin", "payload_bytes": 2624,)"
         R"( "payload_checksum": 7, "resident_bytes": 2624, "policy": "raw-blocks", "runtime_kernel": "k"})";
}

}  // namespace

// --load Q4K_MANIFEST IQ_MANIFEST TENSOR_PLAN ROOT: loads both manifests,
// validates them against the plan, reads every pack file and checks its size
// and checksum; prints one line per tensor.
int load_mode(char** argv) {
  try {
    const std::filesystem::path root = argv[5];
    auto under = [&](const std::filesystem::path& p) { return p.is_absolute() ? p : root / p; };
    // "-" stands for a manifest the packs do not have
    const bool has_q = std::string(argv[2]) != "-", has_i = std::string(argv[3]) != "-";
    const auto q = has_q ? load_q4k_manifest(argv[2]) : Q4KManifest{};
    const auto i = has_i ? load_iq_manifest(argv[3]) : IQManifest{};
    if (has_q) validate_q4k_manifest_tensors_against_plan(select_q4k_tensors(q, {}, 0), argv[4]);
    if (has_i) validate_iq_manifest_tensors_against_plan(i.tensors, argv[4]);
    int bad = 0;
    for (const auto& t : q.tensors) {
      const bool ok = byte_checksum(load_binary_file(under(t.payload_path), t.payload_bytes, "payload")) ==
                          t.payload_checksum &&
                      byte_checksum(load_binary_file(under(t.metadata_path), t.metadata_bytes, "metadata")) ==
                          t.metadata_checksum &&
                      (t.blocks_path.empty() ||
                       byte_checksum(load_binary_file(under(t.blocks_path), t.source_bytes, "blocks")) ==
                           t.source_checksum);
      std::printf("q4k %s layer=%d role=%s rows=%u cols=%u policy=%s ok=%d\n", t.name.c_str(), t.layer,
                  t.role.c_str(), t.rows, t.cols, t.policy.c_str(), ok ? 1 : 0);
      bad += ok ? 0 : 1;
    }
    for (const auto& t : i.tensors) {
      const bool ok =
          byte_checksum(load_binary_file(under(t.payload_path), t.payload_bytes, "payload")) == t.payload_checksum;
      std::printf("raw %s type=%s layer=%d blocks=%llu ok=%d\n", t.name.c_str(), t.type.c_str(), t.layer,
                  static_cast<unsigned long long>(t.block_count), ok ? 1 : 0);
      bad += ok ? 0 : 1;
    }
    return bad == 0 ? 0 : 1;
  } catch (const std::exception& e) {
    std::printf("error %s\n", e.what());
    return 1;
  }
}

// --load-set TENSOR_PLAN ROOT MANIFEST...: each manifest read by the loader its
// producer needs (pack_manifest_kind), validated against the plan, every pack
// file's size and checksum checked; one line per tensor, as --load prints.
int load_set_mode(int argc, char** argv) {
  try {
    const std::filesystem::path plan = argv[2], root = argv[3];
    auto under = [&](const std::filesystem::path& p) { return p.is_absolute() ? p : root / p; };
    int bad = 0;
    for (int a = 4; a < argc; ++a) {
      if (pack_manifest_kind(argv[a]) == PackManifestKind::Q4K) {
        const auto q = load_q4k_manifest(argv[a]);
        validate_q4k_manifest_tensors_against_plan(select_q4k_tensors(q, {}, 0), plan);
        for (const auto& t : q.tensors) {
          const bool ok =
              byte_checksum(load_binary_file(under(t.payload_path), t.payload_bytes, "payload")) ==
                  t.payload_checksum &&
              byte_checksum(load_binary_file(under(t.metadata_path), t.metadata_bytes, "metadata")) ==
                  t.metadata_checksum &&
              (t.blocks_path.empty() ||
               byte_checksum(load_binary_file(under(t.blocks_path), t.source_bytes, "blocks")) == t.source_checksum);
          std::printf("q4k %s layer=%d role=%s rows=%u cols=%u policy=%s ok=%d\n", t.name.c_str(), t.layer,
                      t.role.c_str(), t.rows, t.cols, t.policy.c_str(), ok ? 1 : 0);
          bad += ok ? 0 : 1;
        }
      } else {
        const auto i = load_iq_manifest(argv[a]);
        validate_iq_manifest_tensors_against_plan(i.tensors, plan);
        for (const auto& t : i.tensors) {
          const bool ok =
              byte_checksum(load_binary_file(under(t.payload_path), t.payload_bytes, "payload")) == t.payload_checksum;
          std::printf("raw %s type=%s layer=%d blocks=%llu kernel=%s ok=%d\n", t.name.c_str(), t.type.c_str(),
                      t.layer, static_cast<unsigned long long>(t.block_count), t.runtime_kernel.c_str(), ok ? 1 : 0);
          bad += ok ? 0 : 1;
        }
      }
    }
    return bad == 0 ? 0 : 1;
  } catch (const std::exception& e) {
    std::printf("error %s\n", e.what());
    return 1;
  }
}

int main(int argc, char** argv) {
  if (argc == 6 && std::string(argv[1]) == "--load") return load_mode(argv);
  if (argc >= 5 && std::string(argv[1]) == "--load-set") return load_set_mode(argc, argv);
  g_dir = std::filesystem::temp_directory_path() / ("rtxllm_selftest_" + std::to_string(::getpid()));
  std::filesystem::create_directories(g_dir);

  // ---- layer role plan ----
  run("llama layer plan validates", [] {
    const auto st = stages_of(kLlama);
    const auto seg = build_layer_phase_segments(st);
    CHECK(seg.size() == 2 && seg[0].phase == LayerPhase::Attention && seg[0].begin == 0 && seg[0].count == 2);
    CHECK(seg[1].phase == LayerPhase::Ffn && seg[1].begin == 2 && seg[1].count == 2);
    const auto v = validate_layer_phase_plan(st, seg);
    CHECK(v.passed && v.message == "layer phase plan validated" && v.expected_phases.size() == 2);
  });
  run("llama layer with output validates", [] {
    auto roles = kLlama;
    roles.push_back("output.weight");
    const auto st = stages_of(roles);
    const auto v = validate_layer_phase_plan(st, build_layer_phase_segments(st));
    CHECK(v.passed && v.expected_phases.back() == LayerPhase::Output && v.observed_phases.size() == 3);
  });
  run("hybrid plan with ssm validates", [] {
    const auto st = stages_of({"attn_gate.weight", "attn_qkv.weight", "ffn_gate_exps.weight", "ffn_up_exps.weight",
                               "ffn_down_exps.weight", "ssm_alpha.weight", "ssm_out.weight", "output.weight"});
    const auto v = validate_layer_phase_plan(st, build_layer_phase_segments(st));
    CHECK(v.passed && v.expected_phases.size() == 4 && v.expected_phases[2] == LayerPhase::Ssm);
  });
  run("unknown role rejected", [] {
    const auto st = stages_of({"attn_qkv.weight", "ffn_mystery.weight"});
    const auto v = validate_layer_phase_plan(st, build_layer_phase_segments(st));
    CHECK(!v.passed && v.message == "layer phase plan contains unknown role-plan roles");
    CHECK(count_unknown_layer_roles(st) == 1 && count_unknown_layer_phases(st) == 0);
  });
  run("unknown phase rejected", [] {
    const auto st = stages_of({"attn_qkv.weight", "ffn_down.weight", "token_embd.weight"});
    std::vector<LayerStageDescriptor> s2 = st;
    s2[2].layer_local = false;  // not ranked, but its phase is unknown
    const auto v = validate_layer_phase_plan(s2, build_layer_phase_segments(s2));
    CHECK(!v.passed && v.message == "layer phase plan contains unknown execution phases");
  });
  run("phase order and segment count checked", [] {
    auto st = stages_of({"ffn_down.weight", "attn_qkv.weight"});
    CHECK(validate_layer_phase_plan(st, build_layer_phase_segments(st)).message ==
          "layer phase plan phase order mismatch");
    st = stages_of({"attn_qkv.weight", "ffn_up.weight", "attn_output.weight"});
    CHECK(validate_layer_phase_plan(st, build_layer_phase_segments(st)).message ==
          "layer phase plan segment count mismatch");
    CHECK(validate_layer_phase_plan({}, {}).message == "layer phase plan requires at least one stage");
  });
  run("role ranks and phase names", [] {
    CHECK(layer_role_rank("attn_q.weight") < layer_role_rank("attn_k.weight"));
    CHECK(layer_role_rank("attn_qkv.weight") == 20 && layer_role_rank("ssm_out.weight") == 110);
    CHECK(layer_role_rank("output") == 10000 && layer_role_rank("x") == 5000);
    CHECK(std::string(layer_phase_name(LayerPhase::Ffn)) == "ffn");
    const auto counts = build_layer_phase_counts(stages_of(kLlama));
    CHECK(counts.at("attention") == 2 && counts.at("ffn") == 2);
  });
  run("execution plan counts", [] {
    const auto seg = build_layer_phase_segments(stages_of(kLlama));
    const auto a = build_layer_execution_plan(seg, false), b = build_layer_execution_plan(seg, true);
    CHECK(a.stage_count == 4 && a.phase_count == 2 && a.matvec_kernels_per_replay == 4 &&
          a.total_kernels_per_replay == 4);
    CHECK(b.activation_feedbacks_per_replay == 4 && b.total_kernels_per_replay == 8 &&
          b.phases[1].total_kernels_per_replay == 4);
  });

  // ---- executor ----
  const auto seg = build_layer_phase_segments(stages_of(kLlama));
  const LayerExecutionPlan chained = build_layer_execution_plan(seg, true);
  const std::vector<LayerStageWorkspaceDescriptor> dims = {{6144, 4096}, {4096, 4096}, {28672, 4096}, {4096, 14336}};
  run("workspace plan", [&] {
    const auto ws = build_layer_executor_workspace_plan(chained, dims);
    CHECK(ws.phases.size() == 2 && ws.phases[0].max_rows == 6144 && ws.phases[0].max_cols == 4096);
    CHECK(ws.phases[1].max_rows == 28672 && ws.phases[1].max_cols == 14336 && ws.max_cols == 14336);
    CHECK(ws.logical_values_per_replay == 6144ull * 4096 + 4096ull * 4096 + 28672ull * 4096 + 4096ull * 14336);
    auto bad = dims;
    bad[1].rows = 0;
    expect_throw([&] { build_layer_executor_workspace_plan(chained, bad); }, "empty stage");
    expect_throw([&] { build_layer_executor_workspace_plan(chained, {dims[0]}); }, "stage count mismatch");
  });
  run("allocation plan is aligned and complete", [&] {
    const auto ws = build_layer_executor_workspace_plan(chained, dims);
    const auto aux = build_gated_ffn_aux_workspace_descriptors(ws, true, true);
    CHECK(aux.size() == 2 && aux[0].name == "ffn_gate_cache" && aux[1].values == 14336);
    const auto a = build_layer_executor_workspace_allocation_plan(ws, aux, 4, 256);
    CHECK(a.phases[0].activation_offset == 0 && a.phases[0].activation_bytes == 4096 * 4);
    CHECK(a.phases[0].logits_offset == 4096 * 4 && a.phases[0].logits_bytes == 6144 * 4);
    CHECK(a.phases[1].activation_offset % 256 == 0 && a.auxiliaries[0].offset == a.phase_bytes);
    CHECK(a.total_bytes == a.phase_bytes + a.auxiliary_bytes && a.total_bytes % 256 == 0);
    auto dup = aux;
    dup[1].name = dup[0].name;
    expect_throw([&] { build_layer_executor_workspace_allocation_plan(ws, dup, 4, 256); }, "duplicated");
    expect_throw([&] { build_layer_executor_workspace_allocation_plan(ws, 0, 256); }, "element size");
    expect_throw([&] { build_ssm_recurrent_aux_workspace_descriptors(ws, true); }, "phase is not present");
  });
  run("bind, dataflow and usage", [&] {
    const auto ws = build_layer_executor_workspace_plan(chained, dims);
    const auto aux = build_gated_ffn_aux_workspace_descriptors(ws, true, false);
    const auto a = build_layer_executor_workspace_allocation_plan(ws, aux, 4, 256);
    std::vector<unsigned char> arena(a.total_bytes);
    const auto rt = bind_layer_executor_workspace_runtime(ws, a, arena.data());
    CHECK(reinterpret_cast<unsigned char*>(rt.phases[1].logits) == arena.data() + a.phases[1].logits_offset);
    CHECK(find_layer_aux_workspace_runtime(rt, "ffn_gate_cache").data ==
          reinterpret_cast<float*>(arena.data() + a.auxiliaries[0].offset));
    expect_throw([&] { bind_layer_executor_workspace_runtime(ws, a, nullptr); }, "base is null");
    const auto df = build_layer_executor_dataflow_plan(chained, dims, rt);
    CHECK(df.activation_feedback_edges.size() == 4 && df.wrap_feedbacks == 1 && df.phase_crossing_feedbacks == 2);
    CHECK(find_layer_activation_feedback_edge(df, 3).target_stage == 0 &&
          find_layer_activation_feedback_edge(df, 1).crosses_phase);
    const auto u1 = measure_layer_executor_workspace_usage(ws, a, 4);
    const auto u2 = measure_layer_executor_workspace_usage(rt, 4);
    CHECK(u1.total_high_water_bytes == u2.total_high_water_bytes && u1.total_slack_bytes == u2.total_slack_bytes);
    CHECK(u1.total_high_water_bytes == 4u * (4096 + 6144 + 14336 + 28672 + 14336) &&
          u1.total_high_water_bytes + u1.total_slack_bytes == a.total_bytes);
    CHECK(find_layer_workspace_phase_index_for_stage(a, 2) == 1);
    expect_throw([&] { find_layer_workspace_runtime_phase_index_for_stage(rt, 9); }, "does not cover stage");
  });
  run("replay by phase and counter validation", [&] {
    std::vector<std::size_t> launched, fed;
    auto stage = [&](std::size_t i) { launched.push_back(i); };
    auto feedback = [&](std::size_t i) { fed.push_back(i); };
    auto phase = [&](const LayerPhaseExecution& p) { return replay_layer_phase(p, 4, stage, feedback); };
    auto never = [](const LayerPhaseExecution&) -> LayerReplayCounters { throw std::runtime_error("never"); };
    const auto c = replay_layer_execution_plan_by_phase(chained, 4, phase, phase, never, never);
    CHECK(launched == (std::vector<std::size_t>{0, 1, 2, 3}) && fed == launched);
    CHECK(c.phase_callbacks == 2 && c.attention_phase_callbacks == 1 && c.ffn_phase_callbacks == 1 &&
          c.total_callbacks == 8);
    auto short_phase = [&](const LayerPhaseExecution& p) {
      auto r = replay_layer_phase(p, 4, stage, feedback);
      --r.stage_callbacks;
      return r;
    };
    expect_throw([&] { replay_layer_execution_plan_by_phase(chained, 4, short_phase, phase, never, never); },
                 "stage callback count mismatch");
    LayerExecutionPlan broken = chained;
    broken.total_kernels_per_replay += 1;
    expect_throw([&] { replay_layer_execution_plan(broken, 4, stage, feedback); }, "kernel count mismatch");
    LayerPhaseExecution unknown = chained.phases[0];
    unknown.phase = LayerPhase::Unknown;
    expect_throw([&] { replay_layer_phase(unknown, 4, stage, feedback); }, "unknown phase");
  });

  // ---- admission ----
  run("admission decisions", [] {
    RequestEstimate r;
    r.weight_bytes = 3000, r.prompt_tokens = 10, r.max_new_tokens = 6, r.kv_bytes_per_token = 100;
    r.kv_cache_bytes = 400, r.workspace_bytes = 300, r.workspace_high_water_bytes = 200, r.graph_bytes = 50;
    auto d = decide_admission(ResidencyPolicy::Strict, MemoryBudget{10000, 0}, r);
    CHECK(d.admit && d.required_bytes == 3000 + 1600 + 400 + 300 + 50 && d.breakdown.workspace_slack_bytes == 100);
    CHECK(d.reason == "fits strict VRAM budget");
    d = decide_admission(ResidencyPolicy::Balanced, MemoryBudget{6000, 1000}, r);
    CHECK(!d.admit && d.usable_bytes == 5000 && d.breakdown.over_budget_bytes == 350);
    CHECK(d.reason == "rejected: required 5350 bytes, usable 5000 bytes, over budget 350 bytes");
    d = decide_admission(ResidencyPolicy::Overflow, MemoryBudget{100, 200}, r);
    CHECK(d.admit && d.host_spill_allowed && d.usable_bytes == 0);
    r.kv_bytes_per_token = ~std::size_t{0};
    bool overflowed = false;
    try {
      decide_admission(ResidencyPolicy::Strict, MemoryBudget{}, r);
    } catch (const std::overflow_error&) {
      overflowed = true;
    }
    CHECK(overflowed);
  });

  // ---- pack manifests ----
  run("q4k manifest fields", [] {
    const auto p = write("q.json", R"({"model": "m.gguf", "policy": "split-native", "tensor_count": 1,)"
                                   R"( "note": {"nested": [1, 2, {"x": null}], "ok": true, "f": -1.5e3},)"
                                   R"( "tensors": [)" + q4k_record() + "]}");
    const auto m = load_q4k_manifest(p);
    CHECK(m.model == "m.gguf" && m.tensor_count == 1 && m.tensors.size() == 1);
    const auto& t = m.tensors[0];
    CHECK(t.layer == 3 && t.role == "ffn_down.weight" && t.rows == 16 && t.cols == 512);
    CHECK(t.metadata_path == "b/c.bin" && t.runtime_kernel == "split-native" && t.metadata_checksum == 33);
    CHECK((t.dimensions == std::vector<std::uint64_t>{512, 16}));
    CHECK(q4k_policy_format(t.policy) == 4 && q4k_policy_format("auto") == -1);
  });
  run("q4k manifest rejections", [] {
    std::string rec = q4k_record();
    const std::string no_meta_sum = rec.replace(rec.find("\"metadata_checksum\": 33,"), 24, "");
    expect_throw([&] { load_q4k_manifest(write("q1.json", "{\"tensors\": [" + no_meta_sum + "]}")); },
                 "manifest field missing: metadata_checksum");
    std::string bad_cols = q4k_record();
    bad_cols.replace(bad_cols.find("\"cols\": 512"), 11, "\"cols\": 500");
    expect_throw([&] { load_q4k_manifest(write("q2.json", "{\"tensors\": [" + bad_cols + "]}")); },
                 "invalid Q4_K shape");
    std::string bad_dims = q4k_record();
    bad_dims.replace(bad_dims.find("[512, 16]"), 9, "[16, 512]");
    expect_throw([&] { load_q4k_manifest(write("q3.json", "{\"tensors\": [" + bad_dims + "]}")); },
                 "dimensions disagree");
    expect_throw([&] { load_q4k_manifest(write("q4.json", "{\"tensors\": []}")); }, "manifest contains no tensors");
    expect_throw([&] { load_q4k_manifest(write("q5.json", "{\"tensors\": [" + q4k_record() + ",]}")); },
                 "manifest JSON");
    expect_throw([&] { load_q4k_manifest(write("q6.json", "{\"tensors\": [\"unterminated]}")); }, "manifest JSON");
    expect_throw([&] { load_q4k_manifest(g_dir / "missing.json"); }, "failed to open manifest");
  });
  run("q4k select", [] {
    std::string second = q4k_record();
    second.replace(second.find("blk.3.ffn_down.weight"), 21, "output.weight");
    const auto m = load_q4k_manifest(write("q7.json", "{\"tensors\": [" + q4k_record() + "," + second + "]}"));
    CHECK(m.tensors[1].layer == -1 && m.tensors[1].role == "output");
    CHECK(select_q4k_tensors(m, {}, 1).size() == 1 && select_q4k_tensors(m, {}, 0).size() == 2);
    CHECK(select_q4k_tensors(m, {"output.weight"}, 0)[0].name == "output.weight");
    expect_throw([&] { select_q4k_tensors(m, {"nope"}, 0); }, "manifest tensor not found: nope");
  });
  run("iq manifest fields and rejections", [] {
    const auto m = load_iq_manifest(write("i.json", R"({"types": ["IQ2_S"], "tensors": [)" + iq_record() + "," +
                                                         iq_record(R"("layer": null,)") + "," + iq_record("") + "]}"));
    CHECK(m.types.size() == 1 && m.tensors[0].layer == 2 && m.tensors[1].layer == -1 && m.tensors[2].layer == 0);
    CHECK(m.tensors[0].block_type_size == 82 && m.tensors[0].payload_path == "p.bin");
    CHECK(select_iq_tensor(m, "").name == "blk.2.ffn_gate.weight");
    expect_throw([&] { select_iq_tensor(m, "x"); }, "IQ manifest tensor not found: x");
    expect_throw([&] { load_iq_manifest(write("i1.json", "{\"tensors\": [" + iq_record(R"("layer": 1,)", "Q8_0") + "]}")); },
                 "unsupported raw quant manifest tensor type: Q8_0");
    expect_throw([&] { load_iq_manifest(write("i2.json", "{\"tensors\": [" + iq_record(R"("layer": 1,)", "IQ2_S", "32") + "]}")); },
                 "invalid block metadata");
    expect_throw([&] { load_iq_manifest(write("i3.json", "{\"tensors\": [" + iq_record(R"("layer": 1,)", "IQ2_S", "256", "9") + "]}")); },
                 "source/payload byte mismatch");
  });
  run("tensor plan validation", [] {
    const auto q = load_q4k_manifest(write("q8.json", "{\"tensors\": [" + q4k_record() + "]}"));
    const auto i = load_iq_manifest(write("i4.json", "{\"tensors\": [" + iq_record() + "]}"));
    auto plan = [](const std::string& q4_type, const std::string& dims, const std::string& span,
                   const std::string& off) {
      return R"({"tensors": [{"name": "blk.3.ffn_down.weight", "type": ")" + q4_type + R"(", "dimensions": )" +
             dims + R"(, "span_bytes": )" + span + R"(, "absolute_offset": )" + off +
             R"(}, {"name": "blk.2.ffn_gate.weight", "type": "IQ2_S", "dimensions": [512, 16], "span_bytes": 2624,)"
             R"( "absolute_offset": 8704}]})";
    };
    const auto good = write("plan.json", plan("Q4_K", "[512, 16]", "4608", "4096"));
    CHECK(validate_q4k_manifest_tensors_against_plan(q.tensors, good).checked_tensors == 1);
    CHECK(validate_iq_manifest_tensors_against_plan(i.tensors, good).checked_tensors == 1);
    expect_throw([&] { validate_q4k_manifest_tensors_against_plan(q.tensors, write("p1.json", plan("Q5_K", "[512, 16]", "4608", "4096"))); },
                 "type mismatch");
    expect_throw([&] { validate_q4k_manifest_tensors_against_plan(q.tensors, write("p2.json", plan("Q4_K", "[512, 32]", "4608", "4096"))); },
                 "dimensions mismatch");
    expect_throw([&] { validate_q4k_manifest_tensors_against_plan(q.tensors, write("p3.json", plan("Q4_K", "[512, 16]", "4600", "4096"))); },
                 "source byte mismatch");
    expect_throw([&] { validate_q4k_manifest_tensors_against_plan(q.tensors, write("p4.json", plan("Q4_K", "[512, 16]", "4608", "77"))); },
                 "source offset mismatch");
    CHECK(validate_q4k_manifest_tensors_against_plan(q.tensors, write("p5.json", plan("Q4_K", "[512, 16]", "4608", "0")))
              .checked_tensors == 1);  // an unknown offset is not compared
    expect_throw([&] { validate_iq_manifest_tensors_against_plan(i.tensors, write("p6.json", R"({"tensors": [{"name": "a", "type": "IQ2_S", "span_bytes": 1}]})")); },
                 "tensor plan is missing manifest tensor");
    expect_throw([&] { validate_iq_manifest_tensors_against_plan(i.tensors, write("p7.json", R"({"tensors": [{"name": "a", "type": "IQ2_S", "span_bytes": 1}, {"name": "a", "type": "IQ2_S", "span_bytes": 1}]})")); },
                 "duplicate tensor: a");
    expect_throw([&] { validate_iq_manifest_tensors_against_plan(i.tensors, ""); }, "tensor plan path is empty");
  });
  run("binary files and checksums", [] {
    const auto p = write("blob.bin", std::string("\x01\x02\xff", 3));
    const auto b = load_binary_file(p, 3, "blob");
    CHECK(b.size() == 3 && byte_checksum(b) == 258);
    expect_throw([&] { load_binary_file(p, 4, "blob"); }, "blob size mismatch: expected 4 bytes, got 3");
    expect_throw([&] { load_binary_file(g_dir / "none.bin", 1, "blob"); }, "failed to open blob");
  });

  std::filesystem::remove_all(g_dir);
  if (g_failed != 0) {
    std::fprintf(stderr, "runtime selftest: %d of %d cases failed\n", g_failed, g_cases);
    return 1;
  }
  std::printf("runtime selftest: %d cases passed\n", g_cases);
  return 0;
}
