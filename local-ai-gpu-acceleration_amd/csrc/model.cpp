// Llama decode runner (batch 1, or a batch of 2..8 sequences) on one MI355X:
// arena layout, synthetic weight fill, the per-step launch sequence and its
// hipGraph.
//
// Structure follows the reference's layer-slice runner
// (runtime/apps/mixed_sequence_benchmark_runner/main.cpp: arena setup
// 3764-3791, per-stage launches 4002-4279, capture 4801-4823, replay
// 4825-4836), for a real Llama layer instead of its synthetic stages.
#include <algorithm>
#include <cmath>
#include <cstdio>
#include <cstring>
#include <map>
#include <memory>
#include <new>
#include <string>
#include <vector>

#include "layer.h"
#include "rtxllm/admission.h"
#include "rtxllm/decode_kernels.h"
#include "rtxllm/hip_graph_bucket.h"
#include "rtxllm/layer_executor.h"
#include "rtxllm/layer_plan.h"
#include "rtxllm/llama.h"
#include "rtxllm/pack_manifest.h"
#include "rtxllm/vram_arena.h"
#include "synth.h"
#include "xq.h"

static_assert(RTXLLM_LLAMA_STATUS_CONTEXT_FULL == rtxllm::kStatusContextFull, "status bits of the C-ABI");
static_assert(RTXLLM_LLAMA_STATUS_WAIT_TIMEOUT == RTXLLM_STATUS_WAIT_TIMEOUT, "status bits of the C-ABI");

struct rtxllm_llama {
  rtxllm_llama_config cfg{};
  rtxllm::VramSuperallocator arena;
  rtxllm::HipGraphBucket graph;
  // context-bucketed step graphs by attention span, and the step's graph
  // bucket descriptor (admission and graph-memory accounting)
  std::map<std::uint32_t, rtxllm::HipGraphBucket> span_graphs;
  rtxllm::HipGraphBucketDescriptor graph_desc;
  std::uint32_t span = 0;  // positions the attention launches cover: max_ctx, or a bucket's span while capturing
  std::uint32_t q_rows = 0, kv_rows = 0, nslots = 0;
  std::uint32_t key_slots = 0;  // argmax slots of the LM-head launch (per sequence)
  std::size_t partial_floats = 0;  // attention partial records per sequence
  std::uint32_t batch = 1, pages_per_seq = 0;
  std::uint32_t groups_o = 1, groups_down = 1;  // panel groups of the batch o / down matvecs
  // role plans of the layer-slice executor: one decoder layer (attention
  // phase: qkv (+ attention), o; ffn phase: gate/up, down) and the head
  // (output phase: LM head + argmax)
  rtxllm::LayerExecutionPlan layer_plan, head_plan;
  rtxllm::AdmissionDecision admission;
  // Batch 1: the matvecs of IQ2_S / IQ3_S tensors read copies in the unit
  // layouts ("<role>_units"), rebuilt from "<role>" before the next launch
  // after the layer's weights change (upload, synthesis, packs).
  struct UnitCopy {
    std::string role;
    int fmt;  // the unit layout
    std::uint32_t rows, cols;
  };
  std::vector<UnitCopy> unit_copies;
  std::vector<char> units_dirty;  // [copy * n_layers + layer]
};

namespace {

using rtxllm::ArenaSpec;

std::size_t blocks_of(std::uint32_t rows, std::uint32_t cols) {
  return static_cast<std::size_t>(rows) * (cols / 256u);
}

// Configurable tensor formats (the unit layouts are the runner's own copies).
bool format_ok(int fmt) {
  return fmt >= RTXLLM_FMT_Q4K_RAW && fmt < RTXLLM_FMT_COUNT && fmt != RTXLLM_FMT_IQ2S_UNITS &&
         fmt != RTXLLM_FMT_IQ3S_UNITS;
}

std::string layer_name(const char* role, std::uint32_t layer) {
  return "L" + std::to_string(layer) + "." + role;
}

// Payload and (for Q4_K split layouts) metadata regions of one weight tensor.
void add_tensor(std::vector<ArenaSpec>& specs, const std::string& name, int fmt, std::uint32_t rows,
                std::uint32_t cols) {
  const std::size_t nb = blocks_of(rows, cols);
  specs.push_back({name, nb * rtxllm_format_payload_bytes(fmt)});
  if (rtxllm_format_meta_bytes(fmt) != 0u) specs.push_back({name + "_meta", nb * rtxllm_format_meta_bytes(fmt)});
}

struct TensorRef {
  const std::uint8_t* payload;
  const std::uint8_t* meta;
};

TensorRef tensor(const rtxllm_llama* m, const std::string& name) {
  const auto* base = static_cast<const std::uint8_t*>(m->arena.arena_ptr(name));
  const std::uint8_t* meta =
      m->arena.has_arena(name + "_meta") ? static_cast<const std::uint8_t*>(m->arena.arena_ptr(name + "_meta")) : nullptr;
  return {base, meta};
}

template <class T>
T* region(const rtxllm_llama* m, const std::string& name) {
  return static_cast<T*>(m->arena.arena_ptr(name));
}

rtxllm::KvLayer kv_layer(const rtxllm_llama* m, std::uint32_t layer) {
  rtxllm::KvLayer kv{};
  kv.k = region<std::uint16_t>(m, layer_name("k_cache", layer));
  kv.v = region<std::uint16_t>(m, layer_name("v_cache", layer));
  kv.block_table = region<std::int32_t>(m, layer_name("block_table", layer));
  kv.page_size = m->cfg.page_size;
  kv.n_kv = m->cfg.n_kv_heads;
  kv.capacity = m->cfg.max_ctx;  // per sequence
  return kv;
}

void mark_units_dirty(rtxllm_llama* m) {
  std::fill(m->units_dirty.begin(), m->units_dirty.end(), 1);
}

// The unit layout of a GGUF IQ format (-1: none).
int units_of(int fmt) {
  return fmt == RTXLLM_FMT_IQ2S ? RTXLLM_FMT_IQ2S_UNITS : fmt == RTXLLM_FMT_IQ3S ? RTXLLM_FMT_IQ3S_UNITS : -1;
}

// The copy of `role` (-1: the role's matvec reads the GGUF layout).
int unit_copy(const rtxllm_llama* m, const char* role) {
  for (std::size_t i = 0; i < m->unit_copies.size(); ++i)
    if (m->unit_copies[i].role == role) return static_cast<int>(i);
  return -1;
}

// Rebuild the unit copies of the layers whose weights changed (stream ordered
// after the writes; a device-to-device regrouping, no allocation).
hipError_t ensure_units(rtxllm_llama* m, hipStream_t stream) {
  const std::uint32_t L = m->cfg.n_layers;
  for (std::size_t i = 0; i < m->unit_copies.size(); ++i) {
    const rtxllm_llama::UnitCopy& u = m->unit_copies[i];
    for (std::uint32_t l = 0; l < L; ++l) {
      if (!m->units_dirty[i * L + l]) continue;
      const auto* raw = static_cast<const std::uint8_t*>(m->arena.arena_ptr(layer_name(u.role.c_str(), l)));
      auto* out = static_cast<std::uint8_t*>(m->arena.arena_ptr(layer_name((u.role + "_units").c_str(), l)));
      const hipError_t st = u.fmt == RTXLLM_FMT_IQ2S_UNITS ? rtxllm_iq2s_units_pack(raw, u.rows, u.cols, out, stream)
                                                           : rtxllm_iq3s_units_pack(raw, u.rows, u.cols, out, stream);
      if (st != hipSuccess) return st;
      m->units_dirty[i * L + l] = 0;
    }
  }
  return hipSuccess;
}

// The tensor a batch-1 matvec of `role` (format fmt) reads, and its format.
TensorRef tensor_for(const rtxllm_llama* m, const char* role, std::uint32_t l, int fmt, int& read_fmt) {
  const int u = unit_copy(m, role);
  read_fmt = u >= 0 ? m->unit_copies[static_cast<std::size_t>(u)].fmt : fmt;
  return tensor(m, layer_name(u >= 0 ? (std::string(role) + "_units").c_str() : role, l));
}

hipError_t synth_tensor(rtxllm_llama* m, const std::string& name, int fmt, std::uint32_t rows, std::uint32_t cols,
                        std::uint64_t seed, hipStream_t stream) {
  const std::size_t nb = blocks_of(rows, cols);
  auto* dst = region<std::uint8_t>(m, name);
  constexpr float kLo = 1e-4f, kHi = 2e-3f;
  if (fmt == RTXLLM_FMT_Q4K_SPLIT_NATIVE)
    return rtxllm::launch_synth_q4k_native(seed, nb, kLo, kHi, dst, region<std::uint8_t>(m, name + "_meta"), stream);
  if (rtxllm_format_meta_bytes(fmt) != 0u) return hipErrorInvalidValue;
  return rtxllm::launch_synth_raw(fmt, seed, nb, kLo, kHi, dst, stream);
}

}  // namespace

namespace {

// The model's plan without allocating: the validated config, the derived sizes
// in m, the arena specs, and the strict admission decision (m.admission) of
// weights, KV cache, workspace and the step graph's memory against the
// device's free bytes less guard_bytes.
hipError_t plan_model(const rtxllm_llama_config& c, std::size_t guard_bytes, rtxllm_llama* m,
                      std::vector<ArenaSpec>& specs) {
  const bool shapes_ok = c.hidden != 0u && c.hidden % 256u == 0u && c.hidden <= 16384u && c.n_heads != 0u &&
                         c.n_kv_heads != 0u && c.n_heads % c.n_kv_heads == 0u && c.n_heads / c.n_kv_heads <= 8u &&
                         (c.n_heads * rtxllm::kHeadDim) % 256u == 0u && c.ffn != 0u && c.ffn % 256u == 0u &&
                         c.vocab != 0u && c.n_layers != 0u && c.page_size != 0u && c.max_ctx != 0u &&
                         c.max_ctx % c.page_size == 0u && c.rms_eps >= 0.0f && c.rope_theta > 0.0f;
  if (!shapes_ok || !format_ok(c.fmt_qkv) || !format_ok(c.fmt_o) || !format_ok(c.fmt_gate_up) ||
      !format_ok(c.fmt_down) || !format_ok(c.fmt_lm_head))
    return hipErrorInvalidValue;
  const std::uint32_t batch = c.batch == 0u ? 1u : c.batch;
  if (batch > 8u) return hipErrorInvalidValue;
  if (batch > 1u) {
    // the batch matvecs take 512-column panels; the fused epilogues (qkv,
    // gate/up, LM head) need one panel group of at most 8 panels
    const std::uint32_t q_cols = c.n_heads * rtxllm::kHeadDim;
    const int mm_fmts[] = {c.fmt_qkv, c.fmt_o, c.fmt_gate_up, c.fmt_down, c.fmt_lm_head};
    for (int f : mm_fmts)
      if (f != RTXLLM_FMT_Q4K_RAW && f != RTXLLM_FMT_Q4K_SPLIT_NATIVE && f != RTXLLM_FMT_Q5K &&
          f != RTXLLM_FMT_IQ2S && f != RTXLLM_FMT_IQ3S)
        return hipErrorInvalidValue;
    if (c.hidden % 512u != 0u || c.hidden > 4096u || q_cols % 512u != 0u || c.ffn % 512u != 0u)
      return hipErrorInvalidValue;
  }

  m->cfg = c;
  m->q_rows = c.n_heads * rtxllm::kHeadDim;
  m->kv_rows = c.n_kv_heads * rtxllm::kHeadDim;
  m->nslots = c.hidden / rtxllm::kXGroup;
  m->partial_floats = rtxllm::attention_partials_floats(c.n_heads, c.n_kv_heads, c.max_ctx);
  m->batch = batch;
  m->span = c.max_ctx;
  if (batch == 1u) {
    const rtxllm_llama::UnitCopy roles[] = {{"qkv", c.fmt_qkv, m->q_rows + 2u * m->kv_rows, c.hidden},
                                            {"o", c.fmt_o, c.hidden, m->q_rows},
                                            {"gate_up", c.fmt_gate_up, 2u * c.ffn, c.hidden},
                                            {"down", c.fmt_down, c.hidden, c.ffn}};
    for (const auto& r : roles)
      if (units_of(r.fmt) >= 0) m->unit_copies.push_back({r.role, units_of(r.fmt), r.rows, r.cols});
  }
  m->units_dirty.assign(m->unit_copies.size() * c.n_layers, 1);
  m->pages_per_seq = c.max_ctx / c.page_size;
  const std::size_t B = batch;

  const std::size_t kv_halves =
      B * m->pages_per_seq * c.n_kv_heads * c.page_size * rtxllm::kHeadDim;
  specs.clear();
  for (std::uint32_t l = 0; l < c.n_layers; ++l) {
    add_tensor(specs, layer_name("qkv", l), c.fmt_qkv, m->q_rows + 2u * m->kv_rows, c.hidden);
    add_tensor(specs, layer_name("o", l), c.fmt_o, c.hidden, m->q_rows);
    add_tensor(specs, layer_name("gate_up", l), c.fmt_gate_up, 2u * c.ffn, c.hidden);
    for (const auto& u : m->unit_copies)
      add_tensor(specs, layer_name((u.role + "_units").c_str(), l), u.fmt, u.rows, u.cols);
    add_tensor(specs, layer_name("down", l), c.fmt_down, c.hidden, c.ffn);
    specs.push_back({layer_name("attn_norm", l), 4u * c.hidden});
    specs.push_back({layer_name("ffn_norm", l), 4u * c.hidden});
    specs.push_back({layer_name("k_cache", l), 2u * kv_halves});
    specs.push_back({layer_name("v_cache", l), 2u * kv_halves});
    specs.push_back({layer_name("block_table", l), 4u * B * m->pages_per_seq});
  }
  specs.push_back({"embed", blocks_of(c.vocab, c.hidden) * 176u});
  add_tensor(specs, "lm_head", c.fmt_lm_head, c.vocab, c.hidden);
  specs.push_back({"out_norm", 4u * c.hidden});
  specs.push_back({"h", 4u * B * c.hidden});
  specs.push_back({"xq", rtxllm::xq_bytes(c.hidden)});
  specs.push_back({"sumsq", 4u * m->nslots});
  specs.push_back({"q", B * c.n_kv_heads * rtxllm::kQ16BytesPerKv});
  specs.push_back({"att", 4u * B * m->q_rows});
  specs.push_back({"xq_att", rtxllm::xq_bytes(m->q_rows)});
  specs.push_back({"attn_partials", 4u * B * m->partial_floats});
  specs.push_back({"act", 4u * B * c.ffn});
  specs.push_back({"logits", 4u * B * c.vocab});
  m->key_slots = batch == 1u ? rtxllm::logits_key_slots(c.fmt_lm_head, c.vocab, c.hidden)
                             : rtxllm::mm_logits_key_slots(c.fmt_lm_head, c.vocab, c.hidden);
  if (m->key_slots == 0u) return hipErrorInvalidValue;
  specs.push_back({"argkeys", 8u * B * m->key_slots});
  specs.push_back({"token", 4u * B});
  specs.push_back({"pos", 4u * B});
  specs.push_back({"status", 4u * B});
  if (batch > 1u) {
    const std::uint32_t widest = std::max({c.hidden, m->q_rows, c.ffn});
    specs.push_back({"x16", rtxllm_x16_bytes(widest)});
    m->groups_o = rtxllm::mm_panel_groups(c.fmt_o, c.hidden, m->q_rows);
    m->groups_down = rtxllm::mm_panel_groups(c.fmt_down, c.hidden, c.ffn);
    if (m->groups_o == 0u || m->groups_down == 0u) return hipErrorInvalidValue;
    specs.push_back({"mm_work", 4u * B * c.hidden * std::max(m->groups_o, m->groups_down)});
  }
  specs.push_back({"inv_freq", 4u * rtxllm::kHeadDim / 2u});
  specs.push_back({"rope", 8u * static_cast<std::size_t>(c.max_ctx) * (rtxllm::kHeadDim / 2u)});
  // the layer-slice role plans, validated once
  {
    static const std::vector<rtxllm::LayerStageDescriptor> kLayer = {
        {"attn_qkv.weight"}, {"attn_output.weight"}, {"ffn_gate_up.weight"}, {"ffn_down.weight"}};
    static const std::vector<rtxllm::LayerStageDescriptor> kHeadStages = {{"output.weight", false}};
    for (const auto* stages : {&kLayer, &kHeadStages}) {
      const auto segments = rtxllm::build_layer_phase_segments(*stages);
      if (stages == &kLayer && !rtxllm::validate_layer_phase_plan(*stages, segments).passed)
        return hipErrorInvalidValue;
      (stages == &kLayer ? m->layer_plan : m->head_plan) = rtxllm::build_layer_execution_plan(segments, false);
    }
  }
  // strict admission: weights, KV cache, workspace and the step graph's
  // memory against the device's free bytes
  {
    rtxllm::RequestEstimate req;
    for (const auto& spec : specs) {
      const std::size_t b = (spec.bytes + 255u) & ~std::size_t{255};
      const std::string& n = spec.name;
      const bool kv = n.find("k_cache") != std::string::npos || n.find("v_cache") != std::string::npos ||
                      n.find("block_table") != std::string::npos;
      const bool weight = n.find(".qkv") != std::string::npos || n.find(".o") != std::string::npos ||
                          n.find(".gate_up") != std::string::npos || n.find(".down") != std::string::npos ||
                          n.find("_norm") != std::string::npos || n == "embed" || n.rfind("lm_head", 0) == 0;
      (kv ? req.kv_cache_bytes : weight ? req.weight_bytes : req.workspace_bytes) += b;
    }
    req.workspace_high_water_bytes = req.workspace_bytes;
    rtxllm::HipGraphBucketDescriptor gd;
    gd.name = "decode";
    gd.batch_bucket = batch;
    gd.phase_count = static_cast<std::uint32_t>(c.n_layers * m->layer_plan.phase_count + m->head_plan.phase_count);
    gd.kernel_launches_per_replay = batch > 1u ? 1u + 8u * c.n_layers + 2u : 1u + 6u * c.n_layers + 2u;
    gd.workspace_high_water_bytes = req.workspace_bytes;
    req.graph_bytes = rtxllm::estimate_hip_graph_bucket_allocation(gd).total_bytes;
    m->graph_desc = gd;
    std::size_t free_b = 0, total_b = 0;
    const hipError_t mi = hipMemGetInfo(&free_b, &total_b);
    if (mi != hipSuccess) return mi;
    m->admission =
        rtxllm::decide_admission(rtxllm::ResidencyPolicy::Strict, rtxllm::MemoryBudget{free_b, guard_bytes}, req);
  }
  return hipSuccess;
}

}  // namespace

extern "C" hipError_t rtxllm_llama_admission(const rtxllm_llama_config* cfg, size_t guard_bytes, int* admitted,
                                             size_t* required_bytes, size_t* usable_bytes, char* reason,
                                             size_t reason_len) {
  if (cfg == nullptr) return hipErrorInvalidValue;
  std::unique_ptr<rtxllm_llama> m(new (std::nothrow) rtxllm_llama());
  if (!m) return hipErrorOutOfMemory;
  std::vector<ArenaSpec> specs;
  const hipError_t st = plan_model(*cfg, guard_bytes, m.get(), specs);
  if (st != hipSuccess) return st;
  if (admitted != nullptr) *admitted = m->admission.admit ? 1 : 0;
  if (required_bytes != nullptr) *required_bytes = m->admission.required_bytes;
  if (usable_bytes != nullptr) *usable_bytes = m->admission.usable_bytes;
  if (reason != nullptr && reason_len > 0) std::snprintf(reason, reason_len, "%s", m->admission.reason.c_str());
  return hipSuccess;
}

extern "C" hipError_t rtxllm_llama_create(const rtxllm_llama_config* cfg, rtxllm_llama** out) {
  if (cfg == nullptr || out == nullptr) return hipErrorInvalidValue;
  *out = nullptr;
  const rtxllm_llama_config& c = *cfg;
  std::unique_ptr<rtxllm_llama> m(new (std::nothrow) rtxllm_llama());
  if (!m) return hipErrorOutOfMemory;
  std::vector<ArenaSpec> specs;
  {
    const hipError_t pst = plan_model(c, 0u, m.get(), specs);
    if (pst != hipSuccess) return pst;
  }
  if (!m->admission.admit) return hipErrorOutOfMemory;
  const std::size_t B = m->batch;
  try {
    m->arena.initialize(specs);
    m->arena.reset();
  } catch (const std::exception&) {
    return hipErrorOutOfMemory;
  }

  // RoPE frequencies theta^(-2i/d), computed in double and rounded once; identity block tables.
  std::vector<float> inv_freq(rtxllm::kHeadDim / 2u);
  for (std::uint32_t i = 0; i < inv_freq.size(); ++i)
    inv_freq[i] = static_cast<float>(std::pow(static_cast<double>(c.rope_theta),
                                              -2.0 * static_cast<double>(i) / static_cast<double>(rtxllm::kHeadDim)));
  hipError_t st = hipMemcpy(m->arena.arena_ptr("inv_freq"), inv_freq.data(), 4u * inv_freq.size(), hipMemcpyHostToDevice);
  if (st != hipSuccess) return st;
  // rotary table: (cos, sin) of the fp32 angle pos * inv_freq[i] (the product
  // rounded to fp32, as the textbook RoPE evaluates it), each rounded once
  // from double, for every position of the cache
  const std::size_t half = rtxllm::kHeadDim / 2u;
  std::vector<float> rope(2u * c.max_ctx * half);
  for (std::uint32_t p = 0; p < c.max_ctx; ++p)
    for (std::size_t i = 0; i < half; ++i) {
      const float angle = static_cast<float>(p) * inv_freq[i];
      rope[2u * (p * half + i)] = static_cast<float>(std::cos(static_cast<double>(angle)));
      rope[2u * (p * half + i) + 1u] = static_cast<float>(std::sin(static_cast<double>(angle)));
    }
  st = hipMemcpy(m->arena.arena_ptr("rope"), rope.data(), 4u * rope.size(), hipMemcpyHostToDevice);
  if (st != hipSuccess) return st;
  // sequence s owns pages [s * pages_per_seq, (s + 1) * pages_per_seq)
  std::vector<std::int32_t> table(B * m->pages_per_seq);
  for (std::uint32_t i = 0; i < table.size(); ++i) table[i] = static_cast<std::int32_t>(i);
  for (std::uint32_t l = 0; l < c.n_layers; ++l) {
    st = hipMemcpy(m->arena.arena_ptr(layer_name("block_table", l)), table.data(), 4u * table.size(),
                   hipMemcpyHostToDevice);
    if (st != hipSuccess) return st;
  }
  // staged columns of sequences >= batch and the q16 columns of absent query
  // heads stay zero
  for (const char* name : {"x16", "q"}) {
    std::size_t n = 0;
    void* p = rtxllm_llama_region(m.get(), name, 0u, &n);
    if (p == nullptr) continue;
    st = hipMemset(p, 0, n);
    if (st != hipSuccess) return st;
  }
  st = hipDeviceSynchronize();
  if (st != hipSuccess) return st;
  *out = m.release();
  return hipSuccess;
}

extern "C" void rtxllm_llama_destroy(rtxllm_llama* m) { delete m; }

extern "C" void* rtxllm_llama_region(rtxllm_llama* m, const char* name, uint32_t layer, size_t* bytes) {
  if (m == nullptr || name == nullptr) return nullptr;
  static const char* kPerLayer[] = {"qkv",       "qkv_meta",  "qkv_units", "o",           "o_meta",
                                    "o_units",   "gate_up",   "gate_up_meta", "gate_up_units", "down",
                                    "down_meta", "down_units", "attn_norm", "ffn_norm",  "k_cache",
                                    "v_cache",   "block_table"};
  std::string key = name;
  for (const char* p : kPerLayer)
    if (key == p) {
      if (layer >= m->cfg.n_layers) return nullptr;
      key = layer_name(name, layer);
      break;
    }
  if (!m->arena.has_arena(key)) return nullptr;
  const rtxllm::ArenaView v = m->arena.arena(key);
  if (bytes != nullptr) *bytes = v.bytes;
  return static_cast<std::uint8_t*>(m->arena.base()) + v.offset;
}

extern "C" hipError_t rtxllm_llama_upload(rtxllm_llama* m, const char* name, uint32_t layer, size_t offset,
                                          const void* src, size_t bytes) {
  std::size_t size = 0;
  auto* base = static_cast<std::uint8_t*>(rtxllm_llama_region(m, name, layer, &size));
  if (base == nullptr || src == nullptr || offset > size || bytes > size - offset) return hipErrorInvalidValue;
  // positions must have a KV slot and tokens a row of the embedding table
  const std::string key = name;
  if (key == "pos" || key == "token") {
    if (offset % 4u != 0u || bytes % 4u != 0u) return hipErrorInvalidValue;
    const std::uint32_t limit = key == "pos" ? m->cfg.max_ctx : m->cfg.vocab;
    for (std::size_t i = 0; i < bytes / 4u; ++i) {
      std::uint32_t v;
      std::memcpy(&v, static_cast<const std::uint8_t*>(src) + 4u * i, 4u);
      if (v >= limit) return hipErrorInvalidValue;
    }
  }
  const int u = unit_copy(m, name);
  if (u >= 0) m->units_dirty[static_cast<std::size_t>(u) * m->cfg.n_layers + layer] = 1;
  return hipMemcpy(base + offset, src, bytes, hipMemcpyHostToDevice);
}

extern "C" hipError_t rtxllm_llama_download(rtxllm_llama* m, const char* name, uint32_t layer, size_t offset,
                                            void* dst, size_t bytes) {
  std::size_t size = 0;
  auto* base = static_cast<std::uint8_t*>(rtxllm_llama_region(m, name, layer, &size));
  if (base == nullptr || dst == nullptr || offset > size || bytes > size - offset) return hipErrorInvalidValue;
  return hipMemcpy(dst, base + offset, bytes, hipMemcpyDeviceToHost);
}

namespace {

// One tensor read from a pack: its format, GGUF shape and stream bytes.
struct PackTensor {
  int fmt = -1;
  std::uint64_t rows = 0, cols = 0;
  std::vector<std::uint8_t> payload, meta;
};

std::filesystem::path under(const std::filesystem::path& root, const std::filesystem::path& p) {
  return p.is_absolute() || root.empty() ? p : root / p;
}

void verify(const std::vector<std::uint8_t>& bytes, std::uint64_t checksum, const std::string& what) {
  if (rtxllm::byte_checksum(bytes) != checksum) throw std::runtime_error("checksum mismatch: " + what);
}

struct ManifestRef {
  rtxllm::PackManifestKind kind;
  std::string path;
};

// GGUF tensors of the manifests, by name. A Q4_K tensor is read in the layout
// the runner's config wants for it (`want` maps a tensor name to its format):
// a split layout from its payload + metadata files (the manifest's policy
// must be that layout), the raw blocks from blocks_path. A tensor named in
// two manifests is refused.
std::map<std::string, PackTensor> read_packs(const std::vector<ManifestRef>& manifests,
                                             const std::filesystem::path& root,
                                             const std::map<std::string, int>& want) {
  std::map<std::string, PackTensor> out;
  auto keep = [&](const std::string& name, PackTensor&& pt) {
    if (!out.emplace(name, std::move(pt)).second) throw std::runtime_error("tensor in two manifests: " + name);
  };
  for (const ManifestRef& ref : manifests) {
    if (ref.kind != rtxllm::PackManifestKind::Q4K) continue;
    const rtxllm::Q4KManifest man = rtxllm::load_q4k_manifest(ref.path);
    for (const auto& t : man.tensors) {
      const auto w = want.find(t.name);
      if (w == want.end()) continue;
      PackTensor pt;
      pt.fmt = w->second;
      pt.rows = t.rows, pt.cols = t.cols;
      const std::uint64_t blocks = static_cast<std::uint64_t>(t.rows) * (t.cols / 256u);
      if (pt.fmt == RTXLLM_FMT_Q4K_RAW) {
        if (t.blocks_path.empty()) throw std::runtime_error("raw Q4_K blocks not in the pack: " + t.name);
        pt.payload = rtxllm::load_binary_file(under(root, t.blocks_path), blocks * 144u, "q4k blocks");
        verify(pt.payload, t.source_checksum, t.name + " blocks");
      } else {
        if (rtxllm::q4k_policy_format(t.policy) != pt.fmt)
          throw std::runtime_error("Q4_K pack layout " + t.policy + " is not the configured one: " + t.name);
        pt.payload = rtxllm::load_binary_file(under(root, t.payload_path), t.payload_bytes, "q4k payload");
        pt.meta = rtxllm::load_binary_file(under(root, t.metadata_path), t.metadata_bytes, "q4k metadata");
        verify(pt.payload, t.payload_checksum, t.name + " payload");
        verify(pt.meta, t.metadata_checksum, t.name + " metadata");
        if (pt.payload.size() != blocks * rtxllm_format_payload_bytes(pt.fmt) ||
            pt.meta.size() != blocks * rtxllm_format_meta_bytes(pt.fmt))
          throw std::runtime_error("Q4_K pack stream sizes disagree with the shape: " + t.name);
      }
      keep(t.name, std::move(pt));
    }
  }
  for (const ManifestRef& ref : manifests) {
    if (ref.kind != rtxllm::PackManifestKind::RawBlocks) continue;
    const rtxllm::IQManifest man = rtxllm::load_iq_manifest(ref.path);
    static const std::map<std::string, int> kType = {
        {"IQ2_S", RTXLLM_FMT_IQ2S}, {"IQ3_S", RTXLLM_FMT_IQ3S}, {"Q5_K", RTXLLM_FMT_Q5K}};
    for (const auto& t : man.tensors) {
      const auto w = want.find(t.name);
      if (w == want.end()) continue;
      PackTensor pt;
      pt.fmt = kType.at(t.type);
      if (pt.fmt != w->second) throw std::runtime_error("pack type " + t.type + " is not the configured one: " + t.name);
      if (t.dimensions.size() != 2u) throw std::runtime_error("raw-block pack without 2-D dimensions: " + t.name);
      pt.cols = t.dimensions[0], pt.rows = t.dimensions[1];
      if (t.block_count != pt.rows * (pt.cols / 256u) || t.block_type_size != rtxllm_format_payload_bytes(pt.fmt))
        throw std::runtime_error("raw-block pack geometry disagrees with its dimensions: " + t.name);
      pt.payload = rtxllm::load_binary_file(under(root, t.payload_path), t.payload_bytes, "raw blocks");
      verify(pt.payload, t.payload_checksum, t.name);
      keep(t.name, std::move(pt));
    }
  }
  return out;
}

hipError_t load_manifests(rtxllm_llama* m, const std::vector<ManifestRef>& manifests, const char* payload_root,
                          char* err, size_t err_len);

}  // namespace

extern "C" hipError_t rtxllm_llama_load_packs(rtxllm_llama* m, const char* q4k_manifest, const char* iq_manifest,
                                              const char* payload_root, char* err, size_t err_len) {
  std::vector<ManifestRef> refs;
  if (q4k_manifest != nullptr && *q4k_manifest != '\0') refs.push_back({rtxllm::PackManifestKind::Q4K, q4k_manifest});
  if (iq_manifest != nullptr && *iq_manifest != '\0') refs.push_back({rtxllm::PackManifestKind::RawBlocks, iq_manifest});
  return load_manifests(m, refs, payload_root, err, err_len);
}

extern "C" hipError_t rtxllm_llama_load_pack_set(rtxllm_llama* m, const char* const* manifests, uint32_t count,
                                                 const char* payload_root, char* err, size_t err_len) {
  std::vector<ManifestRef> refs;
  try {
    if (manifests == nullptr && count != 0) throw std::runtime_error("manifests is null");
    for (uint32_t i = 0; i < count; ++i) {
      if (manifests[i] == nullptr || *manifests[i] == '\0') throw std::runtime_error("empty manifest path");
      refs.push_back({rtxllm::pack_manifest_kind(manifests[i]), manifests[i]});
    }
  } catch (const std::exception& e) {
    if (err != nullptr && err_len > 0) std::snprintf(err, err_len, "%s", e.what());
    return hipErrorInvalidValue;
  }
  return load_manifests(m, refs, payload_root, err, err_len);
}

namespace {

hipError_t load_manifests(rtxllm_llama* m, const std::vector<ManifestRef>& manifests, const char* payload_root,
                          char* err, size_t err_len) {
  auto report = [&](const std::string& what) {
    if (err != nullptr && err_len > 0) {
      const std::size_t n = std::min(what.size(), err_len - 1u);
      std::memcpy(err, what.data(), n);
      err[n] = '\0';
    }
  };
  if (m == nullptr) return hipErrorInvalidValue;
  const rtxllm_llama_config& c = m->cfg;
  const std::uint32_t H = c.hidden, Q = m->q_rows, KV = m->kv_rows, F = c.ffn;
  // every tensor the model needs: GGUF name -> (format, rows, cols)
  struct Need {
    int fmt;
    std::uint64_t rows, cols;
  };
  std::map<std::string, Need> need;
  for (std::uint32_t l = 0; l < c.n_layers; ++l) {
    const std::string b = "blk." + std::to_string(l) + ".";
    need[b + "attn_q.weight"] = {c.fmt_qkv, Q, H};
    need[b + "attn_k.weight"] = {c.fmt_qkv, KV, H};
    need[b + "attn_v.weight"] = {c.fmt_qkv, KV, H};
    need[b + "attn_output.weight"] = {c.fmt_o, H, Q};
    need[b + "ffn_gate.weight"] = {c.fmt_gate_up, F, H};
    need[b + "ffn_up.weight"] = {c.fmt_gate_up, F, H};
    need[b + "ffn_down.weight"] = {c.fmt_down, H, F};
  }
  need["token_embd.weight"] = {RTXLLM_FMT_Q5K, c.vocab, H};
  need["output.weight"] = {c.fmt_lm_head, c.vocab, H};
  std::map<std::string, int> want;
  for (const auto& kv : need) want[kv.first] = kv.second.fmt;
  try {
    const auto packs = read_packs(manifests, payload_root != nullptr ? payload_root : "", want);
    auto get = [&](const std::string& name) -> const PackTensor& {
      const auto it = packs.find(name);
      if (it == packs.end()) throw std::runtime_error("tensor missing from the packs: " + name);
      const Need& n = need.at(name);
      if (it->second.rows != n.rows || it->second.cols != n.cols)
        throw std::runtime_error("tensor shape disagrees with the model: " + name);
      return it->second;
    };
    // Every upload is planned and checked first (tensor present, shape, region
    // size), then performed: a refused pack set leaves the weights untouched.
    struct Upload {
      std::string region;
      std::vector<const std::vector<std::uint8_t>*> parts;  // stacked in order
      std::size_t interleave_rows;                         // > 0: parts[0], parts[1] interleaved by row
    };
    std::vector<Upload> plan;
    auto add = [&](const std::string& region, std::vector<const std::vector<std::uint8_t>*> parts,
                   std::size_t rows = 0) {
      std::size_t bytes = 0;
      for (const auto* p : parts) bytes += p->size();
      if (bytes == 0) return;  // no metadata stream for this format
      std::size_t size = 0;
      if (rtxllm_llama_region(m, region.c_str(), 0u, &size) == nullptr || size != bytes)
        throw std::runtime_error("region size mismatch: " + region);
      if (rows > 0 && (parts.size() != 2 || parts[0]->size() != parts[1]->size() || parts[0]->size() % rows != 0))
        throw std::runtime_error("gate/up streams differ: " + region);
      plan.push_back({region, std::move(parts), rows});
    };
    for (std::uint32_t l = 0; l < c.n_layers; ++l) {
      const std::string b = "blk." + std::to_string(l) + ".", L = "L" + std::to_string(l) + ".";
      const auto &q = get(b + "attn_q.weight"), &k = get(b + "attn_k.weight"), &v = get(b + "attn_v.weight");
      add(L + "qkv", {&q.payload, &k.payload, &v.payload});
      add(L + "qkv_meta", {&q.meta, &k.meta, &v.meta});
      const auto& o = get(b + "attn_output.weight");
      add(L + "o", {&o.payload});
      add(L + "o_meta", {&o.meta});
      const auto &g = get(b + "ffn_gate.weight"), &u = get(b + "ffn_up.weight");
      add(L + "gate_up", {&g.payload, &u.payload}, F);
      add(L + "gate_up_meta", {&g.meta, &u.meta}, F);
      const auto& d = get(b + "ffn_down.weight");
      add(L + "down", {&d.payload});
      add(L + "down_meta", {&d.meta});
    }
    add("embed", {&get("token_embd.weight").payload});
    const auto& lm = get("output.weight");
    add("lm_head", {&lm.payload});
    add("lm_head_meta", {&lm.meta});
    // stack rows (q | k | v) or interleave them (gate_i, up_i) stream by stream
    std::vector<std::uint8_t> staging;
    mark_units_dirty(m);
    for (const Upload& up : plan) {
      staging.clear();
      if (up.interleave_rows > 0) {
        const auto &a = *up.parts[0], &bb = *up.parts[1];
        const std::size_t rb = a.size() / up.interleave_rows;
        staging.resize(a.size() + bb.size());
        for (std::size_t i = 0; i < up.interleave_rows; ++i) {
          std::memcpy(staging.data() + (2 * i) * rb, a.data() + i * rb, rb);
          std::memcpy(staging.data() + (2 * i + 1) * rb, bb.data() + i * rb, rb);
        }
      } else {
        for (const auto* p : up.parts) staging.insert(staging.end(), p->begin(), p->end());
      }
      void* dst = rtxllm_llama_region(m, up.region.c_str(), 0u, nullptr);
      const hipError_t st = hipMemcpy(dst, staging.data(), staging.size(), hipMemcpyHostToDevice);
      if (st != hipSuccess) throw std::runtime_error(std::string("upload failed: ") + hipGetErrorString(st));
    }
  } catch (const std::exception& e) {
    report(e.what());
    return hipErrorInvalidValue;
  }
  report("");
  return hipSuccess;
}

}  // namespace

extern "C" hipError_t rtxllm_llama_memory(const rtxllm_llama* m, size_t* required_bytes, size_t* usable_bytes,
                                          size_t* arena_bytes) {
  if (m == nullptr) return hipErrorInvalidValue;
  if (required_bytes != nullptr) *required_bytes = m->admission.required_bytes;
  if (usable_bytes != nullptr) *usable_bytes = m->admission.usable_bytes;
  if (arena_bytes != nullptr) *arena_bytes = m->arena.total_bytes();
  return hipSuccess;
}

extern "C" void rtxllm_llama_weights_changed(rtxllm_llama* m) {
  if (m != nullptr) mark_units_dirty(m);
}

extern "C" hipError_t rtxllm_llama_synth_weights(rtxllm_llama* m, uint64_t seed, hipStream_t stream) {
  if (m == nullptr) return hipErrorInvalidValue;
  mark_units_dirty(m);
  const rtxllm_llama_config& c = m->cfg;
  hipError_t st = hipSuccess;
  for (std::uint32_t l = 0; l < c.n_layers && st == hipSuccess; ++l) {
    const std::uint64_t ls = seed + 4096u * (static_cast<std::uint64_t>(l) + 1u);
    st = synth_tensor(m, layer_name("qkv", l), c.fmt_qkv, m->q_rows + 2u * m->kv_rows, c.hidden, ls + 1u, stream);
    if (st == hipSuccess) st = synth_tensor(m, layer_name("o", l), c.fmt_o, c.hidden, m->q_rows, ls + 2u, stream);
    if (st == hipSuccess)
      st = synth_tensor(m, layer_name("gate_up", l), c.fmt_gate_up, 2u * c.ffn, c.hidden, ls + 3u, stream);
    if (st == hipSuccess) st = synth_tensor(m, layer_name("down", l), c.fmt_down, c.hidden, c.ffn, ls + 4u, stream);
  }
  if (st == hipSuccess) st = synth_tensor(m, "embed", RTXLLM_FMT_Q5K, c.vocab, c.hidden, seed + 5u, stream);
  if (st == hipSuccess) st = synth_tensor(m, "lm_head", c.fmt_lm_head, c.vocab, c.hidden, seed + 6u, stream);
  return st;
}

namespace {

enum Stage { kEmbed = 0, kQkv = 1, kAttention = 2, kO = 3, kGateUp = 4, kDown = 5, kHead = 6 };

// One stage of layer l for a batch of B > 1 sequences, on the matrix cores:
// every stage ends with the next matvec's input staged in x16 (residual +
// RMSNorm fused into the per-sequence staging kernel).
hipError_t launch_stage_batch(rtxllm_llama* m, std::uint32_t l, int stage, bool embed, const float* next_norm,
                              hipStream_t stream) {
  const rtxllm_llama_config& c = m->cfg;
  const std::uint32_t B = m->batch;
  auto* h = region<float>(m, "h");
  void* x16 = m->arena.arena_ptr("x16");
  auto* work = region<float>(m, "mm_work");
  auto* pos = region<std::uint32_t>(m, "pos");
  auto* token = region<std::uint32_t>(m, "token");
  switch (stage) {
    case kEmbed:
      return rtxllm::launch_rms_stage_batch(h, nullptr, 0u, embed ? region<std::uint8_t>(m, "embed") : nullptr, token,
                                            c.vocab, next_norm, c.rms_eps, c.hidden, B, x16, stream);
    case kQkv: {
      const TensorRef t = tensor(m, layer_name("qkv", l));
      return rtxllm::launch_mm_qkv_batch(c.fmt_qkv, t.payload, t.meta, c.hidden, x16, B, m->q_rows, m->kv_rows,
                                         region<float2>(m, "rope"), c.max_ctx, pos, m->arena.arena_ptr("q"), kv_layer(m, l),
                                         m->pages_per_seq, stream);
    }
    case kAttention: {
      return rtxllm::launch_attention_batch(m->arena.arena_ptr("q"), kv_layer(m, l), c.n_heads, pos, m->span, B,
                                            m->pages_per_seq, region<float>(m, "attn_partials"),
                                            region<float>(m, "att"), nullptr, x16, stream);
    }
    case kO: {
      const TensorRef t = tensor(m, layer_name("o", l));
      hipError_t st = rtxllm::launch_mm_batch(c.fmt_o, t.payload, t.meta, c.hidden, m->q_rows, x16, B, work, stream);
      if (st != hipSuccess) return st;
      return rtxllm::launch_rms_stage_batch(h, work, m->groups_o, nullptr, nullptr, 0u,
                                            region<float>(m, layer_name("ffn_norm", l)), c.rms_eps, c.hidden, B, x16,
                                            stream);
    }
    case kGateUp: {
      const TensorRef t = tensor(m, layer_name("gate_up", l));
      // act [B][ffn] goes to the down projection in fp32: its waves stage it
      return rtxllm::launch_mm_gate_up_batch(c.fmt_gate_up, t.payload, t.meta, 2u * c.ffn, c.hidden, x16, B,
                                             region<float>(m, "act"), stream);
    }
    case kDown: {
      const TensorRef t = tensor(m, layer_name("down", l));
      hipError_t st = rtxllm::launch_mm_batch_self(c.fmt_down, t.payload, t.meta, c.hidden, c.ffn,
                                                   region<float>(m, "act"), B, work, stream);
      if (st != hipSuccess) return st;
      return rtxllm::launch_rms_stage_batch(h, work, m->groups_down, nullptr, nullptr, 0u, next_norm, c.rms_eps,
                                            c.hidden, B, x16, stream);
    }
    case kHead: {
      const TensorRef t = tensor(m, "lm_head");
      auto* keys = region<unsigned long long>(m, "argkeys");
      std::uint32_t count = 0u;
      const hipError_t st = rtxllm::launch_mm_logits_batch(c.fmt_lm_head, t.payload, t.meta, c.vocab, c.hidden, x16,
                                                           B, region<float>(m, "logits"), keys, m->key_slots, &count,
                                                           stream);
      if (st != hipSuccess) return st;
      return rtxllm::launch_argmax_finalize_batch(keys, m->key_slots, count, B, token, pos, 1u, c.max_ctx,
                                                  region<std::uint32_t>(m, "status"), stream);
    }
    default: return hipErrorInvalidValue;
  }
}

// One stage of layer l; next_norm is the norm weight the down stage stages the
// residual with (the next layer's attn_norm, or out_norm after the last layer).
hipError_t launch_stage(rtxllm_llama* m, std::uint32_t l, int stage, bool embed, const float* next_norm,
                        hipStream_t stream) {
  if (m->batch > 1u) return launch_stage_batch(m, l, stage, embed, next_norm, stream);
  const rtxllm_llama_config& c = m->cfg;
  auto* h = region<float>(m, "h");
  void* xq = m->arena.arena_ptr("xq");
  auto* sumsq = region<float>(m, "sumsq");
  auto* pos = region<std::uint32_t>(m, "pos");
  const rtxllm::NormIn in{xq, sumsq, m->nslots, c.hidden, c.rms_eps};
  switch (stage) {
    case kEmbed:
      return rtxllm::launch_embed_q5k(embed ? region<std::uint8_t>(m, "embed") : nullptr, c.hidden, c.vocab,
                                      region<std::uint32_t>(m, "token"), h, next_norm, xq, sumsq, m->nslots, stream);
    case kQkv: {
      int f = 0;
      const TensorRef t = tensor_for(m, "qkv", l, c.fmt_qkv, f);
      return rtxllm::launch_qkv(f, t.payload, t.meta, c.hidden, in, m->q_rows, m->kv_rows,
                                region<float2>(m, "rope"), c.max_ctx, pos, m->arena.arena_ptr("q"), kv_layer(m, l),
                                stream);
    }
    case kAttention:
      return rtxllm::launch_attention(m->arena.arena_ptr("q"), kv_layer(m, l), c.n_heads, pos, m->span,
                                      region<float>(m, "attn_partials"), region<float>(m, "att"),
                                      m->arena.arena_ptr("xq_att"), stream);
    case kO: {
      int f = 0;
      const TensorRef t = tensor_for(m, "o", l, c.fmt_o, f);
      return rtxllm::launch_residual(f, t.payload, t.meta, c.hidden, m->q_rows, m->arena.arena_ptr("xq_att"),
                                     nullptr, h,
                                     region<float>(m, layer_name("ffn_norm", l)), xq, sumsq, stream);
    }
    case kGateUp: {
      int f = 0;
      const TensorRef t = tensor_for(m, "gate_up", l, c.fmt_gate_up, f);
      return rtxllm::launch_gate_up(f, t.payload, t.meta, 2u * c.ffn, c.hidden, in, region<float>(m, "act"),
                                    region<std::uint32_t>(m, "status"), stream);
    }
    case kDown: {
      int f = 0;
      const TensorRef t = tensor_for(m, "down", l, c.fmt_down, f);
      return rtxllm::launch_residual(f, t.payload, t.meta, c.hidden, c.ffn, nullptr, region<float>(m, "act"), h,
                                     next_norm, xq, sumsq, stream);
    }
    case kHead: {
      const TensorRef t = tensor(m, "lm_head");
      auto* keys = region<unsigned long long>(m, "argkeys");
      std::uint32_t count = 0u;
      const hipError_t st = rtxllm::launch_logits(c.fmt_lm_head, t.payload, t.meta, c.vocab, c.hidden, in,
                                                  region<float>(m, "logits"), keys, m->key_slots, &count, stream);
      if (st != hipSuccess) return st;
      return rtxllm::launch_argmax_finalize(keys, count, region<std::uint32_t>(m, "token"), pos, 1u, c.max_ctx,
                                            region<std::uint32_t>(m, "status"), stream);
    }
    default: return hipErrorInvalidValue;
  }
}

}  // namespace

extern "C" hipError_t rtxllm_llama_forward(rtxllm_llama* m, uint32_t first, uint32_t last, int flags,
                                           hipStream_t stream) {
  if (m == nullptr || first > last || last > m->cfg.n_layers) return hipErrorInvalidValue;
  const float* out_norm = region<float>(m, "out_norm");
  const float* first_norm = first < last ? region<float>(m, layer_name("attn_norm", first)) : out_norm;
  hipError_t st = ensure_units(m, stream);
  if (st == hipSuccess) st = launch_stage(m, 0u, kEmbed, (flags & RTXLLM_LLAMA_EMBED) != 0, first_norm, stream);
  // Each layer replays the layer plan by phase: stage i of the plan is one of
  // qkv (with the attention over the updated cache), o, gate/up, down (their
  // activation hand-off is fused into the stages, so no feedback launches).
  static constexpr int kLayerStages[] = {kQkv, kO, kGateUp, kDown};
  try {
    for (std::uint32_t l = first; l < last && st == hipSuccess; ++l) {
      const float* next_norm = l + 1u < last ? region<float>(m, layer_name("attn_norm", l + 1u)) : out_norm;
      auto launch = [&](std::size_t i) {
        if (st == hipSuccess) st = launch_stage(m, l, kLayerStages[i], false, next_norm, stream);
        if (st == hipSuccess && kLayerStages[i] == kQkv) st = launch_stage(m, l, kAttention, false, next_norm, stream);
      };
      auto phase = [&](const rtxllm::LayerPhaseExecution& p) {
        return rtxllm::replay_layer_phase(p, m->layer_plan.stage_count, launch, [](std::size_t) {});
      };
      auto none = [](const rtxllm::LayerPhaseExecution&) -> rtxllm::LayerReplayCounters {
        throw std::runtime_error("the decoder layer has no such phase");
      };
      rtxllm::replay_layer_execution_plan_by_phase(m->layer_plan, m->layer_plan.stage_count, phase, phase, none, none);
    }
    if (st == hipSuccess && (flags & RTXLLM_LLAMA_HEAD)) {
      auto head = [&](std::size_t) {
        if (st == hipSuccess) st = launch_stage(m, 0u, kHead, false, out_norm, stream);
      };
      rtxllm::replay_layer_execution_plan(m->head_plan, m->head_plan.stage_count, head, [](std::size_t) {});
    }
  } catch (const std::exception&) {
    return hipErrorInvalidValue;
  }
  return st;
}

extern "C" hipError_t rtxllm_llama_launch_stage(rtxllm_llama* m, uint32_t layer, int stage, hipStream_t stream) {
  if (m == nullptr || layer >= m->cfg.n_layers || stage < kEmbed || stage > kHead) return hipErrorInvalidValue;
  const float* next_norm = layer + 1u < m->cfg.n_layers ? region<float>(m, layer_name("attn_norm", layer + 1u))
                                                        : region<float>(m, "out_norm");
  if (stage == kEmbed) next_norm = region<float>(m, layer_name("attn_norm", 0u));
  const hipError_t st = ensure_units(m, stream);
  if (st != hipSuccess) return st;
  return launch_stage(m, layer, stage, stage == kEmbed, next_norm, stream);
}

extern "C" hipError_t rtxllm_llama_step(rtxllm_llama* m, hipStream_t stream) {
  if (m == nullptr) return hipErrorInvalidValue;
  return rtxllm_llama_forward(m, 0u, m->cfg.n_layers, RTXLLM_LLAMA_EMBED | RTXLLM_LLAMA_HEAD, stream);
}

extern "C" uint32_t rtxllm_llama_launches_per_step(const rtxllm_llama* m) {
  if (m == nullptr) return 0u;
  // batch, per layer: qkv 1, attention 2 (partials; combine + staging of att),
  // o 2 and down 2 (matvec; residual + RMSNorm staging), gate/up 1 (the down
  // matvec stages act itself)
  return m->batch > 1u ? 1u + 8u * m->cfg.n_layers + 2u : 1u + 6u * m->cfg.n_layers + 2u;
}

namespace {

// Capture one step (attention over m->span positions) into `bucket`.
hipError_t capture_step(rtxllm_llama* m, rtxllm::HipGraphBucket& bucket, hipStream_t stream) {
  hipError_t st = ensure_units(m, stream);  // before the capture: the graph holds the step alone
  if (st != hipSuccess) return st;
  st = hipStreamBeginCapture(stream, hipStreamCaptureModeThreadLocal);
  if (st != hipSuccess) return st;
  const hipError_t launch = rtxllm_llama_step(m, stream);
  hipGraph_t g = nullptr;
  st = hipStreamEndCapture(stream, &g);
  if (launch != hipSuccess) {
    if (g != nullptr) (void)hipGraphDestroy(g);
    return launch;
  }
  if (st != hipSuccess) return st;
  try {
    bucket.instantiate(g);
  } catch (const std::exception&) {
    return hipErrorInvalidValue;
  }
  return hipSuccess;
}

rtxllm::HipGraphBucketDescriptor span_descriptor(const rtxllm_llama* m, std::uint32_t span) {
  rtxllm::HipGraphBucketDescriptor d = m->graph_desc;
  d.name = "decode_span_" + std::to_string(span);
  d.query_bucket = span;
  return d;
}

}  // namespace

extern "C" hipError_t rtxllm_llama_graph_capture(rtxllm_llama* m, hipStream_t stream) {
  if (m == nullptr || stream == nullptr) return hipErrorInvalidValue;
  return capture_step(m, m->graph, stream);
}

extern "C" hipError_t rtxllm_llama_graph_capture_span(rtxllm_llama* m, uint32_t span, hipStream_t stream) {
  if (m == nullptr || stream == nullptr || span == 0u || span > m->cfg.max_ctx) return hipErrorInvalidValue;
  // strict admission of the bucket's graph memory
  std::size_t free_b = 0, total_b = 0;
  const hipError_t mi = hipMemGetInfo(&free_b, &total_b);
  if (mi != hipSuccess) return mi;
  try {
    if (rtxllm::estimate_hip_graph_bucket_allocation(span_descriptor(m, span)).total_bytes > free_b)
      return hipErrorOutOfMemory;
  } catch (const std::exception&) {
    return hipErrorInvalidValue;
  }
  rtxllm::HipGraphBucket bucket;
  m->span = span;
  const hipError_t st = capture_step(m, bucket, stream);
  m->span = m->cfg.max_ctx;
  if (st != hipSuccess) return st;
  m->span_graphs[span] = std::move(bucket);
  return hipSuccess;
}

extern "C" hipError_t rtxllm_llama_graph_replay_span(rtxllm_llama* m, uint32_t span, hipStream_t stream) {
  if (m == nullptr) return hipErrorInvalidValue;
  const auto it = m->span_graphs.find(span);
  if (it == m->span_graphs.end()) return hipErrorInvalidValue;
  const hipError_t st = ensure_units(m, stream);
  if (st != hipSuccess) return st;
  try {
    it->second.replay(stream);
  } catch (const std::exception&) {
    return hipErrorLaunchFailure;
  }
  return hipSuccess;
}

extern "C" uint32_t rtxllm_llama_graph_span_for(const rtxllm_llama* m, uint32_t position) {
  if (m == nullptr) return 0u;
  const auto it = m->span_graphs.upper_bound(position);
  return it == m->span_graphs.end() ? 0u : it->first;
}

extern "C" size_t rtxllm_llama_graph_bytes(const rtxllm_llama* m) {
  if (m == nullptr) return 0u;
  std::vector<rtxllm::HipGraphBucketDescriptor> ds;
  if (m->graph.instantiated()) ds.push_back(m->graph_desc);
  for (const auto& kv : m->span_graphs) ds.push_back(span_descriptor(m, kv.first));
  if (ds.empty()) return 0u;
  try {
    return rtxllm::build_hip_graph_bucket_plan(ds).total_bytes;
  } catch (const std::exception&) {
    return 0u;
  }
}

extern "C" hipError_t rtxllm_llama_graph_replay(rtxllm_llama* m, hipStream_t stream) {
  if (m == nullptr || !m->graph.instantiated()) return hipErrorInvalidValue;
  const hipError_t st = ensure_units(m, stream);
  if (st != hipSuccess) return st;
  try {
    m->graph.replay(stream);
  } catch (const std::exception&) {
    return hipErrorLaunchFailure;
  }
  return hipSuccess;
}

extern "C" hipError_t rtxllm_llama_status(rtxllm_llama* m, uint32_t* status, hipStream_t stream) {
  if (m == nullptr || status == nullptr) return hipErrorInvalidValue;
  hipError_t st = hipMemcpyAsync(status, m->arena.arena_ptr("status"), 4u * m->batch, hipMemcpyDeviceToHost, stream);
  if (st == hipSuccess) st = hipStreamSynchronize(stream);
  return st;
}

extern "C" hipError_t rtxllm_llama_clear_status(rtxllm_llama* m, hipStream_t stream) {
  if (m == nullptr) return hipErrorInvalidValue;
  hipError_t st = hipMemsetAsync(m->arena.arena_ptr("status"), 0, 4u * m->batch, stream);
  if (st == hipSuccess) st = hipStreamSynchronize(stream);
  return st;
}
