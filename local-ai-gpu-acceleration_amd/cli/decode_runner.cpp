// rtxllm_decode_runner: the Llama decode step as a command with the reference
// runner's pass / fail contract (runtime/apps/mixed_sequence_benchmark_runner/
// main.cpp:3736-3762 and 5813; tools/bench/native_harness.py:131-165 reads the
// exit code and the one JSON object printed):
//   0  every gate passed;
//   1  an error (bad arguments, unreadable model, a failed HIP call);
//   2  strict admission refused the model (nothing was allocated);
//   3  a gate failed.
// The gates: the step's logits are finite, each token is the argmax of its
// logits, no sequence reached the context end, a hipGraph replay of the step
// equals the eager step bit for bit, and, with --expect-logits, the first
// step's logits match the given ones within --tolerance (normwise: max |a - b|
// / max |b| per sequence) and each token matches the expected argmax where the
// expected top two differ by more than the tolerance. Then --warmup and
// --steps graph replays are timed with HIP events.
//
// Weights come from the device-side synthetic generator (--seed) or from a
// GGUF Llama model (--gguf), packed by the library's producer into
// --pack-dir and loaded with rtxllm_llama_load_pack_set, the norm vectors read
// from its F32 tensors. The KV cache holds seeded N(0, 1) fp16 values.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cmath>
#include <cstdint>
#include <cstdio>
#include <cstring>
#include <fstream>
#include <stdexcept>
#include <string>
#include <thread>
#include <vector>

#include "../csrc/json_value.h"
#include "../csrc/synth.h"  // enum rtxllm_format
#include "rtxllm/decode_kernels.h"
#include "rtxllm/llama.h"
#include "rtxllm/pack_producer.h"

namespace {

namespace J = rtxllm::json;

struct Options {
  std::string label = "decode";
  std::string shape = "8b";
  std::string gguf, pack_dir, expect_logits, policy = "auto";
  std::uint64_t seed = 0x5EED0004ull;
  std::uint32_t batch = 1, steps = 20, warmup = 3, max_ctx = 4096, page_size = 64;
  long long position = -1, token = -1;
  double tolerance = 1e-3;
  std::uint64_t guard_mib = 0;
};

struct Failure : std::runtime_error {
  int code;
  Failure(int c, const std::string& m) : std::runtime_error(m), code(c) {}
};

void hip(hipError_t st, const char* what) {
  if (st != hipSuccess) throw Failure(1, std::string(what) + ": " + hipGetErrorString(st));
}

int usage() {
  std::fprintf(stderr,
               "usage: rtxllm_decode_runner [--shape 8b|small] [--seed N] [--gguf MODEL.gguf --pack-dir DIR "
               "[--policy P]] [--batch B] [--steps N] [--warmup N] [--max-ctx N] [--page-size N] "
               "[--position P] [--token T] [--expect-logits FILE.f32] [--tolerance X] [--guard-mib N] "
               "[--label S]\n");
  return 1;
}

std::uint64_t splitmix64(std::uint64_t x) {
  x += 0x9E3779B97F4A7C15ull;
  x = (x ^ (x >> 30)) * 0xBF58476D1CE4E5B9ull;
  x = (x ^ (x >> 27)) * 0x94D049BB133111EBull;
  return x ^ (x >> 31);
}

int format_of(const std::string& type, const std::string& policy, std::uint64_t rows, std::uint64_t cols) {
  if (type == "Q5_K") return RTXLLM_FMT_Q5K;
  if (type == "IQ2_S") return RTXLLM_FMT_IQ2S;
  if (type == "IQ3_S") return RTXLLM_FMT_IQ3S;
  if (type == "Q4_K") {
    const std::string p = rtxllm::resolve_q4k_policy(policy, rows, cols);
    if (p == "split-native") return RTXLLM_FMT_Q4K_SPLIT_NATIVE;
    if (p == "split-half") return RTXLLM_FMT_Q4K_SPLIT_HALF;
    if (p == "split-compact") return RTXLLM_FMT_Q4K_SPLIT_COMPACT;
    return RTXLLM_FMT_Q4K_SPLIT_PREDECODED;
  }
  throw Failure(1, "tensor type " + type + " has no decode kernel (Q4_K, Q5_K, IQ2_S, IQ3_S)");
}

// The model shape and per-role formats of a GGUF Llama model (its llama.* keys
// and block-0 tensor types; q / k / v and gate / up must share a type).
rtxllm_llama_config config_from_gguf(const rtxllm::GgufHeader& h, const Options& o) {
  if (h.architecture != "llama") throw Failure(1, "architecture '" + h.architecture + "' is not llama");
  auto key = [&](const char* k) {
    const double v = h.number(std::string("llama.") + k, -1.0);
    if (v < 0.0) throw Failure(1, std::string("GGUF key missing: llama.") + k);
    return v;
  };
  auto tensor = [&](const std::string& name) {
    const rtxllm::GgufTensorInfo* t = h.tensor(name);
    if (t == nullptr || t->dimensions.size() != 2) throw Failure(1, "GGUF tensor missing or not 2-D: " + name);
    return t;
  };
  rtxllm_llama_config c{};
  c.hidden = static_cast<std::uint32_t>(key("embedding_length"));
  c.n_layers = static_cast<std::uint32_t>(key("block_count"));
  c.n_heads = static_cast<std::uint32_t>(key("attention.head_count"));
  c.n_kv_heads = static_cast<std::uint32_t>(h.number("llama.attention.head_count_kv", c.n_heads));
  c.ffn = static_cast<std::uint32_t>(key("feed_forward_length"));
  c.rope_theta = static_cast<float>(h.number("llama.rope.freq_base", 500000.0));
  c.rms_eps = static_cast<float>(h.number("llama.attention.layer_norm_rms_epsilon", 1e-6));
  const auto* embd = tensor("token_embd.weight");
  if (embd->type != "Q5_K") throw Failure(1, "token_embd.weight must be Q5_K, not " + embd->type);
  c.vocab = static_cast<std::uint32_t>(embd->dimensions[1]);
  auto fmt = [&](std::initializer_list<const char*> names) {
    std::string type;
    const rtxllm::GgufTensorInfo* first = nullptr;
    for (const char* n : names) {
      const auto* t = tensor(std::string("blk.0.") + n);
      if (first == nullptr) first = t, type = t->type;
      else if (t->type != type) throw Failure(1, std::string("blk.0.") + n + " differs in type from its partners");
    }
    return format_of(type, o.policy, first->dimensions[1], first->dimensions[0]);
  };
  c.fmt_qkv = fmt({"attn_q.weight", "attn_k.weight", "attn_v.weight"});
  c.fmt_o = fmt({"attn_output.weight"});
  c.fmt_gate_up = fmt({"ffn_gate.weight", "ffn_up.weight"});
  c.fmt_down = fmt({"ffn_down.weight"});
  const auto* out = tensor("output.weight");
  c.fmt_lm_head = format_of(out->type, o.policy, out->dimensions[1], out->dimensions[0]);
  return c;
}

rtxllm_llama_config config_from_shape(const Options& o) {
  rtxllm_llama_config c{};
  if (o.shape == "8b") {
    c.hidden = 4096, c.n_heads = 32, c.n_kv_heads = 8, c.ffn = 14336, c.vocab = 128256, c.n_layers = 32;
  } else if (o.shape == "small") {
    c.hidden = 512, c.n_heads = 4, c.n_kv_heads = 2, c.ffn = 1024, c.vocab = 1000, c.n_layers = 2;
  } else {
    throw Failure(1, "unknown --shape " + o.shape + " (8b, small)");
  }
  c.rope_theta = 500000.0f, c.rms_eps = 1e-6f;
  c.fmt_qkv = RTXLLM_FMT_IQ3S, c.fmt_o = RTXLLM_FMT_IQ3S, c.fmt_gate_up = RTXLLM_FMT_IQ2S;
  c.fmt_down = RTXLLM_FMT_Q4K_SPLIT_NATIVE, c.fmt_lm_head = RTXLLM_FMT_Q5K;
  return c;
}

void upload(rtxllm_llama* m, const char* name, std::uint32_t layer, const void* src, std::size_t bytes) {
  hip(rtxllm_llama_upload(m, name, layer, 0, src, bytes), name);
}

template <class T>
std::vector<T> download(rtxllm_llama* m, const char* name, std::size_t count) {
  std::vector<T> out(count);
  hip(rtxllm_llama_download(m, name, 0, 0, out.data(), count * sizeof(T)), name);
  return out;
}

// Norm vectors 1 + N(0, 0.02) and the fp16 KV cache ~ N(0, 1), from the
// library's seeded host generator (the seeds bench.py and the tests use).
void seed_norms_and_cache(rtxllm_llama* m, const rtxllm_llama_config& c, std::uint64_t seed, bool norms) {
  const int threads = static_cast<int>(std::min(16u, std::max(1u, std::thread::hardware_concurrency())));
  std::vector<float> v(c.hidden);
  if (norms) {
    for (std::uint32_t l = 0; l < c.n_layers; ++l) {
      rtxllm_synth_normal_f32(seed + 100 + 2 * l, c.hidden, 1.0f, 0.02f, v.data(), threads);
      upload(m, "attn_norm", l, v.data(), 4u * c.hidden);
      rtxllm_synth_normal_f32(seed + 101 + 2 * l, c.hidden, 1.0f, 0.02f, v.data(), threads);
      upload(m, "ffn_norm", l, v.data(), 4u * c.hidden);
    }
    rtxllm_synth_normal_f32(seed + 99, c.hidden, 1.0f, 0.02f, v.data(), threads);
    upload(m, "out_norm", 0, v.data(), 4u * c.hidden);
  }
  std::size_t bytes = 0;
  if (rtxllm_llama_region(m, "k_cache", 0, &bytes) == nullptr) throw Failure(1, "no k_cache region");
  std::vector<std::uint16_t> k(bytes / 2u), vv(bytes / 2u);
  const bool shared = c.batch > 1u;  // a batch's sequences share one seeded image per role
  for (std::uint32_t l = 0; l < c.n_layers; ++l) {
    if (!shared || l == 0u) {
      const std::uint64_t sk = shared ? seed + 300 : seed + 300 + 2 * l, sv = shared ? seed + 301 : seed + 301 + 2 * l;
      rtxllm_synth_normal_f16(sk, k.size(), 0.0f, 1.0f, k.data(), threads);
      rtxllm_synth_normal_f16(sv, vv.size(), 0.0f, 1.0f, vv.data(), threads);
    }
    upload(m, "k_cache", l, k.data(), bytes);
    upload(m, "v_cache", l, vv.data(), bytes);
  }
}

// The F32 norm vectors of a GGUF Llama model, read at their absolute offsets.
void gguf_norms(rtxllm_llama* m, const rtxllm::GgufHeader& h, const rtxllm_llama_config& c) {
  std::ifstream in(h.path, std::ios::binary);
  if (!in) throw Failure(1, "failed to open " + h.path.string());
  const auto rows = rtxllm::gguf_tensor_spans(h);
  auto read = [&](const std::string& name, const char* region, std::uint32_t layer) {
    for (const auto& r : rows) {
      if (r.name != name) continue;
      if (r.type != "F32" || r.dimensions.size() != 1 || r.dimensions[0] != c.hidden || r.span_bytes < 4u * c.hidden)
        throw Failure(1, name + " must be F32 [" + std::to_string(c.hidden) + "]");
      std::vector<float> v(c.hidden);
      in.seekg(static_cast<std::streamoff>(r.absolute_offset));
      in.read(reinterpret_cast<char*>(v.data()), static_cast<std::streamsize>(4u * c.hidden));
      if (!in) throw Failure(1, "short read of " + name);
      upload(m, region, layer, v.data(), 4u * c.hidden);
      return;
    }
    throw Failure(1, "GGUF tensor missing: " + name);
  };
  for (std::uint32_t l = 0; l < c.n_layers; ++l) {
    read("blk." + std::to_string(l) + ".attn_norm.weight", "attn_norm", l);
    read("blk." + std::to_string(l) + ".ffn_norm.weight", "ffn_norm", l);
  }
  read("output_norm.weight", "out_norm", 0);
}

std::uint32_t host_argmax(const float* x, std::uint32_t n) {  // lowest index on ties
  std::uint32_t best = 0;
  for (std::uint32_t i = 1; i < n; ++i)
    if (x[i] > x[best]) best = i;
  return best;
}

double percentile(std::vector<double> v, double p) {
  std::sort(v.begin(), v.end());
  const double idx = p * static_cast<double>(v.size() - 1);
  const std::size_t lo = static_cast<std::size_t>(idx);
  const std::size_t hi = std::min(lo + 1, v.size() - 1);
  return v[lo] + (v[hi] - v[lo]) * (idx - static_cast<double>(lo));
}

J::Json config_json(const rtxllm_llama_config& c) {
  J::Json o = J::object();
  for (const auto& kv : {std::pair<const char*, std::uint32_t>{"hidden", c.hidden},
                         {"n_heads", c.n_heads},
                         {"n_kv_heads", c.n_kv_heads},
                         {"ffn", c.ffn},
                         {"vocab", c.vocab},
                         {"n_layers", c.n_layers},
                         {"max_ctx", c.max_ctx},
                         {"page_size", c.page_size},
                         {"batch", c.batch}})
    J::set(o, kv.first, J::integer(kv.second));
  J::set(o, "rope_theta", J::real(c.rope_theta));
  J::set(o, "rms_eps", J::real(c.rms_eps));
  for (const auto& kv : {std::pair<const char*, int>{"fmt_qkv", c.fmt_qkv},
                         {"fmt_o", c.fmt_o},
                         {"fmt_gate_up", c.fmt_gate_up},
                         {"fmt_down", c.fmt_down},
                         {"fmt_lm_head", c.fmt_lm_head}})
    J::set(o, kv.first, J::integer_signed(kv.second));
  return o;
}

int run(const Options& o) {
  J::Json out = J::object();
  J::set(out, "path", J::string("rtxllm_decode_runner"));
  J::set(out, "label", J::string(o.label));
  rtxllm::GgufHeader gh;
  rtxllm_llama_config c{};
  if (!o.gguf.empty()) {
    if (o.pack_dir.empty()) throw Failure(1, "--gguf needs --pack-dir");
    gh = rtxllm::read_gguf_header(o.gguf);
    c = config_from_gguf(gh, o);
  } else {
    c = config_from_shape(o);
  }
  c.max_ctx = o.max_ctx, c.page_size = o.page_size, c.batch = o.batch;
  J::set(out, "source", J::string(o.gguf.empty() ? "synthetic" : o.gguf));
  J::set(out, "config", config_json(c));

  // strict admission first, against free memory less the guard
  int admitted = 0;
  std::size_t required = 0, usable = 0;
  char reason[512] = {0};
  const hipError_t ad = rtxllm_llama_admission(&c, static_cast<std::size_t>(o.guard_mib) << 20, &admitted, &required,
                                               &usable, reason, sizeof reason);
  if (ad == hipErrorInvalidValue) throw Failure(1, "the model configuration is not supported");
  hip(ad, "rtxllm_llama_admission");
  J::set(out, "admitted", J::boolean(admitted != 0));
  J::set(out, "admission_reason", J::string(reason));
  J::set(out, "required_bytes", J::integer(required));
  J::set(out, "usable_bytes", J::integer(usable));
  J::set(out, "guard_mib", J::integer(o.guard_mib));
  if (!admitted) {
    std::printf("%s\n", J::dump(out).c_str());
    return 2;
  }
  rtxllm_llama* m = nullptr;
  const hipError_t cr = rtxllm_llama_create(&c, &m);
  if (cr == hipErrorOutOfMemory) {  // free memory changed since the decision
    J::set(out, "admitted", J::boolean(false));
    std::printf("%s\n", J::dump(out).c_str());
    return 2;
  }
  hip(cr, "rtxllm_llama_create");
  struct Guard {
    rtxllm_llama* m;
    ~Guard() { rtxllm_llama_destroy(m); }
  } guard{m};

  hipStream_t stream = nullptr;
  hip(hipStreamCreate(&stream), "hipStreamCreate");
  struct StreamGuard {
    hipStream_t s;
    ~StreamGuard() { (void)hipStreamDestroy(s); }
  } sguard{stream};

  if (o.gguf.empty()) {
    hip(rtxllm_llama_synth_weights(m, o.seed, stream), "rtxllm_llama_synth_weights");
    hip(hipStreamSynchronize(stream), "synchronize");
    seed_norms_and_cache(m, c, o.seed, true);
  } else {
    rtxllm::PackOptions po;
    po.q4k_policy = o.policy;
    po.write_blocks = c.fmt_down == RTXLLM_FMT_Q4K_RAW;
    const rtxllm::PackSetPaths p = rtxllm::pack_gguf(o.gguf, o.pack_dir, po);
    std::vector<std::string> paths;
    for (const auto* x : {&p.q4k_manifest, &p.iq_manifest, &p.q5k_manifest})
      if (!x->empty()) paths.push_back(x->string());
    std::vector<const char*> ptrs;
    for (const auto& s : paths) ptrs.push_back(s.c_str());
    char err[1024] = {0};
    if (rtxllm_llama_load_pack_set(m, ptrs.data(), static_cast<std::uint32_t>(ptrs.size()), nullptr, err,
                                   sizeof err) != hipSuccess)
      throw Failure(1, std::string("rtxllm_llama_load_pack_set: ") + err);
    gguf_norms(m, gh, c);
    seed_norms_and_cache(m, c, o.seed, false);
    J::set(out, "pack_dir", J::string(p.tensor_plan.parent_path().string()));
  }

  // initial tokens and positions
  const std::uint32_t B = c.batch;
  const std::uint64_t replays = 1ull + o.warmup + o.steps;  // graph check + warmup + timed
  long long pos0 = o.position;
  if (pos0 < 0) pos0 = static_cast<long long>(c.max_ctx) - static_cast<long long>(replays) - 2;
  if (pos0 < 0 || static_cast<std::uint64_t>(pos0) + replays >= c.max_ctx)
    throw Failure(1, "--position + 1 + warmup + steps must stay below --max-ctx");
  std::vector<std::uint32_t> tok0(B), posv(B, static_cast<std::uint32_t>(pos0));
  for (std::uint32_t s = 0; s < B; ++s)
    tok0[s] = o.token >= 0 ? static_cast<std::uint32_t>(o.token)
                           : static_cast<std::uint32_t>(splitmix64(o.seed ^ (0xA5A5ull + s)) % c.vocab);
  if (o.token >= static_cast<long long>(c.vocab)) throw Failure(1, "--token must be below the vocabulary size");
  auto set_state = [&]() {
    upload(m, "token", 0, tok0.data(), 4u * B);
    upload(m, "pos", 0, posv.data(), 4u * B);
    hip(rtxllm_llama_clear_status(m, stream), "rtxllm_llama_clear_status");
  };

  // ---- gates -------------------------------------------------------------------------
  set_state();
  hip(rtxllm_llama_step(m, stream), "rtxllm_llama_step");
  hip(hipStreamSynchronize(stream), "synchronize");
  const std::size_t V = c.vocab;
  const std::vector<float> logits = download<float>(m, "logits", B * V);
  const std::vector<std::uint32_t> tok1 = download<std::uint32_t>(m, "token", B);
  std::vector<std::uint32_t> status(B);
  hip(rtxllm_llama_status(m, status.data(), stream), "rtxllm_llama_status");
  bool finite = true, argmax_ok = true, status_clear = true;
  for (float x : logits) finite = finite && std::isfinite(x);
  for (std::uint32_t s = 0; s < B; ++s) {
    argmax_ok = argmax_ok && tok1[s] == host_argmax(logits.data() + s * V, c.vocab);
    status_clear = status_clear && status[s] == 0u;
  }

  bool checked = false, passed = true;
  double worst = 0.0;
  J::Json token_expected = J::array();
  if (!o.expect_logits.empty()) {
    checked = true;
    std::ifstream in(o.expect_logits, std::ios::binary);
    std::vector<float> want(B * V);
    in.read(reinterpret_cast<char*>(want.data()), static_cast<std::streamsize>(4u * want.size()));
    if (!in || in.peek() != std::ifstream::traits_type::eof())
      throw Failure(1, "--expect-logits must hold exactly batch x vocab float32 values");
    for (std::uint32_t s = 0; s < B; ++s) {
      double num = 0.0, den = 0.0;
      for (std::size_t i = 0; i < V; ++i) {
        num = std::max(num, std::fabs(static_cast<double>(logits[s * V + i]) - want[s * V + i]));
        den = std::max(den, std::fabs(static_cast<double>(want[s * V + i])));
      }
      const double rel = den > 0.0 ? num / den : num;
      if (!(rel <= o.tolerance)) passed = false;
      worst = std::max(worst, rel);
      const float* w = want.data() + s * V;
      const std::uint32_t t = host_argmax(w, c.vocab);
      float second = -INFINITY;
      for (std::uint32_t i = 0; i < c.vocab; ++i)
        if (i != t) second = std::max(second, w[i]);
      token_expected.items.push_back(J::integer(t));
      if (static_cast<double>(w[t]) - second > o.tolerance * std::fabs(static_cast<double>(w[t])) && tok1[s] != t)
        passed = false;
    }
  }

  // the captured step against the eager one, from the same state
  set_state();
  hip(rtxllm_llama_graph_capture(m, stream), "rtxllm_llama_graph_capture");
  set_state();
  hip(rtxllm_llama_graph_replay(m, stream), "rtxllm_llama_graph_replay");
  hip(hipStreamSynchronize(stream), "synchronize");
  const std::vector<float> glogits = download<float>(m, "logits", B * V);
  const std::vector<std::uint32_t> gtok = download<std::uint32_t>(m, "token", B);
  const bool graph_match = std::memcmp(glogits.data(), logits.data(), 4u * logits.size()) == 0 && gtok == tok1;

  // ---- timing --------------------------------------------------------------------------
  for (std::uint32_t i = 0; i < o.warmup; ++i) hip(rtxllm_llama_graph_replay(m, stream), "replay");
  std::vector<hipEvent_t> ev(o.steps + 1u);
  for (auto& e : ev) hip(hipEventCreate(&e), "hipEventCreate");
  hip(hipEventRecord(ev[0], stream), "hipEventRecord");
  for (std::uint32_t i = 0; i < o.steps; ++i) {
    hip(rtxllm_llama_graph_replay(m, stream), "replay");
    hip(hipEventRecord(ev[i + 1u], stream), "hipEventRecord");
  }
  hip(hipStreamSynchronize(stream), "synchronize");
  std::vector<double> ms(o.steps);
  float total = 0.0f;
  for (std::uint32_t i = 0; i < o.steps; ++i) {
    float t = 0.0f;
    hip(hipEventElapsedTime(&t, ev[i], ev[i + 1u]), "hipEventElapsedTime");
    ms[i] = t;
  }
  if (o.steps > 0u) hip(hipEventElapsedTime(&total, ev[0], ev[o.steps]), "hipEventElapsedTime");
  for (auto& e : ev) (void)hipEventDestroy(e);
  hip(rtxllm_llama_status(m, status.data(), stream), "rtxllm_llama_status");
  for (std::uint32_t s = 0; s < B; ++s) status_clear = status_clear && status[s] == 0u;
  const std::vector<std::uint32_t> tok_end = download<std::uint32_t>(m, "token", B);

  const bool gates = finite && argmax_ok && status_clear && graph_match;
  J::Json g = J::object();
  J::set(g, "logits_finite", J::boolean(finite));
  J::set(g, "token_is_argmax", J::boolean(argmax_ok));
  J::set(g, "status_clear", J::boolean(status_clear));
  J::set(g, "graph_matches_eager", J::boolean(graph_match));
  J::set(out, "gates", std::move(g));
  J::set(out, "gates_passed", J::boolean(gates));
  J::set(out, "reference_checked", J::boolean(checked));
  if (checked) {
    J::set(out, "reference_passed", J::boolean(passed));
    J::set(out, "reference_tolerance", J::real(o.tolerance));
    J::set(out, "max_logit_rel_error", J::real(worst));
    J::set(out, "token_expected", std::move(token_expected));
  }
  J::Json t1 = J::array(), te = J::array();
  for (std::uint32_t s = 0; s < B; ++s) {
    t1.items.push_back(J::integer(tok1[s]));
    te.items.push_back(J::integer(tok_end[s]));
  }
  J::set(out, "position", J::integer(static_cast<std::uint64_t>(pos0)));
  J::set(out, "token_observed", std::move(t1));
  J::set(out, "tokens_after", std::move(te));
  J::set(out, "warmup", J::integer(o.warmup));
  J::set(out, "steps", J::integer(o.steps));
  if (o.steps > 0u) {
    const double mean = static_cast<double>(total) / o.steps;
    J::set(out, "ms_per_step", J::real(mean));
    J::set(out, "tok_s", J::real(B * 1000.0 / mean));
    J::Json lat = J::object();
    J::set(lat, "p50", J::real(percentile(ms, 0.50)));
    J::set(lat, "p95", J::real(percentile(ms, 0.95)));
    J::set(lat, "p99", J::real(percentile(ms, 0.99)));
    J::set(lat, "max", J::real(*std::max_element(ms.begin(), ms.end())));
    J::set(out, "latency_ms", std::move(lat));
  }
  J::set(out, "launches_per_step", J::integer(rtxllm_llama_launches_per_step(m)));
  J::set(out, "graph_bytes", J::integer(rtxllm_llama_graph_bytes(m)));
  std::size_t req = 0, use = 0, arena = 0;
  hip(rtxllm_llama_memory(m, &req, &use, &arena), "rtxllm_llama_memory");
  J::set(out, "arena_bytes", J::integer(arena));
  std::printf("%s\n", J::dump(out).c_str());
  return gates && (!checked || passed) ? 0 : 3;
}

}  // namespace

int main(int argc, char** argv) {
  Options o;
  try {
    for (int i = 1; i < argc; ++i) {
      const std::string a = argv[i];
      auto value = [&]() -> std::string {
        if (i + 1 >= argc) throw std::invalid_argument(a + " needs a value");
        return argv[++i];
      };
      auto u32 = [&]() {
        const unsigned long long v = std::stoull(value());
        if (v > UINT32_MAX) throw std::invalid_argument(a + " is out of range");
        return static_cast<std::uint32_t>(v);
      };
      if (a == "--shape") o.shape = value();
      else if (a == "--seed") o.seed = std::stoull(value(), nullptr, 0);
      else if (a == "--gguf") o.gguf = value();
      else if (a == "--pack-dir") o.pack_dir = value();
      else if (a == "--policy") o.policy = value();
      else if (a == "--batch") o.batch = u32();
      else if (a == "--steps") o.steps = u32();
      else if (a == "--warmup") o.warmup = u32();
      else if (a == "--max-ctx") o.max_ctx = u32();
      else if (a == "--page-size") o.page_size = u32();
      else if (a == "--position") o.position = std::stoll(value());
      else if (a == "--token") o.token = std::stoll(value());
      else if (a == "--expect-logits") o.expect_logits = value();
      else if (a == "--tolerance") o.tolerance = std::stod(value());
      else if (a == "--guard-mib") o.guard_mib = std::stoull(value());
      else if (a == "--label") o.label = value();
      else if (a == "-h" || a == "--help") return usage() - 1;
      else throw std::invalid_argument("unknown argument " + a);
    }
    if (o.batch == 0u || o.batch > 8u) throw std::invalid_argument("--batch must be 1..8");
  } catch (const std::exception& e) {
    std::fprintf(stderr, "rtxllm_decode_runner: %s\n", e.what());
    return usage();
  }
  try {
    return run(o);
  } catch (const Failure& f) {
    std::fprintf(stderr, "rtxllm_decode_runner: %s\n", f.what());
    return f.code;
  } catch (const std::exception& e) {
    std::fprintf(stderr, "rtxllm_decode_runner: %s\n", e.what());
    return 1;
  }
}
