// rtxllm_gguf_pack: GGUF file -> resident packs, from the command line.
//
//   rtxllm_gguf_pack --model MODEL.gguf --output-dir DIR [--policy P]
//                    [--write-blocks] [--type T]... [--tensor NAME]...
//                    [--layer N] [--limit N]
//
// The options of the reference's producers (tools/bench/q4k_resident_pack.py
// main, iq_resident_pack.py main, q5k_resident_pack.py main) in one run: every
// selected Q4_K, IQ2_S / IQ3_S and Q5_K tensor goes to DIR/q4k, DIR/iq and
// DIR/q5k, each with manifest.json and manifest.md, and DIR/tensor_plan.json
// holds the GGUF tensor plan. Prints json= / markdown= / tensors= /
// resident_bytes= lines per manifest like the reference producers. Exit 0, or
// 1 with the reason on stderr.
#include <cstdio>
#include <cstdlib>
#include <fstream>
#include <iterator>
#include <stdexcept>
#include <string>

#include "rtxllm/pack_producer.h"
#include "../csrc/json_value.h"

namespace {

int usage() {
  std::fprintf(stderr,
               "usage: rtxllm_gguf_pack --model MODEL.gguf --output-dir DIR [--policy auto|auto-lossy|split-native|"
               "split-half|split-compact|split-predecoded] [--write-blocks] [--type Q4_K|Q5_K|IQ2_S|IQ3_S]... "
               "[--tensor NAME]... [--layer N] [--limit N]\n");
  return 1;
}

void report(const std::filesystem::path& manifest) {
  if (manifest.empty()) return;
  std::ifstream in(manifest, std::ios::binary);
  const std::string text((std::istreambuf_iterator<char>(in)), std::istreambuf_iterator<char>());
  const rtxllm::json::Json m = rtxllm::json::Reader(text).document();
  std::uint64_t n = 0, resident = 0;
  rtxllm::json::as_u64(*m.find("tensor_count"), n);
  rtxllm::json::as_u64(*m.find("resident_bytes"), resident);
  std::printf("json=%s\nmarkdown=%s\ntensors=%llu\nresident_bytes=%llu\n", manifest.string().c_str(),
              (manifest.parent_path() / "manifest.md").string().c_str(), static_cast<unsigned long long>(n),
              static_cast<unsigned long long>(resident));
}

}  // namespace

int main(int argc, char** argv) {
  std::string model, out_dir;
  rtxllm::PackOptions opt;
  for (int i = 1; i < argc; ++i) {
    const std::string a = argv[i];
    auto value = [&]() -> std::string {
      if (i + 1 >= argc) throw std::invalid_argument(a + " needs a value");
      return argv[++i];
    };
    try {
      if (a == "--model") model = value();
      else if (a == "--output-dir") out_dir = value();
      else if (a == "--policy") opt.q4k_policy = value();
      else if (a == "--write-blocks") opt.write_blocks = true;
      else if (a == "--type") opt.types.push_back(value());
      else if (a == "--tensor") opt.names.push_back(value());
      else if (a == "--layer") opt.layer = std::stoi(value());
      else if (a == "--limit") opt.limit = std::stoull(value());
      else if (a == "-h" || a == "--help") return usage() - 1;
      else throw std::invalid_argument("unknown argument " + a);
    } catch (const std::exception& e) {
      std::fprintf(stderr, "rtxllm_gguf_pack: %s\n", e.what());
      return usage();
    }
  }
  if (model.empty() || out_dir.empty()) return usage();
  try {
    const rtxllm::PackSetPaths p = rtxllm::pack_gguf(model, out_dir, opt);
    std::printf("tensor_plan=%s\n", p.tensor_plan.string().c_str());
    report(p.q4k_manifest);
    report(p.iq_manifest);
    report(p.q5k_manifest);
  } catch (const std::exception& e) {
    std::fprintf(stderr, "rtxllm_gguf_pack: %s\n", e.what());
    return 1;
  }
  return 0;
}
