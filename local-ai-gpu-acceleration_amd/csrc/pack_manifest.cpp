// Tensor-pack manifest and tensor-plan loaders (host). A small JSON reader
// builds a value tree; the loaders apply the reference's field and
// validation rules to it (see include/rtxllm/pack_manifest.h).
#include "rtxllm/pack_manifest.h"

#include "json_value.h"

#include <algorithm>
#include <cstring>
#include <fstream>
#include <map>
#include <memory>
#include <stdexcept>
#include <string_view>
#include <unordered_map>
#include <utility>

namespace rtxllm {
namespace {

[[noreturn]] void fail(const std::string& what) { throw std::runtime_error(what); }

// ---- field access (required fields throw, optional ones default) --------------------

using json::Json;
using json::Reader;
using json::as_u64;
using json::read_text;

const Json& need(const Json& obj, const char* key) {
  const Json* v = obj.find(key);
  if (v == nullptr) fail(std::string("manifest field missing: ") + key);
  return *v;
}
std::string str(const Json& obj, const char* key) {
  const Json& v = need(obj, key);
  if (v.kind != Json::String) fail(std::string("manifest string value expected: ") + key);
  return v.text;
}
std::string opt_str(const Json& obj, const char* key) {
  const Json* v = obj.find(key);
  return v != nullptr && v->kind == Json::String ? v->text : std::string();
}
std::uint64_t u64(const Json& obj, const char* key) {
  std::uint64_t x = 0;
  if (!as_u64(need(obj, key), x)) fail(std::string("manifest integer value expected: ") + key);
  return x;
}
std::uint64_t opt_u64(const Json& obj, const char* key) {
  const Json* v = obj.find(key);
  std::uint64_t x = 0;
  return v != nullptr && as_u64(*v, x) ? x : 0;
}
std::vector<std::uint64_t> opt_u64_array(const Json& obj, const char* key) {
  const Json* v = obj.find(key);
  std::vector<std::uint64_t> out;
  if (v == nullptr || v->kind == Json::Null) return out;
  if (v->kind != Json::Array) fail(std::string("manifest array value expected: ") + key);
  for (const Json& e : v->items) {
    std::uint64_t x = 0;
    if (!as_u64(e, x)) fail(std::string("manifest array integer expected: ") + key);
    out.push_back(x);
  }
  return out;
}
std::vector<std::string> opt_str_array(const Json& obj, const char* key) {
  const Json* v = obj.find(key);
  std::vector<std::string> out;
  if (v == nullptr || v->kind != Json::Array) return out;
  for (const Json& e : v->items)
    if (e.kind == Json::String) out.push_back(e.text);
  return out;
}

// The document's "tensors" records.
const std::vector<Json>& tensor_records(const Json& doc, const char* what) {
  const Json* t = doc.find("tensors");
  if (t == nullptr) fail(std::string(what) + " does not contain tensors array");
  if (t->kind != Json::Array) fail(std::string(what) + " tensors field is not an array");
  for (const Json& e : t->items)
    if (e.kind != Json::Object) fail(std::string(what) + " tensors array holds a non-object");
  return t->items;
}

std::string dims_text(const std::vector<std::uint64_t>& d) {
  std::string s = "[";
  for (std::size_t i = 0; i < d.size(); ++i) s += (i ? ", " : "") + std::to_string(d[i]);
  return s + "]";
}

// "blk.<layer>.<role>" -> (layer, role); other names: role = name without a
// trailing ".weight", layer -1.
void name_metadata(const std::string& name, int& layer, std::string& role) {
  static const std::string kPrefix = "blk.";
  static const std::string kWeight = ".weight";
  layer = -1;
  if (name.compare(0, kPrefix.size(), kPrefix) != 0) {
    role = name;
    if (role.size() >= kWeight.size() && role.compare(role.size() - kWeight.size(), kWeight.size(), kWeight) == 0)
      role.resize(role.size() - kWeight.size());
    return;
  }
  const std::size_t dot = name.find('.', kPrefix.size());
  if (dot == std::string::npos) {
    role = name;
    return;
  }
  layer = std::stoi(name.substr(kPrefix.size(), dot - kPrefix.size()));
  role = name.substr(dot + 1);
}

struct PlanEntry {
  std::string type;
  std::vector<std::uint64_t> dimensions;
  std::uint64_t span_bytes = 0;
  std::uint64_t absolute_offset = 0;
};

std::unordered_map<std::string, PlanEntry> load_plan(const std::filesystem::path& path) {
  if (path.empty()) fail("tensor plan path is empty");
  const Json doc = Reader(read_text(path, "tensor plan")).document();
  std::unordered_map<std::string, PlanEntry> out;
  for (const Json& t : tensor_records(doc, "tensor plan")) {
    PlanEntry e;
    const std::string name = str(t, "name");
    e.type = str(t, "type");
    e.dimensions = opt_u64_array(t, "dimensions");
    e.span_bytes = u64(t, "span_bytes");
    e.absolute_offset = opt_u64(t, "absolute_offset");
    if (!out.emplace(name, std::move(e)).second) fail("tensor plan contains duplicate tensor: " + name);
  }
  if (out.empty()) fail("tensor plan contains no tensor entries: " + path.string());
  return out;
}

// The checks both manifest kinds share: present, same type, same dimensions,
// same span, same offset when both are known.
const PlanEntry& check_plan_entry(const std::unordered_map<std::string, PlanEntry>& plan, const std::string& name,
                                  const std::string& type, const std::vector<std::uint64_t>& dims,
                                  std::uint64_t source_bytes, bool span_only_if_known, std::uint64_t source_offset) {
  const auto it = plan.find(name);
  if (it == plan.end()) fail("tensor plan is missing manifest tensor: " + name);
  const PlanEntry& p = it->second;
  if (p.type != type) fail("tensor plan type mismatch for " + name + ": manifest " + type + ", plan " + p.type);
  if (p.dimensions != dims)
    fail("tensor plan dimensions mismatch for " + name + ": manifest " + dims_text(dims) + ", plan " +
         dims_text(p.dimensions));
  if ((!span_only_if_known || source_bytes != 0) && p.span_bytes != source_bytes)
    fail("tensor plan source byte mismatch for " + name + ": manifest " + std::to_string(source_bytes) + ", plan " +
         std::to_string(p.span_bytes));
  if (source_offset != 0 && p.absolute_offset != 0 && p.absolute_offset != source_offset)
    fail("tensor plan source offset mismatch for " + name + ": manifest " + std::to_string(source_offset) +
         ", plan " + std::to_string(p.absolute_offset));
  return p;
}

}  // namespace

std::uint64_t byte_checksum(const std::vector<std::uint8_t>& bytes) {
  std::uint64_t sum = 0;
  for (const std::uint8_t b : bytes) sum += b;
  return sum;
}

std::vector<std::uint8_t> load_binary_file(const std::filesystem::path& path, std::uint64_t expected_bytes,
                                           const char* label) {
  std::ifstream in(path, std::ios::binary | std::ios::ate);
  if (!in) fail(std::string("failed to open ") + label + ": " + path.string());
  const auto size = static_cast<std::uint64_t>(in.tellg());
  if (size != expected_bytes)
    fail(std::string(label) + " size mismatch: expected " + std::to_string(expected_bytes) + " bytes, got " +
         std::to_string(size));
  std::vector<std::uint8_t> data(static_cast<std::size_t>(size));
  in.seekg(0);
  if (size != 0 && !in.read(reinterpret_cast<char*>(data.data()), static_cast<std::streamsize>(size)))
    fail(std::string("failed to read ") + label + ": " + path.string());
  return data;
}

int q4k_policy_format(const std::string& policy) {
  static const std::map<std::string, int> kFormats = {
      {"split-predecoded", 1}, {"split-half", 2}, {"split-compact", 3}, {"split-native", 4}};
  const auto it = kFormats.find(policy);
  return it == kFormats.end() ? -1 : it->second;
}

Q4KManifest load_q4k_manifest(const std::filesystem::path& path) {
  const Json doc = Reader(read_text(path, "manifest")).document();
  if (doc.kind != Json::Object) fail("manifest is not a JSON object: " + path.string());
  Q4KManifest m;
  m.path = path;
  m.model = opt_str(doc, "model");
  m.tensor_plan = opt_str(doc, "tensor_plan");
  m.generated_at = opt_str(doc, "generated_at");
  m.policy = opt_str(doc, "policy");
  m.tensor_count = opt_u64(doc, "tensor_count");
  m.payload_bytes = opt_u64(doc, "payload_bytes");
  m.metadata_bytes = opt_u64(doc, "metadata_bytes");
  m.resident_bytes = opt_u64(doc, "resident_bytes");
  for (const Json& o : tensor_records(doc, "manifest")) {
    Q4KManifestTensor t;
    t.name = str(o, "name");
    t.dimensions = opt_u64_array(o, "dimensions");
    const std::uint64_t rows = u64(o, "rows"), cols = u64(o, "cols");
    if (rows > UINT32_MAX || cols > UINT32_MAX) fail("manifest tensor shape exceeds 32 bits: " + t.name);
    t.rows = static_cast<std::uint32_t>(rows);
    t.cols = static_cast<std::uint32_t>(cols);
    t.block_count = opt_u64(o, "block_count");
    t.source_offset = opt_u64(o, "source_offset");
    t.source_bytes = opt_u64(o, "source_bytes");
    t.policy = opt_str(o, "policy");
    t.metadata_format = opt_str(o, "metadata_format");
    t.runtime_kernel = opt_str(o, "runtime_kernel");
    if (t.runtime_kernel.empty()) t.runtime_kernel = t.policy;
    t.payload_path = str(o, "payload_path");
    t.metadata_path = str(o, "metadata_path");
    t.blocks_path = opt_str(o, "blocks_path");
    t.source_checksum = u64(o, "source_checksum");
    t.payload_checksum = u64(o, "payload_checksum");
    t.metadata_checksum = u64(o, "metadata_checksum");
    t.payload_bytes = u64(o, "payload_bytes");
    t.metadata_bytes = u64(o, "metadata_bytes");
    t.resident_bytes = opt_u64(o, "resident_bytes");
    name_metadata(t.name, t.layer, t.role);
    if (t.rows == 0 || t.cols == 0 || t.cols % 256u != 0u) fail("manifest tensor has invalid Q4_K shape: " + t.name);
    if (t.dimensions.empty()) {
      t.dimensions = {t.cols, t.rows};
    } else if (t.dimensions.size() != 2u || t.dimensions[0] != t.cols || t.dimensions[1] != t.rows) {
      fail("manifest tensor dimensions disagree with rows/cols: " + t.name);
    }
    m.tensors.push_back(std::move(t));
  }
  if (m.tensors.empty()) fail("manifest contains no tensors");
  return m;
}

std::vector<Q4KManifestTensor> select_q4k_tensors(const Q4KManifest& manifest, const std::vector<std::string>& names,
                                                  std::size_t limit) {
  std::vector<Q4KManifestTensor> out;
  if (!names.empty()) {
    for (const auto& n : names) {
      const auto it = std::find_if(manifest.tensors.begin(), manifest.tensors.end(),
                                   [&](const Q4KManifestTensor& t) { return t.name == n; });
      if (it == manifest.tensors.end()) fail("manifest tensor not found: " + n);
      out.push_back(*it);
    }
    return out;
  }
  const std::size_t n = limit == 0 ? manifest.tensors.size() : std::min(limit, manifest.tensors.size());
  out.assign(manifest.tensors.begin(), manifest.tensors.begin() + static_cast<std::ptrdiff_t>(n));
  return out;
}

Q4KTensorPlanValidation validate_q4k_manifest_tensors_against_plan(const std::vector<Q4KManifestTensor>& selected,
                                                                   const std::filesystem::path& tensor_plan_path) {
  const auto plan = load_plan(tensor_plan_path);
  for (const auto& t : selected) {
    const PlanEntry& p =
        check_plan_entry(plan, t.name, "Q4_K", t.dimensions, t.source_bytes, true, t.source_offset);
    if (p.dimensions.size() != 2u || p.dimensions[0] != t.cols || p.dimensions[1] != t.rows)
      fail("tensor plan rows/cols mismatch for " + t.name + ": manifest rows/cols " + std::to_string(t.rows) + "/" +
           std::to_string(t.cols) + ", plan dims " + dims_text(p.dimensions));
  }
  return {tensor_plan_path, selected.size()};
}

IQManifest load_iq_manifest(const std::filesystem::path& path) {
  const Json doc = Reader(read_text(path, "manifest")).document();
  if (doc.kind != Json::Object) fail("manifest is not a JSON object: " + path.string());
  IQManifest m;
  m.path = path;
  m.model = opt_str(doc, "model");
  m.tensor_plan = opt_str(doc, "tensor_plan");
  m.generated_at = opt_str(doc, "generated_at");
  m.types = opt_str_array(doc, "types");
  m.tensor_count = opt_u64(doc, "tensor_count");
  m.source_bytes = opt_u64(doc, "source_bytes");
  m.payload_bytes = opt_u64(doc, "payload_bytes");
  m.resident_bytes = opt_u64(doc, "resident_bytes");
  for (const Json& o : tensor_records(doc, "IQ manifest")) {
    IQManifestTensor t;
    t.name = str(o, "name");
    t.type = str(o, "type");
    const Json* layer = o.find("layer");
    t.layer = layer != nullptr && layer->kind == Json::Null ? -1 : static_cast<int>(opt_u64(o, "layer"));
    t.role = opt_str(o, "role");
    t.dimensions = opt_u64_array(o, "dimensions");
    t.element_count = u64(o, "element_count");
    t.block_size = u64(o, "block_size");
    t.block_type_size = u64(o, "block_type_size");
    t.block_count = u64(o, "block_count");
    t.source_offset = u64(o, "source_offset");
    t.source_bytes = u64(o, "source_bytes");
    t.source_checksum = u64(o, "source_checksum");
    t.payload_path = str(o, "payload_path");
    t.payload_bytes = u64(o, "payload_bytes");
    t.payload_checksum = u64(o, "payload_checksum");
    t.resident_bytes = u64(o, "resident_bytes");
    t.policy = opt_str(o, "policy");
    t.runtime_kernel = opt_str(o, "runtime_kernel");
    if (t.type != "IQ2_S" && t.type != "IQ3_S" && t.type != "Q5_K")
      fail("unsupported raw quant manifest tensor type: " + t.type);
    if (t.block_count == 0 || t.block_size != 256 || t.payload_bytes == 0)
      fail("IQ manifest tensor has invalid block metadata: " + t.name);
    if (t.source_bytes != t.payload_bytes) fail("IQ manifest tensor source/payload byte mismatch: " + t.name);
    m.tensors.push_back(std::move(t));
  }
  if (m.tensors.empty()) fail("IQ manifest contains no tensors");
  return m;
}

PackManifestKind pack_manifest_kind(const std::filesystem::path& path) {
  const Json doc = Reader(read_text(path, "manifest")).document();
  const std::string producer = opt_str(doc, "path");
  if (producer == "q4k_resident_pack") return PackManifestKind::Q4K;
  if (producer == "iq_resident_pack" || producer == "q5k_resident_pack") return PackManifestKind::RawBlocks;
  if (!producer.empty()) fail("unknown pack producer " + producer + ": " + path.string());
  const auto& recs = tensor_records(doc, "manifest");
  if (!recs.empty() && recs.front().find("metadata_path") != nullptr) return PackManifestKind::Q4K;
  if (!recs.empty() && recs.front().find("type") != nullptr) return PackManifestKind::RawBlocks;
  fail("cannot tell the kind of manifest " + path.string());
}

IQManifestTensor select_iq_tensor(const IQManifest& manifest, const std::string& name) {
  if (name.empty()) return manifest.tensors.front();
  for (const auto& t : manifest.tensors)
    if (t.name == name) return t;
  fail("IQ manifest tensor not found: " + name);
}

IQTensorPlanValidation validate_iq_manifest_tensors_against_plan(const std::vector<IQManifestTensor>& selected,
                                                                 const std::filesystem::path& tensor_plan_path) {
  const auto plan = load_plan(tensor_plan_path);
  for (const auto& t : selected)
    (void)check_plan_entry(plan, t.name, t.type, t.dimensions, t.source_bytes, false, t.source_offset);
  return {tensor_plan_path, selected.size()};
}

}  // namespace rtxllm
