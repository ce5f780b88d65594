// GGUF -> resident packs (host code, C++17, no GPU work). The reading of the
// container, the tensor plan, the per-producer records and the manifests
// follow the reference's Python producers (see include/rtxllm/pack_producer.h
// for the file:line of each); the code is written for this library.
#include "rtxllm/pack_producer.h"

#include <algorithm>
#include <chrono>
#include <cstring>
#include <ctime>
#include <fstream>
#include <map>
#include <set>
#include <sstream>
#include <stdexcept>

#include "json_value.h"
#include "q4k_split.h"

namespace rtxllm {
namespace {

namespace J = json;
namespace fs = std::filesystem;

[[noreturn]] void fail(const std::string& what) { throw std::runtime_error(what); }

// ---- GGUF block formats (gguf_block_formats.py:14-22) and ggml type ids --------------

struct BlockFormat {
  const char* name;
  std::uint64_t block_size, type_size;
};
constexpr BlockFormat kBlockFormats[] = {{"F32", 1, 4},      {"F16", 1, 2},      {"Q8_0", 32, 34},
                                         {"Q4_K", 256, 144}, {"Q5_K", 256, 176}, {"IQ2_S", 256, 82},
                                         {"IQ3_S", 256, 110}};

const BlockFormat* block_format(const std::string& type) {
  for (const auto& f : kBlockFormats)
    if (type == f.name) return &f;
  return nullptr;
}

// The public ggml type ids of GGUF (gguf_inspect.py:29-65).
std::string ggml_type_name(std::uint32_t id) {
  static const char* const kNames[] = {"F32",     "F16",     "Q4_0",    "Q4_1",   "",       "",        "Q5_0",
                                       "Q5_1",    "Q8_0",    "Q8_1",    "Q2_K",   "Q3_K",   "Q4_K",    "Q5_K",
                                       "Q6_K",    "Q8_K",    "IQ2_XXS", "IQ2_XS", "IQ3_XXS", "IQ1_S",  "IQ4_NL",
                                       "IQ3_S",   "IQ2_S",   "IQ4_XS",  "I8",     "I16",    "I32",     "I64",
                                       "F64",     "IQ1_M",   "BF16",    "Q4_0_4_4", "Q4_0_4_8", "Q4_0_8_8",
                                       "TQ1_0",   "TQ2_0"};
  if (id < sizeof(kNames) / sizeof(kNames[0]) && kNames[id][0] != '\0') return kNames[id];
  return "unknown:" + std::to_string(id);
}

std::uint64_t element_count(const std::vector<std::uint64_t>& dims) {
  if (dims.empty()) fail("tensor dimensions must be a non-empty list");
  std::uint64_t n = 1;
  for (const std::uint64_t d : dims) {
    if (d != 0 && n > UINT64_MAX / d) fail("tensor element count overflows");
    n *= d;
  }
  return n;
}

// Bytes of a tensor's data (gguf_block_formats.py:34-44).
std::uint64_t expected_data_bytes(const std::string& type, const std::vector<std::uint64_t>& dims) {
  const BlockFormat* f = block_format(type);
  if (f == nullptr) fail("unsupported tensor type " + type);
  const std::uint64_t n = element_count(dims);
  if (n % f->block_size != 0)
    fail(type + " element count " + std::to_string(n) + " is not divisible by block size " +
         std::to_string(f->block_size));
  return n / f->block_size * f->type_size;
}

// ---- GGUF reading -----------------------------------------------------------------------

class GgufReader {
 public:
  GgufReader(const fs::path& path, std::uint64_t size) : in_(path, std::ios::binary), size_(size) {
    if (!in_) fail("failed to open GGUF file: " + path.string());
  }
  std::uint64_t pos() const { return pos_; }
  void exact(void* dst, std::uint64_t n) {
    if (n > size_ - pos_) fail("unexpected end of GGUF data at byte " + std::to_string(pos_));
    in_.read(static_cast<char*>(dst), static_cast<std::streamsize>(n));
    if (!in_) fail("failed to read GGUF data at byte " + std::to_string(pos_));
    pos_ += n;
  }
  void skip(std::uint64_t n) {
    if (n > size_ - pos_) fail("unexpected end of GGUF data at byte " + std::to_string(pos_));
    in_.seekg(static_cast<std::streamoff>(n), std::ios::cur);
    pos_ += n;
  }
  template <class T>
  T scalar() {
    T v;
    exact(&v, sizeof(T));  // GGUF is little-endian, as is every host this builds for
    return v;
  }
  std::string string() {
    const std::uint64_t n = scalar<std::uint64_t>();
    if (n > size_ - pos_) fail("GGUF string longer than the file at byte " + std::to_string(pos_));
    std::string s(static_cast<std::size_t>(n), '\0');
    if (n) exact(&s[0], n);
    return s;
  }

 private:
  std::ifstream in_;
  std::uint64_t size_, pos_ = 0;
};

// Byte size of a scalar GGUF value type (gguf_inspect.py:13-27), 0 for
// string / array / unknown.
std::uint64_t scalar_bytes(std::uint32_t t) {
  switch (t) {
    case 0: case 1: case 7: return 1;
    case 2: case 3: return 2;
    case 4: case 5: case 6: return 4;
    case 10: case 11: case 12: return 8;
    default: return 0;
  }
}

// Reads one metadata value: integers into *as_int (when non-null and the type
// is an integer), strings into *as_string, every scalar number (integers,
// floats, bools) into *as_num; arrays are walked and dropped.
void read_value(GgufReader& r, std::uint32_t type, int depth, std::int64_t* as_int, bool* is_int,
                std::string* as_string, bool* is_string, double* as_num = nullptr, bool* is_num = nullptr) {
  if (depth > 64) fail("GGUF metadata arrays nested too deep");
  if (is_int) *is_int = false;
  if (is_string) *is_string = false;
  if (is_num) *is_num = false;
  if (as_num != nullptr && (type == 6 || type == 7 || type == 12)) {
    double v = 0.0;
    if (type == 6) v = r.scalar<float>();
    else if (type == 7) v = r.scalar<std::uint8_t>() != 0u ? 1.0 : 0.0;
    else v = r.scalar<double>();
    *as_num = v, *is_num = true;
    return;
  }
  if (as_num != nullptr && (type <= 5u || type == 10u || type == 11u)) {
    std::int64_t iv = 0;
    bool ii = false;
    read_value(r, type, depth, &iv, &ii, nullptr, nullptr);
    if (type == 10u && !ii) {
      *as_num = 18446744073709551615.0, *is_num = true;  // above INT64_MAX: only its size matters here
      return;
    }
    if (as_int) *as_int = iv, *is_int = ii;
    *as_num = static_cast<double>(iv), *is_num = true;
    return;
  }
  switch (type) {
    case 0: { const auto v = r.scalar<std::uint8_t>(); if (as_int) *as_int = v, *is_int = true; return; }
    case 1: { const auto v = r.scalar<std::int8_t>(); if (as_int) *as_int = v, *is_int = true; return; }
    case 2: { const auto v = r.scalar<std::uint16_t>(); if (as_int) *as_int = v, *is_int = true; return; }
    case 3: { const auto v = r.scalar<std::int16_t>(); if (as_int) *as_int = v, *is_int = true; return; }
    case 4: { const auto v = r.scalar<std::uint32_t>(); if (as_int) *as_int = v, *is_int = true; return; }
    case 5: { const auto v = r.scalar<std::int32_t>(); if (as_int) *as_int = v, *is_int = true; return; }
    case 10: {
      const auto v = r.scalar<std::uint64_t>();
      if (as_int && v <= static_cast<std::uint64_t>(INT64_MAX)) *as_int = static_cast<std::int64_t>(v), *is_int = true;
      return;
    }
    case 11: { const auto v = r.scalar<std::int64_t>(); if (as_int) *as_int = v, *is_int = true; return; }
    case 6: r.skip(4); return;
    case 7: r.skip(1); return;
    case 12: r.skip(8); return;
    case 8: {
      std::string s = r.string();
      if (as_string) *as_string = std::move(s), *is_string = true;
      return;
    }
    case 9: {
      const auto item = r.scalar<std::uint32_t>();
      const auto n = r.scalar<std::uint64_t>();
      const std::uint64_t w = scalar_bytes(item);
      if (w != 0) {
        if (n > UINT64_MAX / w) fail("GGUF metadata array too long");
        r.skip(n * w);
        return;
      }
      if (item != 8 && item != 9) fail("unsupported GGUF metadata value type: " + std::to_string(item));
      for (std::uint64_t k = 0; k < n; ++k) read_value(r, item, depth + 1, nullptr, nullptr, nullptr, nullptr);
      return;
    }
    default: fail("unsupported GGUF metadata value type: " + std::to_string(type));
  }
}

// The layer of a "blk.<digits>." name, else -1 (gguf_tensor_plan.py:48-50).
int tensor_layer(const std::string& name) {
  if (name.compare(0, 4, "blk.") != 0) return -1;
  std::size_t i = 4;
  while (i < name.size() && name[i] >= '0' && name[i] <= '9') ++i;
  if (i == 4 || i >= name.size() || name[i] != '.' || i - 4 > 9) return -1;
  return std::stoi(name.substr(4, i - 4));
}

std::uint64_t align_up(std::uint64_t v, std::uint64_t a) { return (v + a - 1) / a * a; }

double mib(std::uint64_t v) { return static_cast<double>(v) / (1024.0 * 1024.0); }

// ISO 8601 UTC time with microseconds and "+00:00", as Python's
// datetime.now(timezone.utc).isoformat() writes it.
std::string now_iso() {
  const auto now = std::chrono::system_clock::now();
  const std::time_t t = std::chrono::system_clock::to_time_t(now);
  const auto us = std::chrono::duration_cast<std::chrono::microseconds>(now.time_since_epoch()).count() % 1000000;
  std::tm tm{};
  gmtime_r(&t, &tm);
  char buf[64];
  std::snprintf(buf, sizeof buf, "%04d-%02d-%02dT%02d:%02d:%02d.%06lld+00:00", tm.tm_year + 1900, tm.tm_mon + 1,
                tm.tm_mday, tm.tm_hour, tm.tm_min, tm.tm_sec, static_cast<long long>(us));
  return buf;
}

// ---- pack files -------------------------------------------------------------------------

std::uint64_t checksum(const std::vector<std::uint8_t>& b) {
  std::uint64_t s = 0;
  for (const std::uint8_t x : b) s += x;
  return s;
}

void write_file(const fs::path& p, const std::vector<std::uint8_t>& bytes) {
  std::ofstream out(p, std::ios::binary | std::ios::trunc);
  if (!out) fail("failed to create pack file: " + p.string());
  out.write(reinterpret_cast<const char*>(bytes.data()), static_cast<std::streamsize>(bytes.size()));
  if (!out) fail("failed to write pack file: " + p.string());
}

// The tensor's data bytes at its absolute offset; its span must hold them
// (q4k_resident_pack.py:156-167, iq_resident_pack.py:98-112).
std::vector<std::uint8_t> read_tensor_bytes(const fs::path& model, const TensorPlanRow& row, std::uint64_t expected,
                                            const char* what) {
  if (row.span_bytes < expected) fail(row.name + " span is smaller than expected " + what + " bytes");
  std::error_code ec;
  const std::uint64_t size = fs::file_size(model, ec);
  if (ec) fail("failed to open model file: " + model.string());
  if (row.absolute_offset > size || expected > size - row.absolute_offset) {  // before any allocation
    const std::uint64_t got = row.absolute_offset < size ? size - row.absolute_offset : 0u;
    fail("short read for " + row.name + ": expected " + std::to_string(expected) + ", got " + std::to_string(got));
  }
  std::ifstream in(model, std::ios::binary);
  if (!in) fail("failed to open model file: " + model.string());
  in.seekg(static_cast<std::streamoff>(row.absolute_offset));
  std::vector<std::uint8_t> data(static_cast<std::size_t>(expected));
  in.read(reinterpret_cast<char*>(data.data()), static_cast<std::streamsize>(expected));
  const std::uint64_t got = in ? expected : static_cast<std::uint64_t>(std::max<std::streamsize>(in.gcount(), 0));
  if (got != expected)
    fail("short read for " + row.name + ": expected " + std::to_string(expected) + ", got " + std::to_string(got));
  return data;
}

J::Json dims_json(const std::vector<std::uint64_t>& d) {
  J::Json a = J::array();
  for (const std::uint64_t x : d) a.items.push_back(J::integer(x));
  return a;
}

std::string dims_text(const std::vector<std::uint64_t>& d) {
  std::string s = "[";
  for (std::size_t i = 0; i < d.size(); ++i) s += (i ? ", " : "") + std::to_string(d[i]);
  return s + "]";
}

J::Json layer_json(int layer) { return layer < 0 ? J::null_value() : J::integer_signed(layer); }

struct Q4KPolicy {
  const char* name;
  int format;
  const char* metadata_format;
};
// q4k_resident_pack.py:82-97
constexpr Q4KPolicy kQ4KPolicies[] = {{"split-predecoded", RTXLLM_FMT_Q4K_SPLIT_PREDECODED, "fp32-products"},
                                      {"split-half", RTXLLM_FMT_Q4K_SPLIT_HALF, "fp16-products"},
                                      {"split-compact", RTXLLM_FMT_Q4K_SPLIT_COMPACT, "compact-u8"},
                                      {"split-native", RTXLLM_FMT_Q4K_SPLIT_NATIVE, "native16"}};

const Q4KPolicy& q4k_policy(const std::string& name) {
  for (const auto& p : kQ4KPolicies)
    if (name == p.name) return p;
  fail("unknown Q4_K metadata policy: " + name);
}

J::Json q4k_record(const fs::path& model, const TensorPlanRow& row, const fs::path& out_dir,
                   const std::string& policy_arg, bool write_blocks) {
  // q4k_resident_pack.py:64-72: 2-D, cols first, cols a whole number of blocks
  if (row.dimensions.size() != 2) fail(row.name + " is not a 2D Q4_K tensor");
  const std::uint64_t cols = row.dimensions[0], rows = row.dimensions[1];
  if (cols == 0 || rows == 0 || cols % 256 != 0)
    fail(row.name + " has unsupported Q4_K dimensions: " + dims_text(row.dimensions));
  if (rows > UINT32_MAX || cols > UINT32_MAX) fail(row.name + " is too large for a Q4_K pack");
  const std::uint64_t n_blocks = rows * (cols / 256);
  const std::string policy = resolve_q4k_policy(policy_arg, rows, cols);
  const Q4KPolicy& pol = q4k_policy(policy);
  const std::vector<std::uint8_t> blocks = read_tensor_bytes(model, row, n_blocks * 144u, "Q4_K");
  const std::uint32_t mb = rtxllm_format_meta_bytes(pol.format);
  std::vector<std::uint8_t> payload(static_cast<std::size_t>(n_blocks * 128u)),
      meta(static_cast<std::size_t>(n_blocks * mb));
  for (std::uint64_t b = 0; b < n_blocks; ++b)
    q4k_split_block(pol.format, blocks.data() + b * 144u, payload.data() + b * 128u, meta.data() + b * mb);
  if (pol.format == RTXLLM_FMT_Q4K_SPLIT_HALF) {
    // the reference packs the products with struct.pack("<e"), which refuses
    // a finite value beyond the fp16 range: so does this producer
    for (std::uint64_t b = 0; b < n_blocks; ++b) {
      const std::uint8_t* blk = blocks.data() + b * 144u;
      const float d = f16_to_f32_host(static_cast<std::uint16_t>(blk[0] | (blk[1] << 8)));
      const float dmin = f16_to_f32_host(static_cast<std::uint16_t>(blk[2] | (blk[3] << 8)));
      for (int j = 0; j < 16; ++j) {
        std::uint16_t h;
        std::memcpy(&h, meta.data() + b * mb + 2u * static_cast<unsigned>(j), 2);
        const bool inf = (h & 0x7FFFu) == 0x7C00u;
        const float src = (j & 1) ? dmin : d;
        if (inf && src - src == 0.0f)
          fail(row.name + " split-half metadata: a scale product is beyond the fp16 range");
      }
    }
  }
  const std::string label = sanitize_label(row.name);
  const fs::path pp = out_dir / (label + ".q4k_payload.bin");
  const fs::path mp = out_dir / (label + ".q4k_meta." + pol.metadata_format + ".bin");
  write_file(pp, payload);
  write_file(mp, meta);
  std::string bp;
  if (write_blocks) {
    const fs::path p = out_dir / (label + ".q4k_blocks.bin");
    write_file(p, blocks);
    bp = p.string();
  }
  const std::uint64_t resident = payload.size() + meta.size();
  J::Json r = J::object();
  J::set(r, "name", J::string(row.name));
  J::set(r, "dimensions", dims_json(row.dimensions));
  J::set(r, "rows", J::integer(rows));
  J::set(r, "cols", J::integer(cols));
  J::set(r, "block_count", J::integer(n_blocks));
  J::set(r, "source_offset", J::integer(row.absolute_offset));
  J::set(r, "source_bytes", J::integer(blocks.size()));
  J::set(r, "source_checksum", J::integer(checksum(blocks)));
  J::set(r, "policy", J::string(policy));
  J::set(r, "metadata_format", J::string(pol.metadata_format));
  J::set(r, "payload_path", J::string(pp.string()));
  J::set(r, "payload_bytes", J::integer(payload.size()));
  J::set(r, "payload_checksum", J::integer(checksum(payload)));
  J::set(r, "metadata_path", J::string(mp.string()));
  J::set(r, "metadata_bytes", J::integer(meta.size()));
  J::set(r, "metadata_checksum", J::integer(checksum(meta)));
  J::set(r, "blocks_path", J::string(bp));
  J::set(r, "resident_bytes", J::integer(resident));
  J::set(r, "compression_ratio_vs_fp16",
         J::real(static_cast<double>(rows * cols * 2u) / static_cast<double>(resident)));
  J::set(r, "runtime_kernel", J::string(policy));
  return r;
}

// IQ2_S / IQ3_S (iq_resident_pack.py:115-147) and Q5_K (q5k_resident_pack.py:93-120).
J::Json raw_record(const fs::path& model, const TensorPlanRow& row, const fs::path& out_dir) {
  const BlockFormat* f = block_format(row.type);
  const char* kernel = row.type == "IQ2_S"   ? "iq2s_raw_block_probe"
                       : row.type == "IQ3_S" ? "iq3s_raw_block_probe"
                       : row.type == "Q5_K"  ? "q5_k_raw_pending"
                                             : nullptr;
  if (f == nullptr || kernel == nullptr) fail(row.name + " has unsupported raw-block type: " + row.type);
  const std::uint64_t values = element_count(row.dimensions);
  if (values % f->block_size != 0)
    fail(row.name + " element count " + std::to_string(values) + " is not divisible by " +
         std::to_string(f->block_size));
  const std::uint64_t n_blocks = values / f->block_size;
  const std::string what = row.type == "Q5_K" ? "Q5_K" : "IQ";
  const std::vector<std::uint8_t> payload = read_tensor_bytes(model, row, n_blocks * f->type_size, what.c_str());
  std::string lower = row.type;
  std::transform(lower.begin(), lower.end(), lower.begin(), [](unsigned char c) { return std::tolower(c); });
  const fs::path pp = out_dir / (sanitize_label(row.name) + "." + lower + "_raw_blocks.bin");
  write_file(pp, payload);
  int layer = -1;
  std::string role;
  tensor_role(row.name, layer, role);
  const std::uint64_t sum = checksum(payload);
  J::Json r = J::object();
  J::set(r, "name", J::string(row.name));
  J::set(r, "type", J::string(row.type));
  J::set(r, "layer", layer_json(layer));
  J::set(r, "role", J::string(role));
  J::set(r, "dimensions", dims_json(row.dimensions));
  J::set(r, "element_count", J::integer(values));
  J::set(r, "block_size", J::integer(f->block_size));
  J::set(r, "block_type_size", J::integer(f->type_size));
  J::set(r, "block_count", J::integer(n_blocks));
  J::set(r, "source_offset", J::integer(row.absolute_offset));
  J::set(r, "source_bytes", J::integer(payload.size()));
  J::set(r, "source_checksum", J::integer(sum));
  J::set(r, "payload_path", J::string(pp.string()));
  J::set(r, "payload_bytes", J::integer(payload.size()));
  J::set(r, "payload_checksum", J::integer(sum));
  J::set(r, "resident_bytes", J::integer(payload.size()));
  J::set(r, "policy", J::string("raw-blocks"));
  J::set(r, "runtime_kernel", J::string(kernel));
  return r;
}

J::Json record_of(const fs::path& model, const TensorPlanRow& row, const fs::path& out_dir,
                  const std::string& q4k_policy_arg, bool write_blocks) {
  if (row.type == "Q4_K") return q4k_record(model, row, out_dir, q4k_policy_arg, write_blocks);
  return raw_record(model, row, out_dir);
}

std::uint64_t u64_of(const J::Json& rec, const char* key) {
  const J::Json* v = rec.find(key);
  std::uint64_t x = 0;
  if (v == nullptr || !J::as_u64(*v, x)) fail(std::string("record field missing: ") + key);
  return x;
}
std::string text_of(const J::Json& rec, const char* key) {
  const J::Json* v = rec.find(key);
  return v != nullptr && v->kind == J::Json::String ? v->text : std::string();
}

void write_text(const fs::path& p, const std::string& text) {
  std::ofstream out(p, std::ios::binary | std::ios::trunc);
  if (!out) fail("failed to create " + p.string());
  out << text;
  if (!out) fail("failed to write " + p.string());
}

// manifest.md of each producer (q4k_resident_pack.py:225-257,
// iq_resident_pack.py:150-180, q5k_resident_pack.py:123-151).
std::string markdown(const std::string& kind, const J::Json& m) {
  std::ostringstream o;
  const std::string title = kind == "q4k" ? "Q4_K" : kind == "iq" ? "IQ" : "Q5_K";
  o << "# " << title << " Resident Pack\n\n";
  o << "Generated: `" << text_of(m, "generated_at") << "`\n";
  o << "Model: `" << text_of(m, "model") << "`\n";
  if (kind != "q4k") o << "Tensor plan: `" << text_of(m, "tensor_plan") << "`\n";
  o << "Output dir: `" << text_of(m, "output_dir") << "`\n";
  if (kind == "q4k") o << "Policy: `" << text_of(m, "policy") << "`\n";
  if (kind == "iq") {
    o << "Types: `";
    const J::Json* t = m.find("types");
    for (std::size_t i = 0; t != nullptr && i < t->items.size(); ++i) o << (i ? ", " : "") << t->items[i].text;
    o << "`\n";
  }
  o << "Tensor count: `" << u64_of(m, "tensor_count") << "`\n";
  o << "Resident bytes: `" << u64_of(m, "resident_bytes") << "`\n";
  if (kind == "q4k") {
    o << "Payload bytes: `" << u64_of(m, "payload_bytes") << "`\n";
    o << "Metadata bytes: `" << u64_of(m, "metadata_bytes") << "`\n";
  }
  o << "\n";
  if (kind == "q4k")
    o << "| tensor | dims | policy | payload B | meta B | resident B | checksum |\n|---|---|---|---:|---:|---:|---:|\n";
  else if (kind == "iq")
    o << "| tensor | type | dims | blocks | resident B | checksum |\n|---|---|---|---:|---:|---:|\n";
  else
    o << "| tensor | dims | blocks | resident B | checksum |\n|---|---|---:|---:|---:|\n";
  for (const J::Json& t : m.find("tensors")->items) {
    std::vector<std::uint64_t> dims;
    for (const J::Json& d : t.find("dimensions")->items) {
      std::uint64_t x = 0;
      J::as_u64(d, x);
      dims.push_back(x);
    }
    o << "| " << text_of(t, "name");
    if (kind == "iq") o << " | " << text_of(t, "type");
    o << " | " << dims_text(dims);
    if (kind == "q4k")
      o << " | " << text_of(t, "policy") << " | " << u64_of(t, "payload_bytes") << " | "
        << u64_of(t, "metadata_bytes");
    else
      o << " | " << u64_of(t, "block_count");
    o << " | " << u64_of(t, "resident_bytes") << " | " << u64_of(t, "source_checksum") << " |\n";
  }
  return o.str();
}

std::vector<std::string> split(const char* s, char sep) {
  std::vector<std::string> out;
  if (s == nullptr || *s == '\0') return out;
  std::string cur;
  for (const char* p = s;; ++p) {
    if (*p == sep || *p == '\0') {
      if (!cur.empty()) out.push_back(cur);
      cur.clear();
      if (*p == '\0') break;
    } else {
      cur += *p;
    }
  }
  return out;
}

TensorPlanRow row_from_json(const J::Json& t) {
  auto u = [&](const char* key, bool required) {
    const J::Json* v = t.find(key);
    std::uint64_t x = 0;
    if (v == nullptr || v->kind == J::Json::Null) {
      if (required) fail(std::string("tensor row field missing: ") + key);
      return x;
    }
    if (!J::as_u64(*v, x)) fail(std::string("tensor row integer expected: ") + key);
    return x;
  };
  TensorPlanRow r;
  const J::Json* name = t.find("name");
  const J::Json* type = t.find("type");
  if (t.kind != J::Json::Object || name == nullptr || name->kind != J::Json::String || type == nullptr ||
      type->kind != J::Json::String)
    fail("tensor row needs string name and type");
  r.name = name->text;
  r.type = type->text;
  const J::Json* dims = t.find("dimensions");
  if (dims == nullptr || dims->kind != J::Json::Array) fail("tensor dimensions must be a non-empty list");
  for (const J::Json& d : dims->items) {
    std::uint64_t x = 0;
    if (!J::as_u64(d, x)) fail("tensor dimensions must be non-negative integers");
    r.dimensions.push_back(x);
  }
  r.absolute_offset = u("absolute_offset", true);
  r.span_bytes = u("span_bytes", false);
  r.offset = u("offset", false);
  int layer = -1;
  std::string role;
  tensor_role(r.name, layer, role);
  r.layer = layer;
  return r;
}

J::Json plan_json(const GgufHeader& h, const std::vector<TensorPlanRow>& rows) {
  std::uint64_t non_layer = 0, total = 0;
  std::set<int> layers;
  for (const auto& r : rows) {
    total += r.span_bytes;
    if (r.layer < 0) non_layer += r.span_bytes;
    else layers.insert(r.layer);
  }
  J::Json meta = J::object();
  J::set(meta, "architecture", h.architecture.empty() ? J::null_value() : J::string(h.architecture));
  J::set(meta, "name", h.model_name.empty() ? J::null_value() : J::string(h.model_name));
  J::set(meta, "tensor_count", J::integer(h.tensor_count));
  J::set(meta, "metadata_count", J::integer(h.metadata_count));
  J::set(meta, "tensor_data_offset", J::integer(h.tensor_data_offset));
  J::set(meta, "tensor_data_alignment", J::integer(h.alignment));
  J::Json tensors = J::array();
  for (const auto& r : rows) {
    J::Json t = J::object();
    J::set(t, "name", J::string(r.name));
    J::set(t, "layer", layer_json(r.layer));
    J::set(t, "span_bytes", J::integer(r.span_bytes));
    J::set(t, "span_mib", J::real(mib(r.span_bytes)));
    J::set(t, "offset", J::integer(r.offset));
    J::set(t, "absolute_offset", J::integer(r.absolute_offset));
    J::set(t, "type", J::string(r.type));
    J::set(t, "type_id", J::integer(r.type_id));
    J::set(t, "dimensions", dims_json(r.dimensions));
    tensors.items.push_back(std::move(t));
  }
  // gguf_tensor_plan.py:140-179, without the VRAM budget estimate
  J::Json p = J::object();
  J::set(p, "path", J::string("gguf_tensor_plan"));
  J::set(p, "generated_at", J::string(now_iso()));
  J::set(p, "model_path", J::string(h.path.string()));
  J::set(p, "model_size_bytes", J::integer(h.file_size));
  J::set(p, "model_size_mib", J::real(mib(h.file_size)));
  J::set(p, "metadata", std::move(meta));
  J::set(p, "non_layer_bytes", J::integer(non_layer));
  J::set(p, "non_layer_mib", J::real(mib(non_layer)));
  J::set(p, "tensor_span_bytes", J::integer(total));
  J::set(p, "tensor_span_mib", J::real(mib(total)));
  J::set(p, "layer_count", J::integer(layers.size()));
  J::set(p, "tensors", std::move(tensors));
  return p;
}

int copy_out(const std::string& text, char* out, std::size_t len, char* err, std::size_t err_len) {
  if (out == nullptr || text.size() + 1 > len) {
    if (err != nullptr && err_len > 0)
      std::snprintf(err, err_len, "output buffer too small: %zu bytes needed", text.size() + 1);
    return -2;
  }
  std::memcpy(out, text.c_str(), text.size() + 1);
  return 0;
}

void set_err(char* err, std::size_t err_len, const char* what) {
  if (err != nullptr && err_len > 0) std::snprintf(err, err_len, "%s", what);
}

}  // namespace

// ---- public C++ API ------------------------------------------------------------------------

GgufHeader read_gguf_header(const fs::path& path) {
  GgufHeader h;
  h.path = fs::absolute(path);
  std::error_code ec;
  h.file_size = fs::file_size(path, ec);
  if (ec) fail("failed to stat GGUF file: " + path.string());
  GgufReader r(path, h.file_size);
  char magic[4];
  r.exact(magic, 4);
  if (std::memcmp(magic, "GGUF", 4) != 0) fail("not a GGUF file");
  h.version = r.scalar<std::uint32_t>();
  h.tensor_count = r.scalar<std::uint64_t>();
  h.metadata_count = r.scalar<std::uint64_t>();
  for (std::uint64_t i = 0; i < h.metadata_count; ++i) {
    const std::string key = r.string();
    const auto type = r.scalar<std::uint32_t>();
    std::int64_t iv = 0;
    bool is_int = false, is_str = false, is_num = false;
    std::string sv;
    double nv = 0.0;
    read_value(r, type, 0, &iv, &is_int, &sv, &is_str, &nv, &is_num);
    if (is_num) h.numbers.emplace_back(key, nv);
    if (key == "general.alignment" && is_int) h.alignment = iv > 0 ? static_cast<std::uint64_t>(iv) : 32u;
    if (key == "general.architecture" && is_str) h.architecture = sv;
    if (key == "general.name" && is_str) h.model_name = sv;
  }
  // each tensor info takes at least 8 + 4 + 4 + 8 bytes
  if (h.tensor_count > (h.file_size - r.pos()) / 24u) fail("GGUF tensor count exceeds the file");
  h.tensors.reserve(static_cast<std::size_t>(h.tensor_count));
  for (std::uint64_t i = 0; i < h.tensor_count; ++i) {
    GgufTensorInfo t;
    t.name = r.string();
    const auto n_dims = r.scalar<std::uint32_t>();
    if (n_dims > 64) fail("GGUF tensor with " + std::to_string(n_dims) + " dimensions: " + t.name);
    for (std::uint32_t d = 0; d < n_dims; ++d) t.dimensions.push_back(r.scalar<std::uint64_t>());
    t.type_id = r.scalar<std::uint32_t>();
    t.type = ggml_type_name(t.type_id);
    t.offset = r.scalar<std::uint64_t>();
    h.tensors.push_back(std::move(t));
  }
  h.tensor_info_end_offset = r.pos();
  h.tensor_data_offset = align_up(h.tensor_info_end_offset, h.alignment);
  return h;
}

std::vector<TensorPlanRow> gguf_tensor_spans(const GgufHeader& h) {
  std::vector<const GgufTensorInfo*> order;
  for (const auto& t : h.tensors) order.push_back(&t);
  std::stable_sort(order.begin(), order.end(),
                   [](const GgufTensorInfo* a, const GgufTensorInfo* b) { return a->offset < b->offset; });
  const std::uint64_t data_end = h.file_size >= h.tensor_data_offset ? h.file_size - h.tensor_data_offset : 0;
  std::vector<TensorPlanRow> rows;
  for (std::size_t i = 0; i < order.size(); ++i) {
    const GgufTensorInfo& t = *order[i];
    const std::uint64_t next = i + 1 < order.size() ? order[i + 1]->offset : data_end;
    TensorPlanRow r;
    r.name = t.name;
    r.layer = tensor_layer(t.name);
    r.span_bytes = next > t.offset ? next - t.offset : 0;
    r.offset = t.offset;
    r.absolute_offset = h.tensor_data_offset + t.offset;
    r.type = t.type;
    r.type_id = t.type_id;
    r.dimensions = t.dimensions;
    rows.push_back(std::move(r));
  }
  return rows;
}

std::string sanitize_label(const std::string& name) {
  std::string s;
  bool in_run = false;
  for (const char c : name) {
    const bool keep = (c >= 'A' && c <= 'Z') || (c >= 'a' && c <= 'z') || (c >= '0' && c <= '9') || c == '_' ||
                      c == '.' || c == '-';
    if (keep) {
      s += c;
      in_run = false;
    } else if (!in_run) {
      s += '_';
      in_run = true;
    }
  }
  // leading / trailing whitespace the reference strips first ends up in the
  // "_" runs this strip removes, so the labels agree
  const std::size_t b = s.find_first_not_of("._-");
  if (b == std::string::npos) return "native";
  const std::size_t e = s.find_last_not_of("._-");
  return s.substr(b, e - b + 1);
}

void tensor_role(const std::string& name, int& layer, std::string& role) {
  // ^blk\.(\d+)\.(.+)$ ('.' does not match a newline)
  layer = -1;
  if (name.compare(0, 4, "blk.") == 0) {
    std::size_t i = 4;
    while (i < name.size() && name[i] >= '0' && name[i] <= '9') ++i;
    const bool digits = i > 4, dot = i < name.size() && name[i] == '.';
    const std::string rest = dot ? name.substr(i + 1) : std::string();
    if (digits && dot && !rest.empty() && rest.find('\n') == std::string::npos &&
        name.substr(4, i - 4).find('\n') == std::string::npos) {
      const std::string num = name.substr(4, i - 4);
      if (num.size() > 9) fail("layer index out of range: " + name);
      layer = std::stoi(num);
      role = rest;
      return;
    }
  }
  static const std::string kWeight = ".weight";
  if (name.size() >= kWeight.size() && name.compare(name.size() - kWeight.size(), kWeight.size(), kWeight) == 0)
    role = name.substr(0, name.size() - kWeight.size());
  else
    role = name;
}

std::string resolve_q4k_policy(const std::string& policy, std::uint64_t rows, std::uint64_t cols) {
  if (policy == "auto" || policy.empty()) return "split-native";
  if (policy == "auto-lossy") return rows * (cols / 256) > 65536 ? "split-half" : "split-native";
  return q4k_policy(policy).name;
}

std::string pack_tensor_record(const fs::path& model, const TensorPlanRow& row, const fs::path& out_dir,
                               const std::string& q4k_policy_arg, bool write_blocks) {
  return J::dump(record_of(model, row, fs::absolute(out_dir), q4k_policy_arg, write_blocks));
}

PackSetPaths pack_gguf(const fs::path& gguf, const fs::path& out_dir_arg, const PackOptions& opt) {
  const GgufHeader h = read_gguf_header(gguf);
  const std::vector<TensorPlanRow> rows = gguf_tensor_spans(h);
  static const std::vector<std::string> kTypes = {"Q4_K", "Q5_K", "IQ2_S", "IQ3_S"};
  std::set<std::string> types(opt.types.begin(), opt.types.end());
  if (types.empty()) types.insert(kTypes.begin(), kTypes.end());
  for (const auto& t : types)
    if (std::find(kTypes.begin(), kTypes.end(), t) == kTypes.end()) fail("unsupported pack type: " + t);
  if (opt.q4k_policy != "auto" && opt.q4k_policy != "auto-lossy" && !opt.q4k_policy.empty())
    (void)q4k_policy(opt.q4k_policy);
  const std::set<std::string> names(opt.names.begin(), opt.names.end());

  // the reference's selection per producer: type, requested names, layer, then limit
  auto select = [&](const std::set<std::string>& producer_types) {
    std::vector<const TensorPlanRow*> out;
    for (const auto& r : rows) {
      if (!producer_types.count(r.type) || !types.count(r.type)) continue;
      if (!names.empty() && !names.count(r.name)) continue;
      if (opt.layer >= 0) {
        int layer = -1;
        std::string role;
        tensor_role(r.name, layer, role);
        if (layer != opt.layer) continue;
      }
      out.push_back(&r);
    }
    if (opt.limit != 0 && out.size() > opt.limit) out.resize(static_cast<std::size_t>(opt.limit));
    return out;
  };
  const auto q4k = select({"Q4_K"});
  const auto iq = select({"IQ2_S", "IQ3_S"});
  const auto q5k = select({"Q5_K"});
  if (q4k.empty() && iq.empty() && q5k.empty()) fail("no Q4_K / Q5_K / IQ2_S / IQ3_S tensors selected");

  const fs::path out_dir = fs::absolute(out_dir_arg);
  fs::create_directories(out_dir);
  PackSetPaths paths;
  paths.tensor_plan = out_dir / "tensor_plan.json";
  write_text(paths.tensor_plan, J::dump(plan_json(h, rows)) + "\n");
  const std::string stamp = now_iso();

  auto produce = [&](const std::string& kind, const std::vector<const TensorPlanRow*>& sel) -> fs::path {
    if (sel.empty()) return {};
    const fs::path dir = out_dir / kind;
    fs::create_directories(dir);
    J::Json tensors = J::array();
    std::uint64_t source = 0, payload = 0, metadata = 0, resident = 0;
    std::set<std::string> present;
    for (const TensorPlanRow* r : sel) {
      J::Json rec = record_of(h.path, *r, dir, opt.q4k_policy, opt.write_blocks);
      source += u64_of(rec, "source_bytes");
      payload += u64_of(rec, "payload_bytes");
      resident += u64_of(rec, "resident_bytes");
      if (kind == "q4k") metadata += u64_of(rec, "metadata_bytes");
      present.insert(r->type);
      tensors.items.push_back(std::move(rec));
    }
    J::Json m = J::object();
    J::set(m, "path", J::string(kind + "_resident_pack"));
    J::set(m, "generated_at", J::string(stamp));
    J::set(m, "model", J::string(h.path.string()));
    J::set(m, "tensor_plan", J::string(paths.tensor_plan.string()));
    J::set(m, "output_dir", J::string(dir.string()));
    if (kind == "q4k") {
      J::set(m, "policy", J::string(opt.q4k_policy.empty() ? "auto" : opt.q4k_policy));
      J::set(m, "write_blocks", J::boolean(opt.write_blocks));
    } else {
      // the producer's selected types (sorted), as its --type arguments name them
      J::Json t = J::array();
      for (const auto& ty : types)
        if ((kind == "iq" && (ty == "IQ2_S" || ty == "IQ3_S")) || (kind == "q5k" && ty == "Q5_K"))
          t.items.push_back(J::string(ty));
      J::set(m, "types", std::move(t));
    }
    J::set(m, "tensor_count", J::integer(sel.size()));
    J::set(m, "source_bytes", J::integer(source));
    J::set(m, "payload_bytes", J::integer(payload));
    if (kind == "q4k") J::set(m, "metadata_bytes", J::integer(metadata));
    J::set(m, "resident_bytes", J::integer(resident));
    J::set(m, "tensors", std::move(tensors));
    const fs::path json_path = dir / "manifest.json";
    write_text(json_path, J::dump(m));
    write_text(dir / "manifest.md", markdown(kind, m));
    return json_path;
  };
  paths.q4k_manifest = produce("q4k", q4k);
  paths.iq_manifest = produce("iq", iq);
  paths.q5k_manifest = produce("q5k", q5k);
  return paths;
}

}  // namespace rtxllm

// ---- C-ABI -------------------------------------------------------------------------------

extern "C" int rtxllm_gguf_pack(const char* gguf_path, const char* out_dir, const rtxllm_pack_options* options,
                                char* result, size_t result_len, char* err, size_t err_len) {
  try {
    if (gguf_path == nullptr || out_dir == nullptr) throw std::runtime_error("gguf_path and out_dir are required");
    rtxllm::PackOptions opt;
    if (options != nullptr) {
      if (options->q4k_policy != nullptr) opt.q4k_policy = options->q4k_policy;
      opt.write_blocks = options->write_blocks != 0;
      opt.types = rtxllm::split(options->types, ',');
      opt.names = rtxllm::split(options->names, '\n');
      opt.layer = options->layer;
      opt.limit = options->limit;
    }
    const rtxllm::PackSetPaths p = rtxllm::pack_gguf(gguf_path, out_dir, opt);
    namespace J = rtxllm::json;
    J::Json r = J::object();
    auto path_or_null = [](const std::filesystem::path& x) { return x.empty() ? J::null_value() : J::string(x.string()); };
    J::set(r, "tensor_plan", J::string(p.tensor_plan.string()));
    J::set(r, "q4k_manifest", path_or_null(p.q4k_manifest));
    J::set(r, "iq_manifest", path_or_null(p.iq_manifest));
    J::set(r, "q5k_manifest", path_or_null(p.q5k_manifest));
    return rtxllm::copy_out(J::dump(r), result, result_len, err, err_len);
  } catch (const std::exception& e) {
    rtxllm::set_err(err, err_len, e.what());
    return -1;
  }
}

extern "C" int rtxllm_pack_tensor(const char* model_path, const char* tensor_json, const char* out_dir,
                                  const char* q4k_policy, int write_blocks, char* record, size_t record_len,
                                  char* err, size_t err_len) {
  try {
    if (model_path == nullptr || tensor_json == nullptr || out_dir == nullptr)
      throw std::runtime_error("model_path, tensor_json and out_dir are required");
    const rtxllm::json::Json t = rtxllm::json::Reader(tensor_json).document();
    const rtxllm::TensorPlanRow row = rtxllm::row_from_json(t);
    const std::string rec = rtxllm::pack_tensor_record(model_path, row, out_dir,
                                                       q4k_policy != nullptr ? q4k_policy : "auto", write_blocks != 0);
    return rtxllm::copy_out(rec, record, record_len, err, err_len);
  } catch (const std::exception& e) {
    rtxllm::set_err(err, err_len, e.what());
    return -1;
  }
}

extern "C" int rtxllm_gguf_tensor_plan(const char* gguf_path, char* plan, size_t plan_len, char* err,
                                       size_t err_len) {
  try {
    if (gguf_path == nullptr) throw std::runtime_error("gguf_path is required");
    const rtxllm::GgufHeader h = rtxllm::read_gguf_header(gguf_path);
    return rtxllm::copy_out(rtxllm::json::dump(rtxllm::plan_json(h, rtxllm::gguf_tensor_spans(h))), plan, plan_len,
                            err, err_len);
  } catch (const std::exception& e) {
    rtxllm::set_err(err, err_len, e.what());
    return -1;
  }
}

extern "C" int rtxllm_pack_tensor_shape(const char* type, const uint64_t* dims, uint32_t n_dims, uint64_t* values,
                                        uint64_t* blocks, uint64_t* bytes, char* err, size_t err_len) {
  try {
    if (type == nullptr || (dims == nullptr && n_dims != 0)) throw std::runtime_error("type and dims are required");
    const std::vector<std::uint64_t> d(dims, dims + n_dims);
    const std::uint64_t b = rtxllm::expected_data_bytes(type, d);
    const std::uint64_t n = rtxllm::element_count(d);
    if (values) *values = n;
    if (blocks) *blocks = n / rtxllm::block_format(type)->block_size;
    if (bytes) *bytes = b;
    return 0;
  } catch (const std::exception& e) {
    rtxllm::set_err(err, err_len, e.what());
    return -1;
  }
}

extern "C" int rtxllm_pack_tensor_role(const char* name, int* layer, char* role, size_t role_len) {
  if (name == nullptr || layer == nullptr) return -1;
  std::string r;
  try {
    rtxllm::tensor_role(name, *layer, r);
  } catch (const std::exception&) {
    return -1;
  }
  return rtxllm::copy_out(r, role, role_len, nullptr, 0);
}

extern "C" int rtxllm_pack_sanitize_label(const char* name, char* label, size_t label_len) {
  if (name == nullptr) return -1;
  return rtxllm::copy_out(rtxllm::sanitize_label(name), label, label_len, nullptr, 0);
}
