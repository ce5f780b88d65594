/* GGUF -> resident-pack producer (host code, no GPU work).
 *
 * The counterpart of the reference's pack producers and GGUF inspector,
 * written in C++:
 *  - tools/bench/gguf_inspect.py:159-221: the GGUF v3 header, typed metadata,
 *    tensor infos and the data offset (align_up(end of tensor infos,
 *    general.alignment), default 32);
 *  - tools/bench/gguf_tensor_plan.py:53-80: one row per tensor, its span
 *    running to the next tensor's offset (the last to the end of the file) and
 *    its absolute offset = data offset + offset;
 *  - tools/bench/q4k_resident_pack.py:170-222: Q4_K tensors (2-D, cols % 256
 *    == 0) into a 128-byte-per-block payload file and the metadata file of one
 *    split policy, optionally the raw blocks;
 *  - tools/bench/iq_resident_pack.py:115-147: IQ2_S / IQ3_S tensors as raw
 *    blocks (runtime_kernel "iq2s_raw_block_probe" / "iq3s_raw_block_probe");
 *  - tools/bench/q5k_resident_pack.py:93-120: Q5_K tensors as raw blocks
 *    (runtime_kernel "q5_k_raw_pending").
 * The output is the reference producers' form, field for field: manifest.json
 * (indent 2) and manifest.md per producer, absolute pack paths, pack files
 * named <label>.q4k_payload.bin, <label>.q4k_meta.<metadata_format>.bin,
 * <label>.q4k_blocks.bin and <label>.<type>_raw_blocks.bin with label =
 * sanitize_label(tensor name) (tools/bench/native_harness.py:126-128), byte-sum
 * checksums. The "auto" Q4_K policy is the MI355X choice made here
 * (split-native; "auto-lossy": split-half above 65536 blocks), not the
 * reference's RTX 3060 rule (q4k_resident_pack.py:75-79); the named policies
 * are the reference's. The loaders in rtxllm/pack_manifest.h and
 * rtxllm_llama_load_pack_set (rtxllm/llama.h) read the result. */
#ifndef RTXLLM_PACK_PRODUCER_H
#define RTXLLM_PACK_PRODUCER_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef struct rtxllm_pack_options {
  /* NULL or "auto" (MI355X policy), "auto-lossy", "split-native", "split-half",
   * "split-compact", "split-predecoded" */
  const char* q4k_policy;
  /* nonzero: also write each Q4_K tensor's raw blocks (blocks_path), which
   * the decode runner's raw Q4_K format reads */
  int write_blocks;
  /* comma-separated GGUF types to pack; NULL or "": Q4_K,Q5_K,IQ2_S,IQ3_S */
  const char* types;
  /* newline-separated tensor names; NULL or "": every tensor of those types */
  const char* names;
  /* only tensors named blk.<layer>.*; -1: every tensor */
  int layer;
  /* per manifest, the first `limit` selected tensors after the name and layer
   * filters (iq_resident_pack.py:64-82 order); 0: all */
  uint64_t limit;
} rtxllm_pack_options;

/* Packs `gguf_path` under `out_dir` (created if needed): tensor_plan.json, and
 * for each producer with tensors selected, <out_dir>/q4k, /iq, /q5k holding
 * manifest.json, manifest.md and the pack files. `result` receives a JSON
 * object {"tensor_plan": path, "q4k_manifest": path or null, "iq_manifest":
 * ..., "q5k_manifest": ...}. Returns 0; -1 on an error (message in err); -2
 * when result_len is too small (err says how many bytes are needed). `options`
 * may be NULL (auto policy, no blocks, every tensor). */
int rtxllm_gguf_pack(const char* gguf_path, const char* out_dir, const rtxllm_pack_options* options,
                     char* result, size_t result_len, char* err, size_t err_len);

/* The reference producers' pack_tensor: one tensor-plan row (a JSON object
 * with name, type, dimensions, absolute_offset, span_bytes) of the file at
 * model_path (any file: the row says where the bytes are) -> its pack files in
 * out_dir and its manifest record (JSON, indent 2) in `record`. q4k_policy as
 * in rtxllm_pack_options (Q4_K rows only). Returns 0, -1 (err) or -2 (record
 * too small). */
int rtxllm_pack_tensor(const char* model_path, const char* tensor_json, const char* out_dir, const char* q4k_policy,
                       int write_blocks, char* record, size_t record_len, char* err, size_t err_len);

/* The tensor plan of a GGUF file (tensor_plan.json's document) as JSON. */
int rtxllm_gguf_tensor_plan(const char* gguf_path, char* plan, size_t plan_len, char* err, size_t err_len);

/* Element count, block count and data bytes of a tensor of GGUF type `type`
 * (F32, F16, Q8_0, Q4_K, Q5_K, IQ2_S, IQ3_S) with the given dimensions
 * (gguf_block_formats.py:25-44): -1 with err for an unknown type, empty
 * dimensions or an element count that is not whole blocks. */
int rtxllm_pack_tensor_shape(const char* type, const uint64_t* dims, uint32_t n_dims, uint64_t* values,
                             uint64_t* blocks, uint64_t* bytes, char* err, size_t err_len);

/* "blk.<layer>.<role>" -> layer and role; other names: layer -1 and the name
 * without a trailing ".weight" (iq_resident_pack.py:47-52). Returns 0, or -2
 * when role_len is too small. */
int rtxllm_pack_tensor_role(const char* name, int* layer, char* role, size_t role_len);

/* The file label of a tensor name (native_harness.py:126-128): runs of
 * characters outside [A-Za-z0-9_.-] become "_", then leading and trailing
 * ".", "_", "-" are dropped; "native" when nothing is left. Returns 0 or -2. */
int rtxllm_pack_sanitize_label(const char* name, char* label, size_t label_len);

#ifdef __cplusplus
}  /* extern "C" */

#include <filesystem>
#include <string>
#include <utility>
#include <vector>

namespace rtxllm {

struct GgufTensorInfo {
  std::string name;
  std::vector<std::uint64_t> dimensions;
  std::uint32_t type_id = 0;
  std::string type;  // ggml type name, or "unknown:<id>"
  std::uint64_t offset = 0;
};

struct GgufHeader {
  std::filesystem::path path;
  std::uint64_t file_size = 0;
  std::uint32_t version = 0;
  std::uint64_t tensor_count = 0;
  std::uint64_t metadata_count = 0;
  std::uint64_t tensor_info_end_offset = 0;
  std::uint64_t tensor_data_offset = 0;
  std::uint64_t alignment = 32;
  std::string architecture;  // general.architecture, when a string
  std::string model_name;    // general.name, when a string
  // every scalar numeric metadata value (integer, float or bool types) by key
  std::vector<std::pair<std::string, double>> numbers;
  std::vector<GgufTensorInfo> tensors;
  // numbers[key], or fallback when absent
  double number(const std::string& key, double fallback) const {
    for (const auto& kv : numbers)
      if (kv.first == key) return kv.second;
    return fallback;
  }
  const GgufTensorInfo* tensor(const std::string& name) const {
    for (const auto& t : tensors)
      if (t.name == name) return &t;
    return nullptr;
  }
};

struct TensorPlanRow {
  std::string name;
  int layer = -1;  // -1: not a blk.<layer>. tensor
  std::uint64_t span_bytes = 0;
  std::uint64_t offset = 0;
  std::uint64_t absolute_offset = 0;
  std::string type;
  std::uint32_t type_id = 0;
  std::vector<std::uint64_t> dimensions;
};

struct PackOptions {
  std::string q4k_policy = "auto";
  bool write_blocks = false;
  std::vector<std::string> types;  // empty: Q4_K, Q5_K, IQ2_S, IQ3_S
  std::vector<std::string> names;  // empty: all
  int layer = -1;
  std::uint64_t limit = 0;
};

struct PackSetPaths {
  std::filesystem::path tensor_plan;
  std::filesystem::path q4k_manifest;  // empty: no Q4_K tensor selected
  std::filesystem::path iq_manifest;
  std::filesystem::path q5k_manifest;
};

// Header, metadata and tensor infos; throws std::runtime_error on a malformed
// or truncated file.
GgufHeader read_gguf_header(const std::filesystem::path& path);
// The tensor plan rows in file-offset order.
std::vector<TensorPlanRow> gguf_tensor_spans(const GgufHeader& header);
std::string sanitize_label(const std::string& name);
void tensor_role(const std::string& name, int& layer, std::string& role);
// Q4_K policy actually used for a rows x cols tensor under `policy`.
std::string resolve_q4k_policy(const std::string& policy, std::uint64_t rows, std::uint64_t cols);
// pack_tensor of the reference producers: writes the pack files, returns the
// manifest record as JSON text.
std::string pack_tensor_record(const std::filesystem::path& model, const TensorPlanRow& row,
                               const std::filesystem::path& out_dir, const std::string& q4k_policy,
                               bool write_blocks);
PackSetPaths pack_gguf(const std::filesystem::path& gguf, const std::filesystem::path& out_dir,
                       const PackOptions& options);

}  // namespace rtxllm
#endif

#endif
