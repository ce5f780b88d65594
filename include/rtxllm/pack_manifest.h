/* Tensor-pack loaders: the resident-pack manifests written by the pack
 * producers (manifest.json: a "tensors" array of per-tensor records with the
 * pack files' paths, sizes and byte-sum checksums), the GGUF tensor plan they
 * are checked against, and the pack files themselves.
 *
 * Keeps the interface of the reference's loaders
 * (runtime/loaders/q4k_manifest.h:10-69, iq_manifest.h:9-57): the same
 * structs, function names and validation rules -
 *  * Q4_K (q4k_manifest.cpp:352-409): name, rows, cols, payload_path,
 *    metadata_path, source / payload / metadata checksums and payload /
 *    metadata bytes required; cols % 256 == 0; dimensions, when given, equal
 *    [cols, rows]; runtime_kernel defaults to the policy; layer and role come
 *    from a "blk.<layer>.<role>" name (else role = name without ".weight");
 *  * raw blocks (iq_manifest.cpp:355-407): type IQ2_S, IQ3_S or Q5_K;
 *    block_size 256; block_count and payload_bytes non-zero; source_bytes ==
 *    payload_bytes; "layer": null is -1 and an absent layer is 0;
 *  * tensor plan (q4k_manifest.cpp:439-486, iq_manifest.cpp:425-466): every
 *    selected tensor present with the same type, dimensions and span bytes,
 *    and the same absolute offset when both are non-zero.
 * Failures throw std::runtime_error. The JSON reader is a complete
 * recursive-descent parser (strings with every escape, numbers, nesting).
 * Host code, C++17. */
#ifndef RTXLLM_PACK_MANIFEST_H
#define RTXLLM_PACK_MANIFEST_H

#include <cstddef>
#include <cstdint>
#include <filesystem>
#include <string>
#include <vector>

namespace rtxllm {

struct Q4KManifestTensor {
  std::string name;
  int layer = -1;
  std::string role;
  std::vector<std::uint64_t> dimensions;
  std::uint32_t rows = 0;
  std::uint32_t cols = 0;
  std::uint64_t block_count = 0;
  std::uint64_t source_offset = 0;
  std::uint64_t source_bytes = 0;
  std::string policy;
  std::string metadata_format;
  std::string runtime_kernel;
  std::filesystem::path payload_path;
  std::filesystem::path metadata_path;
  std::filesystem::path blocks_path;
  std::uint64_t source_checksum = 0;
  std::uint64_t payload_checksum = 0;
  std::uint64_t metadata_checksum = 0;
  std::uint64_t payload_bytes = 0;
  std::uint64_t metadata_bytes = 0;
  std::uint64_t resident_bytes = 0;
};

struct Q4KManifest {
  std::filesystem::path path;
  std::filesystem::path model;
  std::filesystem::path tensor_plan;
  std::string generated_at;
  std::string policy;
  std::uint64_t tensor_count = 0;
  std::uint64_t payload_bytes = 0;
  std::uint64_t metadata_bytes = 0;
  std::uint64_t resident_bytes = 0;
  std::vector<Q4KManifestTensor> tensors;
};

struct Q4KTensorPlanValidation {
  std::filesystem::path path;
  std::uint64_t checked_tensors = 0;
};

struct IQManifestTensor {
  std::string name;
  std::string type;
  int layer = -1;
  std::string role;
  std::vector<std::uint64_t> dimensions;
  std::uint64_t element_count = 0;
  std::uint64_t block_size = 0;
  std::uint64_t block_type_size = 0;
  std::uint64_t block_count = 0;
  std::uint64_t source_offset = 0;
  std::uint64_t source_bytes = 0;
  std::uint64_t source_checksum = 0;
  std::filesystem::path payload_path;
  std::uint64_t payload_bytes = 0;
  std::uint64_t payload_checksum = 0;
  std::uint64_t resident_bytes = 0;
  std::string policy;
  std::string runtime_kernel;
};

struct IQManifest {
  std::filesystem::path path;
  std::filesystem::path model;
  std::filesystem::path tensor_plan;
  std::string generated_at;
  std::vector<std::string> types;
  std::uint64_t tensor_count = 0;
  std::uint64_t source_bytes = 0;
  std::uint64_t payload_bytes = 0;
  std::uint64_t resident_bytes = 0;
  std::vector<IQManifestTensor> tensors;
};

struct IQTensorPlanValidation {
  std::filesystem::path path;
  std::uint64_t checked_tensors = 0;
};

Q4KManifest load_q4k_manifest(const std::filesystem::path& path);
// The named tensors in that order (each must exist), or the first `limit`
// (0: all) when names is empty.
std::vector<Q4KManifestTensor> select_q4k_tensors(const Q4KManifest& manifest, const std::vector<std::string>& names,
                                                  std::size_t limit);
Q4KTensorPlanValidation validate_q4k_manifest_tensors_against_plan(const std::vector<Q4KManifestTensor>& selected,
                                                                   const std::filesystem::path& tensor_plan_path);

IQManifest load_iq_manifest(const std::filesystem::path& path);
// The named tensor, or the first one when name is empty.
IQManifestTensor select_iq_tensor(const IQManifest& manifest, const std::string& name);
IQTensorPlanValidation validate_iq_manifest_tensors_against_plan(const std::vector<IQManifestTensor>& selected,
                                                                 const std::filesystem::path& tensor_plan_path);

// Sum of the bytes (the producers' checksum).
std::uint64_t byte_checksum(const std::vector<std::uint8_t>& bytes);
// The whole file, which must be exactly expected_bytes long.
std::vector<std::uint8_t> load_binary_file(const std::filesystem::path& path, std::uint64_t expected_bytes,
                                           const char* label);

// Format id (enum rtxllm_format) of a Q4_K pack policy ("split-predecoded",
// "split-half", "split-compact", "split-native"), or -1.
int q4k_policy_format(const std::string& policy);

// Which loader reads a manifest: its "path" field names the producer
// ("q4k_resident_pack"; "iq_resident_pack" or "q5k_resident_pack" for raw
// blocks); without one, Q4_K records carry "metadata_path" and raw-block
// records "type". Throws when neither tells.
enum class PackManifestKind { Q4K, RawBlocks };
PackManifestKind pack_manifest_kind(const std::filesystem::path& path);

}  // namespace rtxllm

#endif
