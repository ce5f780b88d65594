/* Resident VRAM arena of the decode runner: one hipMalloc split into named,
 * 256-byte aligned sub-arenas.
 *
 * Keeps the interface of the reference's VramSuperallocator
 * (runtime/core/allocator/vram_superallocator.h:25-53: initialize, reset,
 * reset_async, base, total_bytes, arenas, arena_ptr, arena; move-only; throws
 * std::invalid_argument / std::out_of_range / std::runtime_error), so runner
 * code written against it compiles unchanged. reset_async clears with a fill
 * kernel rather than a memset node, so it may be captured into a hipGraph. */
#ifndef RTXLLM_VRAM_ARENA_H
#define RTXLLM_VRAM_ARENA_H

#include <hip/hip_runtime_api.h>

#include <cstddef>
#include <cstdint>
#include <string>
#include <string_view>
#include <vector>

namespace rtxllm {

struct ArenaSpec {
  std::string name;
  std::size_t bytes = 0;
};

struct ArenaView {
  std::string name;
  std::size_t offset = 0;
  std::size_t bytes = 0;
};

class VramSuperallocator {
 public:
  static constexpr std::size_t kAlignment = 256;

  VramSuperallocator() = default;
  VramSuperallocator(const VramSuperallocator&) = delete;
  VramSuperallocator& operator=(const VramSuperallocator&) = delete;
  VramSuperallocator(VramSuperallocator&& other) noexcept;
  VramSuperallocator& operator=(VramSuperallocator&& other) noexcept;
  ~VramSuperallocator();

  /* One hipMalloc of the aligned sum; every spec needs a name and > 0 bytes. */
  void initialize(const std::vector<ArenaSpec>& specs);
  /* Zero the whole pool and wait. */
  void reset();
  /* Zero the whole pool on `stream` (a fill kernel: capture-safe). */
  void reset_async(hipStream_t stream);

  [[nodiscard]] void* base() const { return base_; }
  [[nodiscard]] std::size_t total_bytes() const { return total_bytes_; }
  [[nodiscard]] const std::vector<ArenaView>& arenas() const { return arenas_; }
  [[nodiscard]] void* arena_ptr(std::string_view name) const;
  [[nodiscard]] ArenaView arena(std::string_view name) const;
  [[nodiscard]] bool has_arena(std::string_view name) const;

 private:
  static std::size_t align_up(std::size_t value);
  void release() noexcept;

  void* base_ = nullptr;
  std::size_t total_bytes_ = 0;
  std::vector<ArenaView> arenas_;
};

}  // namespace rtxllm

#endif
