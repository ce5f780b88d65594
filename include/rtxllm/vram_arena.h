/* Resident VRAM arena of the decode runner: one hipMalloc split into named,
 * 256-byte aligned sub-arenas.
 *
 * Keeps the public interface of the reference's VramSuperallocator
 * (runtime/core/allocator/vram_superallocator.h:25-53: initialize, reset,
 * reset_async, base, total_bytes, arenas, arena_ptr, arena; move-only; throws
 * std::invalid_argument for an empty spec list or a spec without a name or
 * bytes, std::out_of_range "unknown VRAM arena" for a name it does not hold,
 * std::runtime_error when the device refuses), so runner code written against
 * it compiles unchanged. The implementation is this library's own:
 *  - the layout is planned (offsets, total, overflow checks) before anything
 *    is allocated, so a rejected spec list leaves the arena as it was;
 *  - the pool is an RAII device block, and moves leave the source empty;
 *  - names are found by binary search over an index sorted by name (the
 *    runner looks regions up per launch); a repeated name resolves to its
 *    first spec, as a front-to-back search would;
 *  - reset_async clears with a fill kernel rather than a memset node, so it
 *    may be captured into a hipGraph. */
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

  /* One hipMalloc of the planned total; every spec needs a name and > 0
   * bytes. Replaces any earlier pool: a spec list that fails validation
   * leaves the arena unchanged, a failed allocation leaves it empty. */
  void initialize(const std::vector<ArenaSpec>& specs);
  /* Zero the whole pool and wait for it. */
  void reset();
  /* Zero the whole pool on `stream` (a fill kernel: capture-safe). */
  void reset_async(hipStream_t stream);

  [[nodiscard]] void* base() const { return pool_.get(); }
  [[nodiscard]] std::size_t total_bytes() const { return pool_.size(); }
  [[nodiscard]] const std::vector<ArenaView>& arenas() const { return arenas_; }
  [[nodiscard]] void* arena_ptr(std::string_view name) const;
  [[nodiscard]] ArenaView arena(std::string_view name) const;
  [[nodiscard]] bool has_arena(std::string_view name) const;

 private:
  // One device allocation, freed when the block is destroyed or replaced.
  class DeviceBlock {
   public:
    DeviceBlock() = default;
    explicit DeviceBlock(std::size_t bytes);
    DeviceBlock(DeviceBlock&& other) noexcept;
    DeviceBlock& operator=(DeviceBlock&& other) noexcept;
    DeviceBlock(const DeviceBlock&) = delete;
    DeviceBlock& operator=(const DeviceBlock&) = delete;
    ~DeviceBlock();
    [[nodiscard]] void* get() const { return ptr_; }
    [[nodiscard]] std::size_t size() const { return bytes_; }

   private:
    void* ptr_ = nullptr;
    std::size_t bytes_ = 0;
  };

  // Position in arenas_ of the first view named `name`, or arenas_.size().
  [[nodiscard]] std::size_t find(std::string_view name) const;

  DeviceBlock pool_;
  std::vector<ArenaView> arenas_;  // in spec order
  std::vector<std::uint32_t> by_name_;  // positions in arenas_, sorted by name (stable)
};

}  // namespace rtxllm

#endif
