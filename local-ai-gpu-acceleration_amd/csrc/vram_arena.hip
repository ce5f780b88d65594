// The decode runner's VRAM arena: one device allocation carved into named
// sub-arenas at 256-byte boundaries (interface: include/rtxllm/vram_arena.h).
//
// Steps of initialize: plan the layout from the spec list (validation and
// overflow checks, nothing allocated yet), free the previous pool, allocate
// the new one, then publish the views and the name index together. Lookups
// binary-search the index; reset clears with a grid-stride fill kernel.
#include "rtxllm/vram_arena.h"

#include <hip/hip_runtime.h>

#include <algorithm>
#include <limits>
#include <numeric>
#include <stdexcept>
#include <string>
#include <utility>

namespace rtxllm {
namespace {

constexpr std::size_t kSizeMax = std::numeric_limits<std::size_t>::max();

std::runtime_error device_error(const std::string& what, hipError_t st) {
  return std::runtime_error("VRAM arena: " + what + ": " + hipGetErrorName(st) + " (" + hipGetErrorString(st) +
                            ")");
}

// Offsets and total of a spec list, or an exception before anything changes.
struct Layout {
  std::vector<ArenaView> views;
  std::size_t total = 0;
};

std::size_t next_boundary(std::size_t v) {
  constexpr std::size_t a = VramSuperallocator::kAlignment;
  if (v > kSizeMax - (a - 1u)) throw std::invalid_argument("VRAM arena sizes overflow the address range");
  return (v + (a - 1u)) / a * a;
}

Layout plan_layout(const std::vector<ArenaSpec>& specs) {
  if (specs.empty()) throw std::invalid_argument("VramSuperallocator requires at least one arena");
  if (specs.size() > std::numeric_limits<std::uint32_t>::max())
    throw std::invalid_argument("VRAM arena: too many sub-arenas");
  Layout plan;
  plan.views.reserve(specs.size());
  std::size_t end = 0;
  for (const ArenaSpec& spec : specs) {
    if (spec.name.empty() || spec.bytes == 0) throw std::invalid_argument("arena name and byte size must be non-empty");
    const std::size_t at = next_boundary(end);
    if (spec.bytes > kSizeMax - at) throw std::invalid_argument("VRAM arena sizes overflow the address range");
    plan.views.push_back(ArenaView{spec.name, at, spec.bytes});
    end = at + spec.bytes;
  }
  plan.total = next_boundary(end);
  return plan;
}

// Zero `words` 16-byte words from p (grid-stride loop).
__global__ __launch_bounds__(256) void arena_fill_zero(uint4* __restrict__ p, std::size_t words) {
  const std::size_t stride = static_cast<std::size_t>(gridDim.x) * blockDim.x;
  for (std::size_t i = static_cast<std::size_t>(blockIdx.x) * blockDim.x + threadIdx.x; i < words; i += stride)
    p[i] = make_uint4(0u, 0u, 0u, 0u);
}

}  // namespace

// ---- the device block --------------------------------------------------------

VramSuperallocator::DeviceBlock::DeviceBlock(std::size_t bytes) {
  void* p = nullptr;
  const hipError_t st = hipMalloc(&p, bytes);
  if (st != hipSuccess) throw device_error("allocating " + std::to_string(bytes) + " bytes", st);
  ptr_ = p;
  bytes_ = bytes;
}

VramSuperallocator::DeviceBlock::DeviceBlock(DeviceBlock&& other) noexcept
    : ptr_(std::exchange(other.ptr_, nullptr)), bytes_(std::exchange(other.bytes_, 0u)) {}

VramSuperallocator::DeviceBlock& VramSuperallocator::DeviceBlock::operator=(DeviceBlock&& other) noexcept {
  if (this != &other) {
    if (ptr_ != nullptr) (void)hipFree(ptr_);
    ptr_ = std::exchange(other.ptr_, nullptr);
    bytes_ = std::exchange(other.bytes_, 0u);
  }
  return *this;
}

VramSuperallocator::DeviceBlock::~DeviceBlock() {
  if (ptr_ != nullptr) (void)hipFree(ptr_);
}

// ---- the arena -----------------------------------------------------------------

VramSuperallocator::VramSuperallocator(VramSuperallocator&& other) noexcept
    : pool_(std::move(other.pool_)),
      arenas_(std::exchange(other.arenas_, {})),
      by_name_(std::exchange(other.by_name_, {})) {}

VramSuperallocator& VramSuperallocator::operator=(VramSuperallocator&& other) noexcept {
  if (this != &other) {
    pool_ = std::move(other.pool_);
    arenas_ = std::exchange(other.arenas_, {});
    by_name_ = std::exchange(other.by_name_, {});
  }
  return *this;
}

VramSuperallocator::~VramSuperallocator() = default;

void VramSuperallocator::initialize(const std::vector<ArenaSpec>& specs) {
  Layout plan = plan_layout(specs);
  std::vector<std::uint32_t> order(plan.views.size());
  std::iota(order.begin(), order.end(), 0u);
  std::stable_sort(order.begin(), order.end(),
                   [&](std::uint32_t a, std::uint32_t b) { return plan.views[a].name < plan.views[b].name; });
  // the old pool goes first: the new one may need its memory
  pool_ = DeviceBlock();
  arenas_.clear();
  by_name_.clear();
  pool_ = DeviceBlock(plan.total);
  arenas_ = std::move(plan.views);
  by_name_ = std::move(order);
}

void VramSuperallocator::reset() {
  if (pool_.get() == nullptr) return;
  reset_async(nullptr);
  const hipError_t st = hipStreamSynchronize(nullptr);
  if (st != hipSuccess) throw device_error("waiting for the clear", st);
}

void VramSuperallocator::reset_async(hipStream_t stream) {
  if (pool_.get() == nullptr) return;
  const std::size_t words = pool_.size() / 16u;  // the total is a multiple of 256 bytes
  const std::size_t want = (words + 255u) / 256u;
  const unsigned blocks = static_cast<unsigned>(std::min<std::size_t>(want, 2048u));
  hipLaunchKernelGGL(arena_fill_zero, dim3(blocks), dim3(256), 0, stream, static_cast<uint4*>(pool_.get()), words);
  const hipError_t st = hipGetLastError();
  if (st != hipSuccess) throw device_error("launching the clear", st);
}

std::size_t VramSuperallocator::find(std::string_view name) const {
  const auto it = std::lower_bound(by_name_.begin(), by_name_.end(), name, [&](std::uint32_t i, std::string_view n) {
    return std::string_view(arenas_[i].name) < n;
  });
  if (it != by_name_.end() && arenas_[*it].name == name) return *it;
  return arenas_.size();
}

void* VramSuperallocator::arena_ptr(std::string_view name) const {
  const std::size_t i = find(name);
  if (i == arenas_.size()) throw std::out_of_range("unknown VRAM arena");
  return static_cast<std::uint8_t*>(pool_.get()) + arenas_[i].offset;
}

ArenaView VramSuperallocator::arena(std::string_view name) const {
  const std::size_t i = find(name);
  if (i == arenas_.size()) throw std::out_of_range("unknown VRAM arena");
  return arenas_[i];
}

bool VramSuperallocator::has_arena(std::string_view name) const { return find(name) != arenas_.size(); }

}  // namespace rtxllm
