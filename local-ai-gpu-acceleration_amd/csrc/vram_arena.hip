// VramSuperallocator on HIP: one hipMalloc, named 256-byte aligned sub-arenas.
#include "rtxllm/vram_arena.h"

#include <hip/hip_runtime.h>

#include <algorithm>
#include <sstream>
#include <stdexcept>

namespace rtxllm {
namespace {

void check_hip(hipError_t st, const char* op) {
  if (st == hipSuccess) return;
  std::ostringstream oss;
  oss << op << " failed: " << hipGetErrorString(st);
  throw std::runtime_error(oss.str());
}

__global__ void zero_kernel(uint4* p, std::size_t n16) {
  const uint4 z = make_uint4(0u, 0u, 0u, 0u);
  for (std::size_t i = blockIdx.x * static_cast<std::size_t>(blockDim.x) + threadIdx.x; i < n16;
       i += static_cast<std::size_t>(gridDim.x) * blockDim.x)
    p[i] = z;
}

}  // namespace

VramSuperallocator::VramSuperallocator(VramSuperallocator&& other) noexcept { *this = std::move(other); }

VramSuperallocator& VramSuperallocator::operator=(VramSuperallocator&& other) noexcept {
  if (this == &other) return *this;
  release();
  base_ = other.base_;
  total_bytes_ = other.total_bytes_;
  arenas_ = std::move(other.arenas_);
  other.base_ = nullptr;
  other.total_bytes_ = 0;
  return *this;
}

VramSuperallocator::~VramSuperallocator() { release(); }

std::size_t VramSuperallocator::align_up(std::size_t v) { return (v + kAlignment - 1) & ~(kAlignment - 1); }

void VramSuperallocator::release() noexcept {
  if (base_ != nullptr) (void)hipFree(base_);
  base_ = nullptr;
  total_bytes_ = 0;
  arenas_.clear();
}

void VramSuperallocator::initialize(const std::vector<ArenaSpec>& specs) {
  release();
  if (specs.empty()) throw std::invalid_argument("VramSuperallocator requires at least one arena");
  std::size_t offset = 0;
  std::vector<ArenaView> views;
  views.reserve(specs.size());
  for (const auto& s : specs) {
    if (s.name.empty() || s.bytes == 0) throw std::invalid_argument("arena name and byte size must be non-empty");
    offset = align_up(offset);
    views.push_back(ArenaView{s.name, offset, s.bytes});
    offset += s.bytes;
  }
  const std::size_t total = align_up(offset);
  void* p = nullptr;
  check_hip(hipMalloc(&p, total), "hipMalloc(superpool)");
  base_ = p;
  total_bytes_ = total;
  arenas_ = std::move(views);
}

void VramSuperallocator::reset() {
  if (base_ == nullptr) return;
  reset_async(nullptr);
  check_hip(hipDeviceSynchronize(), "hipDeviceSynchronize(superpool reset)");
}

void VramSuperallocator::reset_async(hipStream_t stream) {
  if (base_ == nullptr) return;
  const std::size_t n16 = total_bytes_ / 16u;  // total is a multiple of 256
  hipLaunchKernelGGL(zero_kernel, dim3(1024), dim3(256), 0, stream, static_cast<uint4*>(base_), n16);
  check_hip(hipGetLastError(), "zero_kernel(superpool)");
}

void* VramSuperallocator::arena_ptr(std::string_view name) const {
  return static_cast<std::uint8_t*>(base_) + arena(name).offset;
}

ArenaView VramSuperallocator::arena(std::string_view name) const {
  const auto it = std::find_if(arenas_.begin(), arenas_.end(), [&](const ArenaView& v) { return v.name == name; });
  if (it == arenas_.end()) throw std::out_of_range("unknown VRAM arena");
  return *it;
}

bool VramSuperallocator::has_arena(std::string_view name) const {
  return std::any_of(arenas_.begin(), arenas_.end(), [&](const ArenaView& v) { return v.name == name; });
}

}  // namespace rtxllm
