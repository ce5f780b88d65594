// Self-test of the decode runner's VRAM arena (rtxllm::VramSuperallocator in
// librtxllm.so), the interface of the reference's allocator
// (runtime/core/allocator/vram_superallocator.h:25-53).
//
// Without a GPU (or with "--cpu"): spec validation (the thrown types and
// messages), the empty arena's lookups, and a failed allocation leaving the
// arena empty. With a GPU ("--gpu"): the 256-byte layout, name lookup (a
// repeated name resolves to its first spec), moves, reset / reset_async, and
// a rejected spec list leaving a live pool as it was.
// Prints one line per check; exits 0 when all pass, 1 otherwise.
#include <hip/hip_runtime_api.h>

#include <cstdio>
#include <cstring>
#include <functional>
#include <stdexcept>
#include <string>
#include <vector>

#include "rtxllm/vram_arena.h"

namespace {

int failures = 0;

void check(bool ok, const char* what) {
  std::printf("%s %s\n", ok ? "ok  " : "FAIL", what);
  if (!ok) ++failures;
}

template <class E>
bool throws(const std::function<void()>& f, const char* message = nullptr) {
  try {
    f();
  } catch (const E& e) {
    return message == nullptr || std::strcmp(e.what(), message) == 0;
  } catch (...) {
    return false;
  }
  return false;
}

using rtxllm::ArenaSpec;
using rtxllm::VramSuperallocator;

void cpu_checks() {
  VramSuperallocator a;
  check(a.base() == nullptr && a.total_bytes() == 0 && a.arenas().empty(), "a new arena is empty");
  check(throws<std::out_of_range>([&] { (void)a.arena_ptr("kv_pages"); }, "unknown VRAM arena"),
        "arena_ptr of an unknown name throws out_of_range");
  check(throws<std::out_of_range>([&] { (void)a.arena("kv_pages"); }, "unknown VRAM arena"),
        "arena of an unknown name throws out_of_range");
  check(!a.has_arena("kv_pages"), "has_arena is false for an unknown name");
  check(throws<std::invalid_argument>([&] { a.initialize({}); }, "VramSuperallocator requires at least one arena"),
        "no specs: invalid_argument");
  check(throws<std::invalid_argument>([&] { a.initialize({{"", 16}}); },
                                      "arena name and byte size must be non-empty"),
        "an unnamed spec: invalid_argument");
  check(throws<std::invalid_argument>([&] { a.initialize({{"workspace", 16}, {"dma", 0}}); },
                                      "arena name and byte size must be non-empty"),
        "a zero-byte spec: invalid_argument");
  const std::size_t huge = ~static_cast<std::size_t>(0) - 100u;
  check(throws<std::invalid_argument>([&] { a.initialize({{"q4k_payload", 512}, {"iq_payload", huge}}); }),
        "sizes past the address range: invalid_argument");
  check(throws<std::invalid_argument>([&] { a.initialize({{"q4k_payload", huge}}); }),
        "a total past the address range: invalid_argument");
  check(a.base() == nullptr && a.arenas().empty(), "rejected spec lists leave the arena empty");
  a.reset();  // an empty arena: nothing to clear
  a.reset_async(nullptr);
  check(true, "reset of an empty arena is a no-op");
}

void no_device_checks() {
  VramSuperallocator a;
  check(throws<std::runtime_error>([&] { a.initialize({{"workspace", 4096}}); }),
        "no device: the allocation throws runtime_error");
  check(a.base() == nullptr && a.total_bytes() == 0 && a.arenas().empty() && !a.has_arena("workspace"),
        "a failed allocation leaves the arena empty");
}

void gpu_checks() {
  VramSuperallocator a;
  // the reference runner's arena names (main.cpp:3764-3774), one repeated
  a.initialize({{"q4k_payload", 1}, {"q4k_metadata", 300}, {"iq_payload", 256}, {"q4k_payload", 5}, {"kv_pages", 257}});
  const auto& v = a.arenas();
  check(v.size() == 5, "five views");
  check(v[0].offset == 0 && v[1].offset == 256 && v[2].offset == 768 && v[3].offset == 1024 && v[4].offset == 1280,
        "offsets at 256-byte boundaries in spec order");
  check(a.total_bytes() == 1792, "total rounded up to 256 bytes");
  check(reinterpret_cast<std::uintptr_t>(a.base()) % 256u == 0u, "base 256-byte aligned");
  auto* base = static_cast<std::uint8_t*>(a.base());
  check(a.arena_ptr("q4k_payload") == base && a.arena("q4k_payload").bytes == 1,
        "a repeated name resolves to its first spec");
  check(a.arena_ptr("kv_pages") == base + 1280 && a.arena("kv_pages").bytes == 257, "lookup by name");
  check(a.arena("iq_payload").name == "iq_payload" && a.has_arena("q4k_metadata") && !a.has_arena("q4k"),
        "has_arena and arena()");
  check(throws<std::out_of_range>([&] { (void)a.arena_ptr("q4k_payloa"); }, "unknown VRAM arena"),
        "a prefix of a name is unknown");

  // reset: a pattern written over the pool is cleared
  std::vector<std::uint8_t> host(a.total_bytes(), 0xA5u);
  bool ok = hipMemcpy(a.base(), host.data(), host.size(), hipMemcpyHostToDevice) == hipSuccess;
  a.reset();
  ok = ok && hipMemcpy(host.data(), a.base(), host.size(), hipMemcpyDeviceToHost) == hipSuccess;
  bool zero = true;
  for (std::uint8_t b : host) zero = zero && b == 0u;
  check(ok && zero, "reset zeroes the whole pool");
  std::fill(host.begin(), host.end(), 0x3Cu);
  hipStream_t s = nullptr;
  ok = hipStreamCreate(&s) == hipSuccess;
  ok = ok && hipMemcpy(a.base(), host.data(), host.size(), hipMemcpyHostToDevice) == hipSuccess;
  a.reset_async(s);
  ok = ok && hipStreamSynchronize(s) == hipSuccess;
  ok = ok && hipMemcpy(host.data(), a.base(), host.size(), hipMemcpyDeviceToHost) == hipSuccess;
  zero = true;
  for (std::uint8_t b : host) zero = zero && b == 0u;
  check(ok && zero, "reset_async on a stream zeroes the whole pool");
  if (s != nullptr) (void)hipStreamDestroy(s);

  // a rejected spec list leaves the live pool as it was
  check(throws<std::invalid_argument>([&] { a.initialize({{"dma", 0}}); }) && a.base() == base &&
            a.arenas().size() == 5,
        "a rejected spec list keeps the live pool");

  // moves leave the source empty
  VramSuperallocator b(std::move(a));
  check(b.base() == base && b.arenas().size() == 5 && b.arena_ptr("kv_pages") == base + 1280,
        "move construction takes the pool");
  check(a.base() == nullptr && a.total_bytes() == 0 && a.arenas().empty() && !a.has_arena("kv_pages"),
        "the moved-from arena is empty");
  VramSuperallocator c;
  c.initialize({{"workspace", 64}});
  c = std::move(b);
  check(c.base() == base && c.has_arena("iq_payload") && !c.has_arena("workspace"),
        "move assignment replaces the pool");
  check(b.base() == nullptr && b.arenas().empty(), "the moved-from arena is empty after assignment");

  // re-initialize replaces the pool and the names
  c.initialize({{"workspace", 4096}, {"dma", 1}});
  check(c.total_bytes() == 4352 && c.arena("dma").offset == 4096 && !c.has_arena("kv_pages"),
        "initialize replaces an earlier pool");
}

}  // namespace

int main(int argc, char** argv) {
  const bool want_gpu = argc > 1 && std::strcmp(argv[1], "--gpu") == 0;
  cpu_checks();
  int devices = 0;
  if (hipGetDeviceCount(&devices) != hipSuccess) devices = 0;
  if (want_gpu) {
    if (devices == 0) {
      std::printf("FAIL no GPU for --gpu\n");
      return 1;
    }
    gpu_checks();
  } else if (devices == 0) {
    no_device_checks();
  }
  std::printf("%s: %d failure(s)\n", argv[0], failures);
  return failures == 0 ? 0 : 1;
}
