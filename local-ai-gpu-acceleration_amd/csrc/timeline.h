// Per-wave timestamps of the decode-step kernels, for the profiling build
// (build/librtxllm_timeline.so, compiled with RTXLLM_TIMELINE). In the
// library proper every stamp compiles to nothing.
//
// Lane 0 of a wave stores s_memrealtime (the 100 MHz constant clock, one
// count every 10 ns, shared by every CU) into a fixed slot of a device array:
// region r (one kernel role) holds kTlRegion slots, and each kernel derives a
// wave's slot from its workgroup and wave index, so a later launch of the
// same role overwrites the earlier one's stamps: after one decode step the
// array holds the last layer's kernels. Slot layouts (point p of a wave):
//   kTlAttnPartial  ((kv head * chunks + chunk) * 8 + wave) * 4 + p: entry,
//                   scores done (K and q arrived), weighted V sum done, end
//                   (batch 1 only);
//   kTlAttnCombine  head * 4 + p: entry, records merged, end (batch 1);
//   kTlGateUpMq     (workgroup * 16 + wave) * 8 + p: entry, codebook barrier,
//                   rounds 0 .. 4 done (p = 2 .. 6), end;
//   kTlQkv, kTlResidualIq (o), kTlResidualK (down), kTlLogits (LM head)
//                   (workgroup * waves_max + wave) * 2 + p: entry, end;
//   kTlAttnPartialB ((((seq * kv heads + kv head) * chunks + chunk) * 8 + wave)
//                   * 4 + p (batch launches, points as kTlAttnPartial);
//   kTlCombineB     ((seq * blocks + block) * 2 + wave) * 2 + p: entry, end;
//   the batch matvecs kTlMm* ((panel group * workgroups + workgroup) * 8 +
//                   wave) * 16 + p: entry, codebook barrier passed, RMSNorm
//                   scale ready, tiles 0 .. 11 done (p = 3 .. 14), end;
//   kTlSelfStaged   workgroup * waves_max + wave: a self-staging matvec wave
//                   has staged its activation groups (the kernel's own region
//                   holds its entry and end);
//   kTlRmsStage*    ((seq * blocks + block) * 4 + wave) * 2 + p: entry, end,
//                   after the o projection (groups = 1) and after the down
//                   projection or the embedding (others).
// Regions 0-15 live in layer.hip's copy of the array, 16-31 in batch.hip's:
// each translation unit has its own device array.
#pragma once

#include <type_traits>

#include "common.h"

namespace rtxllm {

enum TlRegion : int {
  kTlAttnPartial = 0,
  kTlAttnCombine = 1,
  kTlGateUpMq = 2,
  kTlQkv = 3,
  kTlResidualIq = 4,
  kTlResidualK = 5,
  kTlLogits = 6,
  kTlAttnPartialB = 7,
  kTlCombineB = 8,
  kTlSelfStaged = 9,
  kTlRegions = 16,  // per translation unit
  kTlMmQkv = 16,
  kTlMmO = 17,
  kTlMmGateUp = 18,
  kTlMmDown = 19,
  kTlMmLogits = 20,
  kTlRmsStageO = 21,
  kTlRmsStageOther = 22,
};
constexpr std::uint32_t kTlRegion = 65536;  // slots per region

#ifdef RTXLLM_TIMELINE
static __device__ unsigned long long g_timeline[kTlRegions * kTlRegion];
// region r of the translation unit's array is r % kTlRegions
__device__ __forceinline__ void tl_stamp(int region, std::uint32_t slot) {
  if (region >= 0 && (threadIdx.x & 63u) == 0u)
    g_timeline[static_cast<std::uint32_t>(region % kTlRegions) * kTlRegion + (slot & (kTlRegion - 1u))] =
        __builtin_amdgcn_s_memrealtime();
}
// Host side: copy / clear one translation unit's array (defined in batch.hip
// for its regions 16-31, used by layer.hip's entry points).
hipError_t timeline_read_batch(unsigned long long* host);
hipError_t timeline_clear_batch();
#else
__device__ __forceinline__ void tl_stamp(int, std::uint32_t) {}
#endif

// The region of an mv_kernel epilogue: E::tl_region(fmt) if it declares one,
// else -1 (not recorded).
template <class E, class = void>
struct TlRegionOf {
  static constexpr int value(int) { return -1; }
};
template <class E>
struct TlRegionOf<E, std::void_t<decltype(E::tl_region(0))>> {
  static constexpr int value(int fmt) { return E::tl_region(fmt); }
};

}  // namespace rtxllm
