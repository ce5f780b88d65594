// Host-side launch of mv_kernel: geometry selection and the format switch,
// shared by the matvec entry points and the layer pipeline's fused matvecs.
#pragma once

#include "mv.cuh"

namespace rtxllm {

inline int num_cus() {
  static int cached = 0;
  if (cached == 0) {
    int dev = 0, n = 0;
    if (hipGetDevice(&dev) == hipSuccess &&
        hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) == hipSuccess && n > 0)
      cached = n;
    else
      cached = 256;
  }
  return cached;
}

// Launch geometry of mv_kernel, from sweeps on MI355X at the 8B decode shapes:
//  * one unit (32 columns) per lane for rows of up to 16384 columns (two
//    beyond), ks = ceil(units / 64) waves per row;
//  * small matrices: nrg = 4 / ks row groups per workgroup (at least 1) and one
//    4-row tile per row group: many small workgroups, every tile in flight;
//  * large matrices (more than 16 waves per CU): persistent workgroups, the
//    grid capped at 16 waves per CU; each row group double-buffers its tiles
//    and the workgroup copies its codebook once.
//  * grouped epilogues (group_rows > 0): a group's tiles over as many row
//    groups as fit in 8 waves (nrg divides the group's tile count) and the rest
//    over consecutive rounds; one group per workgroup, or several in turn when
//    that would exceed the wave budget above.
struct MvGeom {
  int upl;
  unsigned ks, nrg, grid;
};

inline bool mv_geom(int fmt, std::uint32_t rows, std::uint32_t cols, int tile, std::uint32_t group_rows, MvGeom& g) {
  const std::uint32_t units = cols / 32u;
  g.upl = units > 512u ? 2 : 1;
  g.ks = (units + 64u * g.upl - 1u) / (64u * g.upl);
  if (g.ks > static_cast<unsigned>(kMaxKs)) return false;
  const std::uint32_t tiles = (rows + tile - 1) / tile;
  std::uint32_t grid;
  const std::uint32_t max_waves = 16u * static_cast<std::uint32_t>(num_cus());
  if (group_rows > 0u) {
    const std::uint32_t tg = group_rows / static_cast<std::uint32_t>(tile);
    g.nrg = 1u;
    while (2u * g.nrg <= tg && tg % (2u * g.nrg) == 0u && g.ks * 2u * g.nrg <= static_cast<unsigned>(kMaxKs))
      g.nrg *= 2u;
    grid = (tiles + tg - 1u) / tg;
    const std::uint32_t cap = max_waves / (g.ks * g.nrg);
    if (grid > cap && cap > 0u) grid = cap;  // workgroups take several groups in turn
  } else {
    g.nrg = g.ks >= 4u ? 1u : 4u / g.ks;
    grid = (tiles + g.nrg - 1) / g.nrg;
    if (static_cast<std::uint64_t>(grid) * g.ks * g.nrg > max_waves) grid = max_waves / (g.ks * g.nrg);
  }
  g.grid = grid < 1u ? 1u : (grid > 1048576u ? 1048576u : grid);
  return true;
}

template <int FMT, bool SELF, class Epi>
inline hipError_t launch_mv_fmt(const QTensor& w, const XSrc& xs, std::uint32_t row_count, const Epi& epi,
                         hipStream_t stream) {
  constexpr int kT = Epi::kTile;
  // the kernel addresses each stream with 32-bit byte offsets
  const std::uint64_t blocks = static_cast<std::uint64_t>(row_count) * (w.cols / 256u);
  if (blocks * FmtBytes<FMT>::payload > 0xFFFFFFFFull || blocks * FmtBytes<FMT>::meta > 0xFFFFFFFFull)
    return hipErrorInvalidValue;
  MvGeom g;
  if (!mv_geom(FMT, row_count, w.cols, kT, EpiGroupRows<Epi>::value, g)) return hipErrorInvalidValue;
  const dim3 grid(g.grid), block(64u * g.ks * g.nrg);
  if (g.upl == 2) {
    hipLaunchKernelGGL((mv_kernel<FMT, 2, kT, SELF, Epi>), grid, block, 0, stream, w, xs, row_count, g.ks, epi);
  } else {
    hipLaunchKernelGGL((mv_kernel<FMT, 1, kT, SELF, Epi>), grid, block, 0, stream, w, xs, row_count, g.ks, epi);
  }
  return hipGetLastError();
}

template <bool SELF, class Epi>
inline hipError_t launch_mv(int fmt, const QTensor& w, const XSrc& xs, std::uint32_t row_count, const Epi& epi,
                     hipStream_t stream) {
  switch (fmt) {
    case RTXLLM_FMT_Q4K_RAW: return launch_mv_fmt<RTXLLM_FMT_Q4K_RAW, SELF>(w, xs, row_count, epi, stream);
    case RTXLLM_FMT_Q4K_SPLIT_PREDECODED:
      return launch_mv_fmt<RTXLLM_FMT_Q4K_SPLIT_PREDECODED, SELF>(w, xs, row_count, epi, stream);
    case RTXLLM_FMT_Q4K_SPLIT_HALF:
      return launch_mv_fmt<RTXLLM_FMT_Q4K_SPLIT_HALF, SELF>(w, xs, row_count, epi, stream);
    case RTXLLM_FMT_Q4K_SPLIT_COMPACT:
      return launch_mv_fmt<RTXLLM_FMT_Q4K_SPLIT_COMPACT, SELF>(w, xs, row_count, epi, stream);
    case RTXLLM_FMT_Q4K_SPLIT_NATIVE:
      return launch_mv_fmt<RTXLLM_FMT_Q4K_SPLIT_NATIVE, SELF>(w, xs, row_count, epi, stream);
    case RTXLLM_FMT_Q5K: return launch_mv_fmt<RTXLLM_FMT_Q5K, SELF>(w, xs, row_count, epi, stream);
    case RTXLLM_FMT_IQ2S: return launch_mv_fmt<RTXLLM_FMT_IQ2S, SELF>(w, xs, row_count, epi, stream);
    case RTXLLM_FMT_IQ3S: return launch_mv_fmt<RTXLLM_FMT_IQ3S, SELF>(w, xs, row_count, epi, stream);
    case RTXLLM_FMT_Q4K_RAW_PREDECODED:
      return launch_mv_fmt<RTXLLM_FMT_Q4K_RAW_PREDECODED, SELF>(w, xs, row_count, epi, stream);
    default: return hipErrorInvalidValue;
  }
}

}  // namespace rtxllm
