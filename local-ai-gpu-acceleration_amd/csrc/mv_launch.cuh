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
//  * large matrices (more row groups than the chip holds at once): a
//    persistent grid of exactly the workgroups that are resident together
//    (the kernel's occupancy, queried once per instantiation and block size),
//    nrg = 1 for the IQ formats; each row group double-buffers its tiles and
//    the workgroup copies its codebook once;
//  * epilogues with pairwise hand-over (max_waves > 8) on large matrices: as
//    many row groups per workgroup as max_waves allows, one workgroup per
//    resident slot;
//  * grouped epilogues (group_rows > 0): a group's tiles over as many row
//    groups as fit in 8 waves (nrg divides the group's tile count) and the rest
//    over consecutive rounds; one group per workgroup, or several in turn when
//    there are more groups than resident workgroups.
struct MvGeom {
  int upl;
  unsigned ks, nrg, grid;
};

// resident(block_threads) = workgroups of that size resident per CU (0: unknown).
template <class Resident>
inline bool mv_geom(int fmt, std::uint32_t rows, std::uint32_t cols, int tile, std::uint32_t group_rows,
                    std::uint32_t max_waves, Resident resident, MvGeom& g) {
  const std::uint32_t units = cols / 32u;
  g.upl = units > 512u ? 2 : 1;
  g.ks = (units + 64u * g.upl - 1u) / (64u * g.upl);
  if (g.ks > static_cast<unsigned>(kMaxKs)) return false;
  const std::uint32_t tiles = (rows + tile - 1) / tile;
  const std::uint32_t cus = static_cast<std::uint32_t>(num_cus());
  std::uint32_t grid;
  if (group_rows > 0u) {
    const std::uint32_t tg = group_rows / static_cast<std::uint32_t>(tile);
    g.nrg = 1u;
    while (2u * g.nrg <= tg && tg % (2u * g.nrg) == 0u && g.ks * 2u * g.nrg <= static_cast<unsigned>(kMaxKs))
      g.nrg *= 2u;
    grid = (tiles + tg - 1u) / tg;
  } else {
    g.nrg = g.ks >= 4u ? 1u : 4u / g.ks;
    grid = (tiles + g.nrg - 1) / g.nrg;
  }
  const std::uint32_t per_cu = static_cast<std::uint32_t>(resident(64u * g.ks * g.nrg));
  if (per_cu > 0u && grid > per_cu * cus) {
    const std::uint32_t nrg_wide = max_waves / g.ks;
    const std::uint32_t per_cu_wide =
        max_waves > static_cast<std::uint32_t>(kMaxKs) && nrg_wide > g.nrg
            ? static_cast<std::uint32_t>(resident(64u * g.ks * nrg_wide))
            : 0u;
    if (group_rows == 0u && per_cu_wide > 0u) {
      g.nrg = nrg_wide;
      grid = per_cu_wide * cus;
    } else if (group_rows == 0u && fmt_is_iq(fmt) && g.nrg > 1u) {
      g.nrg = 1u;
      const std::uint32_t per_cu1 = static_cast<std::uint32_t>(resident(64u * g.ks));
      grid = (per_cu1 > 0u ? per_cu1 : 1u) * cus;
    } else {
      grid = per_cu * cus;  // workgroups take several tiles / groups in turn
    }
  }
  g.grid = grid < 1u ? 1u : (grid > 1048576u ? 1048576u : grid);
  return true;
}

// Resident workgroups per CU of one mv_kernel instantiation at a block size
// (cached; 0 if the query fails).
template <int FMT, int UPL, int TILE, bool SELF, class Epi>
inline int mv_resident(std::uint32_t block_threads) {
  constexpr std::uint32_t kW = EpiWaves<Epi>::value;
  static int cache[kW + 1] = {};
  const std::uint32_t w = block_threads / 64u;
  if (w == 0u || w > kW) return 0;
  if (cache[w] == 0) {
    int n = 0;
    if (hipOccupancyMaxActiveBlocksPerMultiprocessor(
            &n, reinterpret_cast<const void*>(&mv_kernel<FMT, UPL, TILE, SELF, Epi>),
            static_cast<int>(block_threads), 0) != hipSuccess || n <= 0)
      return 0;
    cache[w] = n;
  }
  return cache[w];
}

template <int FMT, bool SELF, class Epi>
inline bool mv_geometry_fmt(std::uint32_t rows, std::uint32_t cols, MvGeom& g) {
  constexpr int kT = Epi::kTile;
  const std::uint32_t units = cols / 32u;
  auto resident = [units](std::uint32_t threads) {
    return units > 512u ? mv_resident<FMT, 2, kT, SELF, Epi>(threads) : mv_resident<FMT, 1, kT, SELF, Epi>(threads);
  };
  return mv_geom(FMT, rows, cols, kT, EpiGroupRows<Epi>::value, EpiWaves<Epi>::value, resident, g);
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
  if (!mv_geometry_fmt<FMT, SELF, Epi>(row_count, w.cols, g)) return hipErrorInvalidValue;
  const dim3 grid(g.grid), block(64u * g.ks * g.nrg);
  if (g.upl == 2) {
    hipLaunchKernelGGL((mv_kernel<FMT, 2, kT, SELF, Epi>), grid, block, 0, stream, w, xs, row_count, g.ks, epi);
  } else {
    hipLaunchKernelGGL((mv_kernel<FMT, 1, kT, SELF, Epi>), grid, block, 0, stream, w, xs, row_count, g.ks, epi);
  }
  return hipGetLastError();
}

// The geometry launch_mv<SELF, Epi> would use for this format and shape.
template <bool SELF, class Epi>
inline bool mv_geometry(int fmt, std::uint32_t rows, std::uint32_t cols, MvGeom& g) {
  switch (fmt) {
    case RTXLLM_FMT_Q4K_RAW: return mv_geometry_fmt<RTXLLM_FMT_Q4K_RAW, SELF, Epi>(rows, cols, g);
    case RTXLLM_FMT_Q4K_SPLIT_PREDECODED:
      return mv_geometry_fmt<RTXLLM_FMT_Q4K_SPLIT_PREDECODED, SELF, Epi>(rows, cols, g);
    case RTXLLM_FMT_Q4K_SPLIT_HALF: return mv_geometry_fmt<RTXLLM_FMT_Q4K_SPLIT_HALF, SELF, Epi>(rows, cols, g);
    case RTXLLM_FMT_Q4K_SPLIT_COMPACT:
      return mv_geometry_fmt<RTXLLM_FMT_Q4K_SPLIT_COMPACT, SELF, Epi>(rows, cols, g);
    case RTXLLM_FMT_Q4K_SPLIT_NATIVE: return mv_geometry_fmt<RTXLLM_FMT_Q4K_SPLIT_NATIVE, SELF, Epi>(rows, cols, g);
    case RTXLLM_FMT_Q5K: return mv_geometry_fmt<RTXLLM_FMT_Q5K, SELF, Epi>(rows, cols, g);
    case RTXLLM_FMT_IQ2S: return mv_geometry_fmt<RTXLLM_FMT_IQ2S, SELF, Epi>(rows, cols, g);
    case RTXLLM_FMT_IQ2S_UNITS: return mv_geometry_fmt<RTXLLM_FMT_IQ2S_UNITS, SELF, Epi>(rows, cols, g);
    case RTXLLM_FMT_IQ3S_UNITS: return mv_geometry_fmt<RTXLLM_FMT_IQ3S_UNITS, SELF, Epi>(rows, cols, g);
    case RTXLLM_FMT_IQ3S: return mv_geometry_fmt<RTXLLM_FMT_IQ3S, SELF, Epi>(rows, cols, g);
    case RTXLLM_FMT_Q4K_RAW_PREDECODED:
      return mv_geometry_fmt<RTXLLM_FMT_Q4K_RAW_PREDECODED, SELF, Epi>(rows, cols, g);
    default: return false;
  }
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
    case RTXLLM_FMT_IQ2S_UNITS: return launch_mv_fmt<RTXLLM_FMT_IQ2S_UNITS, SELF>(w, xs, row_count, epi, stream);
    case RTXLLM_FMT_IQ3S_UNITS: return launch_mv_fmt<RTXLLM_FMT_IQ3S_UNITS, SELF>(w, xs, row_count, epi, stream);
    case RTXLLM_FMT_IQ3S: return launch_mv_fmt<RTXLLM_FMT_IQ3S, SELF>(w, xs, row_count, epi, stream);
    case RTXLLM_FMT_Q4K_RAW_PREDECODED:
      return launch_mv_fmt<RTXLLM_FMT_Q4K_RAW_PREDECODED, SELF>(w, xs, row_count, epi, stream);
    default: return hipErrorInvalidValue;
  }
}

}  // namespace rtxllm
