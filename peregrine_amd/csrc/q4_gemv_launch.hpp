// Launch plumbing for the Q4 GEMV kernel template: one translation unit per
// epilogue instantiates launch_m<EPI, NORM> (q4_gemv_inst_*.hip), so the
// ~200 kernel variants compile in parallel.
#pragma once

#include <stdlib.h>

#include <algorithm>
#include <map>
#include <mutex>
#include <utility>

#include "q4_gemv.hpp"

namespace prg {
namespace gemv_detail {

inline int device_cus() {
  static int cus = [] {
    int dev = 0;
    hipDeviceProp_t prop;
    if (hipGetDevice(&dev) != hipSuccess || hipGetDeviceProperties(&prop, dev) != hipSuccess) return 256;
    return prop.multiProcessorCount;
  }();
  return cus;
}

// Grid size per CU for the persistent GEMV; PEREGRINE_GEMV_BPC overrides it.
inline int gemv_blocks_per_cu() {
  static int bpc = [] {
    const char* e = getenv("PEREGRINE_GEMV_BPC");
    const int v = e ? atoi(e) : 0;
    return v > 0 ? v : 3;
  }();
  return bpc;
}

// Blocks of one kernel instantiation that fit on the device at once
// (occupancy API, cached per kernel and LDS size).
inline int max_resident_blocks(const void* fn, size_t lds) {
  static std::mutex mu;
  static std::map<std::pair<const void*, size_t>, int> cache;
  static int cus = 0;
  std::lock_guard<std::mutex> lock(mu);
  if (cus == 0) {
    int dev = 0;
    hipDeviceProp_t prop;
    if (hipGetDevice(&dev) != hipSuccess || hipGetDeviceProperties(&prop, dev) != hipSuccess) return 1024;
    cus = prop.multiProcessorCount;
  }
  auto key = std::make_pair(fn, lds);
  auto it = cache.find(key);
  if (it != cache.end()) return it->second;
  int per_cu = 0;
  if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, fn, kGemvThreads, lds) != hipSuccess || per_cu < 1)
    per_cu = 1;
  const int total = per_cu * cus;
  cache[key] = total;
  return total;
}

template <int M, int ROWS, int ITERS, int EPI, int NORM, bool TAIL>
int launch_one_t(hipStream_t s, const GemvParams& p, size_t lds) {
  const void* fn = reinterpret_cast<const void*>(&q4_gemv_kernel<M, ROWS, ITERS, EPI, NORM, TAIL>);
  const uint32_t resident = static_cast<uint32_t>(max_resident_blocks(fn, lds));
  // A grid of a few blocks per CU (not the occupancy maximum) gives every
  // wave several groups, so its next group's loads overlap the dequant. For
  // small matrices more waves with partly empty rounds beat fewer full ones
  // (measured: 4096 x 4096 takes 5.5 us at 3 blocks/CU, 6.4 us at 1). With
  // the current kernels decode runs at 621 / 612 / 612 / 611 tok/s with 3 / 4
  // / 5 / 6 blocks per CU (the gate/up kernel's registers cap it at 3 in any
  // case). One 768-thread block per CU (x staged once per CU) spills at
  // K = 12288.
  const uint32_t want = (p.total_groups + kGemvWaves - 1) / kGemvWaves;
  const uint32_t cap = std::min<uint32_t>(resident, static_cast<uint32_t>(device_cus() * gemv_blocks_per_cu()));
  uint32_t blocks = std::max<uint32_t>(1, std::min<uint32_t>(want, cap));
  // per-wave argmax entries must fit the final kernel's kArgmaxMaxWaves
  if (EPI == kEpiArgmax && p.argmax_waves != nullptr)
    blocks = std::min<uint32_t>(blocks, kArgmaxMaxWaves / kGemvWaves);
  hipLaunchKernelGGL((q4_gemv_kernel<M, ROWS, ITERS, EPI, NORM, TAIL>), dim3(blocks), dim3(kGemvThreads), lds, s, p);
  return 0;
}

// K a multiple of 2048 (every model shape) takes the branch-free variant.
template <int M, int ROWS, int ITERS, int EPI, int NORM>
int launch_one(hipStream_t s, const GemvParams& p, size_t lds) {
  if (p.tail_lanes == 64) return launch_one_t<M, ROWS, ITERS, EPI, NORM, false>(s, p, lds);
  return launch_one_t<M, ROWS, ITERS, EPI, NORM, true>(s, p, lds);
}

template <int M, int ROWS, int EPI, int NORM>
int launch_iters(hipStream_t s, const GemvParams& p, int iters, size_t lds) {
  switch (iters) {
    case 1: return launch_one<M, ROWS, 1, EPI, NORM>(s, p, lds);
    case 2: return launch_one<M, ROWS, 2, EPI, NORM>(s, p, lds);
    case 3: return launch_one<M, ROWS, 3, EPI, NORM>(s, p, lds);
    case 4: return launch_one<M, ROWS, 4, EPI, NORM>(s, p, lds);
    case 6: return launch_one<M, ROWS, 6, EPI, NORM>(s, p, lds);
    case 8: return launch_one<M, ROWS, 8, EPI, NORM>(s, p, lds);
    default: return -1;
  }
}

template <int M, int EPI, int NORM>
int launch_rows(hipStream_t s, const GemvParams& p, int rows, int iters, size_t lds) {
  if constexpr (EPI == kEpiArgmax) {
    return launch_iters<M, 8, EPI, NORM>(s, p, iters, lds);
  } else {
    switch (rows) {
      case 1: return launch_iters<M, 1, EPI, NORM>(s, p, iters, lds);
      case 2: return launch_iters<M, 2, EPI, NORM>(s, p, iters, lds);
      case 4: return launch_iters<M, 4, EPI, NORM>(s, p, iters, lds);
      default: return -1;
    }
  }
}

template <int EPI, int NORM>
int launch_m_impl(hipStream_t s, const GemvParams& p, int M, int rows, int iters, size_t lds) {
  if (M == 1) return launch_rows<1, EPI, NORM>(s, p, rows, iters, lds);
  if (M == 2) return launch_rows<2, EPI, NORM>(s, p, rows, iters, lds);
  return -1;
}


}  // namespace gemv_detail

template <int EPI, int NORM>
int launch_m(hipStream_t s, const GemvParams& p, int M, int rows, int iters, size_t lds) {
  return gemv_detail::launch_m_impl<EPI, NORM>(s, p, M, rows, iters, lds);
}

}  // namespace prg
