// Launch helpers shared by the GEMM translation units: per-device launch
// facts (dynamic LDS limit raised, workgroups per CU), the bf16 finite bound
// and the XCD-aware tile order.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include <atomic>

namespace clef {

namespace {

constexpr float kBf16Max = 3.3895313892515355e38f;

// Per-device launch facts of one kernel: whether its dynamic LDS limit has
// been raised (an attribute HIP keeps per device) and how many of its
// workgroups a CU holds. Devices 0..31 are cached, safe to share between host
// threads; any other device is queried on every launch.
struct LaunchCache {
  std::atomic<uint32_t> lds_set{0};
  std::atomic<int> per_cu[32] = {};
};

hipError_t current_device(int& dev) { return hipGetDevice(&dev); }

hipError_t ensure_dynamic_lds(LaunchCache& c, const void* kern, int bytes) {
  int dev = 0;
  if (hipError_t e = current_device(dev)) return e;
  const uint32_t bit = dev >= 0 && dev < 32 ? 1u << dev : 0u;
  if (bit && (c.lds_set.load(std::memory_order_acquire) & bit)) return hipSuccess;
  if (hipError_t e = hipFuncSetAttribute(kern, hipFuncAttributeMaxDynamicSharedMemorySize, bytes)) return e;
  c.lds_set.fetch_or(bit, std::memory_order_release);
  return hipSuccess;
}

// Workgroups per CU (at least 1) and the CU count of the current device.
hipError_t resident_per_cu(LaunchCache& c, const void* kern, int threads, int lds_bytes, int& per_cu, int& cus) {
  int dev = 0;
  if (hipError_t e = current_device(dev)) return e;
  if (hipError_t e = hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev)) return e;
  const bool cached = dev >= 0 && dev < 32;
  per_cu = cached ? c.per_cu[dev].load(std::memory_order_relaxed) : 0;
  if (per_cu > 0) return hipSuccess;
  int nb = 0;
  if (hipError_t e = hipOccupancyMaxActiveBlocksPerMultiprocessor(&nb, kern, threads, lds_bytes)) return e;
  per_cu = nb > 0 ? nb : 1;
  if (cached) c.per_cu[dev].store(per_cu, std::memory_order_relaxed);
  return hipSuccess;
}


// Block -> output tile. Workgroups are dispatched round-robin over the 8
// XCDs (block b runs on XCD b % 8), so block b is renumbered to make each
// XCD's blocks consecutive, then the renumbered order walks 8-tile-tall
// column bands: 32 co-resident blocks of one XCD cover an 8 x 4 patch and
// share its A and B panels in that XCD's L2. 32-bit arithmetic: the
// launchers keep tiles_m * tiles_n below 2^31 (kMaxTiles), and 64-bit
// divisions here cost the persistent kernels registers they spill.
constexpr int64_t kMaxTiles = (int64_t)1 << 30;
__device__ __forceinline__ void tile_of_block(int b, int blocks, int tiles_m, int tiles_n, int& tm, int& tn) {
  const int per = blocks / 8;
  const int r = b < 8 * per ? (b % 8) * per + b / 8 : b;
  const int band = 8 * tiles_n;
  const int group = r / band, within = r - group * band;
  const int first = group * 8;
  const int height = tiles_m - first < 8 ? tiles_m - first : 8;
  tm = first + within % height;
  tn = within / height;
}

}  // namespace

}  // namespace clef
