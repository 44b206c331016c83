// Launch checks, version and pinned host memory of libxp.
#include <hip/hip_runtime.h>

#include <cstdio>
#include <mutex>
#include <unordered_map>

#include "common.h"

namespace xp {

int check_launch(const char* what) {
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return fail(XP_E_HIP, "launch of %s failed: %s", what, hipGetErrorString(e));
  return XP_OK;
}

int64_t wallclock_ticks_per_us() {
  static std::mutex mu;
  static std::unordered_map<int, int64_t> cache;
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess) return 100;
  std::lock_guard<std::mutex> lock(mu);
  auto it = cache.find(dev);
  if (it != cache.end()) return it->second;
  int khz = 0;
  int64_t ticks = 100;  // 100 MHz, the MI300-series constant clock
  if (hipDeviceGetAttribute(&khz, hipDeviceAttributeWallClockRate, dev) == hipSuccess && khz > 0)
    ticks = (khz + 999) / 1000;
  cache[dev] = ticks;
  return ticks;
}

}  // namespace xp

extern "C" {

const char* xp_version(void) { return "libxp 0.1 gfx950"; }

int xp_host_alloc(void** ptr, int64_t bytes, int coherent) {
  XP_REQUIRE(ptr != nullptr && bytes > 0, "xp_host_alloc: bad arguments (bytes=%lld)", (long long)bytes);
  unsigned flags = hipHostMallocMapped | hipHostMallocPortable |
                   (coherent ? hipHostMallocCoherent : hipHostMallocNonCoherent);
  void* p = nullptr;
  hipError_t e = hipHostMalloc(&p, static_cast<size_t>(bytes), flags);
  if (e != hipSuccess)
    return xp::fail(XP_E_HIP, "hipHostMalloc(%lld B, coherent=%d) failed: %s", (long long)bytes, coherent,
                    hipGetErrorString(e));
  *ptr = p;
  return XP_OK;
}

int xp_host_free(void* ptr) {
  if (ptr == nullptr) return XP_OK;
  XP_HIP(hipHostFree(ptr));
  return XP_OK;
}

int xp_host_device_pointer(void** dev, void* host) {
  XP_REQUIRE(dev != nullptr && host != nullptr, "xp_host_device_pointer: null pointer");
  XP_HIP(hipHostGetDevicePointer(dev, host, 0));
  return XP_OK;
}

}  // extern "C"
