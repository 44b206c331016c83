// The static workspace of xp_moe_experts_noalloc, in a translation unit of
// its own. It holds no kernel, so its code object (and with it the array)
// is loaded on a device only when its address is first asked for, not when
// the expert kernels of moe.hip load; processes that never call the no-alloc
// entry point do not give up the array's memory.
#include <mutex>

#include "common.h"

// One copy on every device the library runs on, held until the process
// ends. Host code never passes this name to a kernel: it stands for the
// host-side shadow, and each device's own address comes from
// hipGetSymbolAddress (moe_scratch_address).
static __device__ __align__(256) uint8_t scratch[XP_MOE_SCRATCH_BYTES];

namespace xp {
namespace {

constexpr int kMaxDevices = 64;
std::mutex g_scratch_mu;
uint8_t* g_scratch[kMaxDevices];  // device address of `scratch`, per device

}  // namespace

int moe_scratch_address(uint8_t** out) {
  int dev = -1;
  XP_HIP(hipGetDevice(&dev));
  XP_REQUIRE(dev >= 0 && dev < kMaxDevices, "xp_moe_experts_noalloc: device %d (at most %d devices)", dev,
             kMaxDevices);
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (g_scratch[dev] == nullptr) {
    void* p = nullptr;
    const hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess || p == nullptr)
      return fail(XP_E_HIP, "xp_moe_experts_noalloc: hipGetSymbolAddress(scratch) on device %d failed: %s", dev,
                  hipGetErrorString(e));
    g_scratch[dev] = static_cast<uint8_t*>(p);
  }
  *out = g_scratch[dev];
  return XP_OK;
}

}  // namespace xp
