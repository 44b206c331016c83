// Internal helpers shared by the libxp translation units (not part of the ABI).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include <cstdarg>
#include <cstdio>

#include "../../include/xp.h"

namespace xp {

// Record a failure message for xp_last_error() and return `code`.
int fail(int code, const char* fmt, ...) __attribute__((format(printf, 2, 3)));
// Clear the last error (successful calls do not clear it; the Python side
// only reads it after a non-zero status).
void clear_error();

inline hipStream_t as_stream(void* s) { return reinterpret_cast<hipStream_t>(s); }

// Check the launch that was just enqueued.
int check_launch(const char* what);

// Wall-clock ticks per microsecond of the device's constant clock
// (hipDeviceAttributeWallClockRate), cached per device.
int64_t wallclock_ticks_per_us();

// Device address of the no-alloc expert workspace (scratch.hip) on the
// current device, XP_MOE_SCRATCH_BYTES long; looked up once per device.
int moe_scratch_address(uint8_t** out);

inline bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }
inline bool aligned4(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 3u) == 0; }

}  // namespace xp

#define XP_REQUIRE(cond, ...)                       \
  do {                                              \
    if (!(cond)) return ::xp::fail(XP_E_ARG, __VA_ARGS__); \
  } while (0)

#define XP_HIP(call)                                                          \
  do {                                                                        \
    hipError_t err_ = (call);                                                 \
    if (err_ != hipSuccess)                                                   \
      return ::xp::fail(XP_E_HIP, "%s failed: %s", #call, hipGetErrorString(err_)); \
  } while (0)

// ---- device-side helpers (HIP translation units only) ----
#if defined(__HIP__)
namespace xp {

// Exclusive prefix count of `flag` among the lanes below this one (wave64).
__device__ __forceinline__ unsigned lane_prefix(unsigned long long mask) {
  return __builtin_amdgcn_mbcnt_hi(static_cast<unsigned>(mask >> 32),
                                   __builtin_amdgcn_mbcnt_lo(static_cast<unsigned>(mask), 0u));
}

__device__ __forceinline__ int64_t load_id(const void* p, int elem_bytes, int64_t i) {
  return elem_bytes == 8 ? static_cast<const int64_t*>(p)[i]
                         : static_cast<int64_t>(static_cast<const int32_t*>(p)[i]);
}

// Wave priority by the part of its sequential work a wave has done (done of
// total, uniform over the wave): 3 in the first quarter down to 0 in the
// last. The arbiter issues from the highest priority first and, among
// equal priorities, from the oldest wave. In a kernel whose waves all do
// the same sequential work over several rounds of workgroups, one priority
// lets the first-dispatched workgroups run ahead and the last-dispatched
// finish late, alone, as the CU empties; with the waves that have the most
// left going first, a CU's waves keep the same pace, each round ends
// together and the next one starts full.
__device__ __forceinline__ void progress_priority(int done, int total) {
  const int q = (4 * done) / total;
  if (q == 0)
    __builtin_amdgcn_s_setprio(3);
  else if (q == 1)
    __builtin_amdgcn_s_setprio(2);
  else if (q == 2)
    __builtin_amdgcn_s_setprio(1);
  else
    __builtin_amdgcn_s_setprio(0);
}

}  // namespace xp
#endif  // __HIP__
