// Host-side plumbing shared by the entry points: error reporting, device properties,
// the profiling event ring.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include <cstdarg>
#include <cstdio>

#include "../../include/flashmap_amd.h"

namespace fm {

// Formats the thread's last error and returns `code`.
int fail(int code, const char *fmt, ...) __attribute__((format(printf, 2, 3)));
void clear_error();

// Cached per-device properties.
struct DeviceInfo {
  int cus = 0;
};
int device_info(DeviceInfo *info);  // of the current device

// Records the start/end of a profiled launch on `stream` when profiling is enabled.
void profile_before(hipStream_t stream);
void profile_after(hipStream_t stream);

#define FM_CHECK_HIP(expr)                                                         \
  do {                                                                             \
    hipError_t fm_err_ = (expr);                                                   \
    if (fm_err_ != hipSuccess)                                                     \
      return ::fm::fail(FM_ERR_HIP, "%s failed: %s", #expr, hipGetErrorString(fm_err_)); \
  } while (0)

#define FM_REQUIRE(cond, ...)                                                      \
  do {                                                                             \
    if (!(cond)) return ::fm::fail(FM_ERR_INVALID, __VA_ARGS__);                   \
  } while (0)

}  // namespace fm
