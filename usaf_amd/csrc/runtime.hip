// Library-wide state: per-thread error text, ABI version, device queries.
#include "common.h"

#include <stdio.h>
#include <string.h>

namespace usaf {

static thread_local char g_last_error[1024] = {0};

int set_error(int code, const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_last_error, sizeof(g_last_error), fmt, ap);
  va_end(ap);
  return code;
}

int clear_error() {
  g_last_error[0] = 0;
  return USAF_OK;
}

int device_cu_count() {
  // Up to 64 devices per process; the count never changes for a device.
  static int cached[64] = {0};
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 256;
  if (cached[dev] == 0) {
    int n = 0;
    if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || n <= 0) n = 256;
    cached[dev] = n;
  }
  return cached[dev];
}

}  // namespace usaf

extern "C" int usaf_hip_abi_version(void) { return USAF_HIP_ABI_VERSION; }

extern "C" const char* usaf_hip_last_error(void) { return usaf::g_last_error; }
