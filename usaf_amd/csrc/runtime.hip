// Library-wide state: per-thread error text, ABI version, device queries.
#include "common.h"

#include <stdio.h>
#include <string.h>

#include <atomic>

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
  // Up to 64 devices per process; the count never changes for a device.  Each
  // slot is written once with the same value by whichever thread gets there
  // first, so relaxed atomics suffice.
  static std::atomic<int> cached[64];
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 256;
  int n = cached[dev].load(std::memory_order_relaxed);
  if (n == 0) {
    if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || n <= 0) n = 256;
    cached[dev].store(n, std::memory_order_relaxed);
  }
  return n;
}

}  // namespace usaf

extern "C" int usaf_hip_abi_version(void) { return USAF_HIP_ABI_VERSION; }

extern "C" const char* usaf_hip_last_error(void) { return usaf::g_last_error; }

extern "C" int usaf_hip_init(void) {
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess) {
    (void)hipGetLastError();
    return usaf::set_error(USAF_ERR_RUNTIME, "init: no current HIP device");
  }
  (void)usaf::device_cu_count();
  usaf::prepare_gemm_kernels();
  usaf::prepare_sparse_kernels();
  if (int rc = usaf::prepare_noalloc_scratch()) return rc;
  return usaf::clear_error();
}
