// Error channel and version query of the C ABI (include/dsa_mi355x.h).
#include <hip/hip_runtime.h>

#include <cstdarg>
#include <cstdio>
#include <cstring>

#include "dsa_common.h"

namespace {
thread_local char g_last_error[1024] = "";
}

namespace dsa {

int set_error(int code, const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_last_error, sizeof(g_last_error), fmt, ap);
  va_end(ap);
  return code;
}

int check_launch(const char* what) {
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) {
    return set_error(kHipError, "%s: kernel launch failed: %s", what, hipGetErrorString(e));
  }
  return kOk;
}

int reserve_lds(const void* fn, size_t bytes, std::atomic<int>* per_device, const char* what) {
  int dev = -1;
  const bool cached = hipGetDevice(&dev) == hipSuccess && dev >= 0 && dev < kMaxDevices;
  if (cached && per_device[dev].load(std::memory_order_relaxed) >= (int)bytes) return kOk;
  const hipError_t e = hipFuncSetAttribute(fn, hipFuncAttributeMaxDynamicSharedMemorySize, (int)bytes);
  if (e != hipSuccess)
    return set_error(kHipError, "%s: cannot reserve %zu bytes of LDS: %s", what, bytes, hipGetErrorString(e));
  if (cached) {
    int cur = per_device[dev].load(std::memory_order_relaxed);
    while (cur < (int)bytes && !per_device[dev].compare_exchange_weak(cur, (int)bytes)) {
    }
  }
  return kOk;
}

}  // namespace dsa

extern "C" {

const char* dsa_last_error(void) { return g_last_error; }

void dsa_clear_error(void) { g_last_error[0] = '\0'; }

int dsa_abi_version(void) { return 1; }

}  // extern "C"
