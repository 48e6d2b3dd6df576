// Error reporting and version entry points of libnq_attn.so.
#include <stdarg.h>
#include <stdio.h>

#include "nq_device.hpp"

namespace nq {

static thread_local char g_last_error[512] = "";

int fail(int code, const char *fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_last_error, sizeof(g_last_error), fmt, ap);
  va_end(ap);
  return code;
}

int check_launch(const char *what) {
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return fail(NQ_ELAUNCH, "%s: launch failed: %s", what, hipGetErrorString(e));
  return NQ_OK;
}

int device_cus() {
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

}  // namespace nq

extern "C" int nq_abi_version(void) { return NQ_ABI_VERSION; }

extern "C" const char *nq_last_error(void) { return nq::g_last_error; }
