// Host-side error reporting of the C-ABI: a per-thread message that
// jit_last_error() returns, and the status codes of jit_moe.h; and the device's CU count, which
// some launches size their grids by.
#include <hip/hip_runtime.h>

#include <cstdarg>
#include <cstdio>

#include "jit_moe.h"

namespace jit {

static thread_local char g_msg[512] = "";

void set_error(const char *fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_msg, sizeof g_msg, fmt, ap);
  va_end(ap);
}

int fail(int code, const char *fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_msg, sizeof g_msg, fmt, ap);
  va_end(ap);
  return code;
}

int check_launch(const char *what) {
  const hipError_t e = hipGetLastError();
  if (e != hipSuccess) return fail(JIT_ELAUNCH, "%s: launch failed: %s", what, hipGetErrorString(e));
  return JIT_OK;
}

int cu_count() {
  static int cus[64] = {0};
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 256;
  if (cus[dev] <= 0) {
    int n = 0;
    cus[dev] = hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) == hipSuccess && n > 0 ? n : 256;
  }
  return cus[dev];
}

}  // namespace jit

extern "C" const char *jit_last_error(void) { return jit::g_msg; }

extern "C" int jit_version(void) { return 1; }
