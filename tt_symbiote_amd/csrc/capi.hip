// Error plumbing of the C ABI: one message buffer per calling host thread.
#include "common.h"

namespace {
thread_local char g_error[1024] = "";
}

namespace sym_host {

int set_error(int code, const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_error, sizeof(g_error), fmt, ap);
  va_end(ap);
  return code;
}

int check_launch(const char* what) {
  const hipError_t e = hipGetLastError();
  if (e != hipSuccess) return set_error(SYM_ERR_LAUNCH, "%s: %s", what, hipGetErrorString(e));
  return SYM_OK;
}

int cu_count() {
  static int cus[64] = {0};
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) dev = 0;
  if (cus[dev] <= 0) {
    int n = 0;
    if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess ||
        n <= 0)
      n = 256;
    cus[dev] = n;
  }
  return cus[dev];
}

}  // namespace sym_host

extern "C" const char* sym_last_error(void) { return g_error; }
extern "C" int sym_abi_version(void) { return 2; }
