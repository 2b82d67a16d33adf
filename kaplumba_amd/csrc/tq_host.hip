// Host-side plumbing of the C ABI: error reporting, version, sizes.
#include <cstdarg>
#include <cstring>

#include "tq_common.h"

namespace tq {

static thread_local char g_last_error[512] = "";

void set_error(const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_last_error, sizeof(g_last_error), fmt, ap);
  va_end(ap);
}

int fail(int code, const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_last_error, sizeof(g_last_error), fmt, ap);
  va_end(ap);
  return code;
}

int check_launch(const char* what) {
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return fail(TQ_ERR_HIP, "%s: %s", what, hipGetErrorString(e));
  return TQ_OK;
}

int device_cu_count() {
  static thread_local int cached_dev = -1;
  static thread_local int cached_cus = 0;
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess) return 256;
  if (dev != cached_dev) {
    int cus = 0;
    if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess ||
        cus <= 0)
      cus = 256;
    cached_dev = dev;
    cached_cus = cus;
  }
  return cached_cus;
}

}  // namespace tq

extern "C" {

const char* tq_version(void) { return "kaplumba_tq 0.1.0 gfx950"; }

const char* tq_last_error(void) { return tq::g_last_error; }

int tq_packed_width(int dim, int bits) {
  if (dim <= 0 || bits <= 0) return 0;
  return (dim * bits + 31) / 32;
}

}  // extern "C"
