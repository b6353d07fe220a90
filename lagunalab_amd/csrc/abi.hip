// Library-wide C ABI pieces: version, thread-local error text, device properties.
#include "common.h"

namespace lq {

namespace {
thread_local std::string g_error;
}

void set_error(const char* fmt, ...) {
  char buf[512];
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(buf, sizeof(buf), fmt, ap);
  va_end(ap);
  g_error = buf;
}

void clear_error() { g_error.clear(); }

int device_cu_count() {
  static int cached[64] = {0};
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 256;
  if (cached[dev] == 0) {
    int cus = 0;
    if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess ||
        cus < 1)
      cus = 256;
    cached[dev] = cus;
  }
  return cached[dev];
}

}  // namespace lq

extern "C" int lq_version(void) { return 100; }

extern "C" const char* lq_last_error(void) { return lq::g_error.c_str(); }
