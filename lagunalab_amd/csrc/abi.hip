// Library-wide C ABI pieces: version, thread-local error text, device properties.
#include <atomic>

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
  // one slot per device, filled by whichever host thread asks first (every thread computes the
  // same value, so a relaxed atomic store and load are enough)
  static std::atomic<int> cached[64];
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 256;
  int cus = cached[dev].load(std::memory_order_relaxed);
  if (cus == 0) {
    if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess ||
        cus < 1)
      cus = 256;
    cached[dev].store(cus, std::memory_order_relaxed);
  }
  return cus;
}

}  // namespace lq

extern "C" int lq_version(void) { return 100; }

extern "C" const char* lq_last_error(void) { return lq::g_error.c_str(); }
