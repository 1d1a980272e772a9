// Library-level entry points: version and device check; the per-device CU count the launch plans use.
#include <string.h>

#include <atomic>

#include "k2q_common.h"

namespace {
constexpr int kMaxDevices = 64;
std::atomic<int> g_cus[kMaxDevices];   // 0 until the device's first query; written once, read-only afterwards
}  // namespace

int k2q_cu_count() {
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess) return 256;
  if (dev >= 0 && dev < kMaxDevices) {
    const int c = g_cus[dev].load(std::memory_order_relaxed);
    if (c > 0) return c;
  }
  int n = 0;
  if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || n < 1) return 256;
  if (dev >= 0 && dev < kMaxDevices) g_cus[dev].store(n, std::memory_order_relaxed);
  return n;
}

extern "C" const char* k2q_version(void) { return "k2q 0.1.0 gfx950"; }

extern "C" int k2q_check_device(void) {
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess) return K2Q_EARCH;
  hipDeviceProp_t prop;
  if (hipGetDeviceProperties(&prop, dev) != hipSuccess) return K2Q_EARCH;
  return strncmp(prop.gcnArchName, "gfx950", 6) == 0 ? K2Q_OK : K2Q_EARCH;
}
