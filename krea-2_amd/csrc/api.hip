// Library-level entry points: version and device check.
#include <string.h>

#include "k2q_common.h"

extern "C" const char* k2q_version(void) { return "k2q 0.1.0 gfx950"; }

extern "C" int k2q_check_device(void) {
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess) return K2Q_EARCH;
  hipDeviceProp_t prop;
  if (hipGetDeviceProperties(&prop, dev) != hipSuccess) return K2Q_EARCH;
  return strncmp(prop.gcnArchName, "gfx950", 6) == 0 ? K2Q_OK : K2Q_EARCH;
}
