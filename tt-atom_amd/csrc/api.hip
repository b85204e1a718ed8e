// Library-wide entry points of libttatom_hip: error reporting, version and device checks.
#include <string.h>

#include "common.h"

namespace tta {

static thread_local char g_err[512] = "";

void set_error(const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_err, sizeof(g_err), fmt, ap);
  va_end(ap);
}

}  // namespace tta

// geometry.hip: resolves the allocation-free entry points' device scratch on the current device.
int tta_init_scratch_current_device();

extern "C" const char* tta_last_error(void) { return tta::g_err; }

extern "C" int tta_version(void) { return 1; }

// Verifies that the current device is a gfx950 (MI355X-class) part; the code objects in this
// library are built for gfx950 only.
extern "C" int tta_check_device(char* name_out, int64_t name_len) {
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess) {
    tta::set_error("tta_check_device: no HIP device");
    return tta::kUnsupported;
  }
  hipDeviceProp_t prop;
  if (hipGetDeviceProperties(&prop, dev) != hipSuccess) {
    tta::set_error("tta_check_device: hipGetDeviceProperties failed");
    return tta::kUnsupported;
  }
  if (name_out && name_len > 0) {
    strncpy(name_out, prop.gcnArchName, (size_t)name_len - 1);
    name_out[name_len - 1] = 0;
  }
  if (strncmp(prop.gcnArchName, "gfx950", 6) != 0) {
    tta::set_error("tta_check_device: device %s is not gfx950", prop.gcnArchName);
    return tta::kUnsupported;
  }
  return tta_init_scratch_current_device();
}
