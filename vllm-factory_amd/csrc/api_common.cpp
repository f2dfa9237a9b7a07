// Error reporting and library information for the libvfk C ABI.
#include <stdarg.h>
#include <stdio.h>

#include "../../include/vfk.h"
#include "vfk_host.h"

namespace vfk {

static thread_local char g_last_error[512] = "";

int set_error(int code, const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_last_error, sizeof(g_last_error), fmt, ap);
  va_end(ap);
  return code;
}

void clear_error() { g_last_error[0] = 0; }

}  // namespace vfk

extern "C" int vfk_abi_version(void) { return 19; }

extern "C" const char* vfk_last_error(void) { return vfk::g_last_error; }
