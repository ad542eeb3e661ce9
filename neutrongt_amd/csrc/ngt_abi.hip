// Error reporting and version query shared by every entry point.
#include <stdarg.h>
#include <stdio.h>

#include "ngt_common.h"

namespace ngt {
namespace {
thread_local char g_last_error[512] = "";
}

int set_error(int code, const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_last_error, sizeof(g_last_error), fmt, ap);
  va_end(ap);
  return code;
}

}  // namespace ngt

extern "C" int ngt_abi_version(void) { return NGT_ABI_VERSION; }

extern "C" const char* ngt_last_error(void) { return ngt::g_last_error; }
