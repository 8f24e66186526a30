// Library-wide C-ABI functions: version and the thread-local last-error string.
#include "edf_abi.hpp"

#include <string.h>

namespace edf {

static thread_local char g_last_error[512] = "";

int set_error(int code, const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_last_error, sizeof(g_last_error), fmt, ap);
  va_end(ap);
  return code;
}

int clear_error() {
  g_last_error[0] = '\0';
  return EDF_OK;
}

}  // namespace edf

extern "C" {

int edf_version(void) { return EDF_ABI_VERSION; }

const char* edf_last_error(void) { return edf::g_last_error; }

}  // extern "C"
