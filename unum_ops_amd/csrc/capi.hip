// Error reporting and version entry points of the C ABI.
#include "common.h"

namespace unum {

static thread_local char g_last_error[512] = {0};

void set_error(const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_last_error, sizeof(g_last_error), fmt, ap);
  va_end(ap);
}

void clear_error() { g_last_error[0] = '\0'; }

}  // namespace unum

extern "C" const char* unum_last_error(void) { return unum::g_last_error; }

extern "C" int unum_abi_version(void) { return UNUM_ABI_VERSION; }
