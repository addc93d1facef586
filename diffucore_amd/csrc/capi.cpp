// C ABI plumbing: thread-local error messages and the ABI version.
#include <cstdarg>
#include <cstdio>

#include "../../include/diffucore_amd.h"

namespace dc {

static thread_local char g_err[512];

void set_error(const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_err, sizeof(g_err), fmt, ap);
  va_end(ap);
}

void clear_error() { g_err[0] = '\0'; }

}  // namespace dc

extern "C" const char* dc_last_error(void) { return dc::g_err; }

extern "C" int dc_abi_version(void) { return 13; }
