// Error state and version entry points of the C ABI (no HIP calls here).
#include <stdarg.h>
#include <stdio.h>

#include "lsa_abi_common.h"

namespace lsa {

static thread_local char g_error[1024] = "";

int fail(int code, const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_error, sizeof(g_error), fmt, ap);
  va_end(ap);
  return code;
}

void clear_error() { g_error[0] = '\0'; }

}  // namespace lsa

extern "C" int lsa_abi_version(void) { return LSA_ABI_VERSION; }

extern "C" const char* lsa_last_error(void) { return lsa::g_error; }
