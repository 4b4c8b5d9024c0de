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

static thread_local DecodeDebug g_decode_debug = {0, 0};

const DecodeDebug& decode_debug() { return g_decode_debug; }

}  // namespace lsa

extern "C" int lsa_abi_version(void) { return LSA_ABI_VERSION; }

extern "C" const char* lsa_last_error(void) { return lsa::g_error; }

extern "C" void lsa_debug_decode(int32_t skip_publish, int32_t spin_limit) {
  lsa::g_decode_debug.skip_publish = skip_publish ? 1 : 0;
  lsa::g_decode_debug.spin_limit = spin_limit > 0 ? spin_limit : 0;
}
