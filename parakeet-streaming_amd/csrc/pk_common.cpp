// Per-thread error text for the C ABI.
#include "pk_common.h"

namespace pk {

namespace {
thread_local char g_err[512] = {0};
}

int fail(int code, const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  std::vsnprintf(g_err, sizeof(g_err), fmt, ap);
  va_end(ap);
  return code;
}

void clear_error() { g_err[0] = 0; }

}  // namespace pk

extern "C" const char* pk_last_error(void) { return pk::g_err; }

extern "C" int pk_abi_version(void) { return PK_ABI_VERSION; }
