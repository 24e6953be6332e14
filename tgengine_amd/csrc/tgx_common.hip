// Error reporting and version query of libtgx.
#include "tgx_internal.h"

namespace tgx {

static thread_local char g_last_error[512] = "";

void set_error(const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_last_error, sizeof(g_last_error), fmt, ap);
  va_end(ap);
}

}  // namespace tgx

extern "C" const char* tgx_last_error(void) { return tgx::g_last_error; }

extern "C" int tgx_abi_version(void) { return TGX_ABI_VERSION; }
