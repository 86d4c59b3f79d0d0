// Library-level entry points of the C ABI: version and error reporting.
#include <stdio.h>

#include "../../../include/smx.h"
#include "smx_abi_util.h"

namespace smx {
namespace {
thread_local char g_last_error[512] = "";
}
void set_last_error(const char* func, const char* msg) {
  snprintf(g_last_error, sizeof(g_last_error), "%s: %s", func, msg);
}
}  // namespace smx

extern "C" int smx_abi_version(void) { return SMX_ABI_VERSION; }

extern "C" const char* smx_last_error(void) { return smx::g_last_error; }
