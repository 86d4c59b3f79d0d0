// Host-side argument validation shared by the C-ABI entry points.
#pragma once

#include <stdio.h>
#include <stdlib.h>

namespace smx {
// Records the validation message for smx_last_error() on the calling thread.
void set_last_error(const char* func, const char* msg);
}  // namespace smx

#define SMX_REQUIRE(cond, msg)                  \
  do {                                          \
    if (!(cond)) {                              \
      smx::set_last_error(__func__, (msg));     \
      return SMX_EINVAL;                        \
    }                                           \
  } while (0)
