// C-ABI bookkeeping: ABI version and the per-thread last-error message.
#include <stdarg.h>
#include <stdio.h>

#include "ltv_abi_internal.hpp"

namespace ltv {

static thread_local char g_last_error[512] = {0};

void set_error(const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_last_error, sizeof(g_last_error), fmt, ap);
  va_end(ap);
}

}  // namespace ltv

extern "C" int ltv_abi_version(void) { return 11; }

extern "C" const char* ltv_last_error(void) { return ltv::g_last_error; }
