// ABI version and thread-local error reporting for libntlowbit.so.
#include <stdarg.h>
#include <stdio.h>
#include <string.h>

#include "ntlb_host.h"

namespace ntlb {

static thread_local char g_last_error[512] = "";

void set_error(const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_last_error, sizeof(g_last_error), fmt, ap);
  va_end(ap);
}

void clear_error() { g_last_error[0] = '\0'; }

}  // namespace ntlb

extern "C" int ntlb_abi_version(void) { return NTLB_ABI_VERSION; }

extern "C" const char* ntlb_last_error(void) { return ntlb::g_last_error; }
