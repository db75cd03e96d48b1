// Error reporting and version entry points of libkvc.
#include <cstdarg>

#include "kvc_internal.h"

namespace kvc {

namespace {
thread_local char g_last_error[512] = "";
}

void set_error(const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_last_error, sizeof(g_last_error), fmt, ap);
  va_end(ap);
}

void clear_error() { g_last_error[0] = '\0'; }

}  // namespace kvc

extern "C" const char* kvc_last_error(void) { return kvc::g_last_error; }

extern "C" int kvc_abi_version(void) { return 2; }
