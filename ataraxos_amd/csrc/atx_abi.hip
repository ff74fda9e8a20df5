// Library-wide C ABI pieces: error text and ABI version.
#include <stdarg.h>
#include <stdio.h>

#include "atx_common.hpp"

namespace atx {
namespace {
thread_local char g_last_error[512] = {0};
}

void set_error(const char* fmt, ...) {
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(g_last_error, sizeof(g_last_error), fmt, ap);
    va_end(ap);
}

void clear_error() { g_last_error[0] = '\0'; }

}  // namespace atx

extern "C" const char* atx_last_error(void) { return atx::g_last_error; }

extern "C" int atx_abi_version(void) { return ATX_ABI_VERSION; }
