// Library-wide C ABI pieces: error reporting and version.
#include <cstdarg>
#include <cstdio>

#include "common.hpp"

namespace haste {

static thread_local char g_last_error[1024] = "";

void set_error(const char* fmt, ...) {
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(g_last_error, sizeof(g_last_error), fmt, ap);
    va_end(ap);
}

void clear_error() { g_last_error[0] = '\0'; }

}  // namespace haste

extern "C" const char* haste_last_error(void) { return haste::g_last_error; }

extern "C" int haste_abi_version(void) { return 2; }
