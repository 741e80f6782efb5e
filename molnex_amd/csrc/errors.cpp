// Thread-local last-error message for the C ABI.
#include <stdarg.h>
#include <stdio.h>

#include "common.h"

namespace mnx {

static thread_local char g_msg[1024] = "";

int set_error(int code, const char* fmt, ...) {
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(g_msg, sizeof(g_msg), fmt, ap);
    va_end(ap);
    return code;
}

void clear_error() { g_msg[0] = '\0'; }

}  // namespace mnx

extern "C" {
const char* mnx_last_error(void) { return mnx::g_msg; }
int mnx_abi_version(void) { return 1; }
}
