// C ABI plumbing shared by all scan entry points: per-thread error text,
// launch checking and the ABI version.
#include <cstdarg>
#include <cstdio>

#include "common.h"

namespace mogt {

namespace {
thread_local char g_last_error[512] = {0};
}

int set_error(int code, const char* fmt, ...) {
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(g_last_error, sizeof(g_last_error), fmt, ap);
    va_end(ap);
    return code;
}

void clear_error() { g_last_error[0] = '\0'; }

int check_launch(const char* what) {
    const hipError_t e = hipGetLastError();
    if (e != hipSuccess) return set_error(MOGT_E_LAUNCH, "%s: %s", what, hipGetErrorString(e));
    return MOGT_OK;
}

}  // namespace mogt

extern "C" const char* mogt_last_error(void) { return mogt::g_last_error; }

extern "C" int mogt_abi_version(void) { return 2; }
