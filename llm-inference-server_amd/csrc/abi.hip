// ABI version and the thread-local error string shared by every entry point.
#include <stdarg.h>
#include <stdio.h>

#include "pkv_common.h"

namespace pkv {

static thread_local char g_last_error[512] = "";

int fail(int code, const char* fmt, ...) {
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(g_last_error, sizeof(g_last_error), fmt, ap);
    va_end(ap);
    return code;
}

void clear_error() { g_last_error[0] = '\0'; }

int check_launch(const char* what) {
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return fail(PKV_EHIP, "%s: %s", what, hipGetErrorString(e));
    return PKV_OK;
}

}  // namespace pkv

extern "C" int pkv_abi_version(void) { return PKV_ABI_VERSION; }

extern "C" const char* pkv_last_error(void) { return pkv::g_last_error; }
