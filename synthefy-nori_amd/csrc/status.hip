// Thread-local error reporting for the C ABI (nori_last_error) and launch checks.
#include <stdarg.h>
#include <stdio.h>

#include "nori_common.h"

namespace {
thread_local char g_error[512] = {0};
}

namespace nori {

int fail(int code, const char* fmt, ...) {
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(g_error, sizeof(g_error), fmt, ap);
    va_end(ap);
    return code;
}

void clear_error() { g_error[0] = 0; }

int launch_status(const char* what) {
    hipError_t e = hipGetLastError();
    if (e == hipSuccess) return NORI_OK;
    int code = (e == hipErrorOutOfMemory) ? NORI_ERR_OUT_OF_MEMORY : NORI_ERR_RUNTIME;
    return fail(code, "%s: %s", what, hipGetErrorString(e));
}

}  // namespace nori

extern "C" int nori_abi_version(void) { return NORI_ABI_VERSION; }

extern "C" const char* nori_last_error(void) { return g_error; }
