// Error reporting and version query of the C ABI.
#include <stdarg.h>
#include <stdio.h>

#include "common.hpp"

namespace tpw {

static thread_local char g_last_error[512] = "";

void set_error(const char *fmt, ...) {
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(g_last_error, sizeof(g_last_error), fmt, ap);
    va_end(ap);
}

int check_launch(const char *what) {
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) {
        set_error("%s: kernel launch failed: %s", what, hipGetErrorString(e));
        return TPW_ERR_LAUNCH;
    }
    return TPW_OK;
}

}  // namespace tpw

extern "C" const char *tpw_last_error(void) { return tpw::g_last_error; }

extern "C" int tpw_runtime_version(void) { return HIP_VERSION; }
