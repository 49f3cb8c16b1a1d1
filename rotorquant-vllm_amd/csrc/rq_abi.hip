// Library-wide entry points of the C ABI: version and error text.
#include <stdarg.h>

#include "rq_common.h"

namespace rq {

static thread_local char g_err[512] = "";

void set_error(const char *fmt, ...) {
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(g_err, sizeof(g_err), fmt, ap);
    va_end(ap);
}

int check_launch(const char *what) {
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) {
        set_error("%s launch failed: %s", what, hipGetErrorString(e));
        return RQ_ELAUNCH;
    }
    return RQ_OK;
}

}  // namespace rq

extern "C" int rq_abi_version(void) { return RQ_ABI_VERSION; }

extern "C" const char *rq_last_error(void) { return rq::g_err; }
