// Library-wide C-ABI pieces: the per-thread error message and the ABI version.
#include "me_common.h"

namespace me {

namespace {
thread_local std::string g_last_error;
}

void set_error(const char *fmt, ...) {
    char buf[512];
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(buf, sizeof(buf), fmt, ap);
    va_end(ap);
    g_last_error = buf;
}

int check_launch(const char *what) {
    const hipError_t e = hipGetLastError();
    if (e != hipSuccess) {
        set_error("%s: kernel launch failed: %s", what, hipGetErrorString(e));
        return ME_ERR_HIP;
    }
    return ME_OK;
}

}  // namespace me

extern "C" const char *me_last_error(void) { return me::g_last_error.c_str(); }

extern "C" int me_version(void) { return 2; }
