// Status strings and the thread-local error detail of the C ABI.
#include "fl_common.hpp"

#include <string.h>

namespace {
thread_local char g_err[512] = "";
}

namespace fl {
void set_error(const char* fmt, ...) {
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(g_err, sizeof(g_err), fmt, ap);
    va_end(ap);
}

int check_launch(const char* kernel) {
    const hipError_t e = hipGetLastError();
    if (e == hipSuccess) return FL_OK;
    set_error("%s: launch failed: %s", kernel, hipGetErrorString(e));
    return FL_ELAUNCH;
}
}  // namespace fl

extern "C" {

int fl_abi_version(void) { return 1; }

const char* fl_strerror(int status) {
    switch (status) {
    case FL_OK: return "ok";
    case FL_EINVAL: return "invalid argument";
    case FL_ELAUNCH: return "kernel launch failed";
    case FL_ESCRATCH: return "scratch buffer too small";
    default: return "unknown status";
    }
}

const char* fl_last_error(void) { return g_err; }

}  // extern "C"
