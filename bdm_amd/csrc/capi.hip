// Library-wide entry points: version and per-thread error reporting.
#include <cstdarg>

#include "bdm_common.h"

namespace bdm {

static thread_local std::string g_last_error;

void set_error(const char *fmt, ...) {
    char buffer[512];
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(buffer, sizeof buffer, fmt, ap);
    va_end(ap);
    g_last_error = buffer;
}

int fail(int code, const char *fmt, ...) {
    char buffer[512];
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(buffer, sizeof buffer, fmt, ap);
    va_end(ap);
    g_last_error = buffer;
    return code;
}

int check_launch(const char *what) {
    hipError_t err = hipGetLastError();
    if (err != hipSuccess) return fail(BDM_ERR_LAUNCH, "%s: %s", what, hipGetErrorString(err));
    return BDM_OK;
}

}  // namespace bdm

extern "C" int bdm_version(void) { return 2; }

extern "C" const char *bdm_last_error_string(void) { return bdm::g_last_error.c_str(); }

extern "C" int64_t bdm_snapshot_rows(int64_t events, int32_t interval) {
    if (events <= 0 || interval <= 0) return 0;
    return events / interval;
}
