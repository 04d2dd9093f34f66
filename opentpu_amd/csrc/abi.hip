// Error reporting and the device-property cache behind the C ABI (include/otpu.h).
#include <cstdarg>
#include <cstdio>

#include "otpu_common.h"

static thread_local char g_err[512] = "";

extern "C" const char* otpu_last_error(void) { return g_err; }
extern "C" int otpu_version(void) { return OTPU_ABI_VERSION; }

int otpu_fail(int code, const char* fmt, ...) {
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(g_err, sizeof g_err, fmt, ap);
    va_end(ap);
    return code;
}

int otpu_launch_check(const char* what) {
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return otpu_fail(OTPU_ELAUNCH, "%s: %s", what, hipGetErrorString(e));
    return OTPU_OK;
}

// compute units of the current device, looked up once per device (the only global state)
int otpu_cu_count() {
    static int cache[64] = {0};
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 256;
    int v = __atomic_load_n(&cache[dev], __ATOMIC_RELAXED);
    if (v == 0) {
        if (hipDeviceGetAttribute(&v, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess
            || v <= 0)
            v = 256;
        __atomic_store_n(&cache[dev], v, __ATOMIC_RELAXED);
    }
    return v;
}
