// pico_amd/csrc/runtime.hip -- status reporting and device queries of the
// launcher layer.
#include <stdarg.h>
#include <stdio.h>
#include <string.h>

#include "pk_common.h"

namespace {
thread_local char g_err[512] = "";
}

namespace pk {

int fail(const char* fmt, ...) {
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(g_err, sizeof(g_err), fmt, ap);
    va_end(ap);
    return PK_EINVAL;
}

int launch_status(const char* what) {
    hipError_t e = hipGetLastError();
    if(e == hipSuccess) return PK_OK;
    snprintf(g_err, sizeof(g_err), "%s: launch failed: %s", what, hipGetErrorString(e));
    return (int)e;
}

}  // namespace pk

extern "C" const char* pk_last_error(void) { return g_err; }

extern "C" int pk_device_info(int* cu_count, int* clock_khz, char* arch, int arch_len) {
    int dev = 0;
    hipError_t e = hipGetDevice(&dev);
    if(e != hipSuccess) return (int)e;
    hipDeviceProp_t prop;
    e = hipGetDeviceProperties(&prop, dev);
    if(e != hipSuccess) return (int)e;
    if(cu_count) *cu_count = prop.multiProcessorCount;
    if(clock_khz) *clock_khz = prop.clockRate;
    if(arch && arch_len > 0) {
        strncpy(arch, prop.gcnArchName, (size_t)arch_len - 1);
        arch[arch_len - 1] = 0;
    }
    return PK_OK;
}
