// common.hip -- C-ABI error plumbing and device queries.
#include "common.hpp"

#include <cstdarg>

#include "spbitnet_amd.h"

namespace spb {

namespace {
thread_local char g_err[512] = {0};
constexpr int kMaxDevices = 64;
int g_cu_count[kMaxDevices] = {0};
int g_lds_per_cu[kMaxDevices] = {0};
}  // namespace

void set_error(const char* fmt, ...) {
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(g_err, sizeof(g_err), fmt, ap);
    va_end(ap);
}

void clear_error() { g_err[0] = 0; }

const char* last_error() { return g_err; }

int invalid(const char* fmt, ...) {
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(g_err, sizeof(g_err), fmt, ap);
    va_end(ap);
    return static_cast<int>(hipErrorInvalidValue);
}

int launch_status(const char* what) {
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) {
        set_error("%s: launch failed: %s", what, hipGetErrorString(e));
        return static_cast<int>(e);
    }
    return 0;
}

int device_cu_count() {
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxDevices) return 256;
    int n = g_cu_count[dev];
    if (n == 0) {
        if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess ||
            n <= 0)
            n = 256;
        g_cu_count[dev] = n;
    }
    return n;
}

int device_lds_per_cu() {
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxDevices) return 65536;
    int n = g_lds_per_cu[dev];
    if (n == 0) {
        if (hipDeviceGetAttribute(&n, hipDeviceAttributeMaxSharedMemoryPerMultiprocessor, dev) !=
                hipSuccess ||
            n <= 0)
            n = 65536;
        g_lds_per_cu[dev] = n;
    }
    return n;
}

}  // namespace spb

extern "C" int spb_abi_version(void) { return 100; }

extern "C" const char* spb_last_error_string(void) { return spb::last_error(); }
