// Library identity, error reporting and cached device facts.
#include <stdarg.h>
#include <stdio.h>

#include <mutex>
#include <vector>

#include "common.h"

namespace walsh {

static thread_local char g_err[512] = "";

int set_error(int code, const char *fmt, ...) {
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(g_err, sizeof(g_err), fmt, ap);
    va_end(ap);
    return code;
}

int check_hip(hipError_t e, const char *what) {
    if (e == hipSuccess) return WALSH_OK;
    return set_error(WALSH_EHIP, "%s: %s", what, hipGetErrorString(e));
}

const DeviceInfo &device_info() {
    static std::mutex mu;
    static std::vector<DeviceInfo> cache;
    static std::vector<char> valid;
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess) dev = 0;
    std::lock_guard<std::mutex> lock(mu);
    if ((int)cache.size() <= dev) {
        cache.resize(dev + 1);
        valid.resize(dev + 1, 0);
    }
    if (!valid[dev]) {
        DeviceInfo d{256, 65536};
        int v = 0;
        if (hipDeviceGetAttribute(&v, hipDeviceAttributeMultiprocessorCount, dev) == hipSuccess && v > 0)
            d.cu_count = v;
        if (hipDeviceGetAttribute(&v, hipDeviceAttributeMaxSharedMemoryPerBlock, dev) == hipSuccess && v > 0)
            d.max_shared_per_block = v;
        cache[dev] = d;
        valid[dev] = 1;
    }
    return cache[dev];
}

}  // namespace walsh

WALSH_EXPORT int walsh_abi_version(void) { return WALSH_ABI_VERSION; }
WALSH_EXPORT const char *walsh_last_error(void) { return walsh::g_err; }
WALSH_EXPORT const char *walsh_device_arch(void) { return "gfx950"; }
