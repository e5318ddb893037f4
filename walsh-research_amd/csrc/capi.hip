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
        DeviceInfo d{256, 65536, 163840};
        int v = 0;
        if (hipDeviceGetAttribute(&v, hipDeviceAttributeMultiprocessorCount, dev) == hipSuccess && v > 0)
            d.cu_count = v;
        if (hipDeviceGetAttribute(&v, hipDeviceAttributeMaxSharedMemoryPerBlock, dev) == hipSuccess && v > 0)
            d.max_shared_per_block = v;
        if (hipDeviceGetAttribute(&v, hipDeviceAttributeMaxSharedMemoryPerMultiprocessor, dev) == hipSuccess && v > 0)
            d.lds_per_cu = v;
        cache[dev] = d;
        valid[dev] = 1;
    }
    return cache[dev];
}

Timing &timing() {
    static Timing t{false, -1, 0, 0, nullptr, nullptr};
    return t;
}

}  // namespace walsh

WALSH_EXPORT int walsh_timing_begin(int capacity) {
    using namespace walsh;
    Timing &t = timing();
    if (capacity < 1 || capacity > (1 << 20)) return set_error(WALSH_EINVAL, "walsh_timing_begin: capacity");
    if (t.cap < capacity) {
        for (int i = 0; i < 2 * t.cap; ++i) (void)hipEventDestroy(t.ev[i]);
        delete[] t.ev;
        delete[] t.tags;
        t.ev = new hipEvent_t[2 * capacity];
        t.tags = new int[capacity];
        for (int i = 0; i < 2 * capacity; ++i) {
            const hipError_t e = hipEventCreate(&t.ev[i]);
            if (e != hipSuccess) {
                for (int j = 0; j < i; ++j) (void)hipEventDestroy(t.ev[j]);
                delete[] t.ev;
                delete[] t.tags;
                t.ev = nullptr;
                t.tags = nullptr;
                t.cap = 0;
                return check_hip(e, "walsh_timing_begin: hipEventCreate");
            }
        }
        t.cap = capacity;
    }
    t.n = 0;
    t.tag = -1;
    t.on = true;
    return WALSH_OK;
}

WALSH_EXPORT void walsh_timing_tag(int tag) { walsh::timing().tag = tag; }

WALSH_EXPORT int walsh_timing_end(int *tags, float *ms, int capacity) {
    using namespace walsh;
    Timing &t = timing();
    t.on = false;
    const int n = t.n < capacity ? t.n : capacity;
    for (int i = 0; i < n; ++i) {
        hipError_t e = hipEventSynchronize(t.ev[2 * i + 1]);
        if (e == hipSuccess) e = hipEventElapsedTime(&ms[i], t.ev[2 * i], t.ev[2 * i + 1]);
        if (e != hipSuccess) return check_hip(e, "walsh_timing_end");
        tags[i] = t.tags[i];
    }
    t.n = 0;
    return n;
}

WALSH_EXPORT int walsh_abi_version(void) { return WALSH_ABI_VERSION; }
WALSH_EXPORT const char *walsh_last_error(void) { return walsh::g_err; }
WALSH_EXPORT const char *walsh_device_arch(void) { return "gfx950"; }
