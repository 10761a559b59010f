// Library-wide runtime helpers: error slot, device queries, ABI version.
#include <hip/hip_runtime.h>

#include <mutex>
#include <string>

#include "hxq_common.h"

namespace hxq {

static thread_local std::string g_last_error;

void set_error(const std::string &msg) { g_last_error = msg; }
void clear_error() { g_last_error.clear(); }

int device_cu_count() {
    constexpr int kMaxDev = 64;
    static int cache[kMaxDev] = {0};
    static std::mutex mu;
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxDev) return 256;
    std::lock_guard<std::mutex> lock(mu);
    if (cache[dev] == 0) {
        int n = 0;
        if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess ||
            n <= 0)
            n = 256;
        cache[dev] = n;
    }
    return cache[dev];
}

}  // namespace hxq

extern "C" const char *hxq_last_error(void) { return hxq::g_last_error.c_str(); }

extern "C" int hxq_abi_version(void) { return 1; }
