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

extern "C" int hxq_abi_version(void) { return HXQ_ABI_VERSION; }

extern "C" int hxq_device_clocks(int32_t *clock_khz, int32_t *mem_clock_khz,
                                 int32_t *bus_width_bits) {
    hxq::clear_error();
    HXQ_REQUIRE(clock_khz && mem_clock_khz && bus_width_bits, "output pointers are required");
    int dev = 0;
    HXQ_HIP_TRY(hipGetDevice(&dev));
    int v = 0;
    HXQ_HIP_TRY(hipDeviceGetAttribute(&v, hipDeviceAttributeClockRate, dev));
    *clock_khz = v;
    HXQ_HIP_TRY(hipDeviceGetAttribute(&v, hipDeviceAttributeMemoryClockRate, dev));
    *mem_clock_khz = v;
    HXQ_HIP_TRY(hipDeviceGetAttribute(&v, hipDeviceAttributeMemoryBusWidth, dev));
    *bus_width_bits = v;
    return HXQ_OK;
}
