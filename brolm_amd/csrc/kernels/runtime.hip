// Host-side plumbing shared by every bx_* entry point: error state, device info.
#include "common.h"

#include <map>
#include <mutex>
#include <tuple>
#include <vector>

namespace bx {

static thread_local std::string g_last_error;

void set_error(const std::string& msg) { g_last_error = msg; }

int fail(int code, const std::string& msg) {
    set_error(msg);
    return code;
}

int hip_check(hipError_t e, const char* what) {
    if (e == hipSuccess) return BX_OK;
    set_error(std::string(what) + ": " + hipGetErrorString(e));
    return BX_ELAUNCH;
}

int launch_check(const char* what) { return hip_check(hipGetLastError(), what); }

int num_cus() {
    static std::mutex mu;
    static std::vector<int> cache;
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess) return 256;
    std::lock_guard<std::mutex> lk(mu);
    if ((int)cache.size() <= dev) cache.resize(dev + 1, 0);
    if (cache[dev] == 0) {
        int n = 0;
        if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || n <= 0) n = 256;
        cache[dev] = n;
    }
    return cache[dev];
}

int resident_wgs(const void* fn, int threads, size_t lds) {
    static std::mutex mu;
    static std::map<std::tuple<const void*, int, size_t>, int> cache;
    std::lock_guard<std::mutex> lock(mu);
    const auto key = std::make_tuple(fn, threads, lds);
    auto it = cache.find(key);
    if (it != cache.end()) return it->second;
    int occ = 0;
    if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&occ, fn, threads, lds) != hipSuccess || occ < 1) occ = 1;
    cache.emplace(key, occ);
    return occ;
}

}  // namespace bx

extern "C" {

const char* bx_last_error(void) { return bx::g_last_error.c_str(); }

int bx_abi_version(void) { return 1; }

int bx_device_ok(void) {
    int n = 0;
    if (hipGetDeviceCount(&n) != hipSuccess || n <= 0) return 0;
    hipDeviceProp_t p;
    if (hipGetDeviceProperties(&p, 0) != hipSuccess) return 0;
    return std::string(p.gcnArchName).rfind("gfx950", 0) == 0 ? 1 : 0;
}

}  // extern "C"
