// Host-side plumbing shared by every bx_* entry point: error state, device info.
#include <atomic>
#include "common.h"

#include <link.h>

#include <cstdlib>
#include <cstring>
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

// rocprofv3 injects its tool by LD_PRELOAD of librocprofiler-sdk-tool.so and
// names it in ROCP_TOOL_LIBRARIES.  Under that tool, a process whose kernels
// were launched cooperatively, or through a hipGraph, has ended in a host
// segmentation fault in the profiler's exit path; the launch paths consult
// this to take the plain launch and the eager step instead.
static int find_profiler_tool(struct dl_phdr_info* info, size_t, void* hit) {
    if (info->dlpi_name && std::strstr(info->dlpi_name, "librocprofiler-sdk-tool")) {
        *static_cast<int*>(hit) = 1;
        return 1;
    }
    return 0;
}

std::atomic<uint32_t> g_launch_tag{0};

uint32_t next_launch_tag() {
    uint32_t t;
    do t = g_launch_tag.fetch_add(1u, std::memory_order_relaxed) + 1u;
    while (t == 0u);
    return t;
}

bool profiler_attached() {
    static const bool attached = [] {
        const char* t = std::getenv("ROCP_TOOL_LIBRARIES");
        if (t && t[0]) return true;
        int hit = 0;
        dl_iterate_phdr(find_profiler_tool, &hit);
        return hit != 0;
    }();
    return attached;
}

}  // namespace bx

extern "C" {

int bx_profiler_attached(void) { return bx::profiler_attached() ? 1 : 0; }

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
