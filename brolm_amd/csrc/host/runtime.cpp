// brotensor runtime: ROCm device registration and the one op stream.
#include "brotensor/runtime.h"

#include <hip/hip_runtime_api.h>

#include <cstring>
#include <mutex>
#include <stdexcept>
#include <string>
#include <vector>

#include "brolm_hip.h"
#include "hip_util.h"

namespace {

struct RuntimeState {
    bool ready = false;
    int device = 0;
    hipStream_t stream = nullptr;
    void* linear_ws = nullptr;           // the linear entry points' workspace, for the op stream
    std::size_t linear_ws_bytes = 0;
    std::vector<void (*)()> releases;   // on_shutdown hooks, registration order
};

RuntimeState& state() {
    static RuntimeState s;
    return s;
}

std::mutex& init_mutex() {
    static std::mutex m;
    return m;
}

}  // namespace

namespace hipx {

hipStream_t stream() {
    if (!state().ready) throw std::runtime_error("brotensor: init() has not been called");
    return state().stream;
}

void sync() { check(hipStreamSynchronize(stream()), "hipStreamSynchronize"); }

void* linear_ws() {
    if (!state().ready) throw std::runtime_error("brotensor: init() has not been called");
    return state().linear_ws;
}
std::size_t linear_ws_bytes() { return state().linear_ws_bytes; }

void h2d(void* dst, const void* src, std::size_t n) {
    if (n == 0) return;
    check(hipMemcpyAsync(dst, src, n, hipMemcpyHostToDevice, stream()), "hipMemcpyAsync H2D");
    sync();
}

void d2h(void* dst, const void* src, std::size_t n) {
    if (n == 0) return;
    check(hipMemcpyAsync(dst, src, n, hipMemcpyDeviceToHost, stream()), "hipMemcpyAsync D2H");
    sync();
}

}  // namespace hipx

namespace brotensor {

void init() {
    std::lock_guard<std::mutex> lk(init_mutex());
    RuntimeState& s = state();
    if (s.ready) return;
    int n = 0;
    if (hipGetDeviceCount(&n) != hipSuccess || n <= 0)
        throw std::runtime_error(
            "brotensor::init: no ROCm device found (this build has no CPU compute backend)");
    int chosen = -1;
    for (int d = 0; d < n; ++d) {
        hipDeviceProp_t p;
        if (hipGetDeviceProperties(&p, d) != hipSuccess) continue;
        if (std::strncmp(p.gcnArchName, "gfx950", 6) == 0) {
            chosen = d;
            break;
        }
    }
    if (chosen < 0) throw std::runtime_error("brotensor::init: no gfx950 (MI355X) device found");
    hipx::check(hipSetDevice(chosen), "hipSetDevice");
    hipStream_t st = nullptr;
    hipx::check(hipStreamCreateWithFlags(&st, hipStreamNonBlocking), "hipStreamCreate");
    // the op stream's linear workspace (split-K partials and counters of the
    // decode-batch GEMVs), taken here once so no op allocates under graph
    // capture
    const std::size_t wsb = bx_linear_workspace_bytes();
    void* ws = nullptr;
    hipx::check(hipMalloc(&ws, wsb), "hipMalloc linear workspace");
    hipx::bx(bx_linear_workspace_init(ws, wsb, st), "linear workspace init");
    hipx::check(hipStreamSynchronize(st), "hipStreamSynchronize");
    s.device = chosen;
    s.stream = st;
    s.linear_ws = ws;
    s.linear_ws_bytes = wsb;
    s.ready = true;
}

bool initialized() { return state().ready; }

Device default_device() { return state().ready ? Device::ROCm : Device::CPU; }

Dtype compute_dtype() { return Dtype::FP16; }

void sync_all() {
    if (state().ready) hipx::sync();
}

void* stream() { return hipx::stream(); }

int device_ordinal() { return state().device; }

void on_shutdown(void (*release)()) {
    std::lock_guard<std::mutex> lk(init_mutex());
    std::vector<void (*)()>& r = state().releases;
    for (void (*f)() : r)
        if (f == release) return;
    r.push_back(release);
}

void shutdown() {
    std::vector<void (*)()> hooks;
    {
        std::lock_guard<std::mutex> lk(init_mutex());
        if (!state().ready) return;
        hooks.swap(state().releases);
    }
    (void)hipStreamSynchronize(state().stream);
    for (auto it = hooks.rbegin(); it != hooks.rend(); ++it) (*it)();
    std::lock_guard<std::mutex> lk(init_mutex());
    RuntimeState& s = state();
    (void)hipStreamSynchronize(s.stream);
    if (s.linear_ws) (void)hipFree(s.linear_ws);
    s.linear_ws = nullptr;
    s.linear_ws_bytes = 0;
    (void)hipStreamDestroy(s.stream);
    s.stream = nullptr;
    s.ready = false;
}

}  // namespace brotensor
