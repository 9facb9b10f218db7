// BROLM_PROFILE stage timer on HIP events (the Stage list and the
// enabled / add / reset / report / ScopedStage surface are the reference's,
// include/brolm/detail/profile.h:19-69).
//
// A ScopedStage records an event on the op stream when it opens and another
// when it closes, and queues the pair; it never waits, so profiling does not
// serialise the host with the device.  A stage's time is the device time
// between the stream reaching the two events: for a stage of kernels, the
// time those kernels ran; for a stage that waits on the stream from the host
// (a download, a host-side sample), the span until the host records the
// closing event.  Queued pairs are resolved (hipEventSynchronize on the
// closing event, hipEventElapsedTime) once kResolveAt of them are pending and
// whenever the totals are read.  Events are pooled and released by
// brotensor::shutdown().  Before brotensor::init() (host-only stages) a stage
// is timed on the host clock.
#include "brolm/detail/profile.h"

#include <hip/hip_runtime_api.h>

#include <algorithm>
#include <array>
#include <chrono>
#include <cstdio>
#include <cstdlib>
#include <mutex>
#include <numeric>
#include <string_view>
#include <vector>

#include "brotensor/runtime.h"

namespace brolm::detail::profile {

namespace {

constexpr std::size_t kStages = static_cast<std::size_t>(Stage::COUNT);
constexpr std::array<const char*, kStages> kStageNames = {
    "embed",        "idx_upload", "rms_norm", "qkv_proj",     "qk_norm",          "rope",
    "kv_append",    "attention",  "o_proj",   "mlp_proj",     "swiglu",           "residual_add",
    "final_norm",   "lm_head",    "logits_download", "sample", "other"};
constexpr std::size_t kResolveAt = 4096;

struct Pending {
    Stage stage;
    hipEvent_t open, close;
};

class Timer {
public:
    void add(Stage s, std::uint64_t ns) {
        std::lock_guard<std::mutex> lk(mu_);
        Totals& t = totals_[static_cast<std::size_t>(s)];
        t.ns += ns;
        t.calls += 1;
    }
    // Records the opening event of a device-timed stage; false when the
    // runtime has no stream (host timing then).
    bool open(hipEvent_t& ev) {
        std::lock_guard<std::mutex> lk(mu_);
        if (!brotensor::initialized()) return false;
        ev = take_();
        if (!ev || hipEventRecord(ev, stream_()) != hipSuccess) {
            give_(ev);
            return false;
        }
        return true;
    }
    void close(Stage s, hipEvent_t open_ev) {
        std::lock_guard<std::mutex> lk(mu_);
        hipEvent_t ev = take_();
        if (!brotensor::initialized() || !ev || hipEventRecord(ev, stream_()) != hipSuccess) {
            give_(ev);
            give_(open_ev);
            return;
        }
        pending_.push_back({s, open_ev, ev});
        if (pending_.size() >= kResolveAt) resolve_();
    }
    std::array<std::uint64_t, 2> read(Stage s) {
        std::lock_guard<std::mutex> lk(mu_);
        resolve_();
        const Totals& t = totals_[static_cast<std::size_t>(s)];
        return {t.ns, t.calls};
    }
    void reset() {
        std::lock_guard<std::mutex> lk(mu_);
        resolve_();
        totals_.fill(Totals{});
    }
    void report() {
        std::array<Totals, kStages> t;
        {
            std::lock_guard<std::mutex> lk(mu_);
            resolve_();
            t = totals_;
        }
        const double sum_ms =
            std::accumulate(t.begin(), t.end(), 0.0, [](double a, const Totals& x) { return a + x.ns * 1e-6; });
        if (sum_ms <= 0.0) return;
        std::array<std::size_t, kStages> idx;
        std::iota(idx.begin(), idx.end(), std::size_t{0});
        std::stable_sort(idx.begin(), idx.end(), [&](std::size_t a, std::size_t b) { return t[a].ns > t[b].ns; });
        std::fprintf(stderr, "BROLM_PROFILE (device time between stage events)\n");
        std::fprintf(stderr, "  %-16s %8s %12s %12s %7s\n", "stage", "calls", "ms", "us/call", "share");
        for (std::size_t i : idx) {
            if (t[i].calls == 0) continue;
            const double ms = t[i].ns * 1e-6;
            std::fprintf(stderr, "  %-16s %8llu %12.3f %12.2f %6.1f%%\n", kStageNames[i],
                         static_cast<unsigned long long>(t[i].calls), ms, 1e3 * ms / static_cast<double>(t[i].calls),
                         100.0 * ms / sum_ms);
        }
        std::fprintf(stderr, "  %-16s %8s %12.3f\n", "all stages", "", sum_ms);
    }
    // brotensor::shutdown() hook: drain, fold and destroy every event.
    void release() {
        std::lock_guard<std::mutex> lk(mu_);
        resolve_();
        for (hipEvent_t e : pool_) (void)hipEventDestroy(e);
        pool_.clear();
    }

private:
    struct Totals {
        std::uint64_t ns = 0, calls = 0;
    };
    static hipStream_t stream_() { return static_cast<hipStream_t>(brotensor::stream()); }
    hipEvent_t take_() {
        if (!pool_.empty()) {
            hipEvent_t e = pool_.back();
            pool_.pop_back();
            return e;
        }
        hipEvent_t e = nullptr;
        if (hipEventCreate(&e) != hipSuccess) return nullptr;
        brotensor::on_shutdown(+[] { instance().release(); });
        return e;
    }
    void give_(hipEvent_t e) {
        if (e) pool_.push_back(e);
    }
    void resolve_() {
        for (const Pending& p : pending_) {
            float ms = 0.f;
            if (hipEventSynchronize(p.close) == hipSuccess && hipEventElapsedTime(&ms, p.open, p.close) == hipSuccess) {
                Totals& t = totals_[static_cast<std::size_t>(p.stage)];
                t.ns += static_cast<std::uint64_t>(static_cast<double>(ms) * 1e6);
                t.calls += 1;
            }
            give_(p.open);
            give_(p.close);
        }
        pending_.clear();
    }

public:
    static Timer& instance() {
        static Timer* t = new Timer();   // lives to process end; its events go at shutdown
        return *t;
    }

private:
    std::mutex mu_;
    std::array<Totals, kStages> totals_{};
    std::vector<Pending> pending_;
    std::vector<hipEvent_t> pool_;
};

std::uint64_t host_ns() {
    return static_cast<std::uint64_t>(
        std::chrono::duration_cast<std::chrono::nanoseconds>(std::chrono::steady_clock::now().time_since_epoch())
            .count());
}

}  // namespace

bool enabled() {
    static const bool on = [] {
        const char* env = std::getenv("BROLM_PROFILE");
        const std::string_view v = env ? env : "";
        return !v.empty() && v != "0";
    }();
    return on;
}

void add(Stage s, std::uint64_t ns) { Timer::instance().add(s, ns); }
void reset() { Timer::instance().reset(); }
void report() { Timer::instance().report(); }
std::uint64_t total_ns(Stage s) { return Timer::instance().read(s)[0]; }
std::uint64_t calls(Stage s) { return Timer::instance().read(s)[1]; }

ScopedStage::ScopedStage(Stage s) : stage_(s) {
    if (!enabled()) return;
    hipEvent_t ev = nullptr;
    if (Timer::instance().open(ev)) {
        open_ = ev;
        mode_ = Mode::Device;
    } else {
        t0_ = host_ns();
        mode_ = Mode::Host;
    }
}

ScopedStage::~ScopedStage() {
    if (mode_ == Mode::Device) Timer::instance().close(stage_, static_cast<hipEvent_t>(open_));
    else if (mode_ == Mode::Host) Timer::instance().add(stage_, host_ns() - t0_);
}

}  // namespace brolm::detail::profile
