// BROLM_PROFILE stage timer (reference src/detail/profile.cpp).
#include "brolm/detail/profile.h"

#include <algorithm>
#include <array>
#include <chrono>
#include <cstdio>
#include <cstdlib>

#include "brotensor/runtime.h"

namespace brolm::detail::profile {

namespace {

constexpr int kStages = static_cast<int>(Stage::COUNT);
constexpr const char* kNames[kStages] = {"embed",    "idx_upload", "rms_norm",     "qkv_proj",   "qk_norm",
                                         "rope",     "kv_append",  "attention",    "o_proj",     "mlp_proj",
                                         "swiglu",   "residual_add", "final_norm", "lm_head",    "logits_download",
                                         "sample",   "other"};

struct Accum {
    std::uint64_t ns = 0, calls = 0;
};
std::array<Accum, kStages> g_acc;

std::uint64_t now_ns() {
    return static_cast<std::uint64_t>(std::chrono::duration_cast<std::chrono::nanoseconds>(
                                          std::chrono::steady_clock::now().time_since_epoch())
                                          .count());
}

}  // namespace

bool enabled() {
    static const bool on = [] {
        const char* v = std::getenv("BROLM_PROFILE");
        return v != nullptr && *v != '\0' && !(v[0] == '0' && v[1] == '\0');
    }();
    return on;
}

void add(Stage s, std::uint64_t ns) {
    Accum& a = g_acc[static_cast<std::size_t>(s)];
    a.ns += ns;
    a.calls += 1;
}

void reset() { g_acc.fill(Accum{}); }

std::uint64_t total_ns(Stage s) { return g_acc[static_cast<std::size_t>(s)].ns; }
std::uint64_t calls(Stage s) { return g_acc[static_cast<std::size_t>(s)].calls; }

void report() {
    std::uint64_t total = 0;
    for (const Accum& a : g_acc) total += a.ns;
    if (total == 0) return;
    std::array<int, kStages> order{};
    for (int i = 0; i < kStages; ++i) order[static_cast<std::size_t>(i)] = i;
    std::sort(order.begin(), order.end(),
              [](int a, int b) { return g_acc[static_cast<std::size_t>(a)].ns > g_acc[static_cast<std::size_t>(b)].ns; });
    std::fprintf(stderr, "[brolm profile] %-16s %10s %10s %12s %6s\n", "stage", "total ms", "calls", "us/call", "%");
    for (int i : order) {
        const Accum& a = g_acc[static_cast<std::size_t>(i)];
        if (a.calls == 0) continue;
        std::fprintf(stderr, "[brolm profile] %-16s %10.2f %10llu %12.2f %5.1f%%\n", kNames[i],
                     static_cast<double>(a.ns) / 1e6, static_cast<unsigned long long>(a.calls),
                     static_cast<double>(a.ns) / 1e3 / static_cast<double>(a.calls),
                     100.0 * static_cast<double>(a.ns) / static_cast<double>(total));
    }
    std::fprintf(stderr, "[brolm profile] %-16s %10.2f\n", "TOTAL", static_cast<double>(total) / 1e6);
}

ScopedStage::ScopedStage(Stage s) : stage_(s) {
    if (!enabled()) return;
    brotensor::sync_all();
    t0_ = now_ns();
}

ScopedStage::~ScopedStage() {
    if (t0_ == 0) return;
    brotensor::sync_all();
    add(stage_, now_ns() - t0_);
}

}  // namespace brolm::detail::profile
