#pragma once

// Env-gated per-stage timing (reference include/brolm/detail/profile.h:19-69:
// the Stage list and this surface).  BROLM_PROFILE set to a non-empty value
// other than "0" turns ScopedStage on: it records a HIP event on the op
// stream at each end of the stage and never waits, so the accumulated times
// are device time between those events (kernel time for device stages) and
// the stream is not serialised.  report() prints the table to stderr.
// Profiling runs single-token steps on the per-stage kernels (the fused step
// has no stage boundaries), so its throughput is not the fused step's.
// Thread-safe.

#include <cstdint>

namespace brolm::detail::profile {

enum class Stage : int {
    embed = 0,
    idx_upload,
    rms_norm,
    qkv_proj,
    qk_norm,
    rope,
    kv_append,
    attention,
    o_proj,
    mlp_proj,
    swiglu,
    residual_add,
    final_norm,
    lm_head,
    logits_download,
    sample,
    other,
    COUNT,
};

bool enabled();
void add(Stage s, std::uint64_t ns);
void reset();
void report();
// Accumulated nanoseconds / calls of one stage (for tests and tools).
std::uint64_t total_ns(Stage s);
std::uint64_t calls(Stage s);

class ScopedStage {
public:
    explicit ScopedStage(Stage s);
    ~ScopedStage();
    ScopedStage(const ScopedStage&) = delete;
    ScopedStage& operator=(const ScopedStage&) = delete;

private:
    enum class Mode : std::uint8_t { Off, Device, Host };
    Stage stage_;
    Mode mode_ = Mode::Off;
    void* open_ = nullptr;     // the opening hipEvent_t (Device)
    std::uint64_t t0_ = 0;     // host steady_clock ns at entry (Host: before brotensor::init)
};

}  // namespace brolm::detail::profile
