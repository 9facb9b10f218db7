#pragma once

// Env-gated per-stage timing (reference include/brolm/detail/profile.h:19-69).
// BROLM_PROFILE=1 brackets each stage with sync_all() and accumulates wall
// time; report() prints the table to stderr.  Profiling runs the eager path
// (one kernel group per stage), so its throughput is not the graph's.

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
    Stage stage_;
    std::uint64_t t0_ = 0;
};

}  // namespace brolm::detail::profile
