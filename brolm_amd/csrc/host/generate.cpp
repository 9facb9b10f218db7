// Sampler and logits download (reference src/detail/generate.cpp:38-142) and
// the Qwen3 binding (src/qwen_generate.cpp:12-17).
#include "brolm/detail/generate.h"

#include <algorithm>
#include <cmath>
#include <mutex>
#include <numeric>

#include "brolm/detail/profile.h"
#include "brolm/qwen_generate.h"
#include "brotensor/runtime.h"
#include "brolm_hip.h"
#include "hip_util.h"

namespace brolm::detail {

namespace {

std::vector<float> download_fp32(const brotensor::Tensor& t) { return t.to_host_vector(); }

// Strict '>' scan: the lowest index wins ties.
int argmax(const float* logits, int vocab) {
    int best = 0;
    float best_v = logits[0];
    for (int i = 1; i < vocab; ++i) {
        if (logits[i] > best_v) {
            best_v = logits[i];
            best = i;
        }
    }
    return best;
}

// The device sampler's workspace and result slot, shared by every call and
// released by brotensor::shutdown().
struct SamplerBuffers {
    std::mutex mu;
    brotensor::Tensor ws, tok;
    void reserve(std::size_t ws_bytes) {
        if (static_cast<std::size_t>(ws.rows) * 4 < ws_bytes)
            ws = brotensor::Tensor::empty_on(brotensor::Device::ROCm, static_cast<int>((ws_bytes + 3) / 4), 1,
                                             brotensor::Dtype::FP32);
        if (tok.rows == 0) tok = brotensor::Tensor::empty_on(brotensor::Device::ROCm, 1, 1, brotensor::Dtype::FP32);
        brotensor::on_shutdown(release);
    }
    static void release();
};
SamplerBuffers& sampler_buffers() {
    static SamplerBuffers* b = new SamplerBuffers();   // outlives every caller, freed by release()
    return *b;
}
void SamplerBuffers::release() {
    SamplerBuffers& b = sampler_buffers();
    std::lock_guard<std::mutex> lk(b.mu);
    b.ws = brotensor::Tensor();
    b.tok = brotensor::Tensor();
}

}  // namespace

std::vector<float> last_row_fp32(const brotensor::Tensor& logits) {
    profile::ScopedStage ps(profile::Stage::logits_download);
    if (logits.rows == 1) return download_fp32(logits);
    const int es = brotensor::dtype_size_bytes(logits.dtype);
    brotensor::Tensor last = brotensor::Tensor::view(
        logits.device,
        static_cast<char*>(logits.data) + static_cast<std::size_t>(logits.rows - 1) * logits.cols * es, 1,
        logits.cols, logits.dtype);
    return download_fp32(last);
}

int sample_token_device(const brotensor::Tensor& logits, const SamplingParams& p, std::mt19937_64& rng) {
    profile::ScopedStage ps(profile::Stage::sample);
    if (is_greedy(p)) {
        const std::vector<float> row = last_row_fp32(logits);
        return argmax(row.data(), logits.cols);
    }
    if (logits.dtype != brotensor::Dtype::FP16 || logits.device != brotensor::Device::ROCm)
        throw std::runtime_error("sample_token_device: logits must be FP16 on the ROCm device");
    std::uniform_real_distribution<double> dist(0.0, 1.0);
    const double u = dist(rng);
    const int V = logits.cols;
    const auto* row = static_cast<const uint16_t*>(logits.data) + static_cast<std::size_t>(logits.rows - 1) * V;
    SamplerBuffers& b = sampler_buffers();
    std::lock_guard<std::mutex> lk(b.mu);
    b.reserve(bx_sample_workspace_bytes(V));
    hipx::bx(bx_sample_f16(row, V, p.temperature, p.top_k, p.top_p, u, static_cast<int32_t*>(b.tok.data), b.ws.data,
                           hipx::stream()),
             "sample_token_device");
    int32_t out = 0;
    hipx::d2h(&out, b.tok.data, sizeof(out));
    return out;
}

int sample_token(const float* logits, int vocab, const SamplingParams& p, std::mt19937_64& rng) {
    profile::ScopedStage ps(profile::Stage::sample);
    if (vocab <= 0) return 0;
    if (p.temperature <= 0.0f || p.top_k == 1) return argmax(logits, vocab);
    const float inv_t = 1.0f / p.temperature;
    float max_logit = logits[0] * inv_t;
    for (int i = 1; i < vocab; ++i) max_logit = std::max(max_logit, logits[i] * inv_t);
    std::vector<float> probs(static_cast<std::size_t>(vocab));
    double sum = 0.0;
    for (int i = 0; i < vocab; ++i) {
        const float e = std::exp(logits[i] * inv_t - max_logit);
        probs[static_cast<std::size_t>(i)] = e;
        sum += e;
    }
    const float norm = sum > 0.0 ? static_cast<float>(1.0 / sum) : 0.0f;
    for (float& v : probs) v *= norm;
    std::vector<int> order(static_cast<std::size_t>(vocab));
    std::iota(order.begin(), order.end(), 0);
    std::sort(order.begin(), order.end(), [&](int a, int b) {
        return probs[static_cast<std::size_t>(a)] > probs[static_cast<std::size_t>(b)];
    });
    std::size_t keep = static_cast<std::size_t>(vocab);
    if (p.top_k > 0 && static_cast<std::size_t>(p.top_k) < keep) keep = static_cast<std::size_t>(p.top_k);
    if (p.top_p < 1.0f) {
        double cum = 0.0;
        std::size_t nucleus = 0;
        for (std::size_t i = 0; i < keep; ++i) {
            cum += probs[static_cast<std::size_t>(order[i])];
            ++nucleus;
            if (cum >= static_cast<double>(p.top_p)) break;
        }
        keep = std::max<std::size_t>(nucleus, 1);
    }
    double kept = 0.0;
    for (std::size_t i = 0; i < keep; ++i) kept += probs[static_cast<std::size_t>(order[i])];
    if (kept <= 0.0) return order[0];
    std::uniform_real_distribution<double> dist(0.0, 1.0);
    const double r = dist(rng) * kept;
    double acc = 0.0;
    for (std::size_t i = 0; i < keep; ++i) {
        acc += probs[static_cast<std::size_t>(order[i])];
        if (r < acc) return order[i];
    }
    return order[keep - 1];
}

}  // namespace brolm::detail

namespace brolm::qwen {

std::vector<int32_t> generate(Qwen3Model& model, const std::vector<int32_t>& prompt_ids, int eos_id,
                              const GenerateOptions& opts) {
    return brolm::detail::generate(model, prompt_ids, eos_id, opts);
}

std::string generate_text(Qwen3Model& model, const Tokenizer& tok, std::string_view prompt,
                          const GenerateOptions& opts) {
    const std::vector<int32_t> ids = tok.encode(prompt);
    return tok.decode(generate(model, ids, tok.eos_id(), opts));
}

}  // namespace brolm::qwen
