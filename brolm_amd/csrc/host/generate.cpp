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

namespace {

// softmax(logits / T) with the reference's arithmetic (generate.cpp:68-142):
// FP32 exponentials against the FP32 maximum, their sum in FP64, and one FP32
// reciprocal of that sum applied to every term.
std::vector<float> tempered_probs(const float* logits, int vocab, float temperature) {
    const float inv_t = 1.0f / temperature;
    const float top = inv_t * *std::max_element(logits, logits + vocab, [inv_t](float a, float b) {
        return a * inv_t < b * inv_t;
    });
    std::vector<float> pr(logits, logits + vocab);
    double total = 0.0;
    for (float& v : pr) {
        v = std::exp(v * inv_t - top);
        total += v;
    }
    const float scale = total > 0.0 ? static_cast<float>(1.0 / total) : 0.0f;
    for (float& v : pr) v *= scale;
    return pr;
}

// The candidate ids, most probable first, cut to top_k (0: no cut) and then
// to the shortest prefix whose FP64 running sum reaches top_p (at least one
// id).  Equal probabilities are ordered by id: the reference's std::sort
// leaves their order open, and this is the order its restatement in the test
// oracle uses.
std::vector<int> candidates(const std::vector<float>& pr, int top_k, float top_p) {
    const int V = static_cast<int>(pr.size());
    std::vector<int> ids(pr.size());
    std::iota(ids.begin(), ids.end(), 0);
    auto before = [&pr](int a, int b) {
        const float pa = pr[static_cast<std::size_t>(a)], pb = pr[static_cast<std::size_t>(b)];
        return pa > pb || (pa == pb && a < b);
    };
    const int limit = top_k > 0 && top_k < V ? top_k : V;
    std::partial_sort(ids.begin(), ids.begin() + limit, ids.end(), before);
    ids.resize(static_cast<std::size_t>(limit));
    if (top_p < 1.0f) {
        double run = 0.0;
        std::size_t n = 0;
        while (n < ids.size()) {
            run += pr[static_cast<std::size_t>(ids[n++])];
            if (run >= static_cast<double>(top_p)) break;
        }
        ids.resize(std::max<std::size_t>(n, 1));
    }
    return ids;
}

}  // namespace

int sample_token(const float* logits, int vocab, const SamplingParams& p, std::mt19937_64& rng) {
    profile::ScopedStage ps(profile::Stage::sample);
    if (vocab <= 0) return 0;
    if (p.temperature <= 0.0f || p.top_k == 1) return argmax(logits, vocab);
    const std::vector<float> pr = tempered_probs(logits, vocab, p.temperature);
    const std::vector<int> ids = candidates(pr, p.top_k, p.top_p);
    double mass = 0.0;
    for (int i : ids) mass += pr[static_cast<std::size_t>(i)];
    // a distribution with no mass left takes the first candidate without a draw
    if (mass <= 0.0) return ids.front();
    // one uniform draw in [0, 1) scaled by the kept mass, located against the
    // running sum of the candidates in order
    const double target = std::uniform_real_distribution<double>(0.0, 1.0)(rng) * mass;
    double run = 0.0;
    for (int i : ids) {
        run += pr[static_cast<std::size_t>(i)];
        if (target < run) return i;
    }
    return ids.back();
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
