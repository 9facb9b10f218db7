#pragma once

// Sampler + autoregressive loop (reference include/brolm/detail/generate.h:29-123,
// src/detail/generate.cpp).  Greedy generation (temperature <= 0 or top_k == 1)
// on a model with a device decode step runs the argmax on the device and keeps
// the next token there; the token ids produced are the same as the host loop's
// (same FP16 logits, same lowest-index tie rule).

#include <cstdint>
#include <random>
#include <string>
#include <vector>

#include "brotensor/tensor.h"

namespace brolm::detail {

struct SamplingParams {
    float temperature = 1.0f;  // <= 0 => greedy
    int top_k = 0;             // 0 => disabled
    float top_p = 1.0f;        // >= 1 => disabled
    uint64_t seed = 0;
};

int sample_token(const float* logits, int vocab, const SamplingParams& p, std::mt19937_64& rng);
// sample_token on the device for the last row of FP16 device logits: the same
// RNG draw, only the chosen id is downloaded (greedy: host argmax of the row).
int sample_token_device(const brotensor::Tensor& logits, const SamplingParams& p, std::mt19937_64& rng);
std::vector<float> last_row_fp32(const brotensor::Tensor& logits);

struct GenerateOptions {
    int max_new_tokens = 64;
    SamplingParams sampling;
    bool stop_on_eos = true;
    // Greedy only: keep argmax + token feedback on the device (default on).
    bool device_greedy = true;
    // Sampling (temperature > 0, top_k != 1): softmax, top-k / top-p and the
    // draw on the device (default on); off: download the row, sample on host.
    bool device_sampling = true;
};

inline bool is_greedy(const SamplingParams& p) { return p.temperature <= 0.0f || p.top_k == 1; }

template <class Model>
std::vector<int32_t> generate(Model& model, const std::vector<int32_t>& prompt_ids, int eos_id,
                              const GenerateOptions& opts) {
    std::vector<int32_t> generated;
    if (prompt_ids.empty() || opts.max_new_tokens <= 0) return generated;
    const int vocab = model.config().vocab_size;
    model.allocate_cache(static_cast<int>(prompt_ids.size()) + opts.max_new_tokens);
    std::mt19937_64 rng(opts.sampling.seed);

    brotensor::Tensor logits;
    const bool on_device = opts.device_sampling && !is_greedy(opts.sampling);
    auto pick = [&]() {
        if (on_device) return sample_token_device(logits, opts.sampling, rng);
        const std::vector<float> row = last_row_fp32(logits);
        return sample_token(row.data(), vocab, opts.sampling, rng);
    };
    model.forward_last(prompt_ids.data(), static_cast<int>(prompt_ids.size()), logits);
    int next = pick();
    const bool stop = opts.stop_on_eos && eos_id >= 0;
    if (stop && next == eos_id) return generated;
    generated.push_back(static_cast<int32_t>(next));

    if (opts.device_greedy && is_greedy(opts.sampling)) {
        const int want = opts.max_new_tokens - 1;
        if (want > 0) {
            std::vector<int32_t> tail(static_cast<std::size_t>(want));
            const int got = model.decode_greedy(generated.back(), want, tail.data(), stop ? eos_id : -1);
            for (int i = 0; i < got; ++i) {
                if (stop && tail[static_cast<std::size_t>(i)] == eos_id) break;
                generated.push_back(tail[static_cast<std::size_t>(i)]);
            }
        }
        return generated;
    }

    if (on_device) {
        // the rest on the device: the draws are taken now, in the order the
        // per-token loop below would take them (one per token)
        const int want = opts.max_new_tokens - 1;
        if (want > 0) {
            std::uniform_real_distribution<double> dist(0.0, 1.0);
            std::vector<double> u(static_cast<std::size_t>(want));
            for (double& x : u) x = dist(rng);
            std::vector<int32_t> tail(static_cast<std::size_t>(want));
            const int got = model.decode_sampled(generated.back(), want, u.data(), opts.sampling.temperature,
                                                 opts.sampling.top_k, opts.sampling.top_p, tail.data(),
                                                 stop ? eos_id : -1);
            for (int i = 0; i < got; ++i) {
                if (stop && tail[static_cast<std::size_t>(i)] == eos_id) break;
                generated.push_back(tail[static_cast<std::size_t>(i)]);
            }
        }
        return generated;
    }

    while (static_cast<int>(generated.size()) < opts.max_new_tokens) {
        int32_t cur = generated.back();
        model.forward_last(&cur, 1, logits);
        next = pick();
        if (stop && next == eos_id) break;
        generated.push_back(static_cast<int32_t>(next));
    }
    return generated;
}

}  // namespace brolm::detail
