#pragma once

// Mistral 3.1 text decoder (reference include/brolm/mistral3_text.h:52-131,
// src/mistral3_text.cpp): the dense decoder with per-head QK-norm disabled and
// an untied lm_head.  GGUF checkpoints only on this build (the safetensors
// overloads are outside the quantized decode path).  A single-token forward
// runs the same fused decode step as Qwen3, with the q/k heads rotated
// straight from the projections.

#include <cstdint>
#include <string>
#include <string_view>
#include <vector>

#include "brolm/detail/dense_decoder.h"
#include "brolm/mistral3_config.h"
#include "brotensor/tensor.h"

namespace brotensor::gguf { class File; }

namespace brolm::mistral3 {

// HF name -> ggml name: the Qwen3 map without q_norm / k_norm
// (src/mistral3_text.cpp:70-108).  Empty if the name is no Mistral text weight.
std::string mistral3_hf_to_ggml(std::string_view hf_name);

class TextModel {
public:
    explicit TextModel(const Mistral3Config::Text& cfg);
    ~TextModel();
    TextModel(const TextModel&) = delete;
    TextModel& operator=(const TextModel&) = delete;
    TextModel(TextModel&&) noexcept = default;
    TextModel& operator=(TextModel&&) noexcept = default;

    // Untied checkpoints must carry output.weight (throws otherwise).
    void load_weights(const brotensor::gguf::File& f);
    void load_weights(const std::vector<const brotensor::gguf::File*>& shards);

    void allocate_cache(int max_seq_len) { core_.allocate_cache(max_seq_len); }
    void reset_cache() { core_.reset_cache(); }
    int cache_len() const { return core_.cache_len(); }

    void forward(const int32_t* ids, int L, brotensor::Tensor& logits_out) { core_.forward(ids, L, logits_out); }
    void forward_last(const int32_t* ids, int L, brotensor::Tensor& logits_out) {
        core_.forward_last(ids, L, logits_out);
    }
    void embed_tokens(const int32_t* ids, int L, brotensor::Tensor& out) { core_.embed_tokens(ids, L, out); }
    void forward_embeds(const brotensor::Tensor& embeds, int L, brotensor::Tensor& logits_out) {
        core_.forward_embeds(embeds, L, logits_out);
    }

    // Device-side greedy continuation (DenseDecoder::decode_greedy).
    int decode_greedy(int32_t token, int n, int32_t* out, int eos_id) {
        return core_.decode_greedy(token, n, out, eos_id);
    }
    // Device-side sampled continuation (DenseDecoder::decode_sampled).
    int decode_sampled(int32_t token, int n, const double* u, float temperature, int top_k, float top_p,
                       int32_t* out, int eos_id) {
        return core_.decode_sampled(token, n, u, temperature, top_k, top_p, out, eos_id);
    }

    const Mistral3Config::Text& config() const { return cfg_; }
    brolm::detail::DenseDecoder& core() { return core_; }

private:
    Mistral3Config::Text cfg_;
    brolm::detail::DenseDecoder core_;
};

}  // namespace brolm::mistral3
