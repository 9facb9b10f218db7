#pragma once

// Qwen3 decoder (reference include/brolm/qwen.h:35-157): inference-only,
// KV-cached; a thin wrapper over DenseDecoder with per-head QK-norm enabled.
// GGUF checkpoints only on this build (the safetensors overloads are outside
// the quantized decode path).

#include <cstdint>
#include <string>
#include <string_view>
#include <vector>

#include "brolm/detail/dense_decoder.h"
#include "brotensor/tensor.h"

namespace brotensor::gguf { class File; }

namespace brolm::qwen {

// HF tensor name -> ggml name ("blk.N.attn_q.weight", ...); empty if unknown
// (src/qwen.cpp:173-208).
std::string qwen3_hf_to_ggml(std::string_view hf_name);

struct Qwen3Config {
    int vocab_size = 151936;
    int hidden_size = 1024;
    int intermediate_size = 3072;
    int num_hidden_layers = 28;
    int num_attention_heads = 16;
    int num_key_value_heads = 8;
    int head_dim = 128;
    float rms_norm_eps = 1e-6f;
    float rope_theta = 1000000.0f;
    bool tie_word_embeddings = true;
    int max_position_embeddings = 40960;

    // Metadata keys qwen3.* (src/qwen.cpp:88-149); throws on missing required
    // keys or general.architecture != "qwen3".
    static Qwen3Config from_gguf(const brotensor::gguf::File& f);
};

class Qwen3Model {
public:
    explicit Qwen3Model(const Qwen3Config& cfg);
    ~Qwen3Model();
    Qwen3Model(const Qwen3Model&) = delete;
    Qwen3Model& operator=(const Qwen3Model&) = delete;
    Qwen3Model(Qwen3Model&&) noexcept = default;
    Qwen3Model& operator=(Qwen3Model&&) noexcept = default;

    void load_weights(const brotensor::gguf::File& f);
    void load_weights(const std::vector<const brotensor::gguf::File*>& shards);

    void allocate_cache(int max_seq_len) { core_.allocate_cache(max_seq_len); }
    void reset_cache() { core_.reset_cache(); }
    void truncate_cache(int len) { core_.truncate_cache(len); }
    int cache_len() const { return core_.cache_len(); }

    void forward(const int32_t* ids, int L, brotensor::Tensor& logits_out, brotensor::Tensor* hidden_out = nullptr) {
        core_.forward(ids, L, logits_out, hidden_out);
    }
    void forward_last(const int32_t* ids, int L, brotensor::Tensor& logits_out) {
        core_.forward_last(ids, L, logits_out);
    }
    void embed_tokens(const int32_t* ids, int L, brotensor::Tensor& out) { core_.embed_tokens(ids, L, out); }
    void forward_embeds(const brotensor::Tensor& embeds, int L, brotensor::Tensor& logits_out,
                        brotensor::Tensor* hidden_out = nullptr) {
        core_.forward_embeds(embeds, L, logits_out, hidden_out);
    }

    // Device-side greedy continuation (see DenseDecoder::decode_greedy).
    int decode_greedy(int32_t token, int n, int32_t* out, int eos_id) {
        return core_.decode_greedy(token, n, out, eos_id);
    }
    // Device-side sampled continuation (DenseDecoder::decode_sampled).
    int decode_sampled(int32_t token, int n, const double* u, float temperature, int top_k, float top_p,
                       int32_t* out, int eos_id) {
        return core_.decode_sampled(token, n, u, temperature, top_k, top_p, out, eos_id);
    }

    const Qwen3Config& config() const { return cfg_; }
    brolm::detail::DenseDecoder& core() { return core_; }

private:
    Qwen3Config cfg_;
    brolm::detail::DenseDecoder core_;
};

}  // namespace brolm::qwen
