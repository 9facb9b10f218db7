#pragma once

// LLM2Vec text encoder (reference include/brolm/llm2vec.h:31-114,
// src/llm2vec.cpp): a LLaMA-family decoder run bidirectionally (no causal
// mask, no KV cache) as a token / sentence encoder, QK-norm off.  This build
// loads GGUF checkpoints (llama.cpp names, the Mistral / Llama map); the
// reference's safetensors overloads are outside this build.

#include <cstdint>
#include <string>
#include <vector>

#include "brolm/detail/dense_decoder.h"
#include "brotensor/tensor.h"

namespace brotensor::gguf { class File; }

namespace brolm::llm2vec {

// Flat HF LLaMA config.json; defaults are Meta-Llama-3-8B-Instruct.
struct Config {
    int vocab_size = 128256;
    int hidden_size = 4096;
    int intermediate_size = 14336;
    int num_hidden_layers = 32;
    int num_attention_heads = 32;
    int num_key_value_heads = 8;
    int head_dim = 128;   // hidden_size / num_attention_heads when the key is absent
    float rms_norm_eps = 1e-5f;
    float rope_theta = 5.0e5f;

    static Config load(const std::string& config_json_path);
    static Config from_json_text(const std::string& json_text);
    void validate() const;
};

class Encoder {
public:
    explicit Encoder(const Config& cfg);
    ~Encoder();
    Encoder(const Encoder&) = delete;
    Encoder& operator=(const Encoder&) = delete;
    Encoder(Encoder&&) noexcept = default;
    Encoder& operator=(Encoder&&) noexcept = default;

    // output.weight is optional (the encoder never runs the lm_head).
    void load_weights(const brotensor::gguf::File& f);
    void load_weights(const std::vector<const brotensor::gguf::File*>& shards);

    // hidden_out := (L, hidden_size) post-final-norm FP16 (bidirectional).
    void encode(const int32_t* ids, int L, brotensor::Tensor& hidden_out);
    // emb_out := (hidden_size, 1) FP16: mean of the hidden rows whose host
    // pool_mask entry is non-zero (weighted by it), every row when null.
    void encode_pooled(const int32_t* ids, int L, brotensor::Tensor& emb_out, const float* pool_mask = nullptr);

    const Config& config() const { return cfg_; }
    brolm::detail::DenseDecoder& core() { return core_; }

private:
    Config cfg_;
    brolm::detail::DenseDecoder core_;
};

}  // namespace brolm::llm2vec
