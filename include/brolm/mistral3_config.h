#pragma once

// Mistral 3.1 configuration (reference include/brolm/mistral3_config.h:30-143,
// src/mistral3_config.cpp).  The text section drives the dense decoder; the
// top-level multimodal glue is parsed for API parity.  The Pixtral vision
// section is outside this build (no vision tower here), so it is neither
// stored nor validated.

#include <string>

namespace brotensor::gguf { class File; }

namespace brolm::mistral3 {

struct Mistral3Config {
    // text_config (Mistral dense decoder); defaults are Mistral-Small-3.1-24B.
    struct Text {
        int vocab_size = 131072;
        int hidden_size = 5120;
        int intermediate_size = 32768;
        int num_hidden_layers = 40;
        int num_attention_heads = 32;
        int num_key_value_heads = 8;
        int head_dim = 128;
        float rms_norm_eps = 1e-5f;
        float rope_theta = 1.0e9f;
        bool tie_word_embeddings = false;   // HF Mistral default; the key is absent
        int max_position_embeddings = 131072;
        bool has_sliding_window = false;    // "sliding_window": null -> full causal
        int sliding_window = 0;
    } text;

    int image_token_index = 10;
    int spatial_merge_size = 2;
    bool multimodal_projector_bias = false;

    // config.json of Mistral3ForConditionalGeneration: text_config and
    // vision_config must both be present (src/mistral3_config.cpp:36-93).
    static Mistral3Config load(const std::string& config_json_path);
    static Mistral3Config from_json_text(const std::string& json_text);

    // Text section from a llama.cpp GGUF: keys are prefixed with
    // general.architecture ("llama" or "mistral"), head_dim from
    // <arch>.attention.key_length, vocab from the tokenizer token list, tied
    // iff output.weight is absent (src/mistral3_config.cpp:130-191).
    static Mistral3Config from_gguf(const brotensor::gguf::File& f);

    // Positive dims, GQA divisibility, even head_dim, spatial_merge_size > 0.
    void validate() const;
};

}  // namespace brolm::mistral3
