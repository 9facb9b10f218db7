// Qwen3 facade: config from GGUF metadata, the HF -> ggml tensor-name map and
// the GGUF load overloads (reference include/brolm/qwen.h:35-157).
//
// The metadata keys, the ggml tensor names and the error texts are the
// reference's contract (src/qwen.cpp:88-149, :173-208); the reading is table
// driven (meta_tables.h): every config field is one row naming its key,
// whether it is required, and how a missing key is filled.
#include "brolm/qwen.h"

#include <stdexcept>
#include <string>
#include <string_view>
#include <vector>

#include "brolm/detail/weights.h"
#include "brotensor/gguf.h"
#include "meta_tables.h"

namespace brolm::qwen {

namespace gg = ::brotensor::gguf;
namespace mt = ::brolm::detail::meta;

namespace {

// Integer fields in reading order; GQA defaults to one KV head per query
// head, head_dim to hidden / heads, the context length to the default.
const mt::IntRow<Qwen3Config> kIntFields[] = {
    {"embedding_length", &Qwen3Config::hidden_size, true, nullptr},
    {"feed_forward_length", &Qwen3Config::intermediate_size, true, nullptr},
    {"block_count", &Qwen3Config::num_hidden_layers, true, nullptr},
    {"attention.head_count", &Qwen3Config::num_attention_heads, true, nullptr},
    {"attention.head_count_kv", &Qwen3Config::num_key_value_heads, false,
     [](const Qwen3Config& c) { return c.num_attention_heads; }},
    {"attention.key_length", &Qwen3Config::head_dim, false,
     [](const Qwen3Config& c) { return c.hidden_size / c.num_attention_heads; }},
    {"context_length", &Qwen3Config::max_position_embeddings, false, nullptr},
};
const mt::RealRow<Qwen3Config> kRealFields[] = {
    {"attention.layer_norm_rms_epsilon", &Qwen3Config::rms_norm_eps},
    {"rope.freq_base", &Qwen3Config::rope_theta},
};

// Tied embeddings: the boolean key when present, else "no output.weight".
bool tied(const mt::Reader& m) {
    const gg::Value* v = m.raw("tie_word_embeddings");
    if (v && v->type == gg::ValueType::Bool) return v->scalar.b;
    return m.file().find_tensor("output.weight") == nullptr;
}

}  // namespace

Qwen3Config Qwen3Config::from_gguf(const gg::File& f) {
    const mt::Reader m(f, "qwen::Qwen3Config::from_gguf: ", "qwen3.");
    if (const gg::Value* arch = m.raw("general.architecture", false);
        arch && arch->type == gg::ValueType::String && arch->str != "qwen3")
        m.fail("general.architecture is '" + arch->str + "', expected 'qwen3'");
    Qwen3Config c;
    mt::read_rows(m, kIntFields, kRealFields, c);
    c.vocab_size = mt::vocab_size(m, c.vocab_size);
    c.tie_word_embeddings = tied(m);
    return c;
}

std::string qwen3_hf_to_ggml(std::string_view hf) { return mt::hf_to_ggml(hf, /*with_qk_norm=*/true); }

Qwen3Model::Qwen3Model(const Qwen3Config& cfg) : cfg_(cfg), core_(mt::decoder_config(cfg, /*qk_norm=*/true)) {}
Qwen3Model::~Qwen3Model() = default;

void Qwen3Model::load_weights(const gg::File& f) { load_weights(std::vector<const gg::File*>{&f}); }

void Qwen3Model::load_weights(const std::vector<const gg::File*>& shards) {
    if (shards.empty()) throw std::runtime_error("qwen::Qwen3Model: load_weights: no gguf shards");
    const brolm::detail::weights::GgufSource src(shards, [](std::string_view hf) { return qwen3_hf_to_ggml(hf); });
    core_.load_weights(src);
}

}  // namespace brolm::qwen
