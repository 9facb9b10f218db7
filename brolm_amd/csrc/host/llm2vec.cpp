// LLM2Vec encoder facade (reference src/llm2vec.cpp): config.json, GGUF load
// through the Mistral / Llama tensor-name map, bidirectional encode and masked
// mean pooling over DenseDecoder::forward_encode.
#include "brolm/llm2vec.h"

#include <fstream>
#include <sstream>
#include <stdexcept>
#include <string>
#include <string_view>
#include <vector>

#include "brolm/detail/json.h"
#include "brolm/detail/weights.h"
#include "brolm/mistral3_text.h"
#include "brotensor/gguf.h"
#include "brotensor/ops.h"

namespace brolm::llm2vec {

namespace gg = ::brotensor::gguf;
namespace js = ::brolm::detail::json;
namespace bt = ::brotensor;

namespace {

[[noreturn]] void cfg_fail(const std::string& m) { throw std::runtime_error("llm2vec::Config: " + m); }
[[noreturn]] void enc_fail(const std::string& m) { throw std::runtime_error("llm2vec::Encoder: " + m); }

double num(const js::Value& o, const char* key, double dflt) {
    const js::Value* v = o.find(key);
    if (!v || v->kind == js::Value::Kind::Null) return dflt;
    if (!v->is_number()) cfg_fail(std::string("'") + key + "' is not a number");
    return v->num;
}

brolm::detail::DenseDecoderConfig to_core_config(const Config& c) {
    brolm::detail::DenseDecoderConfig d;
    d.vocab_size = c.vocab_size;
    d.hidden_size = c.hidden_size;
    d.intermediate_size = c.intermediate_size;
    d.num_hidden_layers = c.num_hidden_layers;
    d.num_attention_heads = c.num_attention_heads;
    d.num_key_value_heads = c.num_key_value_heads;
    d.head_dim = c.head_dim;
    d.rms_norm_eps = c.rms_norm_eps;
    d.rope_theta = c.rope_theta;
    d.use_qk_norm = false;          // LLaMA has no QK-norm
    d.tie_word_embeddings = true;   // the lm_head is never run
    return d;
}

}  // namespace

Config Config::load(const std::string& path) {
    std::ifstream f(path, std::ios::binary);
    if (!f) cfg_fail("cannot open '" + path + "'");
    std::ostringstream ss;
    ss << f.rdbuf();
    return from_json_text(ss.str());
}

Config Config::from_json_text(const std::string& text) {
    js::Value root;
    try {
        root = js::parse(text);
    } catch (const std::exception& e) {
        cfg_fail(std::string("json parse: ") + e.what());
    }
    if (!root.is_object()) cfg_fail("root is not a JSON object");
    Config c;
    c.vocab_size = static_cast<int>(num(root, "vocab_size", c.vocab_size));
    c.hidden_size = static_cast<int>(num(root, "hidden_size", c.hidden_size));
    c.intermediate_size = static_cast<int>(num(root, "intermediate_size", c.intermediate_size));
    c.num_hidden_layers = static_cast<int>(num(root, "num_hidden_layers", c.num_hidden_layers));
    c.num_attention_heads = static_cast<int>(num(root, "num_attention_heads", c.num_attention_heads));
    c.num_key_value_heads = static_cast<int>(num(root, "num_key_value_heads", c.num_key_value_heads));
    c.rms_norm_eps = static_cast<float>(num(root, "rms_norm_eps", c.rms_norm_eps));
    c.rope_theta = static_cast<float>(num(root, "rope_theta", c.rope_theta));
    if (const js::Value* hd = root.find("head_dim"); hd && hd->is_number())
        c.head_dim = static_cast<int>(hd->num);
    else
        c.head_dim = c.num_attention_heads > 0 ? c.hidden_size / c.num_attention_heads : 0;
    c.validate();
    return c;
}

void Config::validate() const {
    if (hidden_size <= 0 || intermediate_size <= 0 || num_hidden_layers <= 0 || vocab_size <= 0 || head_dim <= 0)
        cfg_fail("non-positive dimension");
    if (num_attention_heads <= 0 || num_key_value_heads <= 0)
        cfg_fail("num_attention_heads / num_key_value_heads must be positive");
    if (num_attention_heads % num_key_value_heads != 0)
        cfg_fail("num_attention_heads must be a multiple of num_key_value_heads");
    if (head_dim % 2 != 0) cfg_fail("head_dim must be even (RoPE rotates pairs)");
}

Encoder::Encoder(const Config& cfg) : cfg_(cfg), core_(to_core_config(cfg)) {}
Encoder::~Encoder() = default;

void Encoder::load_weights(const gg::File& f) {
    const std::vector<const gg::File*> shards = {&f};
    load_weights(shards);
}

void Encoder::load_weights(const std::vector<const gg::File*>& shards) {
    if (shards.empty()) enc_fail("load_weights: no gguf shards");
    brolm::detail::weights::GgufSource src(
        shards, [](std::string_view hf) { return brolm::mistral3::mistral3_hf_to_ggml(hf); });
    core_.load_weights(src);
}

void Encoder::encode(const int32_t* ids, int L, bt::Tensor& hidden_out) { core_.forward_encode(ids, L, hidden_out); }

void Encoder::encode_pooled(const int32_t* ids, int L, bt::Tensor& emb_out, const float* pool_mask) {
    bt::Tensor hidden;
    core_.forward_encode(ids, L, hidden);
    bt::Tensor mask_dev;
    const float* d_mask = nullptr;
    if (pool_mask) {
        mask_dev = bt::Tensor::from_host_on(bt::Device::ROCm, pool_mask, L, 1);
        d_mask = static_cast<const float*>(mask_dev.data);
    }
    bt::masked_mean_pool_forward(hidden, d_mask, emb_out);
}

}  // namespace brolm::llm2vec
