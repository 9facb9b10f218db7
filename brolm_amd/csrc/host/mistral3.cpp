// Mistral 3.1 text facade (reference src/mistral3_config.cpp,
// src/mistral3_text.cpp): config from config.json / GGUF metadata, the HF ->
// ggml tensor-name map, and the GGUF load overloads over DenseDecoder with
// QK-norm off.
#include "brolm/mistral3_config.h"
#include "brolm/mistral3_generate.h"
#include "brolm/mistral3_text.h"

#include <fstream>
#include <sstream>
#include <stdexcept>
#include <string>
#include <string_view>
#include <vector>

#include "brolm/detail/json.h"
#include "brolm/detail/weights.h"
#include "brotensor/gguf.h"

namespace brolm::mistral3 {

namespace gg = ::brotensor::gguf;
namespace js = ::brolm::detail::json;

namespace {

[[noreturn]] void cfg_fail(const std::string& msg) { throw std::runtime_error("mistral3::Mistral3Config: " + msg); }
[[noreturn]] void model_fail(const std::string& msg) { throw std::runtime_error("mistral3::TextModel: " + msg); }

int json_int(const js::Value& o, const char* key, int dflt) {
    const js::Value* v = o.find(key);
    if (!v || v->kind == js::Value::Kind::Null) return dflt;
    if (!v->is_number()) cfg_fail(std::string("'") + key + "' is not a number");
    return static_cast<int>(v->num);
}
float json_float(const js::Value& o, const char* key, float dflt) {
    const js::Value* v = o.find(key);
    if (!v || v->kind == js::Value::Kind::Null) return dflt;
    if (!v->is_number()) cfg_fail(std::string("'") + key + "' is not a number");
    return static_cast<float>(v->num);
}
bool json_bool(const js::Value& o, const char* key, bool dflt) {
    const js::Value* v = o.find(key);
    if (!v || v->kind == js::Value::Kind::Null) return dflt;
    if (!v->is_bool()) cfg_fail(std::string("'") + key + "' is not a boolean");
    return v->b;
}

const gg::Value& need_meta(const gg::File& f, const std::string& key) {
    const gg::Value* v = f.find_meta(key);
    if (!v) cfg_fail("from_gguf: missing metadata '" + key + "'");
    return *v;
}

int meta_as_int(const gg::Value& v, const std::string& key) {
    switch (v.type) {
        case gg::ValueType::U8: return static_cast<int>(v.scalar.u8);
        case gg::ValueType::I8: return static_cast<int>(v.scalar.i8);
        case gg::ValueType::U16: return static_cast<int>(v.scalar.u16);
        case gg::ValueType::I16: return static_cast<int>(v.scalar.i16);
        case gg::ValueType::U32: return static_cast<int>(v.scalar.u32);
        case gg::ValueType::I32: return static_cast<int>(v.scalar.i32);
        case gg::ValueType::U64: return static_cast<int>(v.scalar.u64);
        case gg::ValueType::I64: return static_cast<int>(v.scalar.i64);
        default: cfg_fail("from_gguf: metadata '" + key + "' is not an integer scalar");
    }
}

float meta_as_f32(const gg::Value& v, const std::string& key) {
    if (v.type == gg::ValueType::F32) return v.scalar.f32;
    if (v.type == gg::ValueType::F64) return static_cast<float>(v.scalar.f64);
    cfg_fail("from_gguf: metadata '" + key + "' is not a float scalar");
}

bool starts_with(std::string_view s, std::string_view p) { return s.size() >= p.size() && s.compare(0, p.size(), p) == 0; }

brolm::detail::DenseDecoderConfig to_core_config(const Mistral3Config::Text& c) {
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
    d.use_qk_norm = false;
    d.tie_word_embeddings = c.tie_word_embeddings;
    return d;
}

}  // namespace

// ---- config ---------------------------------------------------------------

Mistral3Config Mistral3Config::load(const std::string& path) {
    std::ifstream f(path, std::ios::binary);
    if (!f) cfg_fail("cannot open '" + path + "'");
    std::ostringstream ss;
    ss << f.rdbuf();
    return from_json_text(ss.str());
}

Mistral3Config Mistral3Config::from_json_text(const std::string& text) {
    js::Value root;
    try {
        root = js::parse(text);
    } catch (const std::exception& e) {
        cfg_fail(std::string("json parse: ") + e.what());
    }
    if (!root.is_object()) cfg_fail("root is not a JSON object");
    Mistral3Config cfg;
    cfg.image_token_index = json_int(root, "image_token_index", cfg.image_token_index);
    cfg.spatial_merge_size = json_int(root, "spatial_merge_size", cfg.spatial_merge_size);
    cfg.multimodal_projector_bias = json_bool(root, "multimodal_projector_bias", cfg.multimodal_projector_bias);
    const js::Value* tc = root.find("text_config");
    if (!tc) cfg_fail("missing text_config");
    if (!tc->is_object()) cfg_fail("text_config is not an object");
    Text& t = cfg.text;
    t.vocab_size = json_int(*tc, "vocab_size", t.vocab_size);
    t.hidden_size = json_int(*tc, "hidden_size", t.hidden_size);
    t.intermediate_size = json_int(*tc, "intermediate_size", t.intermediate_size);
    t.num_hidden_layers = json_int(*tc, "num_hidden_layers", t.num_hidden_layers);
    t.num_attention_heads = json_int(*tc, "num_attention_heads", t.num_attention_heads);
    t.num_key_value_heads = json_int(*tc, "num_key_value_heads", t.num_key_value_heads);
    t.head_dim = json_int(*tc, "head_dim", t.head_dim);
    t.rms_norm_eps = json_float(*tc, "rms_norm_eps", t.rms_norm_eps);
    t.rope_theta = json_float(*tc, "rope_theta", t.rope_theta);
    t.tie_word_embeddings = json_bool(*tc, "tie_word_embeddings", t.tie_word_embeddings);
    t.max_position_embeddings = json_int(*tc, "max_position_embeddings", t.max_position_embeddings);
    if (const js::Value* sw = tc->find("sliding_window"); sw && sw->is_number()) {
        t.has_sliding_window = true;
        t.sliding_window = static_cast<int>(sw->num);
    }
    if (!root.find("vision_config")) cfg_fail("missing vision_config");
    cfg.validate();
    return cfg;
}

Mistral3Config Mistral3Config::from_gguf(const gg::File& f) {
    const gg::Value& arch = need_meta(f, "general.architecture");
    if (arch.type != gg::ValueType::String) cfg_fail("from_gguf: general.architecture is not a string");
    const std::string a = arch.str + ".";
    Mistral3Config cfg;
    Text& t = cfg.text;
    t.hidden_size = meta_as_int(need_meta(f, a + "embedding_length"), a + "embedding_length");
    t.intermediate_size = meta_as_int(need_meta(f, a + "feed_forward_length"), a + "feed_forward_length");
    t.num_hidden_layers = meta_as_int(need_meta(f, a + "block_count"), a + "block_count");
    t.num_attention_heads = meta_as_int(need_meta(f, a + "attention.head_count"), a + "attention.head_count");
    if (const auto* v = f.find_meta(a + "attention.head_count_kv"))
        t.num_key_value_heads = meta_as_int(*v, a + "attention.head_count_kv");
    else
        t.num_key_value_heads = t.num_attention_heads;
    if (const auto* v = f.find_meta(a + "attention.key_length"))
        t.head_dim = meta_as_int(*v, a + "attention.key_length");
    else
        t.head_dim = t.hidden_size / t.num_attention_heads;
    if (const auto* v = f.find_meta(a + "attention.layer_norm_rms_epsilon"))
        t.rms_norm_eps = meta_as_f32(*v, a + "attention.layer_norm_rms_epsilon");
    if (const auto* v = f.find_meta(a + "rope.freq_base")) t.rope_theta = meta_as_f32(*v, a + "rope.freq_base");
    if (const auto* v = f.find_meta(a + "context_length"))
        t.max_position_embeddings = meta_as_int(*v, a + "context_length");
    if (const auto* toks = f.find_meta("tokenizer.ggml.tokens"); toks && toks->type == gg::ValueType::Array)
        t.vocab_size = static_cast<int>(toks->array.size());
    else if (const auto* vs = f.find_meta(a + "vocab_size"))
        t.vocab_size = meta_as_int(*vs, a + "vocab_size");
    t.tie_word_embeddings = f.find_tensor("output.weight") == nullptr;
    cfg.validate();
    return cfg;
}

void Mistral3Config::validate() const {
    if (text.hidden_size <= 0 || text.intermediate_size <= 0 || text.num_hidden_layers <= 0 ||
        text.vocab_size <= 0 || text.head_dim <= 0)
        cfg_fail("text_config has non-positive dimension");
    if (text.num_attention_heads <= 0 || text.num_key_value_heads <= 0)
        cfg_fail("num_attention_heads / num_key_value_heads must be positive");
    if (text.num_attention_heads % text.num_key_value_heads != 0)
        cfg_fail("num_attention_heads must be a multiple of num_key_value_heads");
    if (text.head_dim % 2 != 0) cfg_fail("head_dim must be even (RoPE rotates pairs)");
    if (spatial_merge_size <= 0) cfg_fail("spatial_merge_size must be positive");
}

// ---- text model -------------------------------------------------------------

std::string mistral3_hf_to_ggml(std::string_view hf_name) {
    if (hf_name == "model.embed_tokens.weight") return "token_embd.weight";
    if (hf_name == "model.norm.weight") return "output_norm.weight";
    if (hf_name == "lm_head.weight") return "output.weight";
    constexpr std::string_view kLayers = "model.layers.";
    if (!starts_with(hf_name, kLayers)) return {};
    const auto dot = hf_name.find('.', kLayers.size());
    if (dot == std::string_view::npos) return {};
    const std::string_view idx = hf_name.substr(kLayers.size(), dot - kLayers.size());
    if (idx.empty()) return {};
    for (char ch : idx)
        if (ch < '0' || ch > '9') return {};
    const std::string_view tail = hf_name.substr(dot + 1);
    static constexpr std::pair<std::string_view, std::string_view> kMap[] = {
        {"self_attn.q_proj.weight", "attn_q.weight"},
        {"self_attn.k_proj.weight", "attn_k.weight"},
        {"self_attn.v_proj.weight", "attn_v.weight"},
        {"self_attn.o_proj.weight", "attn_output.weight"},
        {"input_layernorm.weight", "attn_norm.weight"},
        {"post_attention_layernorm.weight", "ffn_norm.weight"},
        {"mlp.gate_proj.weight", "ffn_gate.weight"},
        {"mlp.up_proj.weight", "ffn_up.weight"},
        {"mlp.down_proj.weight", "ffn_down.weight"},
    };
    for (const auto& [hf, ggml] : kMap) {
        if (tail != hf) continue;
        std::string out = "blk.";
        out.append(idx);
        out.push_back('.');
        out.append(ggml);
        return out;
    }
    return {};
}

TextModel::TextModel(const Mistral3Config::Text& cfg) : cfg_(cfg), core_(to_core_config(cfg)) {}
TextModel::~TextModel() = default;

void TextModel::load_weights(const gg::File& f) {
    const std::vector<const gg::File*> shards = {&f};
    load_weights(shards);
}

void TextModel::load_weights(const std::vector<const gg::File*>& shards) {
    if (shards.empty()) model_fail("load_weights: no gguf shards");
    brolm::detail::weights::GgufSource src(shards, [](std::string_view hf) { return mistral3_hf_to_ggml(hf); });
    core_.load_weights(src);
}

std::vector<int32_t> generate(TextModel& model, const std::vector<int32_t>& prompt_ids, int eos_id,
                              const GenerateOptions& opts) {
    return brolm::detail::generate(model, prompt_ids, eos_id, opts);
}

}  // namespace brolm::mistral3
