// Qwen3 facade: config from GGUF metadata, the HF -> ggml tensor-name map and
// the GGUF load overloads (reference include/brolm/qwen.h:35-157).
//
// The metadata keys, the ggml tensor names and the error texts are the
// reference's contract (src/qwen.cpp:88-149, :173-208); the reading is table
// driven: every config field is one row naming its key, whether it is
// required, and how a missing key is filled.
#include "brolm/qwen.h"

#include <array>
#include <charconv>
#include <optional>
#include <stdexcept>
#include <string>
#include <string_view>
#include <vector>

#include "brolm/detail/weights.h"
#include "brotensor/gguf.h"

namespace brolm::qwen {

namespace gg = ::brotensor::gguf;

namespace {

constexpr const char* kWho = "qwen::Qwen3Config::from_gguf: ";

// A GGUF scalar as a double (every integer width and both float widths);
// nullopt for strings, arrays and booleans.
std::optional<double> scalar_value(const gg::Value& v) {
    using T = gg::ValueType;
    switch (v.type) {
        case T::U8: return v.scalar.u8;
        case T::I8: return v.scalar.i8;
        case T::U16: return v.scalar.u16;
        case T::I16: return v.scalar.i16;
        case T::U32: return v.scalar.u32;
        case T::I32: return v.scalar.i32;
        case T::U64: return static_cast<double>(v.scalar.u64);
        case T::I64: return static_cast<double>(v.scalar.i64);
        case T::F32: return v.scalar.f32;
        case T::F64: return v.scalar.f64;
        default: return std::nullopt;
    }
}
bool is_integer_type(gg::ValueType t) {
    using T = gg::ValueType;
    return t == T::U8 || t == T::I8 || t == T::U16 || t == T::I16 || t == T::U32 || t == T::I32 || t == T::U64 ||
           t == T::I64;
}

// Typed access to a file's metadata with the reference's error texts.
class Meta {
public:
    explicit Meta(const gg::File& f) : f_(f) {}

    std::optional<int> integer(const char* key) const {
        const gg::Value* v = f_.find_meta(key);
        if (!v) return std::nullopt;
        if (!is_integer_type(v->type))
            throw std::runtime_error(std::string(kWho) + "metadata '" + key + "' is not an integer scalar");
        return static_cast<int>(static_cast<long long>(*scalar_value(*v)));
    }
    std::optional<float> real(const char* key) const {
        const gg::Value* v = f_.find_meta(key);
        if (!v) return std::nullopt;
        if (v->type != gg::ValueType::F32 && v->type != gg::ValueType::F64)
            throw std::runtime_error(std::string(kWho) + "metadata '" + key + "' is not a float scalar");
        return static_cast<float>(*scalar_value(*v));
    }
    int required(const char* key) const {
        const std::optional<int> v = integer(key);
        if (!v) throw std::runtime_error(std::string(kWho) + "missing metadata '" + key + "'");
        return *v;
    }
    const gg::Value* raw(const char* key) const { return f_.find_meta(key); }
    const gg::File& file() const { return f_; }

private:
    const gg::File& f_;
};

// Integer fields: key, required, and (when optional) the fallback computed
// from the fields read before it.
struct IntField {
    const char* key;
    int Qwen3Config::* field;
    bool required;
    int (*fallback)(const Qwen3Config&);
};
const std::array<IntField, 7> kIntFields = {{
    {"qwen3.embedding_length", &Qwen3Config::hidden_size, true, nullptr},
    {"qwen3.feed_forward_length", &Qwen3Config::intermediate_size, true, nullptr},
    {"qwen3.block_count", &Qwen3Config::num_hidden_layers, true, nullptr},
    {"qwen3.attention.head_count", &Qwen3Config::num_attention_heads, true, nullptr},
    // GQA defaults to one KV head per query head, head_dim to hidden / heads
    {"qwen3.attention.head_count_kv", &Qwen3Config::num_key_value_heads, false,
     [](const Qwen3Config& c) { return c.num_attention_heads; }},
    {"qwen3.attention.key_length", &Qwen3Config::head_dim, false,
     [](const Qwen3Config& c) { return c.hidden_size / c.num_attention_heads; }},
    {"qwen3.context_length", &Qwen3Config::max_position_embeddings, false,
     [](const Qwen3Config& c) { return c.max_position_embeddings; }},
}};
struct RealField {
    const char* key;
    float Qwen3Config::* field;
};
const std::array<RealField, 2> kRealFields = {{
    {"qwen3.attention.layer_norm_rms_epsilon", &Qwen3Config::rms_norm_eps},
    {"qwen3.rope.freq_base", &Qwen3Config::rope_theta},
}};

// vocab: the tokenizer's token list when present, else qwen3.vocab_size.
void read_vocab(const Meta& m, Qwen3Config& c) {
    const gg::Value* toks = m.raw("tokenizer.ggml.tokens");
    if (toks && toks->type == gg::ValueType::Array) {
        c.vocab_size = static_cast<int>(toks->array.size());
        return;
    }
    if (const std::optional<int> v = m.integer("qwen3.vocab_size")) c.vocab_size = *v;
}
// Tied embeddings: the boolean key when present, else "no output.weight".
void read_tie(const Meta& m, Qwen3Config& c) {
    const gg::Value* v = m.raw("qwen3.tie_word_embeddings");
    c.tie_word_embeddings = (v && v->type == gg::ValueType::Bool) ? v->scalar.b
                                                                   : m.file().find_tensor("output.weight") == nullptr;
}

// ---- HF -> ggml names -----------------------------------------------------

struct NamePair {
    std::string_view hf, ggml;
};
// Whole-model tensors.
constexpr std::array<NamePair, 3> kGlobalNames = {{
    {"model.embed_tokens.weight", "token_embd.weight"},
    {"model.norm.weight", "output_norm.weight"},
    {"lm_head.weight", "output.weight"},
}};
// Per-layer tensors: the suffix after "model.layers.<i>." and after "blk.<i>.".
constexpr std::array<NamePair, 11> kLayerNames = {{
    {"self_attn.q_proj.weight", "attn_q.weight"},
    {"self_attn.k_proj.weight", "attn_k.weight"},
    {"self_attn.v_proj.weight", "attn_v.weight"},
    {"self_attn.o_proj.weight", "attn_output.weight"},
    {"self_attn.q_norm.weight", "attn_q_norm.weight"},
    {"self_attn.k_norm.weight", "attn_k_norm.weight"},
    {"input_layernorm.weight", "attn_norm.weight"},
    {"post_attention_layernorm.weight", "ffn_norm.weight"},
    {"mlp.gate_proj.weight", "ffn_gate.weight"},
    {"mlp.up_proj.weight", "ffn_up.weight"},
    {"mlp.down_proj.weight", "ffn_down.weight"},
}};

brolm::detail::DenseDecoderConfig core_config_of(const Qwen3Config& c) {
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
    d.tie_word_embeddings = c.tie_word_embeddings;
    d.use_qk_norm = true;   // the one architectural switch that makes the dense decoder Qwen3
    return d;
}

}  // namespace

Qwen3Config Qwen3Config::from_gguf(const gg::File& f) {
    const Meta m(f);
    if (const gg::Value* arch = m.raw("general.architecture");
        arch && arch->type == gg::ValueType::String && arch->str != "qwen3")
        throw std::runtime_error(std::string(kWho) + "general.architecture is '" + arch->str + "', expected 'qwen3'");
    Qwen3Config c;
    for (const IntField& fld : kIntFields) {
        if (fld.required) {
            c.*fld.field = m.required(fld.key);
        } else {
            const std::optional<int> v = m.integer(fld.key);
            c.*fld.field = v ? *v : fld.fallback(c);
        }
    }
    for (const RealField& fld : kRealFields)
        if (const std::optional<float> v = m.real(fld.key)) c.*fld.field = *v;
    read_vocab(m, c);
    read_tie(m, c);
    return c;
}

std::string qwen3_hf_to_ggml(std::string_view hf) {
    for (const NamePair& p : kGlobalNames)
        if (hf == p.hf) return std::string(p.ggml);
    constexpr std::string_view kPrefix = "model.layers.";
    if (hf.substr(0, kPrefix.size()) != kPrefix) return {};
    const std::string_view rest = hf.substr(kPrefix.size());
    // the layer index: decimal digits up to the next '.'
    unsigned layer = 0;
    const auto [end, ec] = std::from_chars(rest.data(), rest.data() + rest.size(), layer);
    const std::size_t ndig = static_cast<std::size_t>(end - rest.data());
    if (ec != std::errc() || ndig == 0 || ndig >= rest.size() || rest[ndig] != '.') return {};
    const std::string_view suffix = rest.substr(ndig + 1);
    for (const NamePair& p : kLayerNames)
        if (suffix == p.hf) return "blk." + std::string(rest.substr(0, ndig)) + "." + std::string(p.ggml);
    return {};
}

Qwen3Model::Qwen3Model(const Qwen3Config& cfg) : cfg_(cfg), core_(core_config_of(cfg)) {}
Qwen3Model::~Qwen3Model() = default;

void Qwen3Model::load_weights(const gg::File& f) { load_weights(std::vector<const gg::File*>{&f}); }

void Qwen3Model::load_weights(const std::vector<const gg::File*>& shards) {
    if (shards.empty()) throw std::runtime_error("qwen::Qwen3Model: load_weights: no gguf shards");
    const brolm::detail::weights::GgufSource src(shards, [](std::string_view hf) { return qwen3_hf_to_ggml(hf); });
    core_.load_weights(src);
}

}  // namespace brolm::qwen
