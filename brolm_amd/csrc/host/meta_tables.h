#pragma once
// Table-driven readers shared by the model facades (qwen.cpp, mistral3.cpp):
// a config is a list of rows, each naming its metadata key, the member it
// fills and what happens when the key is missing; the HF -> ggml tensor-name
// map is one table of whole-model names and one of per-layer suffixes.
//
// Only the keys, names and error texts are the reference's contract
// (src/qwen.cpp:88-149, src/mistral3_config.cpp:102-191,
// src/mistral3_text.cpp:70-108); the readers are this build's own.
#include <charconv>
#include <optional>
#include <stdexcept>
#include <string>
#include <string_view>

#include "brolm/detail/dense_decoder.h"
#include "brotensor/gguf.h"

namespace brolm::detail::meta {

namespace gg = ::brotensor::gguf;

// A GGUF scalar as a double (every integer width and both float widths);
// nullopt for strings, arrays and booleans.
inline std::optional<double> scalar_value(const gg::Value& v) {
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

inline bool is_float_type(gg::ValueType t) { return t == gg::ValueType::F32 || t == gg::ValueType::F64; }

// Typed access to one file's metadata.  Keys are looked up as prefix + key
// (the architecture prefix, "qwen3." or "<general.architecture>."), and
// every error text starts with `who`.
class Reader {
public:
    Reader(const gg::File& f, std::string who, std::string prefix = {})
        : f_(f), who_(std::move(who)), prefix_(std::move(prefix)) {}

    [[noreturn]] void fail(const std::string& msg) const { throw std::runtime_error(who_ + msg); }

    const gg::Value* raw(std::string_view key, bool prefixed = true) const {
        return f_.find_meta(prefixed ? full(key) : std::string(key));
    }
    std::optional<int> integer(std::string_view key) const {
        const gg::Value* v = raw(key);
        if (!v) return std::nullopt;
        const std::optional<double> d = scalar_value(*v);
        if (!d || is_float_type(v->type)) fail("metadata '" + full(key) + "' is not an integer scalar");
        return static_cast<int>(static_cast<long long>(*d));
    }
    std::optional<float> real(std::string_view key) const {
        const gg::Value* v = raw(key);
        if (!v) return std::nullopt;
        if (!is_float_type(v->type)) fail("metadata '" + full(key) + "' is not a float scalar");
        return static_cast<float>(*scalar_value(*v));
    }
    int required(std::string_view key) const {
        const std::optional<int> v = integer(key);
        if (!v) fail("missing metadata '" + full(key) + "'");
        return *v;
    }
    const gg::File& file() const { return f_; }

private:
    std::string full(std::string_view key) const { return prefix_ + std::string(key); }

    const gg::File& f_;
    std::string who_, prefix_;
};

// One integer field of config C: required, or filled by `fallback` (from the
// fields read before it) when the key is missing, or left at C's default
// when fallback is null.
template <class C>
struct IntRow {
    std::string_view key;
    int C::* field;
    bool required;
    int (*fallback)(const C&);
};
// One float field: read when present, else C's default stays.
template <class C>
struct RealRow {
    std::string_view key;
    float C::* field;
};

template <class C, class IntRows, class RealRows>
void read_rows(const Reader& m, const IntRows& ints, const RealRows& reals, C& c) {
    for (const IntRow<C>& r : ints) {
        if (r.required) {
            c.*r.field = m.required(r.key);
        } else if (const std::optional<int> v = m.integer(r.key)) {
            c.*r.field = *v;
        } else if (r.fallback) {
            c.*r.field = r.fallback(c);
        }
    }
    for (const RealRow<C>& r : reals)
        if (const std::optional<float> v = m.real(r.key)) c.*r.field = *v;
}

// Vocabulary size: the length of the embedded tokenizer's token list when
// there is one, else <prefix>vocab_size, else `dflt`.
inline int vocab_size(const Reader& m, int dflt) {
    const gg::Value* toks = m.raw("tokenizer.ggml.tokens", false);
    if (toks && toks->type == gg::ValueType::Array) return static_cast<int>(toks->array.size());
    if (const std::optional<int> v = m.integer("vocab_size")) return *v;
    return dflt;
}

// ---- HF -> ggml tensor names ------------------------------------------------

struct NamePair {
    std::string_view hf, ggml;
    bool qk_norm;   // exists only in decoders with per-head q / k RMSNorm
};
inline constexpr NamePair kWholeModel[] = {
    {"model.embed_tokens.weight", "token_embd.weight", false},
    {"model.norm.weight", "output_norm.weight", false},
    {"lm_head.weight", "output.weight", false},
};
// The suffix after "model.layers.<i>." and after "blk.<i>.".
inline constexpr NamePair kPerLayer[] = {
    {"self_attn.q_proj.weight", "attn_q.weight", false},
    {"self_attn.k_proj.weight", "attn_k.weight", false},
    {"self_attn.v_proj.weight", "attn_v.weight", false},
    {"self_attn.o_proj.weight", "attn_output.weight", false},
    {"self_attn.q_norm.weight", "attn_q_norm.weight", true},
    {"self_attn.k_norm.weight", "attn_k_norm.weight", true},
    {"input_layernorm.weight", "attn_norm.weight", false},
    {"post_attention_layernorm.weight", "ffn_norm.weight", false},
    {"mlp.gate_proj.weight", "ffn_gate.weight", false},
    {"mlp.up_proj.weight", "ffn_up.weight", false},
    {"mlp.down_proj.weight", "ffn_down.weight", false},
};

// The ggml name of a dense decoder's HF tensor name; empty when the name is
// not one of its weights (with_qk_norm: the q / k head norms exist).
inline std::string hf_to_ggml(std::string_view hf, bool with_qk_norm) {
    for (const NamePair& p : kWholeModel)
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
    for (const NamePair& p : kPerLayer)
        if (suffix == p.hf && (with_qk_norm || !p.qk_norm))
            return "blk." + std::string(rest.substr(0, ndig)) + "." + std::string(p.ggml);
    return {};
}

// The dense decoder's configuration from a facade's config (Qwen3Config,
// Mistral3Config::Text: the same field names); qk_norm is the architectural
// switch between the two.
template <class C>
DenseDecoderConfig decoder_config(const C& c, bool qk_norm) {
    DenseDecoderConfig d;
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
    d.use_qk_norm = qk_norm;
    return d;
}

}  // namespace brolm::detail::meta
