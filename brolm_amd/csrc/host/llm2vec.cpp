// LLM2Vec encoder facade (reference include/brolm/llm2vec.h:31-114): the flat
// HF LLaMA config.json, GGUF weights through the Mistral / Llama tensor-name
// map, and the bidirectional encode (DenseDecoder::forward_encode) with masked
// mean pooling on the device.
//
// Kept from the reference: the config.json keys, the defaults of Config, the
// validation rules and the error texts (src/llm2vec.cpp:70-120).  The parse is
// a table of (key, member) rows, the validation a table of (rule, message)
// rows checked in order.
#include "brolm/llm2vec.h"

#include <array>
#include <fstream>
#include <iterator>
#include <stdexcept>
#include <string>
#include <string_view>
#include <variant>
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

struct ConfigError : std::runtime_error {
    explicit ConfigError(const std::string& m) : std::runtime_error("llm2vec::Config: " + m) {}
};

// config.json members read into Config; an absent or null member keeps the
// default, a member of another JSON kind is an error.
using Member = std::variant<int Config::*, float Config::*>;
struct JsonField {
    const char* key;
    Member member;
};
const std::array<JsonField, 8> kFields = {{
    {"vocab_size", &Config::vocab_size},
    {"hidden_size", &Config::hidden_size},
    {"intermediate_size", &Config::intermediate_size},
    {"num_hidden_layers", &Config::num_hidden_layers},
    {"num_attention_heads", &Config::num_attention_heads},
    {"num_key_value_heads", &Config::num_key_value_heads},
    {"rms_norm_eps", &Config::rms_norm_eps},
    {"rope_theta", &Config::rope_theta},
}};

void read_field(const js::Value& root, const JsonField& f, Config& c) {
    const js::Value* v = root.find(f.key);
    if (!v || v->kind == js::Value::Kind::Null) return;
    if (!v->is_number()) throw ConfigError(std::string("'") + f.key + "' is not a number");
    std::visit([&](auto m) { c.*m = static_cast<std::remove_reference_t<decltype(c.*m)>>(v->num); }, f.member);
}

// Validation rules in the order they are reported.
struct Rule {
    bool (*bad)(const Config&);
    const char* message;
};
const std::array<Rule, 4> kRules = {{
    {[](const Config& c) {
         return c.hidden_size <= 0 || c.intermediate_size <= 0 || c.num_hidden_layers <= 0 || c.vocab_size <= 0 ||
                c.head_dim <= 0;
     },
     "non-positive dimension"},
    {[](const Config& c) { return c.num_attention_heads <= 0 || c.num_key_value_heads <= 0; },
     "num_attention_heads / num_key_value_heads must be positive"},
    {[](const Config& c) { return c.num_attention_heads % c.num_key_value_heads != 0; },
     "num_attention_heads must be a multiple of num_key_value_heads"},
    {[](const Config& c) { return c.head_dim % 2 != 0; }, "head_dim must be even (RoPE rotates pairs)"},
}};

// The dense decoder this encoder runs: LLaMA (no QK-norm), lm_head tied to the
// embedding because encode never reaches it, so output.weight may be absent.
brolm::detail::DenseDecoderConfig decoder_config(const Config& c) {
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
    d.tie_word_embeddings = true;
    return d;
}

}  // namespace

Config Config::load(const std::string& path) {
    std::ifstream in(path, std::ios::binary);
    if (!in) throw ConfigError("cannot open '" + path + "'");
    return from_json_text(std::string(std::istreambuf_iterator<char>(in), std::istreambuf_iterator<char>()));
}

Config Config::from_json_text(const std::string& text) {
    js::Value root;
    try {
        root = js::parse(text);
    } catch (const std::exception& e) {
        throw ConfigError(std::string("json parse: ") + e.what());
    }
    if (!root.is_object()) throw ConfigError("root is not a JSON object");
    Config c;
    for (const JsonField& f : kFields) read_field(root, f, c);
    // HF LLaMA configs usually leave head_dim out: hidden / heads then.
    const js::Value* hd = root.find("head_dim");
    c.head_dim = (hd && hd->is_number()) ? static_cast<int>(hd->num)
                 : c.num_attention_heads > 0 ? c.hidden_size / c.num_attention_heads
                                             : 0;
    c.validate();
    return c;
}

void Config::validate() const {
    for (const Rule& r : kRules)
        if (r.bad(*this)) throw ConfigError(r.message);
}

Encoder::Encoder(const Config& cfg) : cfg_(cfg), core_(decoder_config(cfg)) {}
Encoder::~Encoder() = default;

void Encoder::load_weights(const gg::File& f) { load_weights(std::vector<const gg::File*>{&f}); }

void Encoder::load_weights(const std::vector<const gg::File*>& shards) {
    if (shards.empty()) throw std::runtime_error("llm2vec::Encoder: load_weights: no gguf shards");
    const brolm::detail::weights::GgufSource src(
        shards, [](std::string_view hf) { return brolm::mistral3::mistral3_hf_to_ggml(hf); });
    core_.load_weights(src);
}

void Encoder::encode(const int32_t* ids, int L, bt::Tensor& hidden_out) { core_.forward_encode(ids, L, hidden_out); }

void Encoder::encode_pooled(const int32_t* ids, int L, bt::Tensor& emb_out, const float* pool_mask) {
    bt::Tensor hidden;
    core_.forward_encode(ids, L, hidden);
    // The pool reads its (L) weights from HBM; null means every row counts.
    const bt::Tensor weights = pool_mask ? bt::Tensor::from_host_on(bt::Device::ROCm, pool_mask, L, 1) : bt::Tensor();
    bt::masked_mean_pool_forward(hidden, pool_mask ? static_cast<const float*>(weights.data) : nullptr, emb_out);
}

}  // namespace brolm::llm2vec
