// Mistral 3.1 text facade (reference include/brolm/mistral3_config.h:30-143,
// include/brolm/mistral3_text.h:52-131): the configuration from config.json
// or GGUF metadata, the HF -> ggml tensor-name map, and the GGUF loads over
// the dense decoder with per-head QK-norm off.
//
// The JSON keys, the GGUF metadata keys (every model key prefixed with the
// file's general.architecture, "llama" or "mistral"), the tensor names and
// the error texts are the reference's contract (src/mistral3_config.cpp:
// 36-93, :130-191, :222-246; src/mistral3_text.cpp:70-110).  Everything
// else is tables: a JSON row per config member, the GGUF rows shared with
// the Qwen3 facade's reader (meta_tables.h), and validation as a list of
// (condition, message) rules.
#include "brolm/mistral3_config.h"
#include "brolm/mistral3_generate.h"
#include "brolm/mistral3_text.h"

#include <fstream>
#include <iterator>
#include <stdexcept>
#include <string>
#include <string_view>
#include <variant>
#include <vector>

#include "brolm/detail/json.h"
#include "brolm/detail/weights.h"
#include "brotensor/gguf.h"
#include "meta_tables.h"

namespace brolm::mistral3 {

namespace gg = ::brotensor::gguf;
namespace js = ::brolm::detail::json;
namespace mt = ::brolm::detail::meta;

using Text = Mistral3Config::Text;

namespace {

constexpr const char* kConfigWho = "mistral3::Mistral3Config: ";

[[noreturn]] void config_error(const std::string& msg) { throw std::runtime_error(kConfigWho + msg); }

// ---- config.json -------------------------------------------------------------

// A JSON member of object type O: its key and the member it sets.  A key that
// is missing or null leaves the default; a value of the wrong JSON type is an
// error naming the key.
template <class O>
struct JsonRow {
    std::string_view key;
    std::variant<int O::*, float O::*, bool O::*> field;
};

template <class O, std::size_t N>
void apply_rows(const js::Value& obj, const JsonRow<O> (&rows)[N], O& out) {
    for (const JsonRow<O>& r : rows) {
        const js::Value* v = obj.find(r.key);
        if (!v || v->kind == js::Value::Kind::Null) continue;
        const std::string quoted = "'" + std::string(r.key) + "'";
        if (std::holds_alternative<bool O::*>(r.field)) {
            if (!v->is_bool()) config_error(quoted + " is not a boolean");
            out.*std::get<bool O::*>(r.field) = v->b;
        } else {
            if (!v->is_number()) config_error(quoted + " is not a number");
            if (auto p = std::get_if<int O::*>(&r.field)) out.**p = static_cast<int>(v->num);
            else out.*std::get<float O::*>(r.field) = static_cast<float>(v->num);
        }
    }
}

// Top-level multimodal glue, kept for API parity.
const JsonRow<Mistral3Config> kTopRows[] = {
    {"image_token_index", &Mistral3Config::image_token_index},
    {"spatial_merge_size", &Mistral3Config::spatial_merge_size},
    {"multimodal_projector_bias", &Mistral3Config::multimodal_projector_bias},
};
// text_config.
const JsonRow<Text> kTextRows[] = {
    {"vocab_size", &Text::vocab_size},
    {"hidden_size", &Text::hidden_size},
    {"intermediate_size", &Text::intermediate_size},
    {"num_hidden_layers", &Text::num_hidden_layers},
    {"num_attention_heads", &Text::num_attention_heads},
    {"num_key_value_heads", &Text::num_key_value_heads},
    {"head_dim", &Text::head_dim},
    {"rms_norm_eps", &Text::rms_norm_eps},
    {"rope_theta", &Text::rope_theta},
    {"tie_word_embeddings", &Text::tie_word_embeddings},
    {"max_position_embeddings", &Text::max_position_embeddings},
};

// sliding_window: a number turns the window on; null or absent keeps full
// causal attention.
void read_window(const js::Value& tc, Text& t) {
    const js::Value* sw = tc.find("sliding_window");
    t.has_sliding_window = sw && sw->is_number();
    t.sliding_window = t.has_sliding_window ? static_cast<int>(sw->num) : 0;
}

// ---- GGUF metadata (keys after "<general.architecture>.") ---------------------

const mt::IntRow<Text> kGgufInts[] = {
    {"embedding_length", &Text::hidden_size, true, nullptr},
    {"feed_forward_length", &Text::intermediate_size, true, nullptr},
    {"block_count", &Text::num_hidden_layers, true, nullptr},
    {"attention.head_count", &Text::num_attention_heads, true, nullptr},
    {"attention.head_count_kv", &Text::num_key_value_heads, false,
     [](const Text& t) { return t.num_attention_heads; }},
    // Mistral 3.1's head_dim (128) is not hidden / heads (160): the derived
    // value is only for files without the key
    {"attention.key_length", &Text::head_dim, false, [](const Text& t) { return t.hidden_size / t.num_attention_heads; }},
    {"context_length", &Text::max_position_embeddings, false, nullptr},
};
const mt::RealRow<Text> kGgufReals[] = {
    {"attention.layer_norm_rms_epsilon", &Text::rms_norm_eps},
    {"rope.freq_base", &Text::rope_theta},
};

// ---- validation ----------------------------------------------------------------

struct Rule {
    bool (*broken)(const Mistral3Config&);
    const char* message;
};
const Rule kRules[] = {
    {[](const Mistral3Config& c) {
         const Text& t = c.text;
         return t.hidden_size <= 0 || t.intermediate_size <= 0 || t.num_hidden_layers <= 0 || t.vocab_size <= 0 ||
                t.head_dim <= 0;
     },
     "text_config has non-positive dimension"},
    {[](const Mistral3Config& c) { return c.text.num_attention_heads <= 0 || c.text.num_key_value_heads <= 0; },
     "num_attention_heads / num_key_value_heads must be positive"},
    {[](const Mistral3Config& c) { return c.text.num_attention_heads % c.text.num_key_value_heads != 0; },
     "num_attention_heads must be a multiple of num_key_value_heads"},
    {[](const Mistral3Config& c) { return c.text.head_dim % 2 != 0; }, "head_dim must be even (RoPE rotates pairs)"},
    {[](const Mistral3Config& c) { return c.spatial_merge_size <= 0; }, "spatial_merge_size must be positive"},
};

}  // namespace

Mistral3Config Mistral3Config::load(const std::string& path) {
    std::ifstream in(path, std::ios::binary);
    if (!in) config_error("cannot open '" + path + "'");
    return from_json_text(std::string(std::istreambuf_iterator<char>(in), std::istreambuf_iterator<char>()));
}

Mistral3Config Mistral3Config::from_json_text(const std::string& text) {
    js::Value root;
    try {
        root = js::parse(text);
    } catch (const std::exception& e) {
        config_error(std::string("json parse: ") + e.what());
    }
    if (!root.is_object()) config_error("root is not a JSON object");
    Mistral3Config cfg;
    apply_rows(root, kTopRows, cfg);
    const js::Value* tc = root.find("text_config");
    if (!tc) config_error("missing text_config");
    if (!tc->is_object()) config_error("text_config is not an object");
    apply_rows(*tc, kTextRows, cfg.text);
    read_window(*tc, cfg.text);
    // the vision tower is outside this build; its section must still exist
    if (!root.find("vision_config")) config_error("missing vision_config");
    cfg.validate();
    return cfg;
}

Mistral3Config Mistral3Config::from_gguf(const gg::File& f) {
    const std::string who = std::string(kConfigWho) + "from_gguf: ";
    const gg::Value* arch = f.find_meta("general.architecture");
    if (!arch) throw std::runtime_error(who + "missing metadata 'general.architecture'");
    if (arch->type != gg::ValueType::String) throw std::runtime_error(who + "general.architecture is not a string");
    const mt::Reader m(f, who, arch->str + ".");
    Mistral3Config cfg;
    mt::read_rows(m, kGgufInts, kGgufReals, cfg.text);
    cfg.text.vocab_size = mt::vocab_size(m, cfg.text.vocab_size);
    // Mistral checkpoints carry their own lm_head; without one it is tied
    cfg.text.tie_word_embeddings = f.find_tensor("output.weight") == nullptr;
    cfg.validate();
    return cfg;
}

void Mistral3Config::validate() const {
    for (const Rule& r : kRules)
        if (r.broken(*this)) config_error(r.message);
}

std::string mistral3_hf_to_ggml(std::string_view hf_name) { return mt::hf_to_ggml(hf_name, /*with_qk_norm=*/false); }

TextModel::TextModel(const Mistral3Config::Text& cfg) : cfg_(cfg), core_(mt::decoder_config(cfg, /*qk_norm=*/false)) {}
TextModel::~TextModel() = default;

void TextModel::load_weights(const gg::File& f) { load_weights(std::vector<const gg::File*>{&f}); }

void TextModel::load_weights(const std::vector<const gg::File*>& shards) {
    if (shards.empty()) throw std::runtime_error("mistral3::TextModel: load_weights: no gguf shards");
    const brolm::detail::weights::GgufSource src(shards, [](std::string_view hf) { return mistral3_hf_to_ggml(hf); });
    core_.load_weights(src);
}

std::vector<int32_t> generate(TextModel& model, const std::vector<int32_t>& prompt_ids, int eos_id,
                              const GenerateOptions& opts) {
    return brolm::detail::generate(model, prompt_ids, eos_id, opts);
}

}  // namespace brolm::mistral3
