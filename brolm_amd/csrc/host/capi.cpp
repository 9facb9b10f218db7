// C facade of the Qwen3 and Mistral 3.1 text stacks (include/brolm_c.h).
#include "brolm_c.h"

#include <algorithm>
#include <chrono>
#include <cstring>
#include <exception>
#include <memory>
#include <random>
#include <string>
#include <vector>

#include "brolm/detail/profile.h"
#include "brolm/llm2vec.h"
#include "brolm/mistral3_generate.h"
#include "brolm/mistral3_text.h"
#include "brolm/qwen.h"
#include "brolm/qwen_generate.h"
#include "brolm/qwen_tokenizer.h"
#include "brolm/synth.h"
#include "brotensor/gguf.h"
#include "brotensor/runtime.h"

// A decoder handle: holds a Qwen3Model or a Mistral 3.1 TextModel; both
// wrap one DenseDecoder.
struct brolm_qwen3 {
    std::unique_ptr<brolm::qwen::Qwen3Model> model;
    std::unique_ptr<brolm::mistral3::TextModel> mistral;
    std::unique_ptr<brolm::llm2vec::Encoder> encoder;
    brolm::detail::DenseDecoder* core = nullptr;
};

struct brolm_tokenizer {
    std::unique_ptr<brolm::qwen::Tokenizer> tok;
};

namespace {

thread_local std::string g_err;

template <typename F>
int guard(F&& f) {
    try {
        f();
        return 0;
    } catch (const std::exception& e) {
        g_err = e.what();
    } catch (...) {
        g_err = "unknown C++ exception";
    }
    return -1;
}

brolm::qwen::Qwen3Config to_cfg(const brolm_qwen3_config& c) {
    brolm::qwen::Qwen3Config q;
    q.vocab_size = c.vocab_size;
    q.hidden_size = c.hidden_size;
    q.intermediate_size = c.intermediate_size;
    q.num_hidden_layers = c.num_hidden_layers;
    q.num_attention_heads = c.num_attention_heads;
    q.num_key_value_heads = c.num_key_value_heads;
    q.head_dim = c.head_dim;
    q.rms_norm_eps = c.rms_norm_eps;
    q.rope_theta = c.rope_theta;
    q.tie_word_embeddings = c.tie_word_embeddings != 0;
    q.max_position_embeddings = c.max_position_embeddings;
    return q;
}

void from_cfg(const brolm::qwen::Qwen3Config& q, brolm_qwen3_config* c) {
    c->vocab_size = q.vocab_size;
    c->hidden_size = q.hidden_size;
    c->intermediate_size = q.intermediate_size;
    c->num_hidden_layers = q.num_hidden_layers;
    c->num_attention_heads = q.num_attention_heads;
    c->num_key_value_heads = q.num_key_value_heads;
    c->head_dim = q.head_dim;
    c->rms_norm_eps = q.rms_norm_eps;
    c->rope_theta = q.rope_theta;
    c->tie_word_embeddings = q.tie_word_embeddings ? 1 : 0;
    c->max_position_embeddings = q.max_position_embeddings;
}

void to_host_f32(const brotensor::Tensor& t, float* dst) {
    const std::vector<float> v = t.to_host_vector();
    std::memcpy(dst, v.data(), v.size() * sizeof(float));
}

brolm::qwen::Qwen3Model& model_of(brolm_qwen3* m) {
    if (!m || !m->core) throw std::runtime_error("null model handle");
    if (!m->model) throw std::runtime_error("this call needs a Qwen3 model handle");
    return *m->model;
}

brolm::detail::DenseDecoder& core_of(brolm_qwen3* m) {
    if (!m || !m->core) throw std::runtime_error("null model handle");
    return *m->core;
}

}  // namespace

namespace {

std::vector<std::string> split_lines(const char* s) {
    std::vector<std::string> out;
    if (!s) return out;
    std::string cur;
    for (const char* p = s; *p; ++p) {
        if (*p == '\n') {
            if (!cur.empty()) out.push_back(cur);
            cur.clear();
        } else {
            cur += *p;
        }
    }
    if (!cur.empty()) out.push_back(cur);
    return out;
}

template <class Make>
brolm_tokenizer* make_tokenizer(Make&& make) {
    brolm_tokenizer* h = nullptr;
    guard([&] { h = new brolm_tokenizer{std::make_unique<brolm::qwen::Tokenizer>(make())}; });
    return h;
}

const brolm::qwen::Tokenizer& tok_of(const brolm_tokenizer* t) {
    if (!t || !t->tok) throw std::runtime_error("null tokenizer");
    return *t->tok;
}

int64_t put_string(const std::string& s, char* out, int64_t cap) {
    if (out && cap > 0) std::memcpy(out, s.data(), static_cast<std::size_t>(std::min<int64_t>(cap, s.size())));
    return static_cast<int64_t>(s.size());
}

}  // namespace

extern "C" {

const char* brolm_last_error(void) { return g_err.c_str(); }

int brolm_init(void) {
    return guard([] { brotensor::init(); });
}

int brolm_shutdown(void) {
    return guard([] { brotensor::shutdown(); });
}

namespace {

int synth_write(const brolm_synth_qwen3_spec* s, const char* path, const char* arch) {
    return guard([&] {
        if (!s || !path) throw std::runtime_error("synth: null argument");
        brolm::synth::Qwen3Spec q;
        q.vocab = s->vocab; q.hidden = s->hidden; q.intermediate = s->intermediate; q.layers = s->layers;
        q.n_q = s->n_q; q.n_kv = s->n_kv; q.head_dim = s->head_dim; q.eps = s->eps; q.theta = s->theta;
        q.context = s->context; q.tied = s->tied != 0;
        q.embed = brotensor::dtype_from_ggml(s->embed_type);
        q.q = brotensor::dtype_from_ggml(s->q_type);
        q.k = brotensor::dtype_from_ggml(s->k_type);
        q.v = brotensor::dtype_from_ggml(s->v_type);
        q.o = brotensor::dtype_from_ggml(s->o_type);
        q.gate = brotensor::dtype_from_ggml(s->gate_type);
        q.up = brotensor::dtype_from_ggml(s->up_type);
        q.down = brotensor::dtype_from_ggml(s->down_type);
        q.output = brotensor::dtype_from_ggml(s->output_type);
        q.stddev = s->stddev;
        q.seed = s->seed;
        q.more_bits_type = s->more_bits_type;
        if (q.more_bits_type >= 0) (void)brotensor::dtype_from_ggml(q.more_bits_type);  // throws if unknown
        q.arch = arch;
        brolm::synth::write_qwen3_gguf(q, path);
    });
}

}  // namespace

int brolm_synth_mistral3_write(const brolm_synth_qwen3_spec* s, const char* path) {
    return synth_write(s, path, "llama");
}

int brolm_synth_qwen3_write(const brolm_synth_qwen3_spec* s, const char* path) {
    return synth_write(s, path, "qwen3");
}

int brolm_synth_normal_bf16(uint64_t key, int64_t n, float stddev, float* out) {
    return guard([&] { brolm::synth::normal_bf16(key, n, stddev, out); });
}

uint64_t brolm_synth_tensor_key(uint64_t seed, const char* name) { return brolm::synth::tensor_key(seed, name); }

int brolm_synth_quantize(int ggml_type, const float* src, int64_t n, uint8_t* dst) {
    return guard([&] { brolm::synth::quantize(brotensor::dtype_from_ggml(ggml_type), src, n, dst); });
}

int brolm_qwen3_hf_to_ggml(const char* hf_name, char* out, int cap) {
    const std::string s = brolm::qwen::qwen3_hf_to_ggml(hf_name ? hf_name : "");
    if (out && cap > 0) {
        const std::size_t n = std::min<std::size_t>(s.size(), static_cast<std::size_t>(cap - 1));
        std::memcpy(out, s.data(), n);
        out[n] = 0;
    }
    return static_cast<int>(s.size());
}

int brolm_qwen3_config_from_gguf(const char* path, brolm_qwen3_config* out) {
    return guard([&] {
        const brotensor::gguf::File f = brotensor::gguf::File::open(path);
        from_cfg(brolm::qwen::Qwen3Config::from_gguf(f), out);
    });
}

int brolm_gguf_tensor_count(const char* path, int64_t* out) {
    return guard([&] {
        const brotensor::gguf::File f = brotensor::gguf::File::open(path);
        *out = static_cast<int64_t>(f.tensor_count());
    });
}

int brolm_gguf_tensor_info(const char* path, const char* name, int* ggml_type, int64_t* dims4, int* ndims,
                           int64_t* nbytes) {
    return guard([&] {
        const brotensor::gguf::File f = brotensor::gguf::File::open(path);
        const auto* t = f.find_tensor(name);
        if (!t) throw std::runtime_error(std::string("gguf: no tensor '") + name + "'");
        *ggml_type = brotensor::dtype_to_ggml(t->dtype);
        *ndims = static_cast<int>(t->dims.size());
        for (int i = 0; i < 4; ++i) dims4[i] = i < *ndims ? t->dims[static_cast<std::size_t>(i)] : 1;
        *nbytes = static_cast<int64_t>(t->nbytes);
    });
}

namespace {

const brotensor::gguf::Value& need_meta(const brotensor::gguf::File& f, const char* key) {
    const brotensor::gguf::Value* v = f.find_meta(key);
    if (!v) throw std::runtime_error(std::string("gguf: no metadata '") + key + "'");
    return *v;
}

}  // namespace

int64_t brolm_gguf_tensor_data(const char* path, const char* name, uint8_t* out, int64_t cap) {
    int64_t n = -1;
    const int rc = guard([&] {
        const brotensor::gguf::File f = brotensor::gguf::File::open(path);
        const auto* t = f.find_tensor(name);
        if (!t) throw std::runtime_error(std::string("gguf: no tensor '") + name + "'");
        if (static_cast<int64_t>(t->nbytes) > cap) throw std::runtime_error("gguf: output buffer too small");
        std::memcpy(out, t->data, t->nbytes);
        n = static_cast<int64_t>(t->nbytes);
    });
    return rc == 0 ? n : -1;
}

int brolm_gguf_meta_int(const char* path, const char* key, int64_t* out) {
    return guard([&] {
        using T = brotensor::gguf::ValueType;
        const brotensor::gguf::File f = brotensor::gguf::File::open(path);
        const auto& v = need_meta(f, key);
        switch (v.type) {
            case T::U8: *out = v.scalar.u8; break;
            case T::I8: *out = v.scalar.i8; break;
            case T::U16: *out = v.scalar.u16; break;
            case T::I16: *out = v.scalar.i16; break;
            case T::U32: *out = v.scalar.u32; break;
            case T::I32: *out = v.scalar.i32; break;
            case T::U64: *out = static_cast<int64_t>(v.scalar.u64); break;
            case T::I64: *out = v.scalar.i64; break;
            case T::Bool: *out = v.scalar.b ? 1 : 0; break;
            default: throw std::runtime_error(std::string("gguf: metadata '") + key + "' is not an integer");
        }
    });
}

int brolm_gguf_meta_f64(const char* path, const char* key, double* out) {
    return guard([&] {
        using T = brotensor::gguf::ValueType;
        const brotensor::gguf::File f = brotensor::gguf::File::open(path);
        const auto& v = need_meta(f, key);
        if (v.type == T::F32) *out = v.scalar.f32;
        else if (v.type == T::F64) *out = v.scalar.f64;
        else throw std::runtime_error(std::string("gguf: metadata '") + key + "' is not a float");
    });
}

int64_t brolm_gguf_meta_str(const char* path, const char* key, char* out, int64_t cap) {
    int64_t n = -1;
    const int rc = guard([&] {
        const brotensor::gguf::File f = brotensor::gguf::File::open(path);
        const auto& v = need_meta(f, key);
        if (v.type != brotensor::gguf::ValueType::String)
            throw std::runtime_error(std::string("gguf: metadata '") + key + "' is not a string");
        if (static_cast<int64_t>(v.str.size()) > cap) throw std::runtime_error("gguf: output buffer too small");
        std::memcpy(out, v.str.data(), v.str.size());
        n = static_cast<int64_t>(v.str.size());
    });
    return rc == 0 ? n : -1;
}

int brolm_gguf_meta_array(const char* path, const char* key, int* elem_type, int64_t* count) {
    return guard([&] {
        const brotensor::gguf::File f = brotensor::gguf::File::open(path);
        const auto& v = need_meta(f, key);
        if (v.type != brotensor::gguf::ValueType::Array)
            throw std::runtime_error(std::string("gguf: metadata '") + key + "' is not an array");
        *elem_type = static_cast<int>(v.array_type);
        *count = static_cast<int64_t>(v.array.size());
    });
}

int brolm_gguf_parse_memory(const uint8_t* data, int64_t size, int64_t* n_tensors) {
    return guard([&] {
        if (size < 0 || (!data && size > 0)) throw std::runtime_error("gguf: bad buffer");
        std::vector<std::uint8_t> bytes(data, data + size);
        const brotensor::gguf::File f = brotensor::gguf::File::from_memory(std::move(bytes));
        *n_tensors = static_cast<int64_t>(f.tensor_count());
    });
}

brolm_qwen3* brolm_qwen3_create(const brolm_qwen3_config* cfg) {
    brolm_qwen3* out = nullptr;
    const int rc = guard([&] {
        if (!cfg) throw std::runtime_error("null config");
        auto h = std::make_unique<brolm_qwen3>();
        h->model = std::make_unique<brolm::qwen::Qwen3Model>(to_cfg(*cfg));
        h->core = &h->model->core();
        out = h.release();
    });
    return rc == 0 ? out : nullptr;
}

namespace {

void from_m3(const brolm::mistral3::Mistral3Config& m, brolm_mistral3_config* c) {
    const auto& t = m.text;
    brolm_mistral3_text_config& o = c->text;
    o.vocab_size = t.vocab_size; o.hidden_size = t.hidden_size; o.intermediate_size = t.intermediate_size;
    o.num_hidden_layers = t.num_hidden_layers; o.num_attention_heads = t.num_attention_heads;
    o.num_key_value_heads = t.num_key_value_heads; o.head_dim = t.head_dim;
    o.rms_norm_eps = t.rms_norm_eps; o.rope_theta = t.rope_theta;
    o.tie_word_embeddings = t.tie_word_embeddings ? 1 : 0; o.max_position_embeddings = t.max_position_embeddings;
    o.has_sliding_window = t.has_sliding_window ? 1 : 0; o.sliding_window = t.sliding_window;
    c->image_token_index = m.image_token_index;
    c->spatial_merge_size = m.spatial_merge_size;
    c->multimodal_projector_bias = m.multimodal_projector_bias ? 1 : 0;
}

}  // namespace

int brolm_mistral3_config_from_gguf(const char* path, brolm_mistral3_config* out) {
    return guard([&] {
        if (!path || !out) throw std::runtime_error("null argument");
        const brotensor::gguf::File f = brotensor::gguf::File::open(path);
        from_m3(brolm::mistral3::Mistral3Config::from_gguf(f), out);
    });
}

int brolm_mistral3_config_from_json(const char* text, brolm_mistral3_config* out) {
    return guard([&] {
        if (!text || !out) throw std::runtime_error("null argument");
        from_m3(brolm::mistral3::Mistral3Config::from_json_text(text), out);
    });
}

int brolm_mistral3_hf_to_ggml(const char* hf_name, char* out, int cap) {
    const std::string s = brolm::mistral3::mistral3_hf_to_ggml(hf_name ? hf_name : "");
    if (out && cap > 0) {
        const std::size_t n = std::min<std::size_t>(s.size(), static_cast<std::size_t>(cap - 1));
        std::memcpy(out, s.data(), n);
        out[n] = 0;
    }
    return static_cast<int>(s.size());
}

brolm_qwen3* brolm_mistral3_text_create(const brolm_mistral3_text_config* cfg) {
    brolm_qwen3* out = nullptr;
    const int rc = guard([&] {
        if (!cfg) throw std::runtime_error("null config");
        brolm::mistral3::Mistral3Config::Text t;
        t.vocab_size = cfg->vocab_size; t.hidden_size = cfg->hidden_size;
        t.intermediate_size = cfg->intermediate_size; t.num_hidden_layers = cfg->num_hidden_layers;
        t.num_attention_heads = cfg->num_attention_heads; t.num_key_value_heads = cfg->num_key_value_heads;
        t.head_dim = cfg->head_dim; t.rms_norm_eps = cfg->rms_norm_eps; t.rope_theta = cfg->rope_theta;
        t.tie_word_embeddings = cfg->tie_word_embeddings != 0;
        t.max_position_embeddings = cfg->max_position_embeddings;
        t.has_sliding_window = cfg->has_sliding_window != 0; t.sliding_window = cfg->sliding_window;
        auto h = std::make_unique<brolm_qwen3>();
        h->mistral = std::make_unique<brolm::mistral3::TextModel>(t);
        h->core = &h->mistral->core();
        out = h.release();
    });
    return rc == 0 ? out : nullptr;
}

int brolm_llm2vec_config_from_json(const char* text, brolm_llm2vec_config* out) {
    return guard([&] {
        if (!text || !out) throw std::runtime_error("null argument");
        const brolm::llm2vec::Config c = brolm::llm2vec::Config::from_json_text(text);
        out->vocab_size = c.vocab_size; out->hidden_size = c.hidden_size;
        out->intermediate_size = c.intermediate_size; out->num_hidden_layers = c.num_hidden_layers;
        out->num_attention_heads = c.num_attention_heads; out->num_key_value_heads = c.num_key_value_heads;
        out->head_dim = c.head_dim; out->rms_norm_eps = c.rms_norm_eps; out->rope_theta = c.rope_theta;
    });
}

brolm_qwen3* brolm_llm2vec_create(const brolm_llm2vec_config* cfg) {
    brolm_qwen3* out = nullptr;
    const int rc = guard([&] {
        if (!cfg) throw std::runtime_error("null config");
        brolm::llm2vec::Config c;
        c.vocab_size = cfg->vocab_size; c.hidden_size = cfg->hidden_size;
        c.intermediate_size = cfg->intermediate_size; c.num_hidden_layers = cfg->num_hidden_layers;
        c.num_attention_heads = cfg->num_attention_heads; c.num_key_value_heads = cfg->num_key_value_heads;
        c.head_dim = cfg->head_dim; c.rms_norm_eps = cfg->rms_norm_eps; c.rope_theta = cfg->rope_theta;
        c.validate();
        auto h = std::make_unique<brolm_qwen3>();
        h->encoder = std::make_unique<brolm::llm2vec::Encoder>(c);
        h->core = &h->encoder->core();
        out = h.release();
    });
    return rc == 0 ? out : nullptr;
}

int brolm_decoder_forward_encode(brolm_qwen3* m, const int32_t* ids, int L, float* hidden) {
    return guard([&] {
        brotensor::Tensor hd;
        core_of(m).forward_encode(ids, L, hd);
        if (hidden) to_host_f32(hd, hidden);
    });
}

int brolm_llm2vec_encode_pooled(brolm_qwen3* m, const int32_t* ids, int L, const float* mask, float* emb) {
    return guard([&] {
        core_of(m);
        if (!m->encoder) throw std::runtime_error("encode_pooled needs an llm2vec handle");
        brotensor::Tensor e;
        m->encoder->encode_pooled(ids, L, e, mask);
        if (emb) to_host_f32(e, emb);
    });
}

void brolm_qwen3_free(brolm_qwen3* m) { delete m; }

int brolm_qwen3_load_gguf(brolm_qwen3* m, const char* path) {
    return guard([&] {
        brotensor::init();
        const brotensor::gguf::File f = brotensor::gguf::File::open(path);
        core_of(m);
        if (m->model) m->model->load_weights(f);
        else if (m->mistral) m->mistral->load_weights(f);
        else m->encoder->load_weights(f);
    });
}

int brolm_qwen3_allocate_cache(brolm_qwen3* m, int n) { return guard([&] { core_of(m).allocate_cache(n); }); }
int brolm_qwen3_reset_cache(brolm_qwen3* m) { return guard([&] { core_of(m).reset_cache(); }); }
int brolm_qwen3_truncate_cache(brolm_qwen3* m, int n) { return guard([&] { core_of(m).truncate_cache(n); }); }
int brolm_qwen3_cache_len(const brolm_qwen3* m) { return (m && m->core) ? m->core->cache_len() : -1; }

int brolm_qwen3_allocate_batch(brolm_qwen3* m, int n_slots, int max_seq_len) {
    return guard([&] { core_of(m).allocate_batch(n_slots, max_seq_len); });
}
int brolm_qwen3_slot_len(const brolm_qwen3* m, int slot) {
    int n = -1;
    const int rc = guard([&] {
        if (!m || !m->core) throw std::invalid_argument("null model handle");
        n = m->core->slot_len(slot);
    });
    return rc == 0 ? n : rc;
}
int brolm_qwen3_truncate_slot(brolm_qwen3* m, int slot, int len) {
    return guard([&] { core_of(m).truncate_slot(slot, len); });
}
int brolm_qwen3_prefill_slot(brolm_qwen3* m, int slot, const int32_t* ids, int L, float* logits) {
    return guard([&] {
        brotensor::Tensor lg;
        core_of(m).prefill_slot(slot, ids, L, lg);
        if (logits) to_host_f32(lg, logits);
    });
}
int brolm_qwen3_forward_batch(brolm_qwen3* m, const int32_t* ids, const int32_t* slots, int M, float* logits) {
    return guard([&] {
        brotensor::Tensor lg;
        core_of(m).forward_batch(ids, slots, M, lg);
        if (logits) to_host_f32(lg, logits);
    });
}
double brolm_qwen3_time_forward_batch(brolm_qwen3* m, const int32_t* ids, const int32_t* slots, int M, int n) {
    double ms = -1.0;
    const int rc = guard([&] {
        if (n <= 0) throw std::invalid_argument("time_forward_batch: n must be positive");
        brolm::detail::DenseDecoder& d = core_of(m);
        brotensor::Tensor lg;
        brotensor::sync_all();
        const auto t0 = std::chrono::steady_clock::now();
        for (int i = 0; i < n; ++i) d.forward_batch(ids, slots, M, lg);
        brotensor::sync_all();
        ms = std::chrono::duration<double, std::milli>(std::chrono::steady_clock::now() - t0).count() / n;
    });
    return rc == 0 ? ms : -1.0;
}

int brolm_qwen3_forward(brolm_qwen3* m, const int32_t* ids, int L, float* logits, float* hidden) {
    return guard([&] {
        brotensor::Tensor lg, hd;
        core_of(m).forward(ids, L, lg, hidden ? &hd : nullptr);
        if (logits) to_host_f32(lg, logits);
        if (hidden) to_host_f32(hd, hidden);
    });
}

int brolm_qwen3_forward_last(brolm_qwen3* m, const int32_t* ids, int L, float* logits) {
    return guard([&] {
        brotensor::Tensor lg;
        core_of(m).forward_last(ids, L, lg);
        if (logits) to_host_f32(lg, logits);
    });
}

int brolm_qwen3_embed_tokens(brolm_qwen3* m, const int32_t* ids, int L, uint16_t* out) {
    return guard([&] {
        brotensor::Tensor e;
        core_of(m).embed_tokens(ids, L, e);
        e.copy_to_host_fp16(out);
    });
}

int brolm_qwen3_forward_embeds(brolm_qwen3* m, const uint16_t* embeds, int L, float* logits, float* hidden) {
    return guard([&] {
        brolm::detail::DenseDecoder& q = core_of(m);
        brotensor::Tensor e = brotensor::Tensor::from_host_fp16(embeds, L, q.config().hidden_size);
        brotensor::Tensor lg, hd;
        q.forward_embeds(e, L, lg, hidden ? &hd : nullptr);
        if (logits) to_host_f32(lg, logits);
        if (hidden) to_host_f32(hd, hidden);
    });
}

int brolm_qwen3_generate(brolm_qwen3* m, const int32_t* prompt, int n_prompt, int max_new, int eos_id,
                         int stop_on_eos, float temperature, int top_k, float top_p, uint64_t seed,
                         int device_greedy, int device_sampling, int32_t* out) {
    int count = -1;
    const int rc = guard([&] {
        brolm::qwen::GenerateOptions o;
        o.max_new_tokens = max_new;
        o.stop_on_eos = stop_on_eos != 0;
        o.sampling.temperature = temperature;
        o.sampling.top_k = top_k;
        o.sampling.top_p = top_p;
        o.sampling.seed = seed;
        o.device_greedy = device_greedy != 0;
        o.device_sampling = device_sampling != 0;
        const std::vector<int32_t> p(prompt, prompt + (n_prompt > 0 ? n_prompt : 0));
        const std::vector<int32_t> g = brolm::detail::generate(core_of(m), p, eos_id, o);
        std::memcpy(out, g.data(), g.size() * sizeof(int32_t));
        count = static_cast<int>(g.size());
    });
    return rc == 0 ? count : -1;
}

brolm_tokenizer* brolm_tokenizer_load(const char* vocab_json, const char* merges_txt, const char* extra_specials) {
    return make_tokenizer([&] {
        if (!vocab_json || !merges_txt) throw std::runtime_error("brolm_tokenizer_load: null path");
        return brolm::qwen::Tokenizer::load(vocab_json, merges_txt, split_lines(extra_specials));
    });
}

brolm_tokenizer* brolm_tokenizer_from_gguf(const char* gguf_path, const char* extra_specials) {
    return make_tokenizer([&] {
        if (!gguf_path) throw std::runtime_error("brolm_tokenizer_from_gguf: null path");
        const brotensor::gguf::File f = brotensor::gguf::File::open(gguf_path);
        return brolm::qwen::Tokenizer::from_gguf(f, split_lines(extra_specials));
    });
}

brolm_tokenizer* brolm_tokenizer_from_json(const char* tokenizer_json, const char* extra_specials) {
    return make_tokenizer([&] {
        if (!tokenizer_json) throw std::runtime_error("brolm_tokenizer_from_json: null path");
        return brolm::qwen::Tokenizer::from_tokenizer_json(tokenizer_json, split_lines(extra_specials));
    });
}

void brolm_tokenizer_free(brolm_tokenizer* t) { delete t; }

int brolm_tokenizer_encode(const brolm_tokenizer* t, const char* text, int64_t len, int add_special, int32_t* ids,
                           int cap) {
    int count = -1;
    const int rc = guard([&] {
        if (!text && len > 0) throw std::runtime_error("brolm_tokenizer_encode: null text");
        const std::vector<int32_t> v =
            tok_of(t).encode(std::string_view(text ? text : "", static_cast<std::size_t>(len)), add_special != 0);
        if (ids && cap > 0) std::memcpy(ids, v.data(), std::min<std::size_t>(cap, v.size()) * sizeof(int32_t));
        count = static_cast<int>(v.size());
    });
    return rc == 0 ? count : -1;
}

int64_t brolm_tokenizer_decode(const brolm_tokenizer* t, const int32_t* ids, int n, char* out, int64_t cap) {
    int64_t len = -1;
    const int rc = guard([&] {
        const std::vector<int32_t> v(ids, ids + (n > 0 ? n : 0));
        len = put_string(tok_of(t).decode(v), out, cap);
    });
    return rc == 0 ? len : -1;
}

int64_t brolm_tokenizer_chat(const brolm_tokenizer* t, const char* const* roles, const char* const* contents, int n,
                             int add_generation_prompt, char* out, int64_t cap) {
    int64_t len = -1;
    const int rc = guard([&] {
        std::vector<std::pair<std::string, std::string>> msgs;
        for (int i = 0; i < n; ++i) msgs.emplace_back(roles[i] ? roles[i] : "", contents[i] ? contents[i] : "");
        len = put_string(tok_of(t).apply_chat_template(msgs, add_generation_prompt != 0), out, cap);
    });
    return rc == 0 ? len : -1;
}

int brolm_tokenizer_register_special(brolm_tokenizer* t, const char* token, int32_t id) {
    return guard([&] {
        if (!t || !t->tok || !token) throw std::runtime_error("brolm_tokenizer_register_special: null argument");
        t->tok->register_special_token(token, id);
    });
}

int brolm_tokenizer_info(const brolm_tokenizer* t, int64_t* info) {
    return guard([&] {
        const brolm::qwen::Tokenizer& k = tok_of(t);
        info[0] = static_cast<int64_t>(k.vocab_count());
        info[1] = static_cast<int64_t>(k.merge_count());
        info[2] = k.eos_id();
        info[3] = k.im_start_id();
        info[4] = k.im_end_id();
        info[5] = k.endoftext_id();
    });
}

int64_t brolm_qwen3_generate_text(brolm_qwen3* m, const brolm_tokenizer* t, const char* prompt, int max_new,
                                  int stop_on_eos, float temperature, int top_k, float top_p, uint64_t seed,
                                  char* out, int64_t cap) {
    int64_t len = -1;
    const int rc = guard([&] {
        brolm::qwen::GenerateOptions o;
        o.max_new_tokens = max_new;
        o.stop_on_eos = stop_on_eos != 0;
        o.sampling.temperature = temperature;
        o.sampling.top_k = top_k;
        o.sampling.top_p = top_p;
        o.sampling.seed = seed;
        len = put_string(brolm::qwen::generate_text(model_of(m), tok_of(t), prompt ? prompt : "", o), out, cap);
    });
    return rc == 0 ? len : -1;
}

int brolm_qwen3_decode_greedy(brolm_qwen3* m, int32_t token, int n, int32_t* out, int eos_id) {
    int count = -1;
    const int rc = guard([&] { count = core_of(m).decode_greedy(token, n, out, eos_id); });
    return rc == 0 ? count : -1;
}

int brolm_qwen3_decode_sampled(brolm_qwen3* m, int32_t token, int n, const double* u, float temperature, int top_k,
                               float top_p, int32_t* out, int eos_id) {
    int count = 0;
    const int rc = guard([&] {
        count = core_of(m).decode_sampled(token, n, u, temperature, top_k, top_p, out, eos_id);
    });
    return rc == 0 ? count : rc;
}

double brolm_qwen3_time_decode_steps(brolm_qwen3* m, int32_t token, int n) {
    double ms = -1.0;
    const int rc = guard([&] { ms = core_of(m).time_decode_steps(token, n); });
    return rc == 0 ? ms : -1.0;
}

int64_t brolm_qwen3_decode_weight_bytes(const brolm_qwen3* m) {
    return (m && m->core) ? m->core->decode_weight_bytes() : -1;
}

int brolm_qwen3_decode_mode(brolm_qwen3* m) {
    int mode = -1;
    const int rc = guard([&] { mode = core_of(m).decode_mode(); });
    return rc == 0 ? mode : -1;
}

int brolm_sample_token_device(const uint16_t* logits_dev, int vocab, float temperature, int top_k, float top_p,
                              uint64_t seed) {
    int tok = -1;
    const int rc = guard([&] {
        if (!logits_dev || vocab <= 0) throw std::runtime_error("sample_token_device: bad arguments");
        brolm::detail::SamplingParams p;
        p.temperature = temperature;
        p.top_k = top_k;
        p.top_p = top_p;
        std::mt19937_64 rng(seed);
        const brotensor::Tensor row = brotensor::Tensor::view(brotensor::Device::ROCm, const_cast<uint16_t*>(logits_dev),
                                                              1, vocab, brotensor::Dtype::FP16);
        tok = brolm::detail::sample_token_device(row, p, rng);
    });
    return rc == 0 ? tok : -1;
}

int brolm_sample_token(const float* logits, int vocab, float temperature, int top_k, float top_p, uint64_t seed) {
    brolm::detail::SamplingParams p;
    p.temperature = temperature;
    p.top_k = top_k;
    p.top_p = top_p;
    std::mt19937_64 rng(seed);
    return brolm::detail::sample_token(logits, vocab, p, rng);
}

void brolm_profile_reset(void) { brolm::detail::profile::reset(); }
void brolm_profile_report(void) { brolm::detail::profile::report(); }
int brolm_profile_enabled(void) { return brolm::detail::profile::enabled() ? 1 : 0; }
int brolm_profile_stage(int stage, uint64_t* ns, uint64_t* calls) {
    namespace pr = brolm::detail::profile;
    if (stage < 0 || stage >= static_cast<int>(pr::Stage::COUNT) || !ns || !calls) return -1;
    *ns = pr::total_ns(static_cast<pr::Stage>(stage));
    *calls = pr::calls(static_cast<pr::Stage>(stage));
    return 0;
}

}  // extern "C"

extern "C" int brolm_prompt_ids(uint64_t seed, int n, int vocab, int32_t* out) {
    // tools/bench_decode.cpp:208-213: std::mt19937_64(seed)() % vocab
    if (n < 0 || vocab <= 0 || (!out && n > 0)) {
        g_err = "prompt_ids: bad arguments";
        return -1;
    }
    std::mt19937_64 rng(seed);
    for (int i = 0; i < n; ++i) out[i] = static_cast<int32_t>(rng() % static_cast<uint64_t>(vocab));
    return 0;
}
