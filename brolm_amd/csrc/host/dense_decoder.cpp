// DenseDecoder (reference src/detail/dense_decoder.cpp), MI355X structure:
// FP32 residual stream, op-surface prefill, fused + graph-captured decode step.
#include "brolm/detail/dense_decoder.h"

#include <hip/hip_runtime_api.h>

#include <algorithm>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <stdexcept>
#include <string>
#include <vector>

#include "brolm/detail/compute.h"
#include "brolm/detail/device.h"
#include "brolm/detail/profile.h"
#include "brolm/detail/weights.h"
#include "brolm_hip.h"
#include "brotensor/ops.h"
#include "brotensor/runtime.h"
#include "hip_util.h"

namespace brolm::detail {

namespace bt = ::brotensor;

namespace {

[[noreturn]] void fail(const std::string& msg) { throw std::runtime_error("DenseDecoder: " + msg); }

bt::Tensor make_idx_device(const int32_t* host, int n) {
    bt::Tensor t = bt::Tensor::empty_on(bt::Device::ROCm, n, 1, bt::Dtype::INT32);
    hipx::h2d(t.data, host, static_cast<std::size_t>(n) * sizeof(int32_t));
    return t;
}

bool env_flag(const char* name) {
    const char* v = std::getenv(name);
    return v != nullptr && *v != '\0' && !(v[0] == '0' && v[1] == '\0');
}

int ggml_of(const bt::Tensor& t) { return bt::dtype_to_ggml(t.dtype); }

std::int64_t tensor_bytes(const bt::Tensor& t) { return static_cast<std::int64_t>(t.bytes()); }

}  // namespace

// ─── decode session ──────────────────────────────────────────────────────────
//
// Device scalars (scal): [0] token fed this step, [1] its position, [2] argmax
// of this step's logits, [3] history count, [4 ..) history of argmax ids.
// The captured step ends with the advance kernel (token <- argmax, pos += 1),
// so back-to-back replays decode greedily with no host round trip; the host
// re-stages token/pos whenever it drives the step itself.

struct DecodeGraphSession {
    static constexpr int kHist = 4096;
    int cap = 0;
    bx_decode_dims dims{};
    std::vector<bx_decode_layer> layers;
    void* ws = nullptr;
    int32_t* scal = nullptr;
    uint16_t* logits = nullptr;
    void* argmax_ws = nullptr;
    int32_t* pinned = nullptr;  // host staging {tok, pos, next, count}
    hipEvent_t staged = nullptr;
    hipGraph_t graph = nullptr;
    hipGraphExec_t exec = nullptr;
    bool use_graph = true;
    // persistent single-launch step (bx_persist_step), used when it covers the shape
    bool use_persist = false;
    void* pws = nullptr;
    std::size_t pws_bytes = 0;
    bx_decode_layer* layers_dev = nullptr;
    uint32_t epoch = 0;
    bool aborted = false;  // a persistent step gave up waiting; the caller redoes its steps
    // device-side sampled decoding: the sampler's workspace and the draws
    void* sample_ws = nullptr;
    double* draws = nullptr;

    ~DecodeGraphSession() {
        // after brotensor::shutdown() the op stream is gone and already drained
        if (bt::initialized()) (void)hipStreamSynchronize(static_cast<hipStream_t>(bt::stream()));
        if (pws) (void)hipFree(pws);
        if (sample_ws) (void)hipFree(sample_ws);
        if (draws) (void)hipFree(draws);
        if (layers_dev) (void)hipFree(layers_dev);
        if (exec) (void)hipGraphExecDestroy(exec);
        if (graph) (void)hipGraphDestroy(graph);
        if (staged) (void)hipEventDestroy(staged);
        if (pinned) (void)hipHostFree(pinned);
        if (ws) (void)hipFree(ws);
        if (scal) (void)hipFree(scal);
        if (logits) (void)hipFree(logits);
        if (argmax_ws) (void)hipFree(argmax_ws);
    }
};

// ─── construction ────────────────────────────────────────────────────────────
//
// One replayable step per row count M: the first step of a given M runs
// eagerly (it also settles every buffer), the second is captured and every
// later one replays the graph.  The kernels read positions, lengths, slots
// and token ids from batch_meta_, so a replay needs only that upload.
struct DenseDecoder::BatchGraphs {
    std::vector<hipGraphExec_t> exec;
    std::vector<char> warmed;
    bool use_graph = true;

    explicit BatchGraphs(int n) : exec(static_cast<std::size_t>(n) + 1, nullptr), warmed(exec.size(), 0) {
        // eager steps under a profiler tool (a graph launch under rocprofv3
        // has ended the process in the profiler's exit path)
        use_graph = !env_flag("BROLM_NO_GRAPH") && !bx_profiler_attached();
    }
    ~BatchGraphs() {
        if (bt::initialized()) (void)hipStreamSynchronize(static_cast<hipStream_t>(bt::stream()));
        for (hipGraphExec_t e : exec)
            if (e) (void)hipGraphExecDestroy(e);
    }
};

// The shape rules and their messages are the reference's
// (src/detail/dense_decoder.cpp:97-112); they are checked in table order.

namespace {

struct ShapeRule {
    bool (*bad)(const DenseDecoderConfig&);
    const char* message;
};
constexpr ShapeRule kShapeRules[] = {
    {[](const DenseDecoderConfig& c) {
         return c.hidden_size <= 0 || c.intermediate_size <= 0 || c.num_hidden_layers <= 0 || c.vocab_size <= 0 ||
                c.head_dim <= 0;
     },
     "config has non-positive dimension"},
    {[](const DenseDecoderConfig& c) { return c.num_attention_heads <= 0 || c.num_key_value_heads <= 0; },
     "num_attention_heads / num_key_value_heads must be positive"},
    {[](const DenseDecoderConfig& c) { return c.num_attention_heads % c.num_key_value_heads != 0; },
     "num_attention_heads must be a multiple of num_key_value_heads"},
    {[](const DenseDecoderConfig& c) { return c.head_dim % 2 != 0; },
     "head_dim must be even (RoPE rotates dimension pairs)"},
};

}  // namespace

DenseDecoder::DenseDecoder(const DenseDecoderConfig& cfg) : cfg_(cfg) {
    for (const ShapeRule& r : kShapeRules)
        if (r.bad(cfg_)) fail(r.message);
    layers_.resize(static_cast<std::size_t>(cfg_.num_hidden_layers));
}

DenseDecoder::~DenseDecoder() = default;
DenseDecoder::DenseDecoder(DenseDecoder&&) noexcept = default;
DenseDecoder& DenseDecoder::operator=(DenseDecoder&&) noexcept = default;

// ─── weights ─────────────────────────────────────────────────────────────────
//
// What a checkpoint must hold is one table: the HF tensor name (the Source
// maps it to the file's own naming), its (rows, cols) in model dimensions,
// how it is uploaded, and the Layer member it lands in.  The names, shapes,
// upload kinds and the lm_head tie rule are the reference's contract
// (src/detail/dense_decoder.cpp:121-192); the table order is the order a
// missing tensor is reported in.
//   carrier  quantized matrices keep their GGUF blocks on the device;
//   dense    norm gammas (and the embedding) are dequantized to FP16;
//   rope     q / k rows (and the QK-norm gammas, as one head over head_dim)
//            are permuted within each head from interleaved to half-split
//            pairs, so RoPE rotates contiguous halves.

namespace {

enum class Dim : std::uint8_t { One, Hidden, Ffn, QWidth, KvWidth, HeadDim, Vocab };
enum class Upload : std::uint8_t { Carrier, Dense, Rope };

struct ModelDims {
    int v, h, f, hd, n_q, n_kv;
    int of(Dim d) const {
        switch (d) {
            case Dim::One: return 1;
            case Dim::Hidden: return h;
            case Dim::Ffn: return f;
            case Dim::QWidth: return n_q * hd;
            case Dim::KvWidth: return n_kv * hd;
            case Dim::HeadDim: return hd;
            case Dim::Vocab: return v;
        }
        return 0;
    }
    // heads a rope-permuted tensor's rows split into
    int heads_of(Dim rows) const { return rows == Dim::QWidth ? n_q : rows == Dim::KvWidth ? n_kv : 1; }
};

struct TensorSpec {
    const char* hf;      // name after "model.layers.<i>." (per layer) or the full name
    const char* label;   // the short name the Source's errors use
    Dim rows, cols;
    Upload how;
};

void upload(const weights::Source& src, const std::string& name, const TensorSpec& t, const ModelDims& d,
            bt::Tensor& dst) {
    const int rows = d.of(t.rows), cols = d.of(t.cols);
    switch (t.how) {
        case Upload::Carrier: src.upload_compute_checked(name, rows, cols, dst, t.label); break;
        case Upload::Dense: src.upload_compute_dequant(name, rows, cols, dst, t.label); break;
        case Upload::Rope:
            src.upload_compute_rope_permuted(name, rows, cols, d.heads_of(t.rows), d.hd, dst, t.label);
            break;
    }
}

}  // namespace

void DenseDecoder::load_weights(const weights::Source& src) {
    struct LayerSlot {
        TensorSpec spec;
        bt::Tensor Layer::* member;
        bool qk_norm_only;
    };
    static const LayerSlot kLayerSlots[] = {
        {{"input_layernorm.weight", "input_layernorm.weight", Dim::Hidden, Dim::One, Upload::Dense},
         &Layer::input_ln, false},
        {{"self_attn.q_proj.weight", "q_proj.weight", Dim::QWidth, Dim::Hidden, Upload::Rope}, &Layer::Wq, false},
        {{"self_attn.k_proj.weight", "k_proj.weight", Dim::KvWidth, Dim::Hidden, Upload::Rope}, &Layer::Wk, false},
        {{"self_attn.v_proj.weight", "v_proj.weight", Dim::KvWidth, Dim::Hidden, Upload::Carrier}, &Layer::Wv, false},
        {{"self_attn.o_proj.weight", "o_proj.weight", Dim::Hidden, Dim::QWidth, Upload::Carrier}, &Layer::Wo, false},
        {{"self_attn.q_norm.weight", "q_norm.weight", Dim::HeadDim, Dim::One, Upload::Rope}, &Layer::q_norm, true},
        {{"self_attn.k_norm.weight", "k_norm.weight", Dim::HeadDim, Dim::One, Upload::Rope}, &Layer::k_norm, true},
        {{"post_attention_layernorm.weight", "post_attention_layernorm.weight", Dim::Hidden, Dim::One,
          Upload::Dense},
         &Layer::post_attn_ln, false},
        {{"mlp.gate_proj.weight", "gate_proj.weight", Dim::Ffn, Dim::Hidden, Upload::Carrier}, &Layer::gate_W, false},
        {{"mlp.up_proj.weight", "up_proj.weight", Dim::Ffn, Dim::Hidden, Upload::Carrier}, &Layer::up_W, false},
        {{"mlp.down_proj.weight", "down_proj.weight", Dim::Hidden, Dim::Ffn, Upload::Carrier}, &Layer::down_W,
         false},
    };
    // Everything derived from the old weights goes: the captured single-token
    // step and the batched steps' graphs hold their pointers, and the FP16
    // layer copies of long passes hold their values (rebuilt by the next pass
    // of 512+ rows).
    invalidate_graph_();
    if (batch_graphs_) batch_graphs_ = std::make_unique<BatchGraphs>(batch_slots_);
    for (Layer& ly : layers_)
        for (bt::Tensor* t : {&ly.q16, &ly.k16, &ly.v16, &ly.o16, &ly.gate16, &ly.up16, &ly.down16}) *t = bt::Tensor();
    f16_state_ = 0;
    const ModelDims d{cfg_.vocab_size, cfg_.hidden_size, cfg_.intermediate_size, cfg_.head_dim,
                      cfg_.num_attention_heads, cfg_.num_key_value_heads};
    upload(src, "model.embed_tokens.weight", {"", "embed_tokens.weight", Dim::Vocab, Dim::Hidden, Upload::Dense}, d,
           embed_tokens_);
    for (std::size_t i = 0; i < layers_.size(); ++i) {
        const std::string prefix = "model.layers." + std::to_string(i) + ".";
        for (const LayerSlot& s : kLayerSlots)
            if (!s.qk_norm_only || cfg_.use_qk_norm) upload(src, prefix + s.spec.hf, s.spec, d, layers_[i].*s.member);
    }
    upload(src, "model.norm.weight", {"", "model.norm.weight", Dim::Hidden, Dim::One, Upload::Dense}, d, final_norm_);
    if (src.has("lm_head.weight")) {
        upload(src, "lm_head.weight", {"", "lm_head.weight", Dim::Vocab, Dim::Hidden, Upload::Carrier}, d, lm_head_);
    } else if (cfg_.tie_word_embeddings) {
        // tied: the head reads its own copy of the FP16 embedding rows
        lm_head_ = embed_tokens_.clone();
    } else {
        fail("load_weights: lm_head.weight missing and tie_word_embeddings is false");
    }
    bt::sync_all();
}

// ─── KV cache ────────────────────────────────────────────────────────────────
//
// One HBM arena holds every layer's cache: layer l's K rows, then its V rows,
// each (capacity, n_kv * head_dim) FP16, so the whole cache is one allocation
// and each layer's K and V are contiguous views the kernels read by row.  A
// call with the current capacity keeps the arena (the captured step bakes its
// pointers in); any other capacity reallocates and drops the step session.
// reset / truncate only move cache_len: rows past it are dead until the next
// forward overwrites them, and RoPE positions restart from cache_len.

void DenseDecoder::allocate_cache(int max_seq_len) {
    if (max_seq_len <= 0) fail("allocate_cache: max_seq_len must be positive");
    const int width = cfg_.num_key_value_heads * cfg_.head_dim;
    if (max_seq_len != max_seq_len_ || kv_arena_.data == nullptr) {
        invalidate_graph_();
        const std::int64_t rows = 2LL * static_cast<std::int64_t>(layers_.size()) * max_seq_len;
        if (rows > INT32_MAX) fail("allocate_cache: KV arena rows exceed the tensor row limit");
        kv_arena_ = bt::Tensor();   // free the old arena before taking the new one
        kv_arena_ = bt::Tensor::empty_on(bt::Device::ROCm, static_cast<int>(rows), width, bt::Dtype::FP16);
        const std::size_t plane = static_cast<std::size_t>(max_seq_len) * width;   // FP16 elements
        auto* base = static_cast<std::uint16_t*>(kv_arena_.data);
        for (std::size_t l = 0; l < layers_.size(); ++l) {
            layers_[l].K_cache = bt::Tensor::view(bt::Device::ROCm, base + (2 * l) * plane, max_seq_len, width,
                                                  bt::Dtype::FP16);
            layers_[l].V_cache = bt::Tensor::view(bt::Device::ROCm, base + (2 * l + 1) * plane, max_seq_len, width,
                                                  bt::Dtype::FP16);
        }
    }
    max_seq_len_ = max_seq_len;
    cache_len_ = 0;
    ensure_rope_table_();
}

void DenseDecoder::ensure_rope_table_() {
    const int half = cfg_.head_dim / 2;
    if (rope_cos_.data && rope_cos_.rows == max_seq_len_) return;
    std::vector<float> c(static_cast<std::size_t>(max_seq_len_) * half), s(c.size());
    bx_rope_table_host(c.data(), s.data(), max_seq_len_, cfg_.head_dim, cfg_.rope_theta);
    rope_cos_ = bt::Tensor::from_host_on(bt::Device::ROCm, c.data(), max_seq_len_, half);
    rope_sin_ = bt::Tensor::from_host_on(bt::Device::ROCm, s.data(), max_seq_len_, half);
}

void DenseDecoder::reset_cache() { cache_len_ = 0; }

void DenseDecoder::truncate_cache(int len) {
    if (len < 0) fail("truncate_cache: len must be non-negative");
    if (len > cache_len_) fail("truncate_cache: len exceeds current cache_len");
    cache_len_ = len;
}

// ─── forward (dense_decoder.cpp:231-329) ────────────────────────────────────

void DenseDecoder::embed_tokens(const int32_t* ids, int L, bt::Tensor& out) {
    if (!ids) fail("embed_tokens: ids pointer is null");
    if (L <= 0) fail("embed_tokens: L must be positive");
    if (embed_tokens_.size() == 0) fail("embed_tokens: weights not loaded");
    for (int i = 0; i < L; ++i)
        if (ids[i] < 0 || ids[i] >= cfg_.vocab_size) fail("embed_tokens: token id out of range");
    bt::Tensor idx = make_idx_device(ids, L);
    bt::embedding_lookup_forward(embed_tokens_, static_cast<const int32_t*>(idx.data), L, out);
    out = out.clone();
}

static void check_forward(const char* what, const int32_t* ids, int L, bool loaded, int max_seq, int cache_len,
                          int vocab) {
    if (!ids) fail(std::string(what) + ": ids pointer is null");
    if (L <= 0) fail(std::string(what) + ": L must be positive");
    if (!loaded) fail(std::string(what) + ": weights not loaded");
    if (max_seq == 0) fail(std::string(what) + ": cache not allocated");
    if (cache_len + L > max_seq) fail(std::string(what) + ": cache_len + L exceeds allocated cache capacity");
    for (int i = 0; i < L; ++i)
        if (ids[i] < 0 || ids[i] >= vocab) fail(std::string(what) + ": token id out of range");
}

void DenseDecoder::forward(const int32_t* ids, int L, bt::Tensor& logits_out, bt::Tensor* hidden_out) {
    check_forward("forward", ids, L, embed_tokens_.size() != 0, max_seq_len_, cache_len_, cfg_.vocab_size);
    {
        profile::ScopedStage ps(profile::Stage::idx_upload);
        ids_dev_ = make_idx_device(ids, L);
    }
    {
        profile::ScopedStage ps(profile::Stage::embed);
        resize_like(h_, L, cfg_.hidden_size, bt::Dtype::FP32, bt::Device::ROCm);
        hipx::bx(bx_embedding_f32(static_cast<const uint16_t*>(embed_tokens_.data), embed_tokens_.rows,
                                  embed_tokens_.cols, static_cast<const int32_t*>(ids_dev_.data), L,
                                  static_cast<float*>(h_.data), bt::stream()),
                 "embedding");
    }
    run_layers_(L, logits_out, hidden_out);
}

void DenseDecoder::forward_last(const int32_t* ids, int L, bt::Tensor& logits_out) {
    check_forward("forward_last", ids, L, embed_tokens_.size() != 0, max_seq_len_, cache_len_, cfg_.vocab_size);
    if (L == 1 && !profile::enabled() && fused_step_ok_()) {
        decode_step_(ids[0], logits_out);
        return;
    }
    {
        profile::ScopedStage ps(profile::Stage::idx_upload);
        ids_dev_ = make_idx_device(ids, L);
    }
    {
        profile::ScopedStage ps(profile::Stage::embed);
        resize_like(h_, L, cfg_.hidden_size, bt::Dtype::FP32, bt::Device::ROCm);
        hipx::bx(bx_embedding_f32(static_cast<const uint16_t*>(embed_tokens_.data), embed_tokens_.rows,
                                  embed_tokens_.cols, static_cast<const int32_t*>(ids_dev_.data), L,
                                  static_cast<float*>(h_.data), bt::stream()),
                 "embedding");
    }
    run_layers_(L, logits_out, nullptr, /*logits_last_row_only=*/true);
}

void DenseDecoder::forward_embeds(const bt::Tensor& embeds, int L, bt::Tensor& logits_out, bt::Tensor* hidden_out) {
    if (L <= 0) fail("forward_embeds: L must be positive");
    if (embed_tokens_.size() == 0) fail("forward_embeds: weights not loaded");
    if (max_seq_len_ == 0) fail("forward_embeds: cache not allocated");
    if (cache_len_ + L > max_seq_len_) fail("forward_embeds: cache_len + L exceeds allocated cache capacity");
    if (embeds.rows != L || embeds.cols != cfg_.hidden_size) fail("forward_embeds: embeds must be (L, hidden_size)");
    if (embeds.dtype != bt::Dtype::FP16 || embeds.device != bt::Device::ROCm)
        fail("forward_embeds: embeds must be FP16 on the ROCm device");
    resize_like(h_, L, cfg_.hidden_size, bt::Dtype::FP32, bt::Device::ROCm);
    hipx::bx(bx_dequant_to_f32(BX_TYPE_F16, embeds.data, static_cast<float*>(h_.data), L, cfg_.hidden_size,
                               bt::stream()),
             "forward_embeds");
    run_layers_(L, logits_out, hidden_out);
}

void DenseDecoder::forward_encode(const int32_t* ids, int L, bt::Tensor& hidden_out) {
    if (!ids) fail("forward_encode: ids pointer is null");
    if (L <= 0) fail("forward_encode: L must be positive");
    if (embed_tokens_.size() == 0) fail("forward_encode: weights not loaded");
    for (int i = 0; i < L; ++i)
        if (ids[i] < 0 || ids[i] >= cfg_.vocab_size) fail("forward_encode: token id out of range");
    ids_dev_ = make_idx_device(ids, L);
    resize_like(h_, L, cfg_.hidden_size, bt::Dtype::FP32, bt::Device::ROCm);
    hipx::bx(bx_embedding_f32(static_cast<const uint16_t*>(embed_tokens_.data), embed_tokens_.rows,
                              embed_tokens_.cols, static_cast<const int32_t*>(ids_dev_.data), L,
                              static_cast<float*>(h_.data), bt::stream()),
             "embedding");
    run_layers_encode_(L, hidden_out);
}

// The encoder's layer stack (dense_decoder.cpp:682-779): run_layers_ with
// full attention over the L rows' own k / v instead of the causal cache.
void DenseDecoder::run_layers_encode_(int L, bt::Tensor& hidden_out) {
    const int HD = cfg_.head_dim, n_q = cfg_.num_attention_heads, n_kv = cfg_.num_key_value_heads;
    const float eps = cfg_.rms_norm_eps;
    auto headnorm = [&](const bt::Tensor& src, int num_heads, const bt::Tensor& gain, bt::Tensor& dst) {
        bt::Tensor v = bt::Tensor::view(src.device, src.data, src.rows * num_heads, HD, src.dtype);
        bt::rms_norm_forward(v, gain, eps, dst);
        dst.rows = src.rows;
        dst.cols = num_heads * HD;
    };
    const bool f16 = prefill_f16_(L);
    auto pick = [f16](const bt::Tensor& q, const bt::Tensor& c) -> const bt::Tensor& {
        return f16 && c.data ? c : q;
    };
    for (Layer& layer : layers_) {
        const bt::Tensor& Wq = pick(layer.Wq, layer.q16);
        const bt::Tensor& Wk = pick(layer.Wk, layer.k16);
        const bt::Tensor& Wv = pick(layer.Wv, layer.v16);
        const bt::Tensor& Wo = pick(layer.Wo, layer.o16);
        const bt::Tensor& Wg = pick(layer.gate_W, layer.gate16);
        const bt::Tensor& Wu = pick(layer.up_W, layer.up16);
        const bt::Tensor& Wd = pick(layer.down_W, layer.down16);
        bt::rms_norm_forward(h_, layer.input_ln, eps, norm_);
        {
            // the fused forms where the shape allows (same results as the ops)
            const bt::Tensor* w[3] = {&Wq, &Wk, &Wv};
            bt::Tensor* y[3] = {&q_, &k_, &v_};
            const int same = Wv.dtype == Wq.dtype ? 3 : 2;
            int done = 0;
            if (Wk.dtype == Wq.dtype && bt::linear_group_forward_batched(w, y, same, norm_)) done = same;
            for (int i = done; i < 3; ++i) linear_batched(*w[i], nullptr, norm_, *y[i]);
        }
        bt::Tensor* q_attn = &q_;
        bt::Tensor* k_attn = &k_;
        if (cfg_.use_qk_norm) {
            headnorm(q_, n_q, layer.q_norm, qn_);
            headnorm(k_, n_kv, layer.k_norm, kn_);
            q_attn = &qn_;
            k_attn = &kn_;
        }
        bt::rope_forward(*q_attn, HD, n_q, 0, cfg_.rope_theta, *q_attn);
        bt::rope_forward(*k_attn, HD, n_kv, 0, cfg_.rope_theta, *k_attn);
        bt::flash_attention_gqa_forward(*q_attn, *k_attn, v_, n_q, n_kv, /*causal=*/false, attn_);
        if (!bt::linear_residual_forward_batched(Wo, attn_, h_)) {
            linear_batched(Wo, nullptr, attn_, proj_);
            bt::add_inplace(h_, proj_);
        }
        bt::rms_norm_forward(h_, layer.post_attn_ln, eps, norm_);
        if (!(Wg.dtype == Wu.dtype && bt::linear_swiglu_forward_batched(Wg, Wu, norm_, gate_))) {
            linear_batched(Wg, nullptr, norm_, gate_);
            linear_batched(Wu, nullptr, norm_, up_);
            bt::silu_forward(gate_, gate_);
            bt::mul_inplace(gate_, up_);
        }
        if (!bt::linear_residual_forward_batched(Wd, gate_, h_)) {
            linear_batched(Wd, nullptr, gate_, proj_);
            bt::add_inplace(h_, proj_);
        }
    }
    bt::rms_norm_forward(h_, final_norm_, eps, norm_);
    hidden_out = norm_.clone();
}

// ─── FP16 layer copies for long prompts ─────────────────────────────────────
//
// A pass over L >= 512 rows is bound by the matrix cores, and the FP16 tiles
// run about a fifth faster than the quantized ones, which dequantize inside
// their K loop.  With HBM to spare (288 GB on this part), the first such pass
// dequantizes every quantized layer matrix once into an FP16 copy held by the
// layer, and every long pass after it multiplies those.  The copies are made
// only if the device keeps at least max(8 GB, 10 %) free afterwards, and never
// for single-token or batched decode, which stay on the quantized weights
// (there the step is bound by weight bytes).  BROLM_PREFILL_F16=0 turns them off.
// The weights multiplied are the FP16 roundings the quantized tiles form, so
// results are those of the op path's tile GEMM to its stated tolerance.

bool DenseDecoder::prefill_f16_(int L) {
    constexpr int kRows = 512;
    if (L < kRows) return false;
    if (f16_state_ != 0) return f16_state_ > 0;
    f16_state_ = -1;
    if (const char* e = std::getenv("BROLM_PREFILL_F16"); e && e[0] == '0') return false;
    auto quant = [](const bt::Tensor& t) { return t.dtype == bt::Dtype::Q4_K || t.dtype == bt::Dtype::Q6_K ||
                                                  t.dtype == bt::Dtype::Q8_0; };
    std::size_t need = 0;
    for (const Layer& ly : layers_)
        for (const bt::Tensor* t : {&ly.Wq, &ly.Wk, &ly.Wv, &ly.Wo, &ly.gate_W, &ly.up_W, &ly.down_W})
            if (quant(*t)) need += static_cast<std::size_t>(t->rows) * t->cols * 2;
    if (need == 0) return false;
    std::size_t free_b = 0, total_b = 0;
    if (hipMemGetInfo(&free_b, &total_b) != hipSuccess) return false;
    const std::size_t keep = std::max<std::size_t>(std::size_t(8) << 30, total_b / 10);
    if (free_b < need + keep) return false;
    for (Layer& ly : layers_) {
        auto copy = [&](const bt::Tensor& w, bt::Tensor& out) {
            if (!quant(w)) return;
            out = bt::Tensor::empty_on(bt::Device::ROCm, w.rows, w.cols, bt::Dtype::FP16);
            hipx::bx(bx_dequant_to_f16(bt::dtype_to_ggml(w.dtype), w.data, static_cast<uint16_t*>(out.data), w.rows,
                                       w.cols, bt::stream()),
                     "FP16 layer copy");
        };
        copy(ly.Wq, ly.q16);
        copy(ly.Wk, ly.k16);
        copy(ly.Wv, ly.v16);
        copy(ly.Wo, ly.o16);
        copy(ly.gate_W, ly.gate16);
        copy(ly.up_W, ly.up16);
        copy(ly.down_W, ly.down16);
    }
    f16_state_ = 1;
    return true;
}

// ─── op-surface layer stack (dense_decoder.cpp:526-681) ─────────────────────

void DenseDecoder::run_layers_(int L, bt::Tensor& logits_out, bt::Tensor* hidden_out, bool logits_last_row_only) {
    const int HD = cfg_.head_dim, n_q = cfg_.num_attention_heads, n_kv = cfg_.num_key_value_heads;
    const float eps = cfg_.rms_norm_eps;
    const int seq_offset = cache_len_;

    auto headnorm = [&](const bt::Tensor& src, int num_heads, const bt::Tensor& gain, bt::Tensor& dst) {
        const int rows = src.rows;
        bt::Tensor v = bt::Tensor::view(src.device, src.data, rows * num_heads, HD, src.dtype);
        bt::rms_norm_forward(v, gain, eps, dst);
        dst.rows = rows;
        dst.cols = num_heads * HD;
    };

    namespace prof = profile;
    using PS = profile::Stage;
    const bool f16 = prefill_f16_(L);
    // the FP16 copy of a quantized matrix when long passes use them
    auto pick = [f16](const bt::Tensor& q, const bt::Tensor& c) -> const bt::Tensor& {
        return f16 && c.data ? c : q;
    };
    for (Layer& layer : layers_) {
        const bt::Tensor& Wq = pick(layer.Wq, layer.q16);
        const bt::Tensor& Wk = pick(layer.Wk, layer.k16);
        const bt::Tensor& Wv = pick(layer.Wv, layer.v16);
        const bt::Tensor& Wo = pick(layer.Wo, layer.o16);
        const bt::Tensor& Wg = pick(layer.gate_W, layer.gate16);
        const bt::Tensor& Wu = pick(layer.up_W, layer.up16);
        const bt::Tensor& Wd = pick(layer.down_W, layer.down16);
        { prof::ScopedStage ps(PS::rms_norm); bt::rms_norm_forward(h_, layer.input_ln, eps, norm_); }
        {
            // one launch for the projections that share a weight dtype
            // (q / k always, v too unless a Q4_K_M layer raised it)
            prof::ScopedStage ps(PS::qkv_proj);
            const bt::Tensor* w[3] = {&Wq, &Wk, &Wv};
            bt::Tensor* y[3] = {&q_, &k_, &v_};
            const int same = Wv.dtype == Wq.dtype ? 3 : 2;
            int done = 0;
            if (Wk.dtype == Wq.dtype && bt::linear_group_forward_batched(w, y, same, norm_)) done = same;
            for (int i = done; i < 3; ++i) linear_batched(*w[i], nullptr, norm_, *y[i]);
        }
        bt::Tensor* q_attn = &q_;
        bt::Tensor* k_attn = &k_;
        if (cfg_.use_qk_norm) {
            prof::ScopedStage ps(PS::qk_norm);
            headnorm(q_, n_q, layer.q_norm, qn_);
            headnorm(k_, n_kv, layer.k_norm, kn_);
            q_attn = &qn_;
            k_attn = &kn_;
        }
        {
            prof::ScopedStage ps(PS::rope);
            bt::rope_forward(*q_attn, HD, n_q, seq_offset, cfg_.rope_theta, *q_attn);
            bt::rope_forward(*k_attn, HD, n_kv, seq_offset, cfg_.rope_theta, *k_attn);
        }
        { prof::ScopedStage ps(PS::kv_append); bt::kv_cache_append(*k_attn, v_, cache_len_, layer.K_cache, layer.V_cache); }
        {
            prof::ScopedStage ps(PS::attention);
            bt::flash_attention_decode(*q_attn, layer.K_cache, layer.V_cache, cache_len_ + L, n_q, n_kv, attn_);
        }
        bool fused_o;
        {
            prof::ScopedStage ps(PS::o_proj);  // o_proj and the residual add in one launch
            fused_o = bt::linear_residual_forward_batched(Wo, attn_, h_);
            if (!fused_o) linear_batched(Wo, nullptr, attn_, proj_);
        }
        if (!fused_o) {
            prof::ScopedStage ps(PS::residual_add);
            bt::add_inplace(h_, proj_);
        }
        { prof::ScopedStage ps(PS::rms_norm); bt::rms_norm_forward(h_, layer.post_attn_ln, eps, norm_); }
        bool fused_mlp;
        {
            prof::ScopedStage ps(PS::mlp_proj);  // gate / up projections with the SwiGLU in one launch
            fused_mlp = Wg.dtype == Wu.dtype && bt::linear_swiglu_forward_batched(Wg, Wu, norm_, gate_);
            if (!fused_mlp) {
                linear_batched(Wg, nullptr, norm_, gate_);
                linear_batched(Wu, nullptr, norm_, up_);
            }
        }
        if (!fused_mlp) {
            prof::ScopedStage ps(PS::swiglu);
            bt::silu_forward(gate_, gate_);
            bt::mul_inplace(gate_, up_);
        }
        bool fused_down;
        {
            prof::ScopedStage ps(PS::mlp_proj);  // down and the residual add in one launch
            fused_down = bt::linear_residual_forward_batched(Wd, gate_, h_);
            if (!fused_down) linear_batched(Wd, nullptr, gate_, proj_);
        }
        if (!fused_down) {
            prof::ScopedStage ps(PS::residual_add);
            bt::add_inplace(h_, proj_);
        }
    }
    {
        prof::ScopedStage ps(PS::final_norm);
        bt::rms_norm_forward(h_, final_norm_, eps, norm_);
        if (hidden_out) *hidden_out = norm_.clone();
    }
    {
        prof::ScopedStage ps(PS::lm_head);
        if (logits_last_row_only && L > 1) {
            bt::Tensor last = bt::Tensor::view(
                norm_.device,
                static_cast<char*>(norm_.data) + static_cast<std::size_t>(L - 1) * norm_.cols * 2, 1, norm_.cols,
                norm_.dtype);
            linear_batched(lm_head_, nullptr, last, logits_out);
        } else {
            linear_batched(lm_head_, nullptr, norm_, logits_out);
        }
    }
    cache_len_ += L;
}

// ─── fused decode step ──────────────────────────────────────────────────────

void DenseDecoder::invalidate_graph_() { graph_.reset(); }

// The step's dims: shapes, layer 0's matrix types, and the second attn_v /
// ffn_down type of a mixed (Q4_K_M-style) file when one exists.
bx_decode_dims DenseDecoder::decode_dims_() const {
    bx_decode_dims d{};
    d.hidden = cfg_.hidden_size; d.intermediate = cfg_.intermediate_size;
    d.n_q = cfg_.num_attention_heads; d.n_kv = cfg_.num_key_value_heads; d.head_dim = cfg_.head_dim;
    d.vocab = cfg_.vocab_size; d.cap = max_seq_len_; d.eps = cfg_.rms_norm_eps;
    const Layer& L0 = layers_[0];
    d.qkv_type_q = ggml_of(L0.Wq); d.qkv_type_k = ggml_of(L0.Wk); d.qkv_type_v = ggml_of(L0.Wv);
    d.o_type = ggml_of(L0.Wo); d.gate_type = ggml_of(L0.gate_W); d.up_type = ggml_of(L0.up_W);
    d.down_type = ggml_of(L0.down_W); d.lm_type = ggml_of(lm_head_);
    d.no_qk_norm = cfg_.use_qk_norm ? 0 : 1;
    for (const Layer& L : layers_) {
        if (ggml_of(L.Wv) != d.qkv_type_v && d.v_alt_type == 0) d.v_alt_type = ggml_of(L.Wv);
        if (ggml_of(L.down_W) != d.down_type && d.down_alt_type == 0) d.down_alt_type = ggml_of(L.down_W);
    }
    return d;
}

// Whether single-token steps can run fused (persistent kernel or the graph of
// per-stage kernels): every layer's types are ones the step kernels read,
// with q/k and gate/up sharing a type, and the shape fits the step's
// workspace.  Otherwise forward_last and decode_greedy take the op path, as
// the reference does for any weight dtype (compute.h:54-86); BROLM_OP_STEP=1
// asks for the op path.
bool DenseDecoder::fused_step_ok_() const {
    if (max_seq_len_ == 0 || layers_.empty() || embed_tokens_.size() == 0) return false;
    if (env_flag("BROLM_OP_STEP")) return false;
    auto known = [](int t) {
        return t == BX_TYPE_Q4_K || t == BX_TYPE_Q6_K || t == BX_TYPE_Q8_0 || t == BX_TYPE_F16;
    };
    for (const Layer& L : layers_) {
        const int t[7] = {ggml_of(L.Wq), ggml_of(L.Wk), ggml_of(L.Wv), ggml_of(L.Wo), ggml_of(L.gate_W),
                          ggml_of(L.up_W), ggml_of(L.down_W)};
        for (int x : t)
            if (!known(x)) return false;
        if (t[0] != t[1] || t[4] != t[5]) return false;
    }
    if (!known(ggml_of(lm_head_))) return false;
    const bx_decode_dims d = decode_dims_();
    return bx_decode_ws_bytes(&d) != 0;
}

// The persistent kernel serves one type per role except attn_v and ffn_down,
// which may take a second type (decode_dims_) in some layers.
static bool persist_types_ok(const bx_decode_dims& d, const std::vector<bx_decode_layer>& ls) {
    for (const bx_decode_layer& L : ls) {
        if (L.type_q != d.qkv_type_q || L.type_k != d.qkv_type_k || L.type_o != d.o_type ||
            L.type_gate != d.gate_type || L.type_up != d.up_type)
            return false;
        if (L.type_v != d.qkv_type_v && L.type_v != d.v_alt_type) return false;
        if (L.type_down != d.down_type && L.type_down != d.down_alt_type) return false;
    }
    return true;
}

DecodeGraphSession& DenseDecoder::session_() {
    if (graph_ && graph_->cap == max_seq_len_) return *graph_;
    graph_.reset();
    if (!fused_step_ok_()) fail(std::string("decode step: unsupported shape or weight types: ") + bx_last_error());
    auto s = std::make_unique<DecodeGraphSession>();
    s->cap = max_seq_len_;
    bx_decode_dims& d = s->dims;
    d = decode_dims_();
    for (const Layer& L : layers_) {
        bx_decode_layer bl{};
        bl.in_ln = L.input_ln.data; bl.q_norm = L.q_norm.data; bl.k_norm = L.k_norm.data;
        bl.post_ln = L.post_attn_ln.data;
        bl.Wq = L.Wq.data; bl.Wk = L.Wk.data; bl.Wv = L.Wv.data; bl.Wo = L.Wo.data;
        bl.Wg = L.gate_W.data; bl.Wu = L.up_W.data; bl.Wd = L.down_W.data;
        bl.Kc = L.K_cache.data; bl.Vc = L.V_cache.data;
        bl.type_q = ggml_of(L.Wq); bl.type_k = ggml_of(L.Wk); bl.type_v = ggml_of(L.Wv); bl.type_o = ggml_of(L.Wo);
        bl.type_gate = ggml_of(L.gate_W); bl.type_up = ggml_of(L.up_W); bl.type_down = ggml_of(L.down_W);
        s->layers.push_back(bl);
    }
    const std::size_t wsb = bx_decode_ws_bytes(&d);
    if (wsb == 0) fail(std::string("decode step: unsupported shape: ") + bx_last_error());
    hipx::check(hipMalloc(&s->ws, wsb), "hipMalloc decode ws");
    hipx::check(hipMalloc(reinterpret_cast<void**>(&s->scal), (4 + DecodeGraphSession::kHist) * sizeof(int32_t)),
                "hipMalloc decode scalars");
    hipx::check(hipMemsetAsync(s->scal, 0, (4 + DecodeGraphSession::kHist) * sizeof(int32_t), hipx::stream()),
                "memset scalars");
    hipx::check(hipMalloc(reinterpret_cast<void**>(&s->logits), static_cast<std::size_t>(cfg_.vocab_size) * 2),
                "hipMalloc logits");
    hipx::check(hipMalloc(&s->argmax_ws, bx_argmax_workspace_bytes(cfg_.vocab_size)), "hipMalloc argmax ws");
    hipx::check(hipHostMalloc(reinterpret_cast<void**>(&s->pinned), 4 * sizeof(int32_t), hipHostMallocDefault),
                "hipHostMalloc");
    hipx::check(hipEventCreateWithFlags(&s->staged, hipEventDisableTiming), "hipEventCreate");
    // no captured graph under a profiler tool: a graph launch under
    // rocprofv3 has ended the process in the profiler's exit path
    const bool no_fused = env_flag("BROLM_NO_GRAPH");
    s->use_graph = !no_fused && !bx_profiler_attached();
    if (!no_fused && !env_flag("BROLM_NO_PERSIST") && persist_types_ok(d, s->layers)) {
        s->pws_bytes = bx_persist_ws_bytes(&d);
        if (s->pws_bytes != 0) {
            hipx::check(hipMalloc(&s->pws, s->pws_bytes), "hipMalloc persist ws");
            hipx::bx(bx_persist_ws_init(&d, s->pws, hipx::stream()), "persist ws init");
            const std::size_t lb = s->layers.size() * sizeof(bx_decode_layer);
            hipx::check(hipMalloc(reinterpret_cast<void**>(&s->layers_dev), lb), "hipMalloc layer table");
            hipx::check(hipMemcpyAsync(s->layers_dev, s->layers.data(), lb, hipMemcpyHostToDevice, hipx::stream()),
                        "upload layer table");
            s->use_persist = true;
        }
    }
    hipx::sync();
    graph_ = std::move(s);
    return *graph_;
}

// Enqueue one fused step on the stream (captured or eager).
static void enqueue_step(DecodeGraphSession& s, const bt::Tensor& embed, const bt::Tensor& final_norm,
                         const bt::Tensor& lm_head, const bt::Tensor& cos, const bt::Tensor& sin) {
    void* st = bt::stream();
    int32_t* tok = s.scal + 0;
    int32_t* pos = s.scal + 1;
    int32_t* next = s.scal + 2;
    int32_t* count = s.scal + 3;
    int32_t* hist = s.scal + 4;
    hipx::bx(bx_decode_embed(&s.dims, static_cast<const uint16_t*>(embed.data), tok, s.ws, st), "decode_embed");
    for (const bx_decode_layer& L : s.layers)
        hipx::bx(bx_decode_layer_run(&s.dims, &L, pos, static_cast<const float*>(cos.data),
                                     static_cast<const float*>(sin.data), s.ws, st),
                 "decode_layer");
    hipx::bx(bx_decode_head(&s.dims, static_cast<const uint16_t*>(final_norm.data), lm_head.data, s.logits, s.ws, st),
             "decode_head");
    hipx::bx(bx_argmax_f16(s.logits, s.dims.vocab, next, s.argmax_ws, st), "decode_argmax");
    hipx::bx(bx_decode_advance(tok, pos, next, hist, count, st), "decode_advance");
}

static void stage_step(DecodeGraphSession& s, int32_t token, int32_t pos) {
    // The previous staging copy must have consumed the pinned buffer.
    hipx::check(hipEventSynchronize(s.staged), "hipEventSynchronize");
    s.pinned[0] = token;
    s.pinned[1] = pos;
    s.pinned[2] = 0;
    s.pinned[3] = 0;
    hipx::check(hipMemcpyAsync(s.scal, s.pinned, 4 * sizeof(int32_t), hipMemcpyHostToDevice, hipx::stream()),
                "stage step");
    hipx::check(hipEventRecord(s.staged, hipx::stream()), "hipEventRecord");
}

// After the launches so far completed: true when a persistent step gave up
// on a wait (its abort flag is set).  A step gives up when its workgroups
// are not all resident together, e.g. while another process's kernels hold
// CUs; its outputs and every later step's are then invalid.  The words are
// re-initialized, the session runs the per-stage graph from here on, and
// s.aborted tells the caller to redo the steps it enqueued since its last
// check (they rewrite the same cache rows).
static bool persist_gave_up(DecodeGraphSession& s) {
    hipx::check(hipStreamSynchronize(hipx::stream()), "hipStreamSynchronize");
    uint32_t site = 0;
    const int st = bx_persist_status(s.pws, &site);
    if (st < 0) hipx::bx(st, "persist status");
    if (st == 0) return false;
    hipx::bx(bx_persist_ws_init(&s.dims, s.pws, hipx::stream()), "persist ws init");
    hipx::check(hipStreamSynchronize(hipx::stream()), "hipStreamSynchronize");
    std::fprintf(stderr, "brolm: persistent decode step gave up waiting at site %u; the per-stage graph runs from here on\n",
                 site);
    s.epoch = 0;
    s.use_persist = false;
    s.aborted = true;
    return true;
}

// False when nothing was enqueued: the runtime refused the launch, or a step
// of the ending epoch cycle gave up (s.aborted).
static bool launch_persist(DecodeGraphSession& s, const bt::Tensor& embed, const bt::Tensor& final_norm,
                           const bt::Tensor& lm_head, const bt::Tensor& cos, const bt::Tensor& sin) {
    if (++s.epoch >= 64) {
        // a cycle of 16-bit tags is used up: re-initialize the words, which
        // also clears the abort flag, so a step of this cycle that gave up is
        // looked for first
        if (persist_gave_up(s)) return false;
        hipx::bx(bx_persist_ws_init(&s.dims, s.pws, hipx::stream()), "persist ws init");
        s.epoch = 1;
    }
    const int rc = bx_persist_step(&s.dims, static_cast<int>(s.layers.size()), s.layers_dev,
                                   static_cast<const uint16_t*>(embed.data),
                                   static_cast<const uint16_t*>(final_norm.data), lm_head.data,
                                   static_cast<const float*>(cos.data), static_cast<const float*>(sin.data), s.scal,
                                   s.logits, s.pws, s.epoch, bt::stream());
    if (rc == BX_ELAUNCH) {
        (void)hipGetLastError();  // the refused launch's status is not the stream's
        return false;
    }
    hipx::bx(rc, "persist step");
    return true;
}

// After the launches completed: false when a persistent step gave up, so
// the caller redoes the steps it enqueued since its last check, now on the
// per-stage graph.
static bool check_persist(DecodeGraphSession& s) {
    if (s.use_persist) (void)persist_gave_up(s);
    const bool ok = !s.aborted;
    s.aborted = false;
    return ok;
}

static void launch_steps(DecodeGraphSession& s, int n, const bt::Tensor& embed, const bt::Tensor& final_norm,
                         const bt::Tensor& lm_head, const bt::Tensor& cos, const bt::Tensor& sin) {
    if (s.use_persist) {
        int i = 0;
        while (i < n && launch_persist(s, embed, final_norm, lm_head, cos, sin)) ++i;
        if (i == n || s.aborted) return;
        // refused: this session runs the per-stage graph from here on (same
        // step, same results to the decode tolerance; decode_mode() says so)
        s.use_persist = false;
        n -= i;
    }
    if (s.use_graph && !s.exec) {
        hipStream_t st = hipx::stream();
        hipx::check(hipStreamBeginCapture(st, hipStreamCaptureModeThreadLocal), "hipStreamBeginCapture");
        try {
            enqueue_step(s, embed, final_norm, lm_head, cos, sin);
        } catch (...) {
            hipGraph_t g = nullptr;
            (void)hipStreamEndCapture(st, &g);
            if (g) (void)hipGraphDestroy(g);
            throw;
        }
        hipx::check(hipStreamEndCapture(st, &s.graph), "hipStreamEndCapture");
        hipx::check(hipGraphInstantiate(&s.exec, s.graph, nullptr, nullptr, 0), "hipGraphInstantiate");
    }
    for (int i = 0; i < n; ++i) {
        if (s.use_graph) hipx::check(hipGraphLaunch(s.exec, hipx::stream()), "hipGraphLaunch");
        else enqueue_step(s, embed, final_norm, lm_head, cos, sin);
    }
}

void DenseDecoder::decode_step_(int32_t token, bt::Tensor& logits_out) {
    DecodeGraphSession& s = session_();
    do {
        stage_step(s, token, cache_len_);
        launch_steps(s, 1, embed_tokens_, final_norm_, lm_head_, rope_cos_, rope_sin_);
        resize_like(logits_out, 1, cfg_.vocab_size, bt::Dtype::FP16, bt::Device::ROCm);
        hipx::check(hipMemcpyAsync(logits_out.data, s.logits, static_cast<std::size_t>(cfg_.vocab_size) * 2,
                                   hipMemcpyDeviceToDevice, hipx::stream()),
                    "copy logits");
    } while (!check_persist(s));
    cache_len_ += 1;
}

int DenseDecoder::decode_greedy(int32_t token, int n, int32_t* out, int eos_id) {
    if (n <= 0) return 0;
    check_forward("decode_greedy", &token, 1, embed_tokens_.size() != 0, max_seq_len_, cache_len_, cfg_.vocab_size);
    if (cache_len_ + n > max_seq_len_) fail("decode_greedy: cache_len + n exceeds allocated cache capacity");
    if (!fused_step_ok_()) {
        // op path, one token at a time: logits to the host, lowest-index argmax
        // (generate.cpp:38-48)
        std::vector<uint16_t> row(static_cast<std::size_t>(cfg_.vocab_size));
        bt::Tensor lg;
        int32_t cur = token;
        for (int i = 0; i < n; ++i) {
            forward_last(&cur, 1, lg);
            hipx::d2h(row.data(), lg.data, row.size() * sizeof(uint16_t));
            int best = 0;
            float bv = bt::fp16_bits_to_fp32(row[0]);
            for (int j = 1; j < cfg_.vocab_size; ++j) {
                const float v = bt::fp16_bits_to_fp32(row[static_cast<std::size_t>(j)]);
                if (v > bv) { bv = v; best = j; }
            }
            out[i] = best;
            cur = best;
            if (eos_id >= 0 && best == eos_id) return i + 1;
        }
        return n;
    }
    DecodeGraphSession& s = session_();
    int done = 0;
    int32_t cur = token;
    while (done < n) {
        const int chunk = std::min(n - done, static_cast<int>(DecodeGraphSession::kHist));
        do {
            stage_step(s, cur, cache_len_);
            launch_steps(s, chunk, embed_tokens_, final_norm_, lm_head_, rope_cos_, rope_sin_);
        } while (!check_persist(s));
        hipx::d2h(out + done, s.scal + 4, static_cast<std::size_t>(chunk) * sizeof(int32_t));
        for (int i = 0; i < chunk; ++i) {
            if (eos_id >= 0 && out[done + i] == eos_id) {
                cache_len_ += i + 1;
                return done + i + 1;
            }
        }
        cache_len_ += chunk;
        done += chunk;
        cur = out[done - 1];
    }
    return done;
}

int DenseDecoder::decode_sampled(int32_t token, int n, const double* u, float temperature, int top_k, float top_p,
                                 int32_t* out, int eos_id) {
    if (n <= 0) return 0;
    if (!u || !out) fail("decode_sampled: null draws or output");
    if (!(temperature > 0.0f)) fail("decode_sampled: temperature must be positive (greedy: decode_greedy)");
    for (int i = 0; i < n; ++i)
        if (!(u[i] >= 0.0 && u[i] < 1.0)) fail("decode_sampled: draws must lie in [0, 1)");
    check_forward("decode_sampled", &token, 1, embed_tokens_.size() != 0, max_seq_len_, cache_len_, cfg_.vocab_size);
    if (cache_len_ + n > max_seq_len_) fail("decode_sampled: cache_len + n exceeds allocated cache capacity");
    const int V = cfg_.vocab_size;
    if (!fused_step_ok_()) {
        // op path, one token at a time, the same device sampler on its logits
        bt::Tensor lg, ws, tok;
        ws = bt::Tensor::empty_on(bt::Device::ROCm, static_cast<int>(bx_sample_workspace_bytes(V) / 4), 1,
                                  bt::Dtype::FP32);
        tok = bt::Tensor::empty_on(bt::Device::ROCm, 1, 1, bt::Dtype::FP32);
        int32_t cur = token;
        for (int i = 0; i < n; ++i) {
            forward_last(&cur, 1, lg);
            hipx::bx(bx_sample_f16(static_cast<const uint16_t*>(lg.data), V, temperature, top_k, top_p, u[i],
                                   static_cast<int32_t*>(tok.data), ws.data, bt::stream()),
                     "decode_sampled");
            hipx::d2h(&cur, tok.data, sizeof(cur));
            out[i] = cur;
            if (eos_id >= 0 && cur == eos_id) return i + 1;
        }
        return n;
    }
    DecodeGraphSession& s = session_();
    if (!s.sample_ws) {
        hipx::check(hipMalloc(&s.sample_ws, bx_sample_workspace_bytes(V)), "hipMalloc sampler workspace");
        hipx::check(hipMalloc(reinterpret_cast<void**>(&s.draws), DecodeGraphSession::kHist * sizeof(double)),
                    "hipMalloc draws");
    }
    int done = 0;
    int32_t cur = token;
    while (done < n) {
        const int chunk = std::min(n - done, static_cast<int>(DecodeGraphSession::kHist));
        do {
            stage_step(s, cur, cache_len_);
            hipx::check(hipMemcpyAsync(s.draws, u + done, static_cast<std::size_t>(chunk) * sizeof(double),
                                       hipMemcpyHostToDevice, hipx::stream()),
                        "upload draws");
            for (int i = 0; i < chunk && !s.aborted; ++i) {
                // the fused step (its argmax advances token and history), then
                // the draw replaces that token
                launch_steps(s, 1, embed_tokens_, final_norm_, lm_head_, rope_cos_, rope_sin_);
                hipx::bx(bx_sample_feed_f16(s.logits, V, temperature, top_k, top_p, s.draws, s.scal + 0,
                                            s.scal + 4, s.scal + 3, s.sample_ws, bt::stream()),
                         "decode_sampled");
            }
        } while (!check_persist(s));
        hipx::d2h(out + done, s.scal + 4, static_cast<std::size_t>(chunk) * sizeof(int32_t));
        for (int i = 0; i < chunk; ++i) {
            if (eos_id >= 0 && out[done + i] == eos_id) {
                cache_len_ += i + 1;
                return done + i + 1;
            }
        }
        cache_len_ += chunk;
        done += chunk;
        cur = out[done - 1];
    }
    return done;
}

double DenseDecoder::time_decode_steps(int32_t token, int n) {
    if (n <= 0) return 0.0;
    check_forward("time_decode_steps", &token, 1, embed_tokens_.size() != 0, max_seq_len_, cache_len_,
                  cfg_.vocab_size);
    if (cache_len_ + n > max_seq_len_) fail("time_decode_steps: cache_len + n exceeds allocated cache capacity");
    DecodeGraphSession& s = session_();
    stage_step(s, token, cache_len_);
    launch_steps(s, 0, embed_tokens_, final_norm_, lm_head_, rope_cos_, rope_sin_);  // capture outside timing
    hipEvent_t e0, e1;
    hipx::check(hipEventCreate(&e0), "hipEventCreate");
    hipx::check(hipEventCreate(&e1), "hipEventCreate");
    hipx::check(hipEventRecord(e0, hipx::stream()), "hipEventRecord");
    launch_steps(s, n, embed_tokens_, final_norm_, lm_head_, rope_cos_, rope_sin_);
    hipx::check(hipEventRecord(e1, hipx::stream()), "hipEventRecord");
    hipx::check(hipEventSynchronize(e1), "hipEventSynchronize");
    float ms = 0.f;
    hipx::check(hipEventElapsedTime(&ms, e0, e1), "hipEventElapsedTime");
    (void)hipEventDestroy(e0);
    (void)hipEventDestroy(e1);
    if (!check_persist(s)) fail("time_decode_steps: a persistent step gave up waiting; the timing is void");
    cache_len_ += n;
    return static_cast<double>(ms) / n;
}

int DenseDecoder::decode_mode() {
    if (embed_tokens_.size() == 0) fail("decode_mode: weights not loaded");
    if (max_seq_len_ == 0) fail("decode_mode: cache not allocated");
    if (!fused_step_ok_()) return 3;
    DecodeGraphSession& s = session_();
    return s.use_persist ? 2 : (s.use_graph ? 1 : 0);
}

std::int64_t DenseDecoder::decode_weight_bytes() const {
    std::int64_t b = 0;
    for (const Layer& L : layers_) {
        b += tensor_bytes(L.Wq) + tensor_bytes(L.Wk) + tensor_bytes(L.Wv) + tensor_bytes(L.Wo);
        b += tensor_bytes(L.gate_W) + tensor_bytes(L.up_W) + tensor_bytes(L.down_W);
        b += tensor_bytes(L.input_ln) + tensor_bytes(L.post_attn_ln) + tensor_bytes(L.q_norm) + tensor_bytes(L.k_norm);
    }
    b += tensor_bytes(lm_head_) + tensor_bytes(final_norm_);
    b += static_cast<std::int64_t>(cfg_.hidden_size) * 2;  // one embedding row
    return b;
}

// ─── multi-sequence batched decode ──────────────────────────────────────────
//
// The reference decodes one sequence per model (one cache, one position).
// Here n_slots sequences keep their own KV rows in one slot-major arena and a
// step takes one token from each of M of them: every projection streams its
// weights once for M rows (the 3..16-row MFMA GEMV), RoPE and the KV append
// take a position per row, and attention runs each row over its own slot's
// keys (split-K, per-row length).  Prompts enter a slot through the op-path
// prefill with the layer caches pointed at the slot's rows.

namespace {
constexpr int kMetaI64PerRow = 4;  // dst row, base row (int64); pos, len, id (int32) fit in two more
}


void DenseDecoder::allocate_batch(int n_slots, int max_seq_len) {
    if (n_slots <= 0 || max_seq_len <= 0) fail("allocate_batch: n_slots and max_seq_len must be positive");
    if (embed_tokens_.size() == 0) fail("allocate_batch: weights not loaded");
    const int width = cfg_.num_key_value_heads * cfg_.head_dim;
    const std::int64_t rows = 2LL * static_cast<std::int64_t>(layers_.size()) * n_slots * max_seq_len;
    if (rows > INT32_MAX) fail("allocate_batch: KV arena rows exceed the tensor row limit");
    batch_kv_ = bt::Tensor();
    batch_kv_ = bt::Tensor::empty_on(bt::Device::ROCm, static_cast<int>(rows), width, bt::Dtype::FP16);
    batch_slots_ = n_slots;
    batch_cap_ = max_seq_len;
    slot_len_.assign(static_cast<std::size_t>(n_slots), 0);
    const int half = cfg_.head_dim / 2;
    std::vector<float> c(static_cast<std::size_t>(max_seq_len) * half), sn(c.size());
    bx_rope_table_host(c.data(), sn.data(), max_seq_len, cfg_.head_dim, cfg_.rope_theta);
    batch_cos_ = bt::Tensor::from_host_on(bt::Device::ROCm, c.data(), max_seq_len, half);
    batch_sin_ = bt::Tensor::from_host_on(bt::Device::ROCm, sn.data(), max_seq_len, half);
    batch_meta_ = bt::Tensor::empty_on(bt::Device::ROCm, n_slots, 2 * kMetaI64PerRow, bt::Dtype::FP32);
    batch_graphs_.reset();
    const int H = cfg_.hidden_size, F = cfg_.intermediate_size, qd = cfg_.num_attention_heads * cfg_.head_dim;
    const auto dev = bt::Device::ROCm;
    bh_ = bt::Tensor::empty_on(dev, n_slots, H, bt::Dtype::FP32);
    bnorm_ = bt::Tensor::empty_on(dev, n_slots, H, bt::Dtype::FP16);
    bq_ = bt::Tensor::empty_on(dev, n_slots, qd, bt::Dtype::FP16);
    bk_ = bt::Tensor::empty_on(dev, n_slots, width, bt::Dtype::FP16);
    bv_ = bt::Tensor::empty_on(dev, n_slots, width, bt::Dtype::FP16);
    battn_ = bt::Tensor::empty_on(dev, n_slots, qd, bt::Dtype::FP16);
    bproj_ = bt::Tensor::empty_on(dev, n_slots, H, bt::Dtype::FP16);
    bgate_ = bt::Tensor::empty_on(dev, n_slots, F, bt::Dtype::FP16);
    bup_ = bt::Tensor::empty_on(dev, n_slots, F, bt::Dtype::FP16);
    blogits_ = bt::Tensor::empty_on(dev, n_slots, cfg_.vocab_size, bt::Dtype::FP16);
    // the batched attention's records and counters, for any M <= n_slots;
    // zeroed once (each launch leaves its counters at zero)
    std::size_t wsb = 0;
    for (int m = 1; m <= n_slots; ++m)
        wsb = std::max(wsb, bx_batch_attention_workspace_bytes(m, cfg_.num_attention_heads,
                                                               cfg_.num_key_value_heads, cfg_.head_dim, max_seq_len));
    bws_ = bt::Tensor::empty_on(dev, 1, static_cast<int>((wsb + 3) / 4), bt::Dtype::FP32);
    hipx::check(hipMemset(bws_.data, 0, bws_.bytes()), "hipMemset batch attention workspace");
    bss_ = bt::Tensor::empty_on(dev, 1, static_cast<int>(bx_linear_ss_floats(H)), bt::Dtype::FP32);
    batch_graphs_ = std::make_unique<BatchGraphs>(n_slots);
}

int DenseDecoder::slot_len(int slot) const {
    if (slot < 0 || slot >= batch_slots_) fail("slot_len: slot out of range");
    return slot_len_[static_cast<std::size_t>(slot)];
}

void DenseDecoder::truncate_slot(int slot, int len) {
    if (slot < 0 || slot >= batch_slots_) fail("truncate_slot: slot out of range");
    if (len < 0 || len > slot_len_[static_cast<std::size_t>(slot)])
        fail("truncate_slot: len must be in [0, slot_len]");
    slot_len_[static_cast<std::size_t>(slot)] = len;
}

void DenseDecoder::prefill_slot(int slot, const int32_t* ids, int L, bt::Tensor& logits_out) {
    if (batch_slots_ == 0) fail("prefill_slot: batch not allocated");
    if (slot < 0 || slot >= batch_slots_) fail("prefill_slot: slot out of range");
    const int len = slot_len_[static_cast<std::size_t>(slot)];
    check_forward("prefill_slot", ids, L, true, batch_cap_, len, cfg_.vocab_size);
    const int width = cfg_.num_key_value_heads * cfg_.head_dim;
    const std::size_t plane = static_cast<std::size_t>(batch_slots_) * batch_cap_ * width;  // FP16 elements
    const std::size_t at = static_cast<std::size_t>(slot) * batch_cap_ * width;
    auto* base = static_cast<std::uint16_t*>(batch_kv_.data);
    // point every layer's cache at the slot's rows for the op-path prefill,
    // then put the single-sequence views (and cache_len) back
    std::vector<bt::Tensor> saved;
    saved.reserve(2 * layers_.size());
    for (std::size_t l = 0; l < layers_.size(); ++l) {
        saved.push_back(std::move(layers_[l].K_cache));
        saved.push_back(std::move(layers_[l].V_cache));
        layers_[l].K_cache = bt::Tensor::view(bt::Device::ROCm, base + 2 * l * plane + at, batch_cap_, width,
                                              bt::Dtype::FP16);
        layers_[l].V_cache = bt::Tensor::view(bt::Device::ROCm, base + (2 * l + 1) * plane + at, batch_cap_, width,
                                              bt::Dtype::FP16);
    }
    const int saved_len = cache_len_;
    auto restore = [&] {
        for (std::size_t l = 0; l < layers_.size(); ++l) {
            layers_[l].K_cache = std::move(saved[2 * l]);
            layers_[l].V_cache = std::move(saved[2 * l + 1]);
        }
        cache_len_ = saved_len;
    };
    try {
        cache_len_ = len;
        ids_dev_ = make_idx_device(ids, L);
        resize_like(h_, L, cfg_.hidden_size, bt::Dtype::FP32, bt::Device::ROCm);
        hipx::bx(bx_embedding_f32(static_cast<const uint16_t*>(embed_tokens_.data), embed_tokens_.rows,
                                  embed_tokens_.cols, static_cast<const int32_t*>(ids_dev_.data), L,
                                  static_cast<float*>(h_.data), bt::stream()),
                 "embedding");
        run_layers_(L, logits_out, nullptr, /*logits_last_row_only=*/true);
    } catch (...) {
        restore();
        throw;
    }
    slot_len_[static_cast<std::size_t>(slot)] = len + L;
    restore();
}

// The batched step for M rows on the op stream (eager, or recorded into a
// graph): every pointer it uses is fixed between allocate_batch calls, and the
// attention split plan is sized by the slot capacity, not the current lengths.
void DenseDecoder::enqueue_batch_(int M) {
    const auto* meta = static_cast<const std::int64_t*>(batch_meta_.data);
    const std::int64_t* base_d = meta + M;
    const int32_t* lens_d = reinterpret_cast<const int32_t*>(meta + 2 * M) + M;
    const int32_t* ids_d = lens_d + M;
    const int HD = cfg_.head_dim, n_q = cfg_.num_attention_heads, n_kv = cfg_.num_key_value_heads;
    const int width = n_kv * HD;
    const float eps = cfg_.rms_norm_eps;
    void* st = bt::stream();
    void* const lws = hipx::linear_ws();
    const size_t lwsb = hipx::linear_ws_bytes();
    bh_.resize(M, cfg_.hidden_size, bt::Dtype::FP32);
    battn_.resize(M, n_q * HD, bt::Dtype::FP16);
    hipx::bx(bx_embedding_f32(static_cast<const uint16_t*>(embed_tokens_.data), embed_tokens_.rows,
                              embed_tokens_.cols, ids_d, M, static_cast<float*>(bh_.data), st),
             "forward_batch embedding");
    const std::int64_t plane_rows = static_cast<std::int64_t>(batch_slots_) * batch_cap_;
    auto* arena = static_cast<std::uint16_t*>(batch_kv_.data);
    const auto* cs = static_cast<const float*>(batch_cos_.data);
    const auto* sn = static_cast<const float*>(batch_sin_.data);
    // The residual RMSNorms ride on the GEMV launches: a residual launch also
    // writes each row's sum of squares of the updated h (per 64 columns, into
    // bss_), and the next q / k / v or gate / up launch normalises h itself
    // while staging it.  A launch outside those forms (fewer than 3 rows, or
    // shapes the split GEMV does not take) returns BX_EUNSUPPORTED without
    // running; then the norm runs on its own and the plain forms take its
    // FP16 output.
    float* ss = static_cast<float*>(bss_.data);
    const float* hf = static_cast<const float*>(bh_.data);
    bool have_ss = false;   // ss holds the row sums of the current h
    auto unsupported = [](int rc, const char* what) {
        if (rc == BX_EUNSUPPORTED) return true;
        hipx::bx(rc, what);
        return false;
    };
    // members [0, n) of the q / k / v projections (or one of them) of
    // RMSNorm(h; gain) in one launch; false when the caller must norm first
    auto group_norm = [&](const bt::Tensor* const* w, bt::Tensor* const* y, int n, const bt::Tensor& gain) {
        if (!have_ss) return false;
        const void* W[3];
        uint16_t* Y[3];
        int N[3];
        for (int i = 0; i < n; ++i) {
            y[i]->resize(M, w[i]->rows, bt::Dtype::FP16);
            W[i] = w[i]->data;
            Y[i] = static_cast<uint16_t*>(y[i]->data);
            N[i] = w[i]->rows;
        }
        return !unsupported(bx_linear_group_norm_f16(bt::dtype_to_ggml(w[0]->dtype), n, W, Y, N, hf,
                                                     static_cast<const uint16_t*>(gain.data), eps, ss, M,
                                                     cfg_.hidden_size, lws, lwsb, st),
                            "forward_batch q / k / v with the norm");
    };
    // q and k of one weight type and v of another (Q4_K and Q6_K) in one
    // launch, normalising h (with_norm: needs the row sums) or from bnorm_
    auto group2 = [&](const bt::Tensor* const* w, bt::Tensor* const* y, const bt::Tensor& gain,
                      bool with_norm = true) {
        if (with_norm && !have_ss) return false;
        const void* W[3];
        uint16_t* Y[3];
        int N[3];
        for (int i = 0; i < 3; ++i) {
            y[i]->resize(M, w[i]->rows, bt::Dtype::FP16);
            W[i] = w[i]->data;
            Y[i] = static_cast<uint16_t*>(y[i]->data);
            N[i] = w[i]->rows;
        }
        const int t1 = bt::dtype_to_ggml(w[0]->dtype), t2 = bt::dtype_to_ggml(w[2]->dtype);
        const int rc = with_norm ? bx_linear_group2_norm_f16(t1, t2, 3, 2, W, Y, N, hf,
                                                             static_cast<const uint16_t*>(gain.data), eps, ss, M,
                                                             cfg_.hidden_size, lws, lwsb, st)
                                 : bx_linear_group2_f16(t1, t2, 3, 2, W, Y, N,
                                                        static_cast<const uint16_t*>(bnorm_.data), M,
                                                        cfg_.hidden_size, lws, lwsb, st);
        return !unsupported(rc, "forward_batch q / k / v");
    };
    auto residual = [&](const bt::Tensor& W, const bt::Tensor& X) {
        const int rc = bx_linear_residual_ss_f16(bt::dtype_to_ggml(W.dtype), W.data,
                                                 static_cast<const uint16_t*>(X.data), static_cast<float*>(bh_.data),
                                                 ss, M, W.rows, W.cols, lws, lwsb, st);
        have_ss = rc == BX_OK;
        if (have_ss || !unsupported(rc, "forward_batch residual projection")) return;
        if (!bt::linear_residual_forward_batched(W, X, bh_)) {
            linear_batched(W, nullptr, X, bproj_);
            bt::add_inplace(bh_, bproj_);
        }
    };
    for (std::size_t l = 0; l < layers_.size(); ++l) {
        Layer& layer = layers_[l];
        {
            // q / k / v: the members that share a weight type in one launch
            // (fused forms: 3 <= M <= 16 on the matrix cores), with the norm
            // when the previous residual launch left the row sums
            const bt::Tensor* w[3] = {&layer.Wq, &layer.Wk, &layer.Wv};
            bt::Tensor* y[3] = {&bq_, &bk_, &bv_};
            const int same = layer.Wk.dtype != layer.Wq.dtype ? 1 : layer.Wv.dtype == layer.Wq.dtype ? 3 : 2;
            int done = 0;
            if (same == 2 && group2(w, y, layer.input_ln)) {
                done = 3;
            } else if (group_norm(w, y, same, layer.input_ln)) {
                done = same;
                while (done < 3 && group_norm(w + done, y + done, 1, layer.input_ln)) ++done;
            }
            if (done < 3) {
                bt::rms_norm_forward(bh_, layer.input_ln, eps, bnorm_);
                if (done == 0 && same == 2 && group2(w, y, layer.input_ln, false)) done = 3;
                if (done == 0 && same > 1 && bt::linear_group_forward_batched(w, y, same, bnorm_)) done = same;
                for (int i = done; i < 3; ++i) linear_batched(*w[i], nullptr, bnorm_, *y[i]);
            }
        }
        // q / k head norms, RoPE, the cache write of k / v and the attention
        // over each row's own keys in one launch
        std::uint16_t* Kp = arena + static_cast<std::size_t>(2 * l) * plane_rows * width;
        std::uint16_t* Vp = Kp + static_cast<std::size_t>(plane_rows) * width;
        const bool qkn = cfg_.use_qk_norm;
        hipx::bx(bx_batch_attention_f16(static_cast<const uint16_t*>(bq_.data), static_cast<const uint16_t*>(bk_.data),
                                        static_cast<const uint16_t*>(bv_.data), M, HD, n_q, n_kv,
                                        qkn ? static_cast<const uint16_t*>(layer.q_norm.data) : nullptr,
                                        qkn ? static_cast<const uint16_t*>(layer.k_norm.data) : nullptr, eps, lens_d,
                                        base_d, batch_cap_, cs, sn, batch_cap_, Kp, Vp, plane_rows,
                                        static_cast<uint16_t*>(battn_.data), bws_.data, st),
                 "forward_batch attention");
        residual(layer.Wo, battn_);
        bool mlp = false;
        if (have_ss && layer.gate_W.dtype == layer.up_W.dtype && layer.gate_W.rows == layer.up_W.rows) {
            bgate_.resize(M, layer.gate_W.rows, bt::Dtype::FP16);
            mlp = !unsupported(bx_linear_swiglu_norm_f16(bt::dtype_to_ggml(layer.gate_W.dtype), layer.gate_W.data,
                                                         layer.up_W.data, hf,
                                                         static_cast<const uint16_t*>(layer.post_attn_ln.data), eps,
                                                         ss, static_cast<uint16_t*>(bgate_.data), M, layer.gate_W.rows,
                                                         layer.gate_W.cols, lws, lwsb, st),
                               "forward_batch gate / up with the norm");
        }
        if (!mlp) {
            bt::rms_norm_forward(bh_, layer.post_attn_ln, eps, bnorm_);
            if (!bt::linear_swiglu_forward_batched(layer.gate_W, layer.up_W, bnorm_, bgate_)) {
                linear_batched(layer.gate_W, nullptr, bnorm_, bgate_);
                linear_batched(layer.up_W, nullptr, bnorm_, bup_);
                bt::silu_forward(bgate_, bgate_);
                bt::mul_inplace(bgate_, bup_);
            }
        }
        residual(layer.down_W, bgate_);
    }
    bt::rms_norm_forward(bh_, final_norm_, eps, bnorm_);
    linear_batched(lm_head_, nullptr, bnorm_, blogits_);
}

void DenseDecoder::forward_batch(const int32_t* ids, const int32_t* slots, int M, bt::Tensor& logits_out) {
    if (batch_slots_ == 0) fail("forward_batch: batch not allocated");
    if (!ids || !slots) fail("forward_batch: null ids or slots");
    if (M <= 0 || M > batch_slots_) fail("forward_batch: M must be in [1, batch_slots]");
    std::vector<char> seen(static_cast<std::size_t>(batch_slots_), 0);
    batch_meta_host_.assign(static_cast<std::size_t>(kMetaI64PerRow) * M, 0);
    std::int64_t* dst = batch_meta_host_.data();
    std::int64_t* base = dst + M;
    auto* pos = reinterpret_cast<int32_t*>(dst + 2 * M);
    int32_t* lens = pos + M;
    int32_t* idv = lens + M;
    for (int r = 0; r < M; ++r) {
        const int s = slots[r];
        if (s < 0 || s >= batch_slots_) fail("forward_batch: slot out of range");
        if (seen[static_cast<std::size_t>(s)]) fail("forward_batch: a slot appears twice");
        seen[static_cast<std::size_t>(s)] = 1;
        const int len = slot_len_[static_cast<std::size_t>(s)];
        if (len >= batch_cap_) fail("forward_batch: slot is full");
        if (ids[r] < 0 || ids[r] >= cfg_.vocab_size) fail("forward_batch: token id out of range");
        base[r] = static_cast<std::int64_t>(s) * batch_cap_;
        dst[r] = base[r] + len;
        pos[r] = len;
        lens[r] = len + 1;
        idv[r] = ids[r];
    }
    hipx::h2d(batch_meta_.data, batch_meta_host_.data(), batch_meta_host_.size() * sizeof(std::int64_t));
    BatchGraphs& g = *batch_graphs_;
    const std::size_t mi = static_cast<std::size_t>(M);
    if (!g.use_graph || !g.warmed[mi]) {
        enqueue_batch_(M);
        g.warmed[mi] = 1;
    } else {
        hipStream_t st = static_cast<hipStream_t>(bt::stream());
        if (!g.exec[mi]) {
            hipx::check(hipStreamBeginCapture(st, hipStreamCaptureModeThreadLocal), "hipStreamBeginCapture");
            hipGraph_t graph = nullptr;
            try {
                enqueue_batch_(M);
            } catch (...) {
                (void)hipStreamEndCapture(st, &graph);
                if (graph) (void)hipGraphDestroy(graph);
                throw;
            }
            hipx::check(hipStreamEndCapture(st, &graph), "hipStreamEndCapture");
            const hipError_t e = hipGraphInstantiate(&g.exec[mi], graph, nullptr, nullptr, 0);
            (void)hipGraphDestroy(graph);
            hipx::check(e, "hipGraphInstantiate");
        }
        hipx::check(hipGraphLaunch(g.exec[mi], st), "hipGraphLaunch");
    }
    logits_out = bt::Tensor::view(bt::Device::ROCm, blogits_.data, M, cfg_.vocab_size, bt::Dtype::FP16);
    for (int r = 0; r < M; ++r) ++slot_len_[static_cast<std::size_t>(slots[r])];
}

}  // namespace brolm::detail
