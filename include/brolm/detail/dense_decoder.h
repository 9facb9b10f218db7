#pragma once

// Dense GQA / SwiGLU / RoPE causal decoder core (reference
// include/brolm/detail/dense_decoder.h:84-239, src/detail/dense_decoder.cpp).
//
// Same public surface and semantics as the reference: load_weights through a
// Source, a per-layer FP16 KV cache of (max_seq, n_kv*head_dim),
// forward / forward_last / embed_tokens / forward_embeds, truncate_cache as
// the speculative-draft seam.  MI355X-specific structure:
//   - the residual stream is FP32 in HBM (H*4 bytes per row);
//   - L > 1 (prefill) runs the op surface (MFMA GEMM + split-K attention);
//   - L == 1 runs the fused decode step (six kernels per layer), captured
//     once into a hipGraph and replayed with the token id and position read
//     from device memory (BROLM_NO_GRAPH=1 launches the same kernels eagerly,
//     so graph and eager decode are bit-identical);
//   - decode_greedy() keeps greedy generation on the device: argmax and the
//     next token feed the following replay without a host round trip.

#include <cstdint>
#include <memory>
#include <vector>

#include "brotensor/tensor.h"
#include "brolm_hip.h"

namespace brolm::detail::weights { class Source; }

namespace brolm::detail {

struct DecodeGraphSession;

struct DenseDecoderConfig {
    int vocab_size = 0;
    int hidden_size = 0;
    int intermediate_size = 0;
    int num_hidden_layers = 0;
    int num_attention_heads = 0;
    int num_key_value_heads = 0;
    int head_dim = 0;
    float rms_norm_eps = 1e-6f;
    float rope_theta = 1000000.0f;
    bool use_qk_norm = false;
    bool tie_word_embeddings = true;
};

class DenseDecoder {
public:
    explicit DenseDecoder(const DenseDecoderConfig& cfg);
    ~DenseDecoder();
    DenseDecoder(const DenseDecoder&) = delete;
    DenseDecoder& operator=(const DenseDecoder&) = delete;
    DenseDecoder(DenseDecoder&&) noexcept;
    DenseDecoder& operator=(DenseDecoder&&) noexcept;

    void load_weights(const brolm::detail::weights::Source& src);
    void allocate_cache(int max_seq_len);
    void reset_cache();
    void truncate_cache(int len);
    int cache_len() const { return cache_len_; }
    int max_seq_len() const { return max_seq_len_; }

    void forward(const int32_t* ids, int L, brotensor::Tensor& logits_out, brotensor::Tensor* hidden_out = nullptr);
    void forward_last(const int32_t* ids, int L, brotensor::Tensor& logits_out);
    void embed_tokens(const int32_t* ids, int L, brotensor::Tensor& out);
    void forward_embeds(const brotensor::Tensor& embeds, int L, brotensor::Tensor& logits_out,
                        brotensor::Tensor* hidden_out = nullptr);
    // Bidirectional, cacheless pass for encoder use (dense_decoder.h:157-169):
    // every layer attends all L tokens (no causal mask, RoPE positions from
    // 0), no lm_head; hidden_out := (L, hidden_size) post-final-norm FP16.
    // Needs no cache allocation and leaves the KV cache untouched.
    void forward_encode(const int32_t* ids, int L, brotensor::Tensor& hidden_out);

    // Greedy decode of up to n tokens starting from `token` at position
    // cache_len(), entirely on the device (argmax feeds the next step).
    // Writes the n sampled ids to out; stops after eos_id when eos_id >= 0.
    // Returns the number of ids written; cache_len advances by that count.
    int decode_greedy(int32_t token, int n, int32_t* out, int eos_id);
    // The same loop with top-k / top-p sampling on the device (temperature >
    // 0): step i draws with u[i] (host values in [0, 1), one per token, taken
    // from the caller's generator in order, as generate.cpp:68-142 draws them).
    int decode_sampled(int32_t token, int n, const double* u, float temperature, int top_k, float top_p,
                       int32_t* out, int eos_id);

    // Replays the captured step n times from `token` at cache_len() and
    // returns the GPU time per step in milliseconds (hipEvents around the
    // replays); cache_len advances by n.  Used by bench.py.
    double time_decode_steps(int32_t token, int n);

    // Bytes of weights one decode step streams (carrier bytes of every
    // per-layer matrix + lm_head + one embedding row + norm gammas).
    std::int64_t decode_weight_bytes() const;

    // How single-token steps run: 2 = persistent single launch, 1 = replayed
    // hipGraph of per-stage kernels, 0 = the same kernels launched eagerly,
    // 3 = the op path (one forward_last per token).  Needs loaded weights and
    // an allocated cache (creates the step session when one is used).
    int decode_mode();

    // ── Multi-sequence batched decode ──────────────────────────────────────
    // An extension beyond the reference's single cache: n_slots independent
    // sequences, each with its own KV rows (slot-major arena, capacity
    // max_seq_len per slot), stepped together so one pass over the weights
    // serves M tokens.  The single-sequence cache above is untouched.
    void allocate_batch(int n_slots, int max_seq_len);
    int batch_slots() const { return batch_slots_; }
    int batch_capacity() const { return batch_cap_; }
    int slot_len(int slot) const;
    void truncate_slot(int slot, int len);
    // Appends L prompt tokens to `slot` (op path, causal over the slot's own
    // rows); logits_out := logits of the last row (1, vocab).
    void prefill_slot(int slot, const int32_t* ids, int L, brotensor::Tensor& logits_out);
    // One decode step of M sequences: row r is token ids[r] of slot slots[r]
    // (distinct slots) at position slot_len(slots[r]); logits_out := (M,
    // vocab) FP16 on the device.  Every listed slot's length advances by one.
    void forward_batch(const int32_t* ids, const int32_t* slots, int M, brotensor::Tensor& logits_out);

    const DenseDecoderConfig& config() const { return cfg_; }

private:
    struct Layer {
        brotensor::Tensor input_ln;
        brotensor::Tensor Wq, Wk, Wv, Wo;
        brotensor::Tensor q_norm, k_norm;
        brotensor::Tensor post_attn_ln;
        brotensor::Tensor gate_W, up_W, down_W;
        brotensor::Tensor K_cache, V_cache;
        // FP16 copies of the quantized matrices for long prompts (empty until
        // the first one, and when they would not fit)
        brotensor::Tensor q16, k16, v16, o16, gate16, up16, down16;
    };

    void run_layers_encode_(int L, brotensor::Tensor& hidden_out);
    void run_layers_(int L, brotensor::Tensor& logits_out, brotensor::Tensor* hidden_out,
                     bool logits_last_row_only = false);
    void decode_step_(int32_t token, brotensor::Tensor& logits_out);
    DecodeGraphSession& session_();
    bool fused_step_ok_() const;
    ::bx_decode_dims decode_dims_() const;
    void invalidate_graph_();
    void ensure_rope_table_();
    bool prefill_f16_(int L);   // FP16 layer copies in use for an L-row pass

    DenseDecoderConfig cfg_;
    brotensor::Tensor embed_tokens_;
    std::vector<Layer> layers_;
    brotensor::Tensor final_norm_;
    brotensor::Tensor lm_head_;

    int cache_len_ = 0;
    int max_seq_len_ = 0;
    // every layer's K then V, (capacity, n_kv*head_dim) FP16 each; the
    // layers' K_cache / V_cache are views into it
    brotensor::Tensor kv_arena_;

    brotensor::Tensor rope_cos_, rope_sin_;  // (cap, hd/2) FP32
    brotensor::Tensor ids_dev_, h_, norm_, q_, k_, v_, qn_, kn_, attn_, proj_, gate_, up_;
    brotensor::Tensor attn_ws_;

    std::unique_ptr<DecodeGraphSession> graph_;
    int f16_state_ = 0;   // FP16 layer copies: 0 not tried, 1 built, -1 declined

    // batched decode: per layer a K plane then a V plane, each
    // (n_slots * capacity, n_kv * head_dim) FP16; slot s, position p is row
    // s * capacity + p of both
    int batch_slots_ = 0;
    int batch_cap_ = 0;
    std::vector<int> slot_len_;
    brotensor::Tensor batch_kv_;
    brotensor::Tensor batch_cos_, batch_sin_;  // (capacity, hd/2) FP32
    brotensor::Tensor batch_meta_;             // per-step row metadata (device)
    std::vector<std::int64_t> batch_meta_host_;
    // the batched step's own activations, sized for n_slots rows at
    // allocate_batch so that a step of any M <= n_slots keeps their addresses
    // (each M's step is captured once into a hipGraph and replayed)
    brotensor::Tensor bh_, bnorm_, bq_, bk_, bv_, battn_, bproj_, bgate_, bup_, blogits_, bws_, bss_;
    struct BatchGraphs;
    std::unique_ptr<BatchGraphs> batch_graphs_;
    void enqueue_batch_(int M);
};

}  // namespace brolm::detail
