/*
 * brolm_c.h — C ABI of libbrolm.so, the C++20 Qwen3 decode stack
 * (include/brolm/qwen.h, include/brolm/qwen_generate.h) for FFI callers
 * (Python ctypes, cgo, ...).  Each entry point forwards to the C++ API named
 * beside it, which mirrors the reference's (paths in wlejon/brolm).
 *
 * Conventions: int returns are 0 on success, -1 on failure with a
 * thread-local message from brolm_last_error(); host buffers are caller-owned;
 * logits come back as FP32 values of the FP16 device logits.
 */
#ifndef BROLM_C_H
#define BROLM_C_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef struct brolm_qwen3 brolm_qwen3;

/* Qwen3Config (include/brolm/qwen.h:35-47). */
typedef struct {
    int vocab_size, hidden_size, intermediate_size, num_hidden_layers;
    int num_attention_heads, num_key_value_heads, head_dim;
    float rms_norm_eps, rope_theta;
    int tie_word_embeddings, max_position_embeddings;
} brolm_qwen3_config;

/* Synthetic checkpoint spec (include/brolm/synth.h); *_type are ggml ids. */
typedef struct {
    int vocab, hidden, intermediate, layers, n_q, n_kv, head_dim;
    float eps, theta;
    int context, tied;
    int embed_type, q_type, k_type, v_type, o_type, gate_type, up_type, down_type, output_type;
    float stddev;
    uint64_t seed;
    int more_bits_type;  /* ggml id for attn_v / ffn_down on use_more_bits layers, -1: none */
} brolm_synth_qwen3_spec;

const char* brolm_last_error(void);
/* brotensor::init(): registers the gfx950 device (fails without one). */
int brolm_init(void);
/* brotensor::shutdown(): after the queued work, frees the runtime's own
 * device buffers (op scratch, RoPE tables, sampler buffers, profiler events)
 * and the op stream.  Models still open stay valid to close.  No-op when
 * not initialised. */
int brolm_shutdown(void);

/* synth::write_qwen3_gguf */
int brolm_synth_qwen3_write(const brolm_synth_qwen3_spec* spec, const char* path);
/* synth::normal_bf16 / synth::quantize (test hooks for the generator). */
int brolm_synth_normal_bf16(uint64_t key, int64_t n, float stddev, float* out);
uint64_t brolm_synth_tensor_key(uint64_t seed, const char* name);
int brolm_synth_quantize(int ggml_type, const float* src, int64_t n, uint8_t* dst);

/* qwen3_hf_to_ggml (src/qwen.cpp:173-208): writes the ggml name to out
 * (NUL-terminated, cap bytes) and returns its length; 0 if unmapped. */
int brolm_qwen3_hf_to_ggml(const char* hf_name, char* out, int cap);
/* Qwen3Config::from_gguf (src/qwen.cpp:88-149). */
int brolm_qwen3_config_from_gguf(const char* path, brolm_qwen3_config* out);
/* GGUF metadata / tensor directory of the product reader (gguf::File). */
int brolm_gguf_tensor_count(const char* path, int64_t* out);
int brolm_gguf_tensor_info(const char* path, const char* name, int* ggml_type, int64_t* dims4, int* ndims,
                           int64_t* nbytes);
/* Tensor bytes as stored (nbytes of brolm_gguf_tensor_info); returns nbytes,
 * or -1 on error or when cap is too small. */
int64_t brolm_gguf_tensor_data(const char* path, const char* name, uint8_t* out, int64_t cap);
/* Metadata of the product reader: integer scalars of any width (and bool),
 * float scalars (F32 / F64), strings (returns the byte length, -1 when absent,
 * not a string or cap too small; no terminator written), arrays (element
 * value type and count). */
int brolm_gguf_meta_int(const char* path, const char* key, int64_t* out);
int brolm_gguf_meta_f64(const char* path, const char* key, double* out);
int64_t brolm_gguf_meta_str(const char* path, const char* key, char* out, int64_t cap);
int brolm_gguf_meta_array(const char* path, const char* key, int* elem_type, int64_t* count);
/* gguf::File::from_memory over a byte buffer: 0 and the tensor count when it
 * parses, nonzero with brolm_last_error() when it is malformed. */
int brolm_gguf_parse_memory(const uint8_t* data, int64_t size, int64_t* n_tensors);

/* Mistral3Config (include/brolm/mistral3_config.h:30-143): the text section
 * and the top-level multimodal glue (the Pixtral vision section is not part
 * of this build). */
typedef struct {
    int vocab_size, hidden_size, intermediate_size, num_hidden_layers;
    int num_attention_heads, num_key_value_heads, head_dim;
    float rms_norm_eps, rope_theta;
    int tie_word_embeddings, max_position_embeddings;
    int has_sliding_window, sliding_window;
} brolm_mistral3_text_config;
typedef struct {
    brolm_mistral3_text_config text;
    int image_token_index, spatial_merge_size, multimodal_projector_bias;
} brolm_mistral3_config;

/* Mistral3Config::from_gguf (src/mistral3_config.cpp:130-191) */
int brolm_mistral3_config_from_gguf(const char* path, brolm_mistral3_config* out);
/* Mistral3Config::from_json_text (src/mistral3_config.cpp:36-93); text is a
 * NUL-terminated config.json document. */
int brolm_mistral3_config_from_json(const char* text, brolm_mistral3_config* out);
/* mistral3_hf_to_ggml (src/mistral3_text.cpp:70-108); same contract as
 * brolm_qwen3_hf_to_ggml. */
int brolm_mistral3_hf_to_ggml(const char* hf_name, char* out, int cap);
/* synth::write_mistral3_gguf: arch "llama", no QK-norm gammas. */
int brolm_synth_mistral3_write(const brolm_synth_qwen3_spec* spec, const char* path);
/* mistral3::TextModel (include/brolm/mistral3_text.h:52-131).  Returns a
 * decoder handle: brolm_qwen3_free, _load_gguf, _allocate_cache,
 * _reset_cache, _truncate_cache, _cache_len, _forward, _forward_last,
 * _embed_tokens, _forward_embeds, _generate (mistral3::generate,
 * include/brolm/mistral3_generate.h:40-43), _decode_greedy,
 * _time_decode_steps, _decode_weight_bytes and _decode_mode accept it;
 * brolm_qwen3_generate_text (Qwen tokenizer) rejects it. */
brolm_qwen3* brolm_mistral3_text_create(const brolm_mistral3_text_config* cfg);

/* llm2vec::Config (include/brolm/llm2vec.h:41-63). */
typedef struct {
    int vocab_size, hidden_size, intermediate_size, num_hidden_layers;
    int num_attention_heads, num_key_value_heads, head_dim;
    float rms_norm_eps, rope_theta;
} brolm_llm2vec_config;
/* llm2vec::Config::from_json_text (src/llm2vec.cpp:70-96). */
int brolm_llm2vec_config_from_json(const char* text, brolm_llm2vec_config* out);
/* llm2vec::Encoder (include/brolm/llm2vec.h:65-114) over GGUF weights: a
 * decoder handle for brolm_qwen3_free / _load_gguf / brolm_decoder_forward_encode. */
brolm_qwen3* brolm_llm2vec_create(const brolm_llm2vec_config* cfg);
/* DenseDecoder::forward_encode (dense_decoder.h:157-169) on any decoder
 * handle: bidirectional, cacheless; hidden (L, hidden_size) FP32 values of the
 * FP16 result.  Encoder::encode on an llm2vec handle. */
int brolm_decoder_forward_encode(brolm_qwen3* m, const int32_t* ids, int L, float* hidden);
/* Encoder::encode_pooled (src/llm2vec.cpp:137-153): emb (hidden_size); mask
 * (host, L floats) or NULL for every token. */
int brolm_llm2vec_encode_pooled(brolm_qwen3* m, const int32_t* ids, int L, const float* mask, float* emb);

/* Qwen3Model (include/brolm/qwen.h:58-157). */
brolm_qwen3* brolm_qwen3_create(const brolm_qwen3_config* cfg);
void brolm_qwen3_free(brolm_qwen3* m);
int brolm_qwen3_load_gguf(brolm_qwen3* m, const char* path);
int brolm_qwen3_allocate_cache(brolm_qwen3* m, int max_seq_len);
int brolm_qwen3_reset_cache(brolm_qwen3* m);
int brolm_qwen3_truncate_cache(brolm_qwen3* m, int len);
int brolm_qwen3_cache_len(const brolm_qwen3* m);
/* forward: logits (L, vocab); hidden (L, hidden) or NULL. */
/* Multi-sequence batched decode (no counterpart in the reference, whose
 * model holds one sequence; dense_decoder.h:84-239 is the one-sequence
 * surface these extend): n_slots sequences with their own KV rows. */
int brolm_qwen3_allocate_batch(brolm_qwen3* m, int n_slots, int max_seq_len);
/* Tokens held by `slot` (>= 0), or a negative error code. */
int brolm_qwen3_slot_len(const brolm_qwen3* m, int slot);
int brolm_qwen3_truncate_slot(brolm_qwen3* m, int slot, int len);
/* Appends L prompt tokens to `slot`; logits (vocab) of the last one. */
int brolm_qwen3_prefill_slot(brolm_qwen3* m, int slot, const int32_t* ids, int L, float* logits);
/* One step of M sequences: ids[r] joins slot slots[r] (distinct slots);
 * logits (M, vocab) row-major. */
int brolm_qwen3_forward_batch(brolm_qwen3* m, const int32_t* ids, const int32_t* slots, int M, float* logits);
/* n calls of forward_batch without reading logits back; wall-clock ms per
 * call (every slot advances by n), or -1 on error. */
double brolm_qwen3_time_forward_batch(brolm_qwen3* m, const int32_t* ids, const int32_t* slots, int M, int n);
int brolm_qwen3_forward(brolm_qwen3* m, const int32_t* ids, int L, float* logits, float* hidden);
/* forward_last: logits (1, vocab). */
int brolm_qwen3_forward_last(brolm_qwen3* m, const int32_t* ids, int L, float* logits);
/* embed_tokens: out (L, hidden) FP16 bits. */
int brolm_qwen3_embed_tokens(brolm_qwen3* m, const int32_t* ids, int L, uint16_t* out);
/* forward_embeds: embeds (L, hidden) FP16 bits from the host. */
int brolm_qwen3_forward_embeds(brolm_qwen3* m, const uint16_t* embeds, int L, float* logits, float* hidden);
/* qwen::generate (include/brolm/qwen_generate.h:45-47); returns the count. */
int brolm_qwen3_generate(brolm_qwen3* m, const int32_t* prompt, int n_prompt, int max_new, int eos_id,
                         int stop_on_eos, float temperature, int top_k, float top_p, uint64_t seed,
                         int device_greedy, int device_sampling, int32_t* out);
/* DenseDecoder::decode_greedy / time_decode_steps / decode_weight_bytes. */
int brolm_qwen3_decode_greedy(brolm_qwen3* m, int32_t token, int n, int32_t* out, int eos_id);
/* Device-side top-k / top-p continuation (DenseDecoder::decode_sampled): n
 * tokens from `token`, step i drawing with u[i] in [0, 1); returns the ids
 * written (stops after eos_id when eos_id >= 0), or a negative error code. */
int brolm_qwen3_decode_sampled(brolm_qwen3* m, int32_t token, int n, const double* u, float temperature, int top_k,
                               float top_p, int32_t* out, int eos_id);
double brolm_qwen3_time_decode_steps(brolm_qwen3* m, int32_t token, int n);
int64_t brolm_qwen3_decode_weight_bytes(const brolm_qwen3* m);
/* DenseDecoder::decode_mode: 2 persistent single launch, 1 captured graph, 0 eager, 3 the op path
 * (one forward_last per token: weight types or shapes the fused step does not take, or
 * BROLM_OP_STEP=1); -1 on error
 * (no counterpart in the reference: reports which of this build's step paths runs). */
int brolm_qwen3_decode_mode(brolm_qwen3* m);

/* sample_token with a fresh std::mt19937_64(seed) (src/detail/generate.cpp:68-142). */
int brolm_sample_token(const float* logits, int vocab, float temperature, int top_k, float top_p, uint64_t seed);
/* The same draw on the device (sample_token_device, include/brolm/detail/generate.h):
 * logits_dev is one FP16 row in device memory; u is the first
 * uniform_real_distribution<double>(0, 1) draw of std::mt19937_64(seed).
 * Returns the token id, or -1 with brolm_last_error(). */
int brolm_sample_token_device(const uint16_t* logits_dev, int vocab, float temperature, int top_k, float top_p,
                              uint64_t seed);

/* Synthetic prompt of tools/bench_decode.cpp:208-213: std::mt19937_64(seed)() % vocab. */
int brolm_prompt_ids(uint64_t seed, int n, int vocab, int32_t* out);

/* BROLM_PROFILE stage table (reference src/detail/profile.cpp), timed with
 * HIP events on the op stream. */
void brolm_profile_reset(void);
void brolm_profile_report(void);
int brolm_profile_enabled(void);
/* Accumulated device nanoseconds and call count of one stage
 * (profile::Stage order: embed = 0 ... other = 16); -1 for a bad index. */
int brolm_profile_stage(int stage, uint64_t* ns, uint64_t* calls);

/* qwen::Tokenizer (include/brolm/qwen_tokenizer.h; reference
 * include/brolm/qwen_tokenizer.h:41-151).  A handle from one of the three
 * loaders; NULL on failure (brolm_last_error).  `extra_specials` is a
 * '\n'-separated list of extra special-token names or NULL. */
typedef struct brolm_tokenizer brolm_tokenizer;
brolm_tokenizer* brolm_tokenizer_load(const char* vocab_json, const char* merges_txt, const char* extra_specials);
brolm_tokenizer* brolm_tokenizer_from_gguf(const char* gguf_path, const char* extra_specials);
brolm_tokenizer* brolm_tokenizer_from_json(const char* tokenizer_json, const char* extra_specials);
void brolm_tokenizer_free(brolm_tokenizer* t);
/* encode: writes up to cap ids, returns the total count (may exceed cap) or -1. */
int brolm_tokenizer_encode(const brolm_tokenizer* t, const char* text, int64_t len, int add_special, int32_t* ids,
                           int cap);
/* decode: writes up to cap bytes (not NUL-terminated), returns the total byte
 * count (may exceed cap) or -1. */
int64_t brolm_tokenizer_decode(const brolm_tokenizer* t, const int32_t* ids, int n, char* out, int64_t cap);
/* apply_chat_template over n (role, content) pairs; same return convention. */
int64_t brolm_tokenizer_chat(const brolm_tokenizer* t, const char* const* roles, const char* const* contents, int n,
                             int add_generation_prompt, char* out, int64_t cap);
int brolm_tokenizer_register_special(brolm_tokenizer* t, const char* token, int32_t id);
/* info[6] = {vocab_count, merge_count, eos_id, im_start_id, im_end_id, endoftext_id}. */
int brolm_tokenizer_info(const brolm_tokenizer* t, int64_t* info);
/* qwen::generate_text (reference src/qwen_generate.cpp:19-25): encode(prompt),
 * generate with eos = tok.eos_id(), decode the new ids; same return
 * convention as brolm_tokenizer_decode. */
int64_t brolm_qwen3_generate_text(brolm_qwen3* m, const brolm_tokenizer* t, const char* prompt, int max_new,
                                  int stop_on_eos, float temperature, int top_k, float top_p, uint64_t seed,
                                  char* out, int64_t cap);

#ifdef __cplusplus
}
#endif
#endif
