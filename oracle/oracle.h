/*
 * oracle.h — CPU restatement of brolm's quantized Qwen3 decode path.
 *
 * TEST INFRASTRUCTURE ONLY.  This library is the checker the parity tests,
 * __graft_entry__.smoke() and bench.py's cpu_baseline leg compare the HIP path
 * against.  Nothing in the product (brolm_amd/, include/) may link, load or
 * call it.
 *
 * What it restates (reference = wlejon/brolm, paths relative to its root):
 *   - GGUF block unpacking Q8_0 / Q4_K / Q6_K.  brolm calls
 *     brotensor::dequant_{q8_0,q4k,q6k}_to_fp16 (include/brolm/detail/weights.h:325-339);
 *     brotensor is an un-vendored, unpinned sibling (CMakeLists.txt:61-75), so
 *     the block layouts follow the published ggml k-quant formats
 *     (llama.cpp ggml-quants.c, block_q8_0 / block_q4_K / block_q6_K; layout
 *     unchanged since the k-quants were introduced in 2023).
 *   - The dense decoder op order of src/detail/dense_decoder.cpp:526-681 in
 *     FP32 on weights dequantized on load, the load rules of :121-192 (rope
 *     row permute weights.h:132-148, tie rule :180-191), cache bookkeeping
 *     :196-227, forward/forward_last :242-294.
 *   - Greedy argmax with lowest-index ties (src/detail/generate.cpp:38-48)
 *     and the generate loop (include/brolm/detail/generate.h:78-123).
 *   - Temperature / top-k / top-p sampling (src/detail/generate.cpp:68-142)
 *     given the uniform draw; pinned by exhaustive draws over tiny
 *     vocabularies against the kept set and renormalised probabilities the
 *     definition fixes (tests/test_sampling.py).
 *
 * Parity status per function (how each is pinned) is stated beside it.
 */
#ifndef BROLM_ORACLE_H
#define BROLM_ORACLE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ggml tensor type ids (GGUF spec). */
enum {
    OR_T_F32 = 0, OR_T_F16 = 1, OR_T_Q8_0 = 8, OR_T_Q4_K = 12, OR_T_Q6_K = 14, OR_T_BF16 = 30
};

/* ---- scalar conversions (IEEE-754 binary16 / bfloat16, RNE, subnormals kept) ---- */
float    or_f16_to_f32(uint16_t h);
uint16_t or_f32_to_f16(float f);
float    or_bf16_to_f32(uint16_t h);
uint16_t or_f32_to_bf16(float f);
void     or_f32_to_f16_array(const float* src, uint16_t* dst, int64_t n);
void     or_f16_to_f32_array(const uint16_t* src, float* dst, int64_t n);

/* ---- block formats ---- */
int64_t or_type_block_elems(int type);   /* 32 / 256, 1 for dense */
int64_t or_type_block_bytes(int type);   /* 34 / 144 / 210, elem bytes for dense */
int64_t or_row_bytes(int type, int64_t cols);
/* 6-bit scale/min unpack of a Q4_K super-block (ggml get_scale_min_k4). */
void or_get_scale_min_k4(int j, const uint8_t* scales12, uint8_t* sc, uint8_t* m);
/* Unpack n elements (multiple of the block size) into FP32. Returns 0 / -1. */
int or_dequant(int type, const void* src, int64_t n, float* dst);

/* ---- GGUF v3 reader (independent of the product's reader) ---- */
typedef struct or_gguf or_gguf;
or_gguf*    or_gguf_open(const char* path);                       /* NULL on error */
or_gguf*    or_gguf_open_memory(const void* data, size_t size);   /* borrows data */
void        or_gguf_close(or_gguf* g);
const char* or_gguf_error(void);
int64_t     or_gguf_n_tensors(const or_gguf* g);
int64_t     or_gguf_find_tensor(const or_gguf* g, const char* name); /* -1 if absent */
const char* or_gguf_tensor_name(const or_gguf* g, int64_t i);
int         or_gguf_tensor_type(const or_gguf* g, int64_t i);
int         or_gguf_tensor_ndims(const or_gguf* g, int64_t i);
int64_t     or_gguf_tensor_dim(const or_gguf* g, int64_t i, int d);
const void* or_gguf_tensor_data(const or_gguf* g, int64_t i);
int64_t     or_gguf_tensor_nbytes(const or_gguf* g, int64_t i);
/* metadata: returns 0 if found and of a numeric/int kind */
int         or_gguf_meta_int(const or_gguf* g, const char* key, int64_t* out);
int         or_gguf_meta_f64(const or_gguf* g, const char* key, double* out);
int         or_gguf_meta_str(const or_gguf* g, const char* key, const char** out);
int         or_gguf_meta_array_len(const or_gguf* g, const char* key, int64_t* out);

/* ---- FP32 ops (used by the decoder below, exported for unit tests) ---- */
void or_rms_norm(const float* x, const float* gamma, float eps, float* y, int rows, int cols);
/* interleaved-pair rotation, pairs (2i,2i+1), angle = (pos0+r)*theta^(-2i/hd) */
void or_rope(float* x, int rows, int hd, int n_heads, int pos0, float theta);
/* Y[M,N] = X[M,K] * W[N,K]^T, FP32, OpenMP over rows of W */
void or_linear(const float* W, const float* X, float* Y, int M, int N, int K);
/* causal GQA attention: q (L, n_q*hd); Kc/Vc (>= pos0+L, n_kv*hd); row r sees keys [0, pos0+r] */
void or_attention(const float* q, const float* Kc, const float* Vc, int L, int pos0,
                  int n_q, int n_kv, int hd, float* out);
float or_silu(float x);

/* ---- FP32 dense decoder on dequantized weights: Qwen3 (general.architecture
 * "qwen3", per-head QK-norm) or Mistral 3.1 text ("llama" / "mistral", no
 * QK-norm) ---- */
typedef struct or_model or_model;
typedef struct {
    int vocab_size, hidden_size, intermediate_size, num_hidden_layers;
    int num_attention_heads, num_key_value_heads, head_dim;
    float rms_norm_eps, rope_theta;
    int tie_word_embeddings, max_position_embeddings;
    int use_qk_norm;
} or_config;

or_model* or_model_load(const or_gguf* g);          /* NULL on error (or_gguf_error) */
void      or_model_free(or_model* m);
void      or_model_config(const or_model* m, or_config* out);
int       or_model_allocate_cache(or_model* m, int max_seq_len);
void      or_model_reset_cache(or_model* m);
int       or_model_truncate_cache(or_model* m, int len);
/* bench helper: K / V rows [0, len) filled with deterministic values, cache_len = len */
int       or_model_fill_cache(or_model* m, int len, uint64_t seed);
int       or_model_cache_len(const or_model* m);
/* logits: (L, V) or (1, V) when last_only; hidden (optional): (L, H) post-final-norm */
int       or_model_forward(or_model* m, const int32_t* ids, int L, int last_only,
                           float* logits, float* hidden);
/* bidirectional, cacheless pass (forward_encode): hidden (L, H) post-final-norm */
int       or_model_forward_encode(or_model* m, const int32_t* ids, int L, float* hidden);
/* dequantized FP32 weights after load-time permutes (for tests). which: see oracle.c */
const float* or_model_weight(const or_model* m, int layer, const char* which, int64_t* rows, int64_t* cols);

/* greedy argmax, lowest index wins ties; margin = top1 - top2 (optional) */
int or_argmax(const float* logits, int vocab, float* margin);
/* sample_token (src/detail/generate.cpp:68-142) given the uniform draw u in
 * [0, 1); equal probabilities in ascending index order; margin (optional):
 * the draw's distance to the chosen interval's nearer end / kept mass */
int or_sample_token(const float* logits, int vocab, float temperature, int top_k, float top_p, double u,
                    double* margin);
/* generate: prefill prompt, then decode; writes <= max_new ids; returns count.
 * margins (optional, max_new floats) receives the top-2 gap at each step. */
int or_generate_greedy(or_model* m, const int32_t* prompt, int n_prompt, int max_new,
                       int eos_id, int32_t* out, float* margins);

int or_num_threads(void);

#ifdef __cplusplus
}
#endif
#endif
