/*
 * brolm_hip.h — C ABI of the MI355X (gfx950) kernel library libbrolm_hip.so.
 *
 * This is the thin layer between the C++20 host (the brotensor-shaped op
 * surface in include/brotensor/ops.h and brolm's DenseDecoder) and the
 * hand-written HIP kernels.  Plain pointers and sizes only; no C++ types.
 *
 * Contract for every entry point:
 *   - Pointers are device pointers (hipMalloc'd or torch-owned) unless stated.
 *   - `stream` is a hipStream_t passed as void* (NULL = the null stream).
 *   - Nothing here allocates device memory; scratch is passed in by the
 *     caller, sized by the matching *_workspace_bytes query (except
 *     bx_argmax_f16_noalloc, whose scratch is a fixed array of the library).
 *     Calls on different streams never share scratch unless the caller
 *     hands them the same workspace.
 *   - Return 0 on success or a negative BX_E* code; bx_last_error() gives a
 *     thread-local message.  Shapes are validated on the host before any
 *     launch, so an invalid shape is an error return, never a device fault.
 *   - FP16 values travel as uint16_t bit patterns (IEEE binary16).
 *
 * Quantized weights ("carriers") live on the device in a repacked layout that
 * is a byte permutation of the GGUF blocks (same byte count; see
 * bx_repack_gguf_rows).  The reference interface each entry point replaces is
 * cited beside it (paths relative to wlejon/brolm; the ops themselves live in
 * the absent sibling brotensor, so the citation is brolm's call site).
 */
#ifndef BROLM_HIP_H
#define BROLM_HIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define BX_OK 0
#define BX_EINVAL (-1)     /* bad argument or shape */
#define BX_ELAUNCH (-2)    /* HIP runtime error */
#define BX_EUNSUPPORTED (-3)

/* ggml tensor type ids accepted by the carrier entry points. */
#define BX_TYPE_F32 0
#define BX_TYPE_F16 1
#define BX_TYPE_Q8_0 8
#define BX_TYPE_Q4_K 12
#define BX_TYPE_Q6_K 14

const char* bx_last_error(void);
int bx_abi_version(void);
/* 1 if a gfx950 device is present and the code objects load. */
int bx_device_ok(void);
/* 1 if a rocprofiler-sdk tool (rocprofv3) is loaded into this process.  No
 * counterpart in the reference.  Under such a tool, bx_persist_step launches
 * its grid without the cooperative API and the host decode session steps
 * eagerly instead of through a hipGraph: with those two launch forms, the
 * profiler's exit path has ended the process with a segmentation fault. */
int bx_profiler_attached(void);

/* ---------------------------------------------------------------- carriers */

/* Repack `rows` GGUF rows of `cols` elements (src: device copy of the GGUF
 * bytes, row-major) into the device carrier layout at dst (same byte count).
 * Replaces the layout handed over by gguf::upload_raw
 * (include/brolm/detail/weights.h:294-305, :324). */
int bx_repack_gguf_rows(int type, const void* src, void* dst, int64_t rows, int64_t cols, void* stream);
/* Inverse of bx_repack_gguf_rows (carrier -> GGUF bytes). */
int bx_unpack_carrier_rows(int type, const void* src, void* dst, int64_t rows, int64_t cols, void* stream);
/* Carrier byte count for (rows, cols) of `type`; -1 if cols is ragged. */
int64_t bx_carrier_bytes(int type, int64_t rows, int64_t cols);

/* K6: dequant_{q8_0,q4k,q6k}_to_fp16 (weights.h:325-339). FP32 values are
 * d*sc*q - dmin*m exactly as the GGUF formula, then RNE to binary16 with
 * subnormals kept. */
int bx_dequant_to_f16(int type, const void* carrier, uint16_t* dst, int64_t rows, int64_t cols, void* stream);
/* Unpack-only debug entry: the same values before the FP16 rounding. */
int bx_dequant_to_f32(int type, const void* carrier, float* dst, int64_t rows, int64_t cols, void* stream);

/* ------------------------------------------------------------------ linear */

/* Workspace of the linear entry points below (no counterpart in the
 * reference: brotensor's ops keep their scratch to themselves).  Decode
 * batches of 3..16 rows over layer-sized matrices split K across
 * workgroups; their partial sums and per-tile-group counters live in `ws`
 * (bx_linear_workspace_bytes() bytes: 32 KB of counters, 64 MB of FP32
 * partials), which the caller allocates and clears once with
 * bx_linear_workspace_init before its first use.  Every launch leaves the
 * counters at zero again, and each counter word carries its launch's tag,
 * so a launch that did not complete cannot make a later one sum early or
 * never.  Launches that may run at the same time (other streams, other
 * threads) take distinct workspaces.  ws = NULL (ws_bytes 0) is accepted: those shapes then take the
 * single-pass launch, and the forms that exist only as split launches (the
 * _norm and _ss forms, group2) return BX_EINVAL. */
size_t bx_linear_workspace_bytes(void);
int bx_linear_workspace_init(void* ws, size_t ws_bytes, void* stream);

/* K1-K4: linear_forward_batched_{q4k,q6k,q8_0,}_fp16(W, bias, X, Y)
 * (include/brolm/detail/compute.h:54-86).  Y[M,N] = X[M,K] . W[N,K]^T (+bias[N]).
 * X, Y, bias FP16; FP32 accumulation.  W is a carrier of `wtype` or dense FP16
 * (wtype BX_TYPE_F16).  M <= 16 runs the GEMV kernels, larger M the prefill
 * GEMM.  ws / ws_bytes: the linear workspace above. */
int bx_linear_f16(int wtype, const void* W, const uint16_t* bias, const uint16_t* X, uint16_t* Y,
                  int M, int N, int K, void* ws, size_t ws_bytes, void* stream);

/* Fused prefill forms of the linears of src/detail/dense_decoder.cpp:526-681
 * (the op sequence linear / silu / mul / add_inplace, with the same
 * roundings).  bx_linear_tiles_ok is 1 when (M, K) qualify: M >= 128 with K a
 * multiple of 64 (the MFMA tile GEMM) or 3 <= M <= 16 with K a multiple of
 * 256 (the MFMA GEMV of decode batches); else 0 and the caller runs the
 * unfused ops.
 * bx_linear_group_f16: n (1..3) weights of one type sharing X (q / k / v
 *   projections), Y[i] (M, N[i]) FP16, one launch.
 * bx_linear_residual_f16: H (M, N) FP32 += f16(X W^T) (o / down projection
 *   and the residual add).
 * bx_linear_swiglu_f16: Y (M, F) = f16(f16(silu(f16(X Wg^T))) * f16(X Wu^T))
 *   (gate / up projections, silu, mul). */
int bx_linear_tiles_ok(int M, int K);
int bx_linear_group_f16(int wtype, int n, const void* const* W, uint16_t* const* Y, const int* N, const uint16_t* X,
                        int M, int K, void* ws, size_t ws_bytes, void* stream);
int bx_linear_residual_f16(int wtype, const void* W, const uint16_t* X, float* H, int M, int N, int K, void* ws,
                           size_t ws_bytes, void* stream);
int bx_linear_swiglu_f16(int wtype, const void* Wg, const void* Wu, const uint16_t* X, uint16_t* Y, int M, int F,
                         int K, void* ws, size_t ws_bytes, void* stream);
/* Decode batches (3 <= M <= 16, K % 256 == 0) with the residual RMSNorm
 * (rms_norm_forward, dense_decoder.cpp:559, :540-550) carried between
 * launches instead of run on its own: bx_linear_residual_ss_f16 is
 * bx_linear_residual_f16 that also writes, per 64 columns of the updated H,
 * each row's sum of squares (ss_out: bx_linear_ss_floats(N) floats); the
 * group / SwiGLU forms then take X = RMSNorm(H; gamma, eps) with the row sums
 * of those partials (ss_in from the launch that last updated H, K = its N).
 * The norm's sum of squares is added in another order than bx_rms_norm's.
 * All three return BX_EUNSUPPORTED, launching nothing, for matrices outside
 * the split batched GEMV (the caller then runs bx_rms_norm and the plain
 * forms). */
size_t bx_linear_ss_floats(int N);
int bx_linear_residual_ss_f16(int wtype, const void* W, const uint16_t* X, float* H, float* ss_out, int M, int N,
                              int K, void* ws, size_t ws_bytes, void* stream);
int bx_linear_group_norm_f16(int wtype, int n, const void* const* W, uint16_t* const* Y, const int* N, const float* H,
                             const uint16_t* gamma, float eps, const float* ss_in, int M, int K, void* ws,
                             size_t ws_bytes, void* stream);
int bx_linear_swiglu_norm_f16(int wtype, const void* Wg, const void* Wu, const float* H, const uint16_t* gamma,
                              float eps, const float* ss_in, uint16_t* Y, int M, int F, int K, void* ws,
                              size_t ws_bytes, void* stream);
/* The q / k / v projections in one decode-batch launch when v's weight type
 * differs from q / k's (the per-weight dispatch of compute.h:54-86 over
 * llama.cpp's Q4_K_M mix): members [0, n1) of type wtype, [n1, n) of type
 * wtype2, Q4_K then Q6_K only; each member's output has exactly the bits of
 * its own launch.  The _norm form takes X = RMSNorm(H) with the row sums of
 * bx_linear_residual_ss_f16, as bx_linear_group_norm_f16.  BX_EUNSUPPORTED,
 * nothing launched, for other types or shapes outside the split GEMV. */
int bx_linear_group2_f16(int wtype, int wtype2, int n, int n1, const void* const* W, uint16_t* const* Y, const int* N,
                         const uint16_t* X, int M, int K, void* ws, size_t ws_bytes, void* stream);
int bx_linear_group2_norm_f16(int wtype, int wtype2, int n, int n1, const void* const* W, uint16_t* const* Y,
                              const int* N, const float* H, const uint16_t* gamma, float eps, const float* ss_in, int M,
                              int K, void* ws, size_t ws_bytes, void* stream);

/* ------------------------------------------------------------- elementwise */

/* K7: embedding_lookup_forward(W, idx_dev, L, out) (dense_decoder.cpp:259-261).
 * W FP16 (V, H); ids must be in [0, V) (checked by the caller on the host). */
int bx_embedding_f16(const uint16_t* W, int V, int H, const int32_t* ids, int L, uint16_t* out, void* stream);
/* Same gather into an FP32 residual stream. */
int bx_embedding_f32(const uint16_t* W, int V, int H, const int32_t* ids, int L, float* out, void* stream);

/* K8/K9: rms_norm_forward(X, gamma, eps, Y) (dense_decoder.cpp:559, :540-550).
 * x_is_f32 selects an FP32 input (the residual stream); Y is FP16. */
int bx_rms_norm(const void* X, int x_is_f32, const uint16_t* gamma, float eps, uint16_t* Y, int rows, int cols,
                void* stream);

/* K10: rope_forward(X, hd, n_heads, seq_offset, theta, Y) (dense_decoder.cpp:587-590),
 * in place allowed (X == Y).  Row r rotates at position seq_offset + r using
 * the FP32 cos/sin table (cap, hd/2) built by bx_rope_table on the host side. */
int bx_rope_f16(const uint16_t* X, uint16_t* Y, int rows, int hd, int n_heads, int seq_offset,
                const float* cos_tab, const float* sin_tab, int tab_rows, void* stream);
/* Host helper: cos/sin table of pos*theta^(-2i/hd), computed in double. */
void bx_rope_table_host(float* cos_out, float* sin_out, int rows, int hd, float theta);

/* K12: kv_cache_append(k, v, cur_len, Kc, Vc) (dense_decoder.cpp:597-598). */
int bx_kv_append_f16(const uint16_t* k, const uint16_t* v, int L, int cols, int cur_len, uint16_t* Kc,
                     uint16_t* Vc, int cap, void* stream);

/* K14: flash_attention_decode(q, Kc, Vc, valid_len, n_q, n_kv, out[, softcap, window])
 * (dense_decoder.cpp:606-607; Gemma form src/gemma2.cpp:365-367).
 * q (L, n_q*hd) FP16, caches (cap, n_kv*hd) FP16, out (L, n_q*hd) FP16.
 * Row r attends keys [max(0, p-window+1), p] with p = valid_len - L + r.
 * workspace: bx_attention_workspace_bytes(L, n_q, hd, valid_len) bytes. */
size_t bx_attention_workspace_bytes(int L, int n_q, int hd, int valid_len);
int bx_attention_decode_f16(const uint16_t* q, const uint16_t* Kc, const uint16_t* Vc, int L, int valid_len,
                            int n_q, int n_kv, int hd, float softcap, int window, uint16_t* out,
                            void* workspace, void* stream);

/* K14b: flash_attention_gqa_forward(q, k, v, nullptr, n_q, n_kv, causal, out)
 * (dense_decoder.cpp:737-745, the encoder's attention): q (L, n_q*hd), K / V
 * (n_keys, n_kv*hd) FP16, out (L, n_q*hd) FP16.  causal = 0: every row
 * attends all n_keys keys; causal = 1: row r attends keys [0, n_keys - L + r].
 * workspace: bx_attention_workspace_bytes(L, n_q, hd, n_keys) bytes. */
int bx_attention_gqa_f16(const uint16_t* q, const uint16_t* K, const uint16_t* V, int L, int n_keys, int n_q,
                         int n_kv, int hd, int causal, uint16_t* out, void* workspace, void* stream);

/* Batched decode of independent sequences (an extension of the one-sequence
 * cache of dense_decoder.cpp:196-227, 585-607): row r of q (rows, n_q*hd) is
 * the newest token of its own sequence, whose rlen = lens_dev[r] keys sit in
 * cache rows base_rows_dev[r] .. + rlen - 1 (the last one its own); max_len >=
 * every rlen sizes the split.  workspace: bx_attention_workspace_bytes(rows,
 * n_q, hd, max_len) bytes. */
int bx_attention_varlen_f16(const uint16_t* q, const uint16_t* Kc, const uint16_t* Vc, int rows,
                            const int32_t* lens_dev, const int64_t* base_rows_dev, int max_len, int n_q, int n_kv,
                            int hd, uint16_t* out, void* workspace, void* stream);
/* rope_forward with a position per row (pos_dev, device int32 < tab_rows). */
int bx_rope_rows_f16(const uint16_t* X, uint16_t* Y, int rows, int hd, int n_heads, const int32_t* pos_dev,
                     const float* cos_tab, const float* sin_tab, int tab_rows, void* stream);
/* kv_cache_append of row r to cache row dst_rows_dev[r] (< cache_rows). */
int bx_kv_append_rows_f16(const uint16_t* k, const uint16_t* v, int rows, int cols, const int64_t* dst_rows_dev,
                          uint16_t* Kc, uint16_t* Vc, int64_t cache_rows, void* stream);
/* Attention of one batched step with its per-head stage in one launch: for row
 * r (its sequence's newest token at position lens_dev[r] - 1, keys in cache
 * rows base_rows_dev[r] .. + lens_dev[r] - 1): the q / k head RMSNorm and RoPE
 * of bx_qk_rope_kv_rows_f16 (same bits), the new k / v rows written to the
 * cache, split attention over the row's keys and the merge of the splits ->
 * out (rows, n_q*hd) FP16.  q, k, v: the raw projections.  workspace:
 * bx_batch_attention_workspace_bytes(rows, ...) bytes, zeroed once before its
 * first use (the kernel leaves its counters at zero; a counter left by a
 * launch that did not complete carries that launch's tag and is ignored);
 * calls sharing one workspace must not overlap.  hd: 64, 128 or 256; n_q / n_kv <= 8. */
size_t bx_batch_attention_workspace_bytes(int rows, int n_q, int n_kv, int hd, int max_len);
int bx_batch_attention_f16(const uint16_t* q, const uint16_t* k, const uint16_t* v, int rows, int hd, int n_q,
                           int n_kv, const uint16_t* q_gain, const uint16_t* k_gain, float eps, const int32_t* lens_dev,
                           const int64_t* base_rows_dev, int max_len, const float* cos_tab, const float* sin_tab,
                           int tab_rows, uint16_t* Kc, uint16_t* Vc, int64_t cache_rows, uint16_t* out,
                           void* workspace, void* stream);
/* The per-head ops of one batched step in one launch (dense_decoder.cpp:
 * 575-607 per row): q / k head RMSNorm with q_gain / k_gain (both null: none),
 * RoPE at pos_dev[r], roped q heads to q_out (may be q), roped k rows and the
 * v rows to cache row dst_rows_dev[r]; bit-identical to rms_norm, rope_rows and
 * kv_append_rows in sequence.  hd: 64, 128 or 256. */
int bx_qk_rope_kv_rows_f16(const uint16_t* q, const uint16_t* k, const uint16_t* v, int rows, int hd, int n_q,
                           int n_kv, const uint16_t* q_gain, const uint16_t* k_gain, float eps, const int32_t* pos_dev,
                           const float* cos_tab, const float* sin_tab, int tab_rows, const int64_t* dst_rows_dev,
                           uint16_t* Kc, uint16_t* Vc, int64_t cache_rows, uint16_t* q_out, void* stream);

/* K15: flash_attention_decode_masked(q, Kc, Vc, mask, n_q, n_kv, out)
 * (dense_decoder.cpp:476-478): one query row attends the keys j < n_keys
 * whose FP32 mask[j] (device) is non-zero.  workspace as above with L = 1,
 * valid_len = n_keys. */
int bx_attention_masked_f16(const uint16_t* q, const uint16_t* Kc, const uint16_t* Vc, const float* mask, int n_keys,
                            int n_q, int n_kv, int hd, uint16_t* out, void* workspace, void* stream);

/* K13: scatter_rows(src, idx_row, dst) (dense_decoder.cpp:473-474):
 * dst row *idx_dev (device int32, must be < dst_rows) = src (one row of
 * `row_bytes` bytes). */
int bx_scatter_row(const void* src, const int32_t* idx_dev, void* dst, int64_t row_bytes, int dst_rows,
                   void* stream);

/* K16: silu_forward(g, g) + mul_inplace(g, u) (dense_decoder.cpp:635-636). */
int bx_silu_mul_f16(uint16_t* g, const uint16_t* u, int64_t n, void* stream);
int bx_silu_f16(const uint16_t* x, uint16_t* y, int64_t n, void* stream);
int bx_mul_f16(uint16_t* a, const uint16_t* b, int64_t n, void* stream);
/* K17: add_inplace(h, proj) (dense_decoder.cpp:616, :645); h FP32 or FP16. */
int bx_add_inplace(void* h, int h_is_f32, const uint16_t* x, int64_t n, void* stream);
/* sample_token (src/detail/generate.cpp:68-142) for temperature > 0 on the
 * device: softmax of logits / temperature, top-k then top-p truncation in
 * descending probability, and the token where the running kept mass first
 * exceeds u * kept (u: the host's uniform_real_distribution<double>(0, 1)
 * draw).  One FP16 logits row (device); *out (device int32).  Equal
 * probabilities resolve to the lowest index.  workspace (device, 256-byte
 * aligned, about 12 bytes per id): bx_sample_workspace_bytes(vocab); vocab up
 * to 4,194,304.  Four stream-ordered launches; calls that share a workspace
 * must be ordered on one stream. */
size_t bx_sample_workspace_bytes(int vocab);
/* bx_sample_f16 inside a device-side decode loop (no reference counterpart:
 * the reference samples on the host, generate.cpp:68-142): the draw is
 * u_dev[*count - 1] (device, each in [0, 1)), and the id is written to *tok and
 * hist[*count - 1], the token and history slots the fused decode step
 * (bx_decode_advance / bx_persist_step) has just filled with its argmax. */
int bx_sample_feed_f16(const uint16_t* logits, int vocab, float temperature, int top_k, float top_p,
                       const double* u_dev, int32_t* tok, int32_t* hist, const int32_t* count, void* workspace,
                       void* stream);
int bx_sample_f16(const uint16_t* logits, int vocab, float temperature, int top_k, float top_p, double u,
                  int32_t* out, void* workspace, void* stream);
/* masked_mean_pool_forward(x, mask, out) (src/llm2vec.cpp:139-153): out[c] =
 * sum_r mask[r] x[r, c] / sum_r mask[r] over the L rows of x (L, cols) FP16,
 * FP32 sums, FP16 out (cols); mask (device FP32, L) or NULL for all rows; an
 * all-zero mask gives zeros. */
int bx_masked_mean_pool_f16(const uint16_t* x, const float* mask, int L, int cols, uint16_t* out, void* stream);
/* FP32 -> FP16 copy (RNE). */
int bx_f32_to_f16(const float* x, uint16_t* y, int64_t n, void* stream);

/* ------------------------------------------------------------ decode step */

/* Fused single-token decode kernels (the captured step of
 * dense_decoder.cpp:335-524, restructured).  Per-step scalars (token id,
 * position) are read from device memory so the step can be graph-captured
 * once and replayed.  All activations are in `ws` (bx_decode_ws_bytes). */
typedef struct {
    int hidden, intermediate, n_q, n_kv, head_dim, vocab, cap;
    float eps;
    int qkv_type_q, qkv_type_k, qkv_type_v, o_type, gate_type, up_type, down_type, lm_type;
    /* 1: no per-head q/k RMSNorm (Mistral / Llama, DenseDecoderConfig
     * use_qk_norm = false): q and k are rounded to FP16 and rotated as they
     * come from the projections; the layers' q_norm / k_norm are not read.
     * 0 (a zero-initialized struct): Qwen3's QK-norm. */
    int no_qk_norm;
    /* A second type that some layers use for attn_v / ffn_down (llama.cpp
     * Q4_K_M raises them to Q6_K on some layers only), or 0 when every
     * layer has qkv_type_v / down_type.  Each layer's own types travel in
     * its bx_decode_layer. */
    int v_alt_type, down_alt_type;
} bx_decode_dims;

typedef struct {
    const void *in_ln, *q_norm, *k_norm, *post_ln;  /* FP16 gammas (q/k norms permuted) */
    const void *Wq, *Wk, *Wv, *Wo, *Wg, *Wu, *Wd;   /* carriers or FP16 */
    void *Kc, *Vc;                                  /* FP16 (cap, n_kv*hd) */
    /* BX_TYPE_* of this layer's matrices.  Layers may differ: a llama.cpp
     * Q4_K_M file stores attn_v / ffn_down as Q6_K in some layers only (the
     * reference dispatches per weight on its dtype, compute.h:54-86).  The
     * bx_decode_dims types describe layer 0 and size the workspaces. */
    int type_q, type_k, type_v, type_o, type_gate, type_up, type_down, type_pad;
} bx_decode_layer;

size_t bx_decode_ws_bytes(const bx_decode_dims* d);
/* Embedding row of *tok_dev into the FP32 residual (ws). */
int bx_decode_embed(const bx_decode_dims* d, const uint16_t* embed, const int32_t* tok_dev, void* ws, void* stream);
/* One layer at position *pos_dev (cos/sin table rows pos). */
int bx_decode_layer_run(const bx_decode_dims* d, const bx_decode_layer* L, const int32_t* pos_dev,
                        const float* cos_tab, const float* sin_tab, void* ws, void* stream);
/* Final norm + lm_head -> logits (FP16, vocab). */
int bx_decode_head(const bx_decode_dims* d, const uint16_t* final_norm, const void* lm_head, uint16_t* logits,
                   void* ws, void* stream);

/* Step feedback for device-side greedy decoding: *tok = *next, *pos += 1,
 * hist[*count] = *next, *count += 1 (hist may be NULL; count must then be
 * NULL too; hist must hold at least as many ids as steps between resets). */
int bx_decode_advance(int32_t* tok_dev, int32_t* pos_dev, const int32_t* next_dev, int32_t* hist, int32_t* count,
                      void* stream);

/* Persistent decode step: the same single-token step (embedding, all layers,
 * final norm, lm_head, greedy argmax, the feedback of bx_decode_advance) as
 * ONE launch with one workgroup per CU (a plain launch after the cooperative
 * launch's occupancy check; a grid that is not all resident aborts); stages hand vectors to
 * each other through tagged words in `ws` instead of kernel boundaries
 * (replaces the captured step of dense_decoder.cpp:335-524 as a whole).
 * bx_persist_ws_bytes returns 0 (with a message) for shapes/format mixes it
 * does not cover.  bx_persist_ws_init (stream-ordered, a fill kernel: no
 * memset node) must run on `ws` before the first step, after an aborted step,
 * and before each cycle of epochs: `epoch` grows by one per launch on that ws
 * through 1..63, then the caller re-initializes ws and restarts at 1 (the
 * hand-off words carry 16-bit tags).  `layers_dev` is a device array of
 * n_layers (<= 126) bx_decode_layer.  scal = {tok, pos, next, count,
 * hist[...]} as for bx_decode_advance.  bx_persist_status reads the abort
 * flag after the launches completed (caller synchronizes): 0 ok, 1 aborted
 * (`site` names the wait that timed out). */
size_t bx_persist_ws_bytes(const bx_decode_dims* d);
int bx_persist_ws_init(const bx_decode_dims* d, void* ws, void* stream);
int bx_persist_step(const bx_decode_dims* d, int n_layers, const bx_decode_layer* layers_dev,
                    const uint16_t* embed, const uint16_t* final_norm, const void* lm_head, const float* cos_tab,
                    const float* sin_tab, int32_t* scal, uint16_t* logits, void* ws, uint32_t epoch, void* stream);
int bx_persist_status(const void* ws, uint32_t* site);
/* Debug timing (no counterpart in the reference): while buf_dev is non-null,
 * every later bx_persist_step writes the device wall clock (wall_clock64, the
 * constant-rate counter) at each stage boundary of each workgroup into
 * buf_dev[wg * 1024 + slot] (wg = the dispatch's workgroup index).  The
 * XCD-partitioned kernel (the default where it has an instantiation): slot 0
 * start; 1 + 9 l + {0 A normed, 1 A words out, 2 B done, 3 C records
 * combined, 4 C partials out, 5 D normed, 6 D words out, 7 E input, 8 E done};
 * 1 + 9 L + {0 head input normed, 1 logits written, 2 step done (logical
 * workgroup 0)}; for layer 14 the sub-stages at 600 + k; slot 1000 the
 * workgroup's logical id (XCD + 8 rank).  The first persistent kernel: slot 0
 * start, 1 + 10 l + {0 A input, 1 A done, 2 B done, 3 C input, 4 C done,
 * 5 D input, 6 D done, 7 E input, 8 E done}, 1 + 10 L + {0 head input, 1 head
 * rows done, 2 step done (workgroup 0)}; for layer 14 also the attention
 * sub-stages (900-907) and the gate/up sub-stages (910 activation cached,
 * 911 gate dots, 912 up dots, 913 all waves done).  slots_per_wg must be >=
 * 1024.  NULL switches it off. */
int bx_persist_trace(uint64_t* buf_dev, int slots_per_wg);

/* Device greedy argmax over FP16 logits, lowest index wins ties
 * (src/detail/generate.cpp:38-48).  Writes the id to *out (device int32).
 * workspace: bx_argmax_workspace_bytes(n). */
size_t bx_argmax_workspace_bytes(int64_t n);
int bx_argmax_f16(const uint16_t* logits, int64_t n, int32_t* out, void* workspace, void* stream);
/* bx_argmax_f16 without a workspace argument and without any allocation: the
 * partials live in a fixed 2 KB device array of the library (one copy per
 * GPU, held until the process ends).  No counterpart in the reference; it is
 * for callers that cannot allocate device memory (code under HIP graph
 * capture, serving loops with a fixed memory budget).  Same result and error
 * behaviour as bx_argmax_f16; n up to 2^31 - 1.  Calls that overlap on one GPU
 * (different streams, or different threads) share the array and race:
 * serialize them. */
int bx_argmax_f16_noalloc(const uint16_t* logits, int64_t n, int32_t* out, void* stream);

#ifdef __cplusplus
}
#endif
#endif
