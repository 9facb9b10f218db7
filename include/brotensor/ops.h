#pragma once

// brotensor op surface used by brolm's Qwen3 decode path, implemented on
// libbrolm_hip (C ABI in include/brolm_hip.h).  Signatures follow brolm's call
// sites (src/detail/dense_decoder.cpp, include/brolm/detail/compute.h:54-86,
// include/brolm/detail/weights.h:325-339).
//
// Conventions (as the reference relies on them):
//   - inputs are const&, outputs are resized by the op; an unallocated output
//     is pinned to the op's device first (include/brolm/detail/device.h:3-9);
//   - every op is ordered on brotensor::stream(); sync_all() is the barrier;
//   - contract violations (dtype, shape, device) throw std::runtime_error.

#include <cstdint>

#include "brotensor/tensor.h"

namespace brotensor {

// K1-K4: Y (M, N) = X (M, K) . W (N, K)^T (+ bias), FP16 in/out, FP32 accumulate.
void linear_forward_batched_fp16(const Tensor& W, const Tensor* bias, const Tensor& X, Tensor& Y);
void linear_forward_batched_q4k_fp16(const Tensor& W, const Tensor* bias, const Tensor& X, Tensor& Y);
void linear_forward_batched_q6k_fp16(const Tensor& W, const Tensor* bias, const Tensor& X, Tensor& Y);
void linear_forward_batched_q8_0_fp16(const Tensor& W, const Tensor* bias, const Tensor& X, Tensor& Y);

// Fused prefill linears (MFMA tile path only).  Each returns false, having
// done nothing, when the shapes or dtypes do not qualify (fewer than 128 rows,
// K not a multiple of 64, mixed weight dtypes, a dtype without a quant
// kernel): the caller then runs the unfused ops, which give the same values.
//   linear_group_forward_batched:    Y[i] = X . W[i]^T, 1..3 weights of one dtype
//   linear_residual_forward_batched: H (FP32) += fp16(X . W^T)
//   linear_swiglu_forward_batched:   Y = fp16(fp16(silu(fp16(X . Wg^T))) * fp16(X . Wu^T))
bool linear_group_forward_batched(const Tensor* const* W, Tensor* const* Y, int n, const Tensor& X);
bool linear_residual_forward_batched(const Tensor& W, const Tensor& X, Tensor& H);
bool linear_swiglu_forward_batched(const Tensor& Wg, const Tensor& Wu, const Tensor& X, Tensor& Y);

// K6: quant carrier -> FP16 tensor of the same (rows, cols).
void dequant_q8_0_to_fp16(const Tensor& raw, Tensor& dst);
void dequant_q4k_to_fp16(const Tensor& raw, Tensor& dst);
void dequant_q6k_to_fp16(const Tensor& raw, Tensor& dst);
// Unpack-only debug entry (FP32 values before the FP16 rounding).
void dequant_to_fp32(const Tensor& raw, Tensor& dst);

// K7: out (L, H) = W[idx_dev[r]] (W FP16; ids must be valid, checked by the caller).
void embedding_lookup_forward(const Tensor& W, const std::int32_t* idx_dev, int L, Tensor& out);

// K8/K9: Y = X * rsqrt(mean(X^2) + eps) * gamma per row; X FP16 or FP32, Y FP16.
void rms_norm_forward(const Tensor& X, const Tensor& gamma, float eps, Tensor& Y);

// K10: interleaved-pair RoPE of n_heads heads of width hd per row, row r at
// position seq_offset + r; X == Y allowed.
void rope_forward(const Tensor& X, int hd, int n_heads, int seq_offset, float theta, Tensor& Y);
// K11: same rotation with a staged (1, hd/2) FP32 cos/sin row (single-row X).
void rope_apply(const Tensor& X, const Tensor& cos, const Tensor& sin, int hd, int n_heads, Tensor& Y);

// K12: Kc[cur_len + r] = k[r], Vc[cur_len + r] = v[r].
void kv_cache_append(const Tensor& k, const Tensor& v, int cur_len, Tensor& Kc, Tensor& Vc);
// K13: dst[idx_row[0]] = src (one row, device-resident row index).
void scatter_rows(const Tensor& src, const Tensor& idx_row, Tensor& dst);

// K14: causal GQA attention of the L rows of q against cache rows
// [0, valid_len) (row r sees keys <= valid_len - L + r); 1/sqrt(hd) inside.
// softcap > 0 applies s -> softcap * tanh(s / softcap); window > 0 limits each
// row to its last `window` keys (src/gemma2.cpp:365-367).
void flash_attention_decode(const Tensor& q, const Tensor& Kc, const Tensor& Vc, int valid_len, int n_q, int n_kv,
                            Tensor& out, float softcap = 0.0f, int window = 0);
// K16: GQA attention of the L rows of q over the n rows of k / v (no cache);
// causal = false lets every row see every key (the encoder's form).
void flash_attention_gqa_forward(const Tensor& q, const Tensor& k, const Tensor& v, int n_q, int n_kv, bool causal,
                                 Tensor& out);
// Mean of the rows of x (L, cols) FP16 weighted by the device FP32 mask (L,)
// or all rows when mask is null -> out (cols, 1) FP16.
void masked_mean_pool_forward(const Tensor& x, const float* mask, Tensor& out);
// K15: single-row attention over the keys whose FP32 mask entry is non-zero
// (mask has Kc.rows entries, device memory).
void flash_attention_decode_masked(const Tensor& q, const Tensor& Kc, const Tensor& Vc, const float* mask, int n_q,
                                   int n_kv, Tensor& out);

// K16/K17
void silu_forward(const Tensor& x, Tensor& y);      // aliasing allowed
void mul_inplace(Tensor& a, const Tensor& b);
void add_inplace(Tensor& a, const Tensor& b);       // a FP16 or FP32, b FP16

// K18: element copies (element size of the tensors' dtype).
void copy_d2d(const Tensor& src, std::int64_t src_off, Tensor& dst, std::int64_t dst_off, std::int64_t n);
void copy_d2d_strided(const Tensor& src, std::int64_t src_off, std::int64_t src_stride, Tensor& dst,
                      std::int64_t dst_off, std::int64_t dst_stride, std::int64_t elem, std::int64_t n);

// Device greedy argmax of an FP16 row vector into a (1,1) INT32 tensor.
void argmax_forward(const Tensor& logits_row, Tensor& out_idx);

}  // namespace brotensor
