// brotensor op surface on libbrolm_hip (see include/brotensor/ops.h).
#include "brotensor/ops.h"

#include <hip/hip_runtime_api.h>

#include <mutex>
#include <stdexcept>
#include <string>
#include <vector>

#include "brolm_hip.h"
#include "brotensor/runtime.h"
#include "hip_util.h"

namespace brotensor {

namespace {

[[noreturn]] void contract(const std::string& op, const std::string& msg) {
    throw std::runtime_error("brotensor::" + op + ": " + msg);
}

void need_device(const Tensor& t, const char* op, const char* what) {
    if (t.device != Device::ROCm || t.data == nullptr)
        contract(op, std::string(what) + " must be an allocated ROCm tensor (this build has no CPU backend)");
}

void need_dtype(const Tensor& t, Dtype dt, const char* op, const char* what) {
    if (t.dtype != dt)
        contract(op, std::string(what) + " dtype " + dtype_name(t.dtype) + ", expected " + dtype_name(dt));
}

// Pin an unallocated output to the device, then size it (adopt_output).
void size_out(Tensor& t, int r, int c, Dtype dt) {
    if (t.data == nullptr) t.device = Device::ROCm;
    if (t.device != Device::ROCm) contract("output", "output tensor lives on the CPU");
    t.resize(r, c, dt);
}

// Scratch shared by every op call (attention split-K partials, argmax
// partials, the RoPE tables), grown on demand and released by
// brotensor::shutdown(), so none of it is left for exit handlers to free.
struct Scratch {
    std::mutex mu;
    void* attn_ws = nullptr;
    std::size_t attn_bytes = 0;
    void* argmax_ws = nullptr;
    std::size_t argmax_bytes = 0;
    void* wdeq = nullptr;          // FP16 copies of quantized weights for long prompts
    std::size_t wdeq_bytes = 0;
    float theta = 0.f;
    int hd = 0, rows = 0;
    float* cos_t = nullptr;
    float* sin_t = nullptr;
};

Scratch& scratch() {
    static Scratch* s = new Scratch();
    return *s;
}

void release_scratch() {
    Scratch& S = scratch();
    std::lock_guard<std::mutex> lk(S.mu);
    for (void* p : {S.attn_ws, S.argmax_ws, S.wdeq, static_cast<void*>(S.cos_t), static_cast<void*>(S.sin_t)})
        if (p) (void)hipFree(p);
    S.attn_ws = S.argmax_ws = S.wdeq = nullptr;
    S.cos_t = S.sin_t = nullptr;
    S.attn_bytes = S.argmax_bytes = S.wdeq_bytes = 0;
    S.rows = S.hd = 0;
}

void* grow(void*& p, std::size_t& have, std::size_t need) {
    if (need <= have && p) return p;
    if (p) {
        hipx::sync();
        (void)hipFree(p);
        p = nullptr;
    }
    std::size_t n = need < 4096 ? 4096 : need;
    on_shutdown(release_scratch);
    hipx::check(hipMalloc(&p, n), "hipMalloc scratch");
    have = n;
    return p;
}

// RoPE table for (theta, hd) with at least `rows` positions.
void rope_table(float theta, int hd, int rows, const float** c, const float** s, int* have_rows) {
    Scratch& S = scratch();
    if (S.cos_t == nullptr || S.theta != theta || S.hd != hd || S.rows < rows) {
        int n = S.rows > rows ? S.rows : rows;
        if (n < 4096) n = 4096;
        while (n < rows) n *= 2;
        std::vector<float> hc((std::size_t)n * (hd / 2)), hs((std::size_t)n * (hd / 2));
        bx_rope_table_host(hc.data(), hs.data(), n, hd, theta);
        hipx::sync();
        if (S.cos_t) (void)hipFree(S.cos_t);
        if (S.sin_t) (void)hipFree(S.sin_t);
        on_shutdown(release_scratch);
        hipx::check(hipMalloc(reinterpret_cast<void**>(&S.cos_t), hc.size() * 4), "hipMalloc rope");
        hipx::check(hipMalloc(reinterpret_cast<void**>(&S.sin_t), hs.size() * 4), "hipMalloc rope");
        hipx::h2d(S.cos_t, hc.data(), hc.size() * 4);
        hipx::h2d(S.sin_t, hs.data(), hs.size() * 4);
        S.theta = theta;
        S.hd = hd;
        S.rows = n;
    }
    *c = S.cos_t;
    *s = S.sin_t;
    *have_rows = S.rows;
}

// Long prompts (M >= kDequantRows rows on the tile GEMM) run the FP16 tiles on
// an FP16 copy of each quantized weight, dequantized once per call into the
// op scratch: at these M the GEMM is bound by the matrix cores, where the
// in-loop dequantization of the quantized tiles costs about a fifth of the
// rate, while the copy costs one pass over the weight.  Either way the matrix
// cores multiply each weight rounded once to FP16, the tile path's stated
// difference from the GEMV path.
constexpr int kDequantRows = 512;

bool dequant_first(const Tensor& W, int M, int K) {
    const bool quant = W.dtype == Dtype::Q4_K || W.dtype == Dtype::Q6_K || W.dtype == Dtype::Q8_0;
    return quant && M >= kDequantRows && bx_linear_tiles_ok(M, K) == 1;
}

// FP16 copies of W[0..n) in the scratch (the caller holds scratch().mu);
// out[i] points at W[i]'s copy.
void dequant_weights(const Tensor* const* W, int n, const void** out) {
    std::size_t total = 0;
    for (int i = 0; i < n; ++i) total += ((std::size_t)W[i]->rows * W[i]->cols * 2 + 255) / 256 * 256;
    Scratch& S = scratch();
    auto* base = static_cast<uint8_t*>(grow(S.wdeq, S.wdeq_bytes, total));
    std::size_t off = 0;
    for (int i = 0; i < n; ++i) {
        uint16_t* dst = reinterpret_cast<uint16_t*>(base + off);
        hipx::bx(bx_dequant_to_f16(dtype_to_ggml(W[i]->dtype), W[i]->data, dst, W[i]->rows, W[i]->cols,
                                   hipx::stream()),
                 "dequantize weights for the FP16 tiles");
        out[i] = dst;
        off += ((std::size_t)W[i]->rows * W[i]->cols * 2 + 255) / 256 * 256;
    }
}

void linear_impl(const char* op, Dtype expect, const Tensor& W, const Tensor* bias, const Tensor& X, Tensor& Y) {
    need_device(W, op, "W");
    need_device(X, op, "X");
    need_dtype(W, expect, op, "W");
    need_dtype(X, Dtype::FP16, op, "X");
    if (X.cols != W.cols)
        contract(op, "X cols " + std::to_string(X.cols) + " != W cols " + std::to_string(W.cols));
    const uint16_t* b = nullptr;
    if (bias) {
        need_device(*bias, op, "bias");
        need_dtype(*bias, Dtype::FP16, op, "bias");
        if (bias->size() != W.rows) contract(op, "bias must have W.rows elements");
        b = static_cast<const uint16_t*>(bias->data);
    }
    if (Y.data == X.data) contract(op, "Y must not alias X");
    size_out(Y, X.rows, W.rows, Dtype::FP16);
    if (dequant_first(W, X.rows, X.cols)) {
        std::lock_guard<std::mutex> lk(scratch().mu);
        const Tensor* w[1] = {&W};
        const void* wf[1];
        dequant_weights(w, 1, wf);
        hipx::bx(bx_linear_f16(BX_TYPE_F16, wf[0], b, static_cast<const uint16_t*>(X.data),
                               static_cast<uint16_t*>(Y.data), X.rows, W.rows, W.cols, hipx::linear_ws(),
                               hipx::linear_ws_bytes(), hipx::stream()),
                 op);
        return;
    }
    hipx::bx(bx_linear_f16(dtype_to_ggml(W.dtype), W.data, b, static_cast<const uint16_t*>(X.data),
                           static_cast<uint16_t*>(Y.data), X.rows, W.rows, W.cols, hipx::linear_ws(),
                           hipx::linear_ws_bytes(), hipx::stream()),
             op);
}

void dequant_impl(const char* op, Dtype expect, const Tensor& raw, Tensor& dst) {
    need_device(raw, op, "raw");
    need_dtype(raw, expect, op, "raw");
    size_out(dst, raw.rows, raw.cols, Dtype::FP16);
    hipx::bx(bx_dequant_to_f16(dtype_to_ggml(raw.dtype), raw.data, static_cast<uint16_t*>(dst.data), raw.rows,
                               raw.cols, hipx::stream()),
             op);
}

}  // namespace

void linear_forward_batched_fp16(const Tensor& W, const Tensor* bias, const Tensor& X, Tensor& Y) {
    linear_impl("linear_forward_batched_fp16", Dtype::FP16, W, bias, X, Y);
}
void linear_forward_batched_q4k_fp16(const Tensor& W, const Tensor* bias, const Tensor& X, Tensor& Y) {
    linear_impl("linear_forward_batched_q4k_fp16", Dtype::Q4_K, W, bias, X, Y);
}
void linear_forward_batched_q6k_fp16(const Tensor& W, const Tensor* bias, const Tensor& X, Tensor& Y) {
    linear_impl("linear_forward_batched_q6k_fp16", Dtype::Q6_K, W, bias, X, Y);
}
void linear_forward_batched_q8_0_fp16(const Tensor& W, const Tensor* bias, const Tensor& X, Tensor& Y) {
    linear_impl("linear_forward_batched_q8_0_fp16", Dtype::Q8_0, W, bias, X, Y);
}

namespace {

bool fused_ok(const Tensor& X, const Tensor& W) {
    const bool quant_kernel = W.dtype == Dtype::FP16 || W.dtype == Dtype::Q4_K || W.dtype == Dtype::Q6_K ||
                              W.dtype == Dtype::Q8_0;
    return quant_kernel && W.device == Device::ROCm && X.device == Device::ROCm && X.dtype == Dtype::FP16 &&
           X.cols == W.cols && bx_linear_tiles_ok(X.rows, X.cols) == 1;
}

}  // namespace

bool linear_group_forward_batched(const Tensor* const* W, Tensor* const* Y, int n, const Tensor& X) {
    if (n < 1 || n > 3) return false;
    for (int i = 0; i < n; ++i)
        if (!fused_ok(X, *W[i]) || W[i]->dtype != W[0]->dtype || Y[i]->data == X.data) return false;
    const void* w[3];
    uint16_t* y[3];
    int N[3];
    for (int i = 0; i < n; ++i) {
        size_out(*Y[i], X.rows, W[i]->rows, Dtype::FP16);
        w[i] = W[i]->data;
        y[i] = static_cast<uint16_t*>(Y[i]->data);
        N[i] = W[i]->rows;
    }
    int wtype = dtype_to_ggml(W[0]->dtype);
    std::unique_lock<std::mutex> lk(scratch().mu, std::defer_lock);
    if (dequant_first(*W[0], X.rows, X.cols)) {
        lk.lock();
        dequant_weights(W, n, w);
        wtype = BX_TYPE_F16;
    }
    hipx::bx(bx_linear_group_f16(wtype, n, w, y, N, static_cast<const uint16_t*>(X.data), X.rows, X.cols,
                                 hipx::linear_ws(), hipx::linear_ws_bytes(), hipx::stream()),
             "linear_group_forward_batched");
    return true;
}

bool linear_residual_forward_batched(const Tensor& W, const Tensor& X, Tensor& H) {
    if (!fused_ok(X, W) || H.dtype != Dtype::FP32 || H.device != Device::ROCm || H.rows != X.rows ||
        H.cols != W.rows)
        return false;
    const void* w = W.data;
    int wtype = dtype_to_ggml(W.dtype);
    std::unique_lock<std::mutex> lk(scratch().mu, std::defer_lock);
    if (dequant_first(W, X.rows, X.cols)) {
        lk.lock();
        const Tensor* ws[1] = {&W};
        dequant_weights(ws, 1, &w);
        wtype = BX_TYPE_F16;
    }
    hipx::bx(bx_linear_residual_f16(wtype, w, static_cast<const uint16_t*>(X.data), static_cast<float*>(H.data), X.rows,
                                    W.rows, W.cols, hipx::linear_ws(), hipx::linear_ws_bytes(), hipx::stream()),
             "linear_residual_forward_batched");
    return true;
}

bool linear_swiglu_forward_batched(const Tensor& Wg, const Tensor& Wu, const Tensor& X, Tensor& Y) {
    if (!fused_ok(X, Wg) || !fused_ok(X, Wu) || Wg.dtype != Wu.dtype || Wg.rows != Wu.rows || Y.data == X.data)
        return false;
    size_out(Y, X.rows, Wg.rows, Dtype::FP16);
    const void* w[2] = {Wg.data, Wu.data};
    int wtype = dtype_to_ggml(Wg.dtype);
    std::unique_lock<std::mutex> lk(scratch().mu, std::defer_lock);
    if (dequant_first(Wg, X.rows, X.cols)) {
        lk.lock();
        const Tensor* ws[2] = {&Wg, &Wu};
        dequant_weights(ws, 2, w);
        wtype = BX_TYPE_F16;
    }
    hipx::bx(bx_linear_swiglu_f16(wtype, w[0], w[1], static_cast<const uint16_t*>(X.data),
                                  static_cast<uint16_t*>(Y.data), X.rows, Wg.rows, Wg.cols, hipx::linear_ws(),
                                  hipx::linear_ws_bytes(), hipx::stream()),
             "linear_swiglu_forward_batched");
    return true;
}

void dequant_q8_0_to_fp16(const Tensor& raw, Tensor& dst) { dequant_impl("dequant_q8_0_to_fp16", Dtype::Q8_0, raw, dst); }
void dequant_q4k_to_fp16(const Tensor& raw, Tensor& dst) { dequant_impl("dequant_q4k_to_fp16", Dtype::Q4_K, raw, dst); }
void dequant_q6k_to_fp16(const Tensor& raw, Tensor& dst) { dequant_impl("dequant_q6k_to_fp16", Dtype::Q6_K, raw, dst); }

void dequant_to_fp32(const Tensor& raw, Tensor& dst) {
    need_device(raw, "dequant_to_fp32", "raw");
    if (!dtype_is_quant(raw.dtype) && raw.dtype != Dtype::FP16) contract("dequant_to_fp32", "unsupported dtype");
    size_out(dst, raw.rows, raw.cols, Dtype::FP32);
    hipx::bx(bx_dequant_to_f32(dtype_to_ggml(raw.dtype), raw.data, static_cast<float*>(dst.data), raw.rows, raw.cols,
                               hipx::stream()),
             "dequant_to_fp32");
}

void embedding_lookup_forward(const Tensor& W, const std::int32_t* idx_dev, int L, Tensor& out) {
    need_device(W, "embedding_lookup_forward", "W");
    need_dtype(W, Dtype::FP16, "embedding_lookup_forward", "W");
    if (L <= 0 || !idx_dev) contract("embedding_lookup_forward", "bad ids");
    size_out(out, L, W.cols, Dtype::FP16);
    hipx::bx(bx_embedding_f16(static_cast<const uint16_t*>(W.data), W.rows, W.cols, idx_dev, L,
                              static_cast<uint16_t*>(out.data), hipx::stream()),
             "embedding_lookup_forward");
}

void rms_norm_forward(const Tensor& X, const Tensor& gamma, float eps, Tensor& Y) {
    need_device(X, "rms_norm_forward", "X");
    need_device(gamma, "rms_norm_forward", "gamma");
    need_dtype(gamma, Dtype::FP16, "rms_norm_forward", "gamma");
    if (X.dtype != Dtype::FP16 && X.dtype != Dtype::FP32) contract("rms_norm_forward", "X must be FP16 or FP32");
    if (gamma.size() != X.cols) contract("rms_norm_forward", "gamma must have X.cols elements");
    if (Y.data == X.data) contract("rms_norm_forward", "Y must not alias X");
    size_out(Y, X.rows, X.cols, Dtype::FP16);
    hipx::bx(bx_rms_norm(X.data, X.dtype == Dtype::FP32, static_cast<const uint16_t*>(gamma.data), eps,
                         static_cast<uint16_t*>(Y.data), X.rows, X.cols, hipx::stream()),
             "rms_norm_forward");
}

void rope_forward(const Tensor& X, int hd, int n_heads, int seq_offset, float theta, Tensor& Y) {
    need_device(X, "rope_forward", "X");
    need_dtype(X, Dtype::FP16, "rope_forward", "X");
    if (hd <= 0 || hd % 2 || n_heads <= 0 || X.cols != hd * n_heads)
        contract("rope_forward", "X cols must equal n_heads * hd with even hd");
    if (seq_offset < 0) contract("rope_forward", "negative seq_offset");
    std::lock_guard<std::mutex> lk(scratch().mu);
    const float *c, *s;
    int rows = 0;
    rope_table(theta, hd, seq_offset + X.rows, &c, &s, &rows);
    if (&Y != &X) size_out(Y, X.rows, X.cols, Dtype::FP16);
    hipx::bx(bx_rope_f16(static_cast<const uint16_t*>(X.data), static_cast<uint16_t*>(Y.data), X.rows, hd, n_heads,
                         seq_offset, c, s, rows, hipx::stream()),
             "rope_forward");
}

void rope_apply(const Tensor& X, const Tensor& cos, const Tensor& sin, int hd, int n_heads, Tensor& Y) {
    need_device(X, "rope_apply", "X");
    need_dtype(X, Dtype::FP16, "rope_apply", "X");
    need_dtype(cos, Dtype::FP32, "rope_apply", "cos");
    need_dtype(sin, Dtype::FP32, "rope_apply", "sin");
    if (X.rows != 1 || X.cols != hd * n_heads || cos.size() != hd / 2 || sin.size() != hd / 2)
        contract("rope_apply", "expects a single row and (1, hd/2) cos/sin");
    if (&Y != &X) size_out(Y, X.rows, X.cols, Dtype::FP16);
    hipx::bx(bx_rope_f16(static_cast<const uint16_t*>(X.data), static_cast<uint16_t*>(Y.data), 1, hd, n_heads, 0,
                         static_cast<const float*>(cos.data), static_cast<const float*>(sin.data), 1, hipx::stream()),
             "rope_apply");
}

void kv_cache_append(const Tensor& k, const Tensor& v, int cur_len, Tensor& Kc, Tensor& Vc) {
    for (const Tensor* t : {&k, &v, static_cast<const Tensor*>(&Kc), static_cast<const Tensor*>(&Vc)}) {
        need_device(*t, "kv_cache_append", "operand");
        need_dtype(*t, Dtype::FP16, "kv_cache_append", "operand");
    }
    if (k.rows != v.rows || k.cols != v.cols || Kc.cols != k.cols || Vc.cols != k.cols || Kc.rows != Vc.rows)
        contract("kv_cache_append", "shape mismatch");
    hipx::bx(bx_kv_append_f16(static_cast<const uint16_t*>(k.data), static_cast<const uint16_t*>(v.data), k.rows,
                              k.cols, cur_len, static_cast<uint16_t*>(Kc.data), static_cast<uint16_t*>(Vc.data),
                              Kc.rows, hipx::stream()),
             "kv_cache_append");
}

void scatter_rows(const Tensor& src, const Tensor& idx_row, Tensor& dst) {
    need_device(src, "scatter_rows", "src");
    need_device(dst, "scatter_rows", "dst");
    need_device(idx_row, "scatter_rows", "idx_row");
    need_dtype(idx_row, Dtype::INT32, "scatter_rows", "idx_row");
    if (src.dtype != dst.dtype || src.cols != dst.cols || src.rows != 1)
        contract("scatter_rows", "src must be one row matching dst");
    hipx::bx(bx_scatter_row(src.data, static_cast<const int32_t*>(idx_row.data), dst.data,
                            dtype_storage_bytes(src.dtype, src.cols), dst.rows, hipx::stream()),
             "scatter_rows");
}

void flash_attention_decode(const Tensor& q, const Tensor& Kc, const Tensor& Vc, int valid_len, int n_q, int n_kv,
                            Tensor& out, float softcap, int window) {
    for (const Tensor* t : {&q, &Kc, &Vc}) {
        need_device(*t, "flash_attention_decode", "operand");
        need_dtype(*t, Dtype::FP16, "flash_attention_decode", "operand");
    }
    if (n_q <= 0 || n_kv <= 0 || q.cols % n_q) contract("flash_attention_decode", "bad head counts");
    const int hd = q.cols / n_q;
    if (Kc.cols != n_kv * hd || Vc.cols != Kc.cols || Vc.rows != Kc.rows)
        contract("flash_attention_decode", "cache shape does not match n_kv * head_dim");
    if (valid_len < q.rows || valid_len > Kc.rows) contract("flash_attention_decode", "valid_len out of range");
    size_out(out, q.rows, q.cols, Dtype::FP16);
    std::lock_guard<std::mutex> lk(scratch().mu);
    Scratch& S = scratch();
    void* ws = grow(S.attn_ws, S.attn_bytes, bx_attention_workspace_bytes(q.rows, n_q, hd, valid_len));
    hipx::bx(bx_attention_decode_f16(static_cast<const uint16_t*>(q.data), static_cast<const uint16_t*>(Kc.data),
                                     static_cast<const uint16_t*>(Vc.data), q.rows, valid_len, n_q, n_kv, hd, softcap,
                                     window, static_cast<uint16_t*>(out.data), ws, hipx::stream()),
             "flash_attention_decode");
}

void flash_attention_gqa_forward(const Tensor& q, const Tensor& k, const Tensor& v, int n_q, int n_kv, bool causal,
                                 Tensor& out) {
    for (const Tensor* t : {&q, &k, &v}) {
        need_device(*t, "flash_attention_gqa_forward", "operand");
        need_dtype(*t, Dtype::FP16, "flash_attention_gqa_forward", "operand");
    }
    if (n_q <= 0 || n_kv <= 0 || q.cols % n_q) contract("flash_attention_gqa_forward", "bad head counts");
    const int hd = q.cols / n_q;
    if (k.cols != n_kv * hd || v.cols != k.cols || v.rows != k.rows)
        contract("flash_attention_gqa_forward", "k / v shape does not match n_kv * head_dim");
    size_out(out, q.rows, q.cols, Dtype::FP16);
    std::lock_guard<std::mutex> lk(scratch().mu);
    Scratch& S = scratch();
    void* ws = grow(S.attn_ws, S.attn_bytes, bx_attention_workspace_bytes(q.rows, n_q, hd, k.rows));
    hipx::bx(bx_attention_gqa_f16(static_cast<const uint16_t*>(q.data), static_cast<const uint16_t*>(k.data),
                                  static_cast<const uint16_t*>(v.data), q.rows, k.rows, n_q, n_kv, hd, causal ? 1 : 0,
                                  static_cast<uint16_t*>(out.data), ws, hipx::stream()),
             "flash_attention_gqa_forward");
}

void masked_mean_pool_forward(const Tensor& x, const float* mask, Tensor& out) {
    need_device(x, "masked_mean_pool_forward", "x");
    need_dtype(x, Dtype::FP16, "masked_mean_pool_forward", "x");
    size_out(out, x.cols, 1, Dtype::FP16);
    hipx::bx(bx_masked_mean_pool_f16(static_cast<const uint16_t*>(x.data), mask, x.rows, x.cols,
                                     static_cast<uint16_t*>(out.data), hipx::stream()),
             "masked_mean_pool_forward");
}

void flash_attention_decode_masked(const Tensor& q, const Tensor& Kc, const Tensor& Vc, const float* mask, int n_q,
                                   int n_kv, Tensor& out) {
    for (const Tensor* t : {&q, &Kc, &Vc}) {
        need_device(*t, "flash_attention_decode_masked", "operand");
        need_dtype(*t, Dtype::FP16, "flash_attention_decode_masked", "operand");
    }
    if (q.rows != 1 || n_q <= 0 || n_kv <= 0 || q.cols % n_q || !mask)
        contract("flash_attention_decode_masked", "expects one query row and a mask");
    const int hd = q.cols / n_q;
    if (Kc.cols != n_kv * hd) contract("flash_attention_decode_masked", "cache shape mismatch");
    size_out(out, 1, q.cols, Dtype::FP16);
    std::lock_guard<std::mutex> lk(scratch().mu);
    Scratch& S = scratch();
    void* ws = grow(S.attn_ws, S.attn_bytes, bx_attention_workspace_bytes(1, n_q, hd, Kc.rows));
    hipx::bx(bx_attention_masked_f16(static_cast<const uint16_t*>(q.data), static_cast<const uint16_t*>(Kc.data),
                                     static_cast<const uint16_t*>(Vc.data), mask, Kc.rows, n_q, n_kv, hd,
                                     static_cast<uint16_t*>(out.data), ws, hipx::stream()),
             "flash_attention_decode_masked");
}

void silu_forward(const Tensor& x, Tensor& y) {
    need_device(x, "silu_forward", "x");
    need_dtype(x, Dtype::FP16, "silu_forward", "x");
    if (&y != &x && y.data != x.data) size_out(y, x.rows, x.cols, Dtype::FP16);
    hipx::bx(bx_silu_f16(static_cast<const uint16_t*>(x.data), static_cast<uint16_t*>(y.data), x.size(),
                         hipx::stream()),
             "silu_forward");
}

void mul_inplace(Tensor& a, const Tensor& b) {
    need_device(a, "mul_inplace", "a");
    need_device(b, "mul_inplace", "b");
    need_dtype(a, Dtype::FP16, "mul_inplace", "a");
    need_dtype(b, Dtype::FP16, "mul_inplace", "b");
    if (a.size() != b.size()) contract("mul_inplace", "size mismatch");
    hipx::bx(bx_mul_f16(static_cast<uint16_t*>(a.data), static_cast<const uint16_t*>(b.data), a.size(),
                        hipx::stream()),
             "mul_inplace");
}

void add_inplace(Tensor& a, const Tensor& b) {
    need_device(a, "add_inplace", "a");
    need_device(b, "add_inplace", "b");
    need_dtype(b, Dtype::FP16, "add_inplace", "b");
    if (a.dtype != Dtype::FP16 && a.dtype != Dtype::FP32) contract("add_inplace", "a must be FP16 or FP32");
    if (a.size() != b.size()) contract("add_inplace", "size mismatch");
    hipx::bx(bx_add_inplace(a.data, a.dtype == Dtype::FP32, static_cast<const uint16_t*>(b.data), a.size(),
                            hipx::stream()),
             "add_inplace");
}

void copy_d2d(const Tensor& src, std::int64_t src_off, Tensor& dst, std::int64_t dst_off, std::int64_t n) {
    need_device(src, "copy_d2d", "src");
    need_device(dst, "copy_d2d", "dst");
    const int es = dtype_size_bytes(src.dtype);
    if (es == 0 || src.dtype != dst.dtype) contract("copy_d2d", "dense matching dtypes required");
    if (src_off < 0 || dst_off < 0 || n < 0 || src_off + n > src.size() || dst_off + n > dst.size())
        contract("copy_d2d", "range out of bounds");
    if (n == 0) return;
    hipx::check(hipMemcpyAsync(static_cast<char*>(dst.data) + dst_off * es,
                               static_cast<const char*>(src.data) + src_off * es, (std::size_t)(n * es),
                               hipMemcpyDeviceToDevice, hipx::stream()),
                "copy_d2d");
}

void copy_d2d_strided(const Tensor& src, std::int64_t src_off, std::int64_t src_stride, Tensor& dst,
                      std::int64_t dst_off, std::int64_t dst_stride, std::int64_t elem, std::int64_t n) {
    need_device(src, "copy_d2d_strided", "src");
    need_device(dst, "copy_d2d_strided", "dst");
    const int es = dtype_size_bytes(src.dtype);
    if (es == 0 || src.dtype != dst.dtype) contract("copy_d2d_strided", "dense matching dtypes required");
    if (n <= 0 || elem <= 0) return;
    if (src_off + (n - 1) * src_stride + elem > src.size() || dst_off + (n - 1) * dst_stride + elem > dst.size())
        contract("copy_d2d_strided", "range out of bounds");
    hipx::check(hipMemcpy2DAsync(static_cast<char*>(dst.data) + dst_off * es, (std::size_t)(dst_stride * es),
                                 static_cast<const char*>(src.data) + src_off * es, (std::size_t)(src_stride * es),
                                 (std::size_t)(elem * es), (std::size_t)n, hipMemcpyDeviceToDevice, hipx::stream()),
                "copy_d2d_strided");
}

void argmax_forward(const Tensor& logits_row, Tensor& out_idx) {
    need_device(logits_row, "argmax_forward", "logits");
    need_dtype(logits_row, Dtype::FP16, "argmax_forward", "logits");
    size_out(out_idx, 1, 1, Dtype::INT32);
    std::lock_guard<std::mutex> lk(scratch().mu);
    Scratch& S = scratch();
    void* ws = grow(S.argmax_ws, S.argmax_bytes, bx_argmax_workspace_bytes(logits_row.size()));
    hipx::bx(bx_argmax_f16(static_cast<const uint16_t*>(logits_row.data), logits_row.size(),
                           static_cast<int32_t*>(out_idx.data), ws, hipx::stream()),
             "argmax_forward");
}

}  // namespace brotensor
