// Multi-sequence batched decode: the per-row forms of RoPE and the KV append
// (each of the M rows is the next token of its own sequence, at its own
// position, in its own slot of a slot-major KV arena), and the two fused with
// the q / k head RMSNorm into one launch.  The attention over
// each row's own keys is bx_attention_varlen_f16 (attention.hip).  These
// extend the single-sequence ops of src/detail/dense_decoder.cpp:585-607
// (rope_forward with one seq_offset, kv_cache_append at one cur_len).
#include "common.h"

namespace bx {
namespace {

// RoPE of one pair (2i, 2i+1) by the table angle (cos c, sin s), FP16 out.
// The arithmetic is fixed (one explicit fused multiply-add each, an FP32
// result, then FP16), so every kernel that rotates with this function rounds
// the same way; left to the compiler, which product it fuses, or a fusion
// with the FP16 conversion, may differ between kernels and move a result
// across an FP16 rounding boundary.
__device__ __forceinline__ void rope_pair(float x0, float x1, float c, float s, uint16_t& y0, uint16_t& y1) {
    y0 = f2h(f32_fence(__builtin_fmaf(x0, c, -f32_fence(x1 * s))));
    y1 = f2h(f32_fence(__builtin_fmaf(x0, s, f32_fence(x1 * c))));
}

// Row r rotates at position pos[r]; rows whose position is outside the table
// are left unwritten (the host validates positions before the launch).
__global__ void rope_rows_kernel(const uint16_t* __restrict__ X, uint16_t* __restrict__ Y, int rows, int hd,
                                 int n_heads, const int32_t* __restrict__ pos, int tab_rows,
                                 const float* __restrict__ cos_t, const float* __restrict__ sin_t) {
    const int half = hd / 2;
    const int64_t i = blockIdx.x * (int64_t)blockDim.x + threadIdx.x;
    if (i >= (int64_t)rows * n_heads * half) return;
    const int p = (int)(i % half);
    const int64_t rh = i / half;
    const int r = (int)(rh / n_heads);
    const int ps = pos[r];
    if (ps < 0 || ps >= tab_rows) return;
    const int64_t off = rh * hd + 2 * p;
    const float c = cos_t[(int64_t)ps * half + p], s = sin_t[(int64_t)ps * half + p];
    uint16_t y0, y1;
    rope_pair(h2f(X[off]), h2f(X[off + 1]), c, s, y0, y1);
    Y[off] = y0;
    Y[off + 1] = y1;
}

// Row r of k / v goes to cache row dst[r] (slot * capacity + position);
// rows outside [0, cache_rows) are skipped.
__global__ void kv_rows_kernel(const uint16_t* __restrict__ k, const uint16_t* __restrict__ v, int rows, int cols,
                               const int64_t* __restrict__ dst, int64_t cache_rows, uint16_t* __restrict__ Kc,
                               uint16_t* __restrict__ Vc) {
    const int64_t i = blockIdx.x * (int64_t)blockDim.x + threadIdx.x;
    if (i >= (int64_t)rows * cols) return;
    const int r = (int)(i / cols), c = (int)(i % cols);
    const int64_t d = dst[r];
    if (d < 0 || d >= cache_rows) return;
    Kc[d * cols + c] = k[i];
    Vc[d * cols + c] = v[i];
}

// The per-head stage of a batched step in one launch: for row r and head h
// (q heads, then k heads), the head RMSNorm (when a gain is given), RoPE at
// pos[r], and the k row (with its v row) written to cache row dst[r].  One
// wavefront per (row, head); lane l holds elements l, l + 64, ... of the head,
// as the one-wavefront rms_norm_kernel does, so the sum of squares, the FP16
// normed values and the rotation round exactly as the separate launches of
// rms_norm, rope_rows and kv_append_rows.  A pair's partner element is in the
// neighbouring lane.
template <int EPL>
__global__ __launch_bounds__(256) void qk_rope_kv_rows_kernel(
    const uint16_t* q, const uint16_t* __restrict__ k, const uint16_t* __restrict__ v, int rows, int n_q, int n_kv, const uint16_t* __restrict__ q_gain, const uint16_t* __restrict__ k_gain, float eps,
    const int32_t* __restrict__ pos, int tab_rows, const float* __restrict__ cos_t, const float* __restrict__ sin_t,
    const int64_t* __restrict__ dst, int64_t cache_rows, uint16_t* __restrict__ Kc, uint16_t* __restrict__ Vc,
    uint16_t* q_out) {
    constexpr int HD = 64 * EPL, half = HD / 2;
    const int item = blockIdx.x * 4 + (threadIdx.x >> 6);
    const int heads = n_q + n_kv;
    if (item >= rows * heads) return;
    const int lane = threadIdx.x & 63;
    const int r = item / heads, h = item - r * heads;
    const bool is_q = h < n_q;
    const int hk = h - n_q;
    const uint16_t* src = is_q ? q + ((int64_t)r * n_q + h) * HD : k + ((int64_t)r * n_kv + hk) * HD;
    const uint16_t* gain = is_q ? q_gain : k_gain;
    float x[EPL];
#pragma unroll
    for (int i = 0; i < EPL; ++i) x[i] = h2f(src[lane + 64 * i]);
    if (gain) {
        float ss = 0.f;
#pragma unroll
        for (int i = 0; i < EPL; ++i) ss += x[i] * x[i];
        ss = wave_sum(ss);
        const float inv = 1.0f / sqrtf(ss / (float)HD + eps);
#pragma unroll
        for (int i = 0; i < EPL; ++i) x[i] = h2f(norm_f16(x[i], inv, h2f(gain[lane + 64 * i])));
    }
    const int ps = pos[r];
    const bool rot = ps >= 0 && ps < tab_rows;
    uint16_t y[EPL];
#pragma unroll
    for (int i = 0; i < EPL; ++i) {
        const int e = lane + 64 * i;
        const float other = __shfl_xor(x[i], 1, 64);
        const float c = rot ? cos_t[(int64_t)ps * half + (e >> 1)] : 1.f;
        const float sn = rot ? sin_t[(int64_t)ps * half + (e >> 1)] : 0.f;
        uint16_t y0, y1;
        if (e & 1) rope_pair(other, x[i], c, sn, y0, y1);
        else rope_pair(x[i], other, c, sn, y0, y1);
        y[i] = (e & 1) ? y1 : y0;
    }
    if (is_q) {
        if (!rot) return;
        uint16_t* o = q_out + ((int64_t)r * n_q + h) * HD;
#pragma unroll
        for (int i = 0; i < EPL; ++i) o[lane + 64 * i] = y[i];
        return;
    }
    const int64_t d = dst[r];
    if (!rot || d < 0 || d >= cache_rows) return;
    const int64_t width = (int64_t)n_kv * HD;
    const uint16_t* vs = v + (int64_t)r * width + (int64_t)hk * HD;
#pragma unroll
    for (int i = 0; i < EPL; ++i) {
        const int e = lane + 64 * i;
        Kc[d * width + (int64_t)hk * HD + e] = y[i];
        Vc[d * width + (int64_t)hk * HD + e] = vs[e];
    }
}

inline unsigned blocks_of(int64_t n, int bs) { return (unsigned)((n + bs - 1) / bs); }

}  // namespace
}  // namespace bx

using namespace bx;

extern "C" {

int bx_rope_rows_f16(const uint16_t* X, uint16_t* Y, int rows, int hd, int n_heads, const int32_t* pos_dev,
                     const float* cos_tab, const float* sin_tab, int tab_rows, void* stream) {
    if (!X || !Y || !pos_dev || !cos_tab || !sin_tab || rows <= 0 || hd <= 0 || hd % 2 || n_heads <= 0 ||
        tab_rows <= 0)
        return fail(BX_EINVAL, "rope_rows: bad arguments");
    const int64_t n = (int64_t)rows * n_heads * (hd / 2);
    rope_rows_kernel<<<blocks_of(n, 256), 256, 0, as_stream(stream)>>>(X, Y, rows, hd, n_heads, pos_dev, tab_rows,
                                                                        cos_tab, sin_tab);
    return launch_check("rope_rows");
}

int bx_kv_append_rows_f16(const uint16_t* k, const uint16_t* v, int rows, int cols, const int64_t* dst_rows_dev,
                          uint16_t* Kc, uint16_t* Vc, int64_t cache_rows, void* stream) {
    if (!k || !v || !dst_rows_dev || !Kc || !Vc || rows <= 0 || cols <= 0 || cache_rows <= 0)
        return fail(BX_EINVAL, "kv_append_rows: bad arguments");
    kv_rows_kernel<<<blocks_of((int64_t)rows * cols, 256), 256, 0, as_stream(stream)>>>(k, v, rows, cols,
                                                                                          dst_rows_dev, cache_rows,
                                                                                          Kc, Vc);
    return launch_check("kv_append_rows");
}

int bx_qk_rope_kv_rows_f16(const uint16_t* q, const uint16_t* k, const uint16_t* v, int rows, int hd, int n_q,
                           int n_kv, const uint16_t* q_gain, const uint16_t* k_gain, float eps, const int32_t* pos_dev,
                           const float* cos_tab, const float* sin_tab, int tab_rows, const int64_t* dst_rows_dev,
                           uint16_t* Kc, uint16_t* Vc, int64_t cache_rows, uint16_t* q_out, void* stream) {
    if (!q || !k || !v || !pos_dev || !cos_tab || !sin_tab || !dst_rows_dev || !Kc || !Vc || !q_out || rows <= 0 ||
        n_q <= 0 || n_kv <= 0 || tab_rows <= 0 || cache_rows <= 0 || (q_gain == nullptr) != (k_gain == nullptr))
        return fail(BX_EINVAL, "qk_rope_kv_rows: bad arguments");
    const unsigned grid = blocks_of((int64_t)rows * (n_q + n_kv), 4);
    hipStream_t st = as_stream(stream);
    switch (hd) {
        case 64:
            qk_rope_kv_rows_kernel<1><<<grid, 256, 0, st>>>(q, k, v, rows, n_q, n_kv, q_gain, k_gain, eps, pos_dev,
                                                            tab_rows, cos_tab, sin_tab, dst_rows_dev, cache_rows, Kc,
                                                            Vc, q_out);
            break;
        case 128:
            qk_rope_kv_rows_kernel<2><<<grid, 256, 0, st>>>(q, k, v, rows, n_q, n_kv, q_gain, k_gain, eps, pos_dev,
                                                            tab_rows, cos_tab, sin_tab, dst_rows_dev, cache_rows, Kc,
                                                            Vc, q_out);
            break;
        case 256:
            qk_rope_kv_rows_kernel<4><<<grid, 256, 0, st>>>(q, k, v, rows, n_q, n_kv, q_gain, k_gain, eps, pos_dev,
                                                            tab_rows, cos_tab, sin_tab, dst_rows_dev, cache_rows, Kc,
                                                            Vc, q_out);
            break;
        default:
            return fail(BX_EUNSUPPORTED, "qk_rope_kv_rows: head_dim must be 64, 128 or 256");
    }
    return launch_check("qk_rope_kv_rows");
}

}  // extern "C"
