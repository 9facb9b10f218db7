// Multi-sequence batched decode: the per-row forms of RoPE and the KV append
// (each of the M rows is the next token of its own sequence, at its own
// position, in its own slot of a slot-major KV arena).  The attention over
// each row's own keys is bx_attention_varlen_f16 (attention.hip).  These
// extend the single-sequence ops of src/detail/dense_decoder.cpp:585-607
// (rope_forward with one seq_offset, kv_cache_append at one cur_len).
#include "common.h"

namespace bx {
namespace {

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
    const float x0 = h2f(X[off]), x1 = h2f(X[off + 1]);
    Y[off] = f2h(x0 * c - x1 * s);
    Y[off + 1] = f2h(x0 * s + x1 * c);
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

}  // extern "C"
