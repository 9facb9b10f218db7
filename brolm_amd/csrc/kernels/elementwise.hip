// Small per-token ops of the decoder (brolm call sites in
// src/detail/dense_decoder.cpp): embedding gather, RMSNorm / per-head
// QK-norm, interleaved-pair RoPE, KV-cache append, SwiGLU, residual add.
#include <cmath>

#include "common.h"

namespace bx {
namespace {

inline unsigned blocks_for(int64_t n, int bs) { return (unsigned)((n + bs - 1) / bs); }

template <typename OutT>
__device__ __forceinline__ void put(OutT* p, float v);
template <>
__device__ __forceinline__ void put<float>(float* p, float v) { *p = v; }
template <>
__device__ __forceinline__ void put<uint16_t>(uint16_t* p, float v) { *p = f2h(v); }

template <typename OutT>
__global__ void embedding_kernel(const uint16_t* __restrict__ W, int H, const int32_t* __restrict__ ids, int L,
                                 OutT* __restrict__ out) {
    const int64_t i = blockIdx.x * (int64_t)blockDim.x + threadIdx.x;
    if (i >= (int64_t)L * H) return;
    const int r = (int)(i / H), c = (int)(i % H);
    put(out + i, h2f(W[(int64_t)ids[r] * H + c]));
}

// One block per row.  y = x * (mean(x^2) + eps)^-1/2 * gamma  (FP32 math).
// EPT > 0: every thread holds at most EPT elements (cols <= NT * EPT), all
// its x and gamma loads issued before any use (one memory round trip instead
// of one per element); EPT = 0: any width, element by element.  Thread t adds
// the squares of elements t, t + NT, ... in that order either way, so both
// forms give the same bits.
template <typename InT, int NT, int EPT>
__global__ __launch_bounds__(NT) void rms_norm_kernel(const InT* __restrict__ X, const uint16_t* __restrict__ gamma,
                                                      float eps, uint16_t* __restrict__ Y, int cols) {
    __shared__ float red[NT / 64];
    const int64_t r = blockIdx.x;
    const InT* x = X + r * cols;
    if constexpr (EPT > 0) {
        float v[EPT], g[EPT];
#pragma unroll
        for (int i = 0; i < EPT; ++i) {
            const int c = threadIdx.x + NT * i;
            const int cc = c < cols ? c : cols - 1;   // clamped: every load issued
            if constexpr (sizeof(InT) == 4) v[i] = x[cc]; else v[i] = h2f(x[cc]);
            g[i] = h2f(gamma[cc]);
        }
        float ss = 0.f;
#pragma unroll
        for (int i = 0; i < EPT; ++i)
            if (threadIdx.x + NT * i < cols) ss += v[i] * v[i];
        ss = block_sum<NT>(ss, red);
        const float inv = 1.0f / sqrtf(ss / (float)cols + eps);
#pragma unroll
        for (int i = 0; i < EPT; ++i) {
            const int c = threadIdx.x + NT * i;
            if (c < cols) Y[r * cols + c] = norm_f16(v[i], inv, g[i]);
        }
        return;
    }
    float ss = 0.f;
    for (int c = threadIdx.x; c < cols; c += NT) {
        float v;
        if constexpr (sizeof(InT) == 4) v = x[c]; else v = h2f(x[c]);
        ss += v * v;
    }
    ss = block_sum<NT>(ss, red);
    const float inv = 1.0f / sqrtf(ss / (float)cols + eps);
    for (int c = threadIdx.x; c < cols; c += NT) {
        float v;
        if constexpr (sizeof(InT) == 4) v = x[c]; else v = h2f(x[c]);
        Y[r * cols + c] = norm_f16(v, inv, h2f(gamma[c]));
    }
}

template <typename InT, int NT>
void rms_norm_launch(const InT* X, const uint16_t* gamma, float eps, uint16_t* Y, int rows, int cols,
                     hipStream_t st) {
    const int ept = (cols + NT - 1) / NT;
    if (ept <= 1) rms_norm_kernel<InT, NT, 1><<<rows, NT, 0, st>>>(X, gamma, eps, Y, cols);
    else if (ept <= 2) rms_norm_kernel<InT, NT, 2><<<rows, NT, 0, st>>>(X, gamma, eps, Y, cols);
    else if (ept <= 4) rms_norm_kernel<InT, NT, 4><<<rows, NT, 0, st>>>(X, gamma, eps, Y, cols);
    else if (ept <= 8) rms_norm_kernel<InT, NT, 8><<<rows, NT, 0, st>>>(X, gamma, eps, Y, cols);
    else if (ept <= 16) rms_norm_kernel<InT, NT, 16><<<rows, NT, 0, st>>>(X, gamma, eps, Y, cols);
    else rms_norm_kernel<InT, NT, 0><<<rows, NT, 0, st>>>(X, gamma, eps, Y, cols);
}

// Pairs (2i, 2i+1) of every head rotate by the table angle of row pos.
__global__ void rope_kernel(const uint16_t* __restrict__ X, uint16_t* __restrict__ Y, int rows, int hd, int n_heads,
                            int seq_offset, const float* __restrict__ cos_t, const float* __restrict__ sin_t) {
    const int half = hd / 2;
    const int64_t i = blockIdx.x * (int64_t)blockDim.x + threadIdx.x;
    const int64_t total = (int64_t)rows * n_heads * half;
    if (i >= total) return;
    const int p = (int)(i % half);
    const int64_t rh = i / half;
    const int r = (int)(rh / n_heads);
    const int64_t off = rh * hd + 2 * p;
    const int pos = seq_offset + r;
    const float c = cos_t[(int64_t)pos * half + p], s = sin_t[(int64_t)pos * half + p];
    const float x0 = h2f(X[off]), x1 = h2f(X[off + 1]);
    Y[off] = f2h(x0 * c - x1 * s);
    Y[off + 1] = f2h(x0 * s + x1 * c);
}

__global__ void kv_append_kernel(const uint16_t* __restrict__ k, const uint16_t* __restrict__ v, int L, int cols,
                                 int cur_len, uint16_t* __restrict__ Kc, uint16_t* __restrict__ Vc) {
    const int64_t i = blockIdx.x * (int64_t)blockDim.x + threadIdx.x;
    if (i >= (int64_t)L * cols) return;
    const int64_t dst = (int64_t)cur_len * cols + i;
    Kc[dst] = k[i];
    Vc[dst] = v[i];
}


__global__ void silu_mul_kernel(uint16_t* __restrict__ g, const uint16_t* __restrict__ u, int64_t n) {
    const int64_t i = blockIdx.x * (int64_t)blockDim.x + threadIdx.x;
    if (i < n) g[i] = f2h(silu_f32(h2f(g[i])) * h2f(u[i]));
}
__global__ void silu_kernel(const uint16_t* __restrict__ x, uint16_t* __restrict__ y, int64_t n) {
    const int64_t i = blockIdx.x * (int64_t)blockDim.x + threadIdx.x;
    if (i < n) y[i] = f2h(silu_f32(h2f(x[i])));
}
__global__ void mul_kernel(uint16_t* __restrict__ a, const uint16_t* __restrict__ b, int64_t n) {
    const int64_t i = blockIdx.x * (int64_t)blockDim.x + threadIdx.x;
    if (i < n) a[i] = f2h(h2f(a[i]) * h2f(b[i]));
}
template <typename T>
__global__ void add_kernel(T* __restrict__ h, const uint16_t* __restrict__ x, int64_t n) {
    const int64_t i = blockIdx.x * (int64_t)blockDim.x + threadIdx.x;
    if (i >= n) return;
    if constexpr (sizeof(T) == 4) h[i] += h2f(x[i]); else h[i] = f2h(h2f(h[i]) + h2f(x[i]));
}
__global__ void scatter_row_kernel(const uint8_t* __restrict__ src, const int32_t* __restrict__ idx,
                                   uint8_t* __restrict__ dst, int64_t row_bytes, int dst_rows) {
    const int r = *idx;
    if (r < 0 || r >= dst_rows) return;  // out-of-range index: no write
    for (int64_t i = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; i < row_bytes; i += (int64_t)gridDim.x * blockDim.x)
        dst[(int64_t)r * row_bytes + i] = src[i];
}

__global__ void f32_to_f16_kernel(const float* __restrict__ x, uint16_t* __restrict__ y, int64_t n) {
    const int64_t i = blockIdx.x * (int64_t)blockDim.x + threadIdx.x;
    if (i < n) y[i] = f2h(x[i]);
}

// One thread per column, rows in order: the sums are deterministic.
__global__ void mean_pool_kernel(const uint16_t* __restrict__ x, const float* __restrict__ mask, int L, int cols,
                                 uint16_t* __restrict__ out) {
    const int c = blockIdx.x * blockDim.x + threadIdx.x;
    if (c >= cols) return;
    float s = 0.f, w = 0.f;
    for (int r = 0; r < L; ++r) {
        const float m = mask ? mask[r] : 1.0f;
        if (m != 0.f) {
            s += m * h2f(x[(int64_t)r * cols + c]);
            w += m;
        }
    }
    out[c] = f2h(w != 0.f ? s / w : 0.f);
}

}  // namespace
}  // namespace bx

using namespace bx;

extern "C" {

int bx_masked_mean_pool_f16(const uint16_t* x, const float* mask, int L, int cols, uint16_t* out, void* stream) {
    if (!x || !out || L <= 0 || cols <= 0) return fail(BX_EINVAL, "masked_mean_pool: bad arguments");
    mean_pool_kernel<<<(cols + 255) / 256, 256, 0, as_stream(stream)>>>(x, mask, L, cols, out);
    return launch_check("masked_mean_pool");
}

int bx_embedding_f16(const uint16_t* W, int V, int H, const int32_t* ids, int L, uint16_t* out, void* stream) {
    if (!W || !ids || !out || V <= 0 || H <= 0 || L <= 0) return fail(BX_EINVAL, "embedding: bad arguments");
    embedding_kernel<uint16_t><<<blocks_for((int64_t)L * H, 256), 256, 0, as_stream(stream)>>>(W, H, ids, L, out);
    return launch_check("embedding");
}

int bx_embedding_f32(const uint16_t* W, int V, int H, const int32_t* ids, int L, float* out, void* stream) {
    if (!W || !ids || !out || V <= 0 || H <= 0 || L <= 0) return fail(BX_EINVAL, "embedding: bad arguments");
    embedding_kernel<float><<<blocks_for((int64_t)L * H, 256), 256, 0, as_stream(stream)>>>(W, H, ids, L, out);
    return launch_check("embedding");
}

int bx_rms_norm(const void* X, int x_is_f32, const uint16_t* gamma, float eps, uint16_t* Y, int rows, int cols,
                void* stream) {
    if (!X || !gamma || !Y || rows <= 0 || cols <= 0) return fail(BX_EINVAL, "rms_norm: bad arguments");
    hipStream_t st = as_stream(stream);
    if (cols <= 512) {
        if (x_is_f32) rms_norm_launch<float, 64>((const float*)X, gamma, eps, Y, rows, cols, st);
        else rms_norm_launch<uint16_t, 64>((const uint16_t*)X, gamma, eps, Y, rows, cols, st);
    } else {
        if (x_is_f32) rms_norm_launch<float, 256>((const float*)X, gamma, eps, Y, rows, cols, st);
        else rms_norm_launch<uint16_t, 256>((const uint16_t*)X, gamma, eps, Y, rows, cols, st);
    }
    return launch_check("rms_norm");
}

void bx_rope_table_host(float* cos_out, float* sin_out, int rows, int hd, float theta) {
    const int half = hd / 2;
    for (int i = 0; i < half; ++i) {
        const double inv = std::pow((double)theta, -2.0 * i / (double)hd);
        for (int p = 0; p < rows; ++p) {
            const double a = (double)p * inv;
            cos_out[(size_t)p * half + i] = (float)std::cos(a);
            sin_out[(size_t)p * half + i] = (float)std::sin(a);
        }
    }
}

int bx_rope_f16(const uint16_t* X, uint16_t* Y, int rows, int hd, int n_heads, int seq_offset, const float* cos_tab,
                const float* sin_tab, int tab_rows, void* stream) {
    if (!X || !Y || !cos_tab || !sin_tab || rows <= 0 || hd <= 0 || hd % 2 || n_heads <= 0)
        return fail(BX_EINVAL, "rope: bad arguments");
    if (seq_offset < 0 || seq_offset + rows > tab_rows) return fail(BX_EINVAL, "rope: position beyond the table");
    const int64_t n = (int64_t)rows * n_heads * (hd / 2);
    rope_kernel<<<blocks_for(n, 256), 256, 0, as_stream(stream)>>>(X, Y, rows, hd, n_heads, seq_offset, cos_tab,
                                                                    sin_tab);
    return launch_check("rope");
}

int bx_kv_append_f16(const uint16_t* k, const uint16_t* v, int L, int cols, int cur_len, uint16_t* Kc, uint16_t* Vc,
                     int cap, void* stream) {
    if (!k || !v || !Kc || !Vc || L <= 0 || cols <= 0) return fail(BX_EINVAL, "kv_append: bad arguments");
    if (cur_len < 0 || cur_len + L > cap) return fail(BX_EINVAL, "kv_append: cur_len + L exceeds the cache capacity");
    kv_append_kernel<<<blocks_for((int64_t)L * cols, 256), 256, 0, as_stream(stream)>>>(k, v, L, cols, cur_len, Kc,
                                                                                         Vc);
    return launch_check("kv_append");
}

int bx_silu_mul_f16(uint16_t* g, const uint16_t* u, int64_t n, void* stream) {
    if (!g || !u || n < 0) return fail(BX_EINVAL, "silu_mul: bad arguments");
    if (n == 0) return BX_OK;
    silu_mul_kernel<<<blocks_for(n, 256), 256, 0, as_stream(stream)>>>(g, u, n);
    return launch_check("silu_mul");
}

int bx_silu_f16(const uint16_t* x, uint16_t* y, int64_t n, void* stream) {
    if (!x || !y || n < 0) return fail(BX_EINVAL, "silu: bad arguments");
    if (n == 0) return BX_OK;
    silu_kernel<<<blocks_for(n, 256), 256, 0, as_stream(stream)>>>(x, y, n);
    return launch_check("silu");
}

int bx_mul_f16(uint16_t* a, const uint16_t* b, int64_t n, void* stream) {
    if (!a || !b || n < 0) return fail(BX_EINVAL, "mul: bad arguments");
    if (n == 0) return BX_OK;
    mul_kernel<<<blocks_for(n, 256), 256, 0, as_stream(stream)>>>(a, b, n);
    return launch_check("mul");
}

int bx_add_inplace(void* h, int h_is_f32, const uint16_t* x, int64_t n, void* stream) {
    if (!h || !x || n < 0) return fail(BX_EINVAL, "add: bad arguments");
    if (n == 0) return BX_OK;
    if (h_is_f32) add_kernel<float><<<blocks_for(n, 256), 256, 0, as_stream(stream)>>>((float*)h, x, n);
    else add_kernel<uint16_t><<<blocks_for(n, 256), 256, 0, as_stream(stream)>>>((uint16_t*)h, x, n);
    return launch_check("add");
}

int bx_scatter_row(const void* src, const int32_t* idx_dev, void* dst, int64_t row_bytes, int dst_rows,
                   void* stream) {
    if (!src || !idx_dev || !dst || row_bytes <= 0 || dst_rows <= 0) return fail(BX_EINVAL, "scatter_row: bad arguments");
    scatter_row_kernel<<<blocks_for(row_bytes, 256) < 64 ? blocks_for(row_bytes, 256) : 64, 256, 0,
                         as_stream(stream)>>>(static_cast<const uint8_t*>(src), idx_dev, static_cast<uint8_t*>(dst),
                                              row_bytes, dst_rows);
    return launch_check("scatter_row");
}

int bx_f32_to_f16(const float* x, uint16_t* y, int64_t n, void* stream) {
    if (!x || !y || n < 0) return fail(BX_EINVAL, "f32_to_f16: bad arguments");
    if (n == 0) return BX_OK;
    f32_to_f16_kernel<<<blocks_for(n, 256), 256, 0, as_stream(stream)>>>(x, y, n);
    return launch_check("f32_to_f16");
}

}  // extern "C"
