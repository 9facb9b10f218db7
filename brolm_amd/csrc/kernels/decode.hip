// Fused single-token decode step: the captured graph body of
// src/detail/dense_decoder.cpp:439-496 (run_layers_ at L == 1, :526-681),
// restructured into six kernels per layer:
//
//   1 norm_qkv   rms_norm(h) in the prologue, GEMV over [Wq; Wk; Wv] (mixed
//                carrier formats by row segment), FP32 q/k/v out
//   2 attn       per (KV head, split): QK-norm + RoPE of q and k, KV-cache
//                write of position pos, split-K attention partials
//   3 combine    merge splits -> FP16 attention output
//   4 o_proj     GEMV + residual add into the FP32 residual stream
//   5 norm_mlp   rms_norm(h) prologue, gate and up rows of the same index in
//                one wavefront, SwiGLU epilogue -> FP16 activation
//   6 down       GEMV + residual add
//
// The token id and position are read from device memory (pos_dev, tok_dev),
// so one capture serves every step; the split count is fixed at capture time
// and the keys per split follow pos on the device.
#include <cmath>

#include "attention_core.h"
#include "gemv_core.h"

namespace bx {
namespace {

constexpr int kThreads = 256;
constexpr int kWaves = kThreads / 64;
constexpr int kMinKeysPerSplit = 32;

struct WsLayout {
    size_t h, qkv, attn, act, part, total;
    int S;
};

WsLayout ws_layout(const bx_decode_dims& d) {
    WsLayout w{};
    const int qd = d.n_q * d.head_dim, kvd = d.n_kv * d.head_dim;
    int S = (2 * num_cus()) / (d.n_kv > 0 ? d.n_kv : 1);
    if (S < 1) S = 1;
    const int smax = (d.cap + kMinKeysPerSplit - 1) / kMinKeysPerSplit;
    if (S > smax) S = smax;
    w.S = S;
    size_t off = 0;
    auto take = [&](size_t bytes) {
        const size_t o = off;
        off += (bytes + 255) / 256 * 256;
        return o;
    };
    w.h = take((size_t)d.hidden * 4);
    w.qkv = take((size_t)(qd + 2 * kvd) * 4);
    w.attn = take((size_t)qd * 2);
    w.act = take((size_t)d.intermediate * 2);
    w.part = take((size_t)d.n_q * S * (d.head_dim + 2) * 4);
    w.total = off;
    return w;
}

// ---- activation staging -------------------------------------------------

// x = fp16(h * rsqrt(mean(h^2) + eps) * gamma), swizzled into LDS (+ sums).
__device__ void stage_norm(const float* __restrict__ h, const uint16_t* __restrict__ gamma, float eps, int K,
                           uint32_t* xs, float* xsum, float* red) {
    float ss = 0.f;
    for (int i = threadIdx.x; i < K; i += kThreads) {
        const float v = h[i];
        ss += v * v;
    }
    ss = block_sum<kThreads>(ss, red);
    const float inv = 1.0f / sqrtf(ss / (float)K + eps);
    for (int g = threadIdx.x; g < K / 4; g += kThreads) {
        const float4 v = *reinterpret_cast<const float4*>(h + 4 * g);
        const u2v gm = *reinterpret_cast<const u2v*>(gamma + 4 * g);
        const uint32_t x0 = f2h(v.x * inv * h2f(gm.x & 0xffff));
        const uint32_t x1 = f2h(v.y * inv * h2f(gm.x >> 16));
        const uint32_t x2 = f2h(v.z * inv * h2f(gm.y & 0xffff));
        const uint32_t x3 = f2h(v.w * inv * h2f(gm.y >> 16));
        store_group<true>(xs, g, x0, x1, x2, x3);
    }
    __syncthreads();
    sums_from_lds(xs, 1, K, K / 2, xsum, K / 16);
    __syncthreads();
}

__device__ void stage_f16(const uint16_t* __restrict__ x, int K, uint32_t* xs, float* xsum) {
    for (int g = threadIdx.x; g < K / 4; g += kThreads) {
        const u2v v = *reinterpret_cast<const u2v*>(x + 4 * g);
        store_group<true>(xs, g, v.x & 0xffff, v.x >> 16, v.y & 0xffff, v.y >> 16);
    }
    __syncthreads();
    sums_from_lds(xs, 1, K, K / 2, xsum, K / 16);
    __syncthreads();
}

// ---- one weight row (M = 1) against the staged activation ---------------

template <int FMT>
__device__ __forceinline__ float row_dot_fmt(const void* W, int64_t N, int K, int64_t n, const uint32_t* xs,
                                             const float* xsum) {
    const int lane = threadIdx.x & 63;
    const int U = K / 32;
    float acc[1] = {0.f};
    for (int u = lane; u < U; u += 64) {
        const auto raw = load_unit<FMT>(W, N, K, n, u);
        if constexpr (FMT == FMT_F16) dot_unit_f16_swz<1>(raw, u, xs, K / 2, acc);
        else dot_unit<1>(raw, u, xs, K / 2, xsum, K / 16, acc);
    }
    return wave_sum(acc[0]);
}

__device__ __forceinline__ float row_dot(int type, const void* W, int64_t N, int K, int64_t n, const uint32_t* xs,
                                         const float* xsum) {
    switch (type) {
        case BX_TYPE_Q4_K: return row_dot_fmt<FMT_Q4_K>(W, N, K, n, xs, xsum);
        case BX_TYPE_Q6_K: return row_dot_fmt<FMT_Q6_K>(W, N, K, n, xs, xsum);
        case BX_TYPE_Q8_0: return row_dot_fmt<FMT_Q8_0>(W, N, K, n, xs, xsum);
        default: return row_dot_fmt<FMT_F16>(W, N, K, n, xs, xsum);
    }
}

struct Seg3 {
    const void* W[3];
    int type[3];
    int rows[3];
};

// ---- kernels ---------------------------------------------------------------

__global__ void embed_kernel(const uint16_t* __restrict__ E, const int32_t* __restrict__ tok, int H,
                             float* __restrict__ h) {
    const int64_t t = *tok;
    for (int i = blockIdx.x * blockDim.x + threadIdx.x; i < H; i += gridDim.x * blockDim.x) h[i] = h2f(E[t * H + i]);
}

// 1: rms_norm + [Wq; Wk; Wv] -> FP32 rows.
__global__ __launch_bounds__(kThreads) void norm_qkv_kernel(const float* __restrict__ h,
                                                            const uint16_t* __restrict__ gamma, float eps, int K,
                                                            Seg3 seg, float* __restrict__ out) {
    extern __shared__ __align__(16) uint32_t smem[];
    uint32_t* xs = smem;
    float* xsum = reinterpret_cast<float*>(smem + K / 2);
    float* red = xsum + K / 16;
    stage_norm(h, gamma, eps, K, xs, xsum, red);
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    const int N = seg.rows[0] + seg.rows[1] + seg.rows[2];
    for (int r = blockIdx.x * kWaves + wave; r < N; r += gridDim.x * kWaves) {
        int sgi = 0, n = r;
        if (n >= seg.rows[0]) { n -= seg.rows[0]; sgi = 1; if (n >= seg.rows[1]) { n -= seg.rows[1]; sgi = 2; } }
        const float v = row_dot(seg.type[sgi], seg.W[sgi], seg.rows[sgi], K, n, xs, xsum);
        if (lane == 0) out[r] = v;
    }
}

// 4 / 6: FP16 activation x, GEMV, residual add into h.
__global__ __launch_bounds__(kThreads) void gemv_resid_kernel(const uint16_t* __restrict__ x, int K, const void* W,
                                                              int type, int N, float* __restrict__ h) {
    extern __shared__ __align__(16) uint32_t smem[];
    uint32_t* xs = smem;
    float* xsum = reinterpret_cast<float*>(smem + K / 2);
    stage_f16(x, K, xs, xsum);
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    for (int r = blockIdx.x * kWaves + wave; r < N; r += gridDim.x * kWaves) {
        const float v = row_dot(type, W, N, K, r, xs, xsum);
        if (lane == 0) h[r] += v;
    }
}

// 5: rms_norm + gate/up rows of index n -> act[n] = fp16(silu(g) * u).
__global__ __launch_bounds__(kThreads) void norm_mlp_kernel(const float* __restrict__ h,
                                                            const uint16_t* __restrict__ gamma, float eps, int K,
                                                            const void* Wg, int tg, const void* Wu, int tu, int F,
                                                            uint16_t* __restrict__ act) {
    extern __shared__ __align__(16) uint32_t smem[];
    uint32_t* xs = smem;
    float* xsum = reinterpret_cast<float*>(smem + K / 2);
    float* red = xsum + K / 16;
    stage_norm(h, gamma, eps, K, xs, xsum, red);
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    for (int r = blockIdx.x * kWaves + wave; r < F; r += gridDim.x * kWaves) {
        const float g = row_dot(tg, Wg, F, K, r, xs, xsum);
        const float u = row_dot(tu, Wu, F, K, r, xs, xsum);
        if (lane == 0) act[r] = f2h(g / (1.0f + __expf(-g)) * u);
    }
}

// Final: rms_norm + lm_head rows -> FP16 logits.
__global__ __launch_bounds__(kThreads) void norm_head_kernel(const float* __restrict__ h,
                                                             const uint16_t* __restrict__ gamma, float eps, int K,
                                                             const void* W, int type, int N,
                                                             uint16_t* __restrict__ logits) {
    extern __shared__ __align__(16) uint32_t smem[];
    uint32_t* xs = smem;
    float* xsum = reinterpret_cast<float*>(smem + K / 2);
    float* red = xsum + K / 16;
    stage_norm(h, gamma, eps, K, xs, xsum, red);
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    for (int r = blockIdx.x * kWaves + wave; r < N; r += gridDim.x * kWaves) {
        const float v = row_dot(type, W, N, K, r, xs, xsum);
        if (lane == 0) logits[r] = f2h(v);
    }
}

// Per-head RMSNorm of a 'hd' FP32 vector into dst (LDS) using one wavefront,
// then the RoPE rotation at table row pos; round to FP16 precision when asked.
__device__ void head_norm_rope(const float* src, const uint16_t* gamma, float eps, int hd, const float* cos_row,
                               const float* sin_row, float* dst, bool round16, float post_scale) {
    const int lane = threadIdx.x & 63;
    float ss = 0.f;
    for (int d = lane; d < hd; d += 64) ss += src[d] * src[d];
    ss = wave_sum(ss);
    const float inv = 1.0f / sqrtf(ss / (float)hd + eps);
    for (int p = lane; p < hd / 2; p += 64) {
        float x0 = src[2 * p] * inv * h2f(gamma[2 * p]);
        float x1 = src[2 * p + 1] * inv * h2f(gamma[2 * p + 1]);
        if (round16) { x0 = h2f(f2h(x0)); x1 = h2f(f2h(x1)); }
        const float c = cos_row[p], s = sin_row[p];
        float y0 = x0 * c - x1 * s, y1 = x0 * s + x1 * c;
        if (round16) { y0 = h2f(f2h(y0)); y1 = h2f(f2h(y1)); }
        dst[2 * p] = y0 * post_scale;
        dst[2 * p + 1] = y1 * post_scale;
    }
}

// 2: attention partials for (split s, KV head g) at position *pos.
__global__ __launch_bounds__(kThreads) void attn_kernel(const float* __restrict__ qkv, const uint16_t* q_norm,
                                                        const uint16_t* k_norm, float eps, int n_q, int n_kv, int hd,
                                                        const int32_t* __restrict__ pos_dev,
                                                        const float* __restrict__ cos_t,
                                                        const float* __restrict__ sin_t, uint16_t* Kc, uint16_t* Vc,
                                                        int S, float* __restrict__ part) {
    extern __shared__ __align__(16) float sm[];
    const int s = blockIdx.x, g = blockIdx.y;
    const int G = n_q / n_kv;
    const int pos = *pos_dev;
    int kps = (pos + 1 + S - 1) / S;
    if (kps < kMinKeysPerSplit) kps = kMinKeysPerSplit;
    const int kb = s * kps, ke = min(pos + 1, (s + 1) * kps);
    float* qs = sm;                  // G * hd
    float* ck = qs + G * hd;         // hd
    float* cv = ck + hd;             // hd
    float* sc = cv + hd;             // G * 256
    float* red = sc + G * 256;       // 64
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    const int qd = n_q * hd, kvd = n_kv * hd;
    const float* cos_row = cos_t + (int64_t)pos * (hd / 2);
    const float* sin_row = sin_t + (int64_t)pos * (hd / 2);
    const float scale = 1.0f / sqrtf((float)hd);
    AttnArgs a{};
    a.Kc = Kc; a.Vc = Vc; a.mask = nullptr; a.L = 1; a.valid_len = pos + 1;
    a.n_q = n_q; a.n_kv = n_kv; a.hd = hd; a.softcap = 0.f; a.window = 0; a.kps = kps; a.S = S; a.ws = part;
    if (kb < ke) {
        // query heads of the group (wave w -> heads w, w+4, ...)
        for (int i = wave; i < G; i += kWaves)
            head_norm_rope(qkv + (int64_t)(g * G + i) * hd, q_norm, eps, hd, cos_row, sin_row, qs + i * hd, false,
                           scale);
        const bool has_cur = kb <= pos && pos < ke;
        if (has_cur && wave == 0) {
            head_norm_rope(qkv + qd + (int64_t)g * hd, k_norm, eps, hd, cos_row, sin_row, ck, true, 1.0f);
            for (int d = lane; d < hd; d += 64) cv[d] = h2f(f2h(qkv[qd + kvd + (int64_t)g * hd + d]));
        }
        __syncthreads();
        if (has_cur) {
            for (int d = threadIdx.x; d < hd; d += kThreads) {
                Kc[(int64_t)pos * kvd + (int64_t)g * hd + d] = f2h(ck[d]);
                Vc[(int64_t)pos * kvd + (int64_t)g * hd + d] = f2h(cv[d]);
            }
        }
        AttnState st;
        attn_state_init(st);
        attn_range(a, g, kb, ke, qs, sc, red, st, ck, cv, has_cur ? pos : -1);
        attn_write_partial(a, 0, g, s, st);
        attn_write_ml(a, 0, g, s, red);
    } else {
        // empty split: m = -inf, l = 0 (its o is never read)
        if (threadIdx.x < G) {
            float* rec = part + ((int64_t)(g * G + threadIdx.x) * S + s) * (hd + 2);
            rec[hd] = -INFINITY;
            rec[hd + 1] = 0.f;
        }
    }
}

// 3: merge the S partials of each query head -> FP16 attention output.
__global__ void combine_kernel(const float* __restrict__ part, int S, int hd, uint16_t* __restrict__ out) {
    const int h = blockIdx.x;
    const float* base = part + (int64_t)h * S * (hd + 2);
    float M = -INFINITY;
    for (int s = 0; s < S; ++s) M = fmaxf(M, base[(int64_t)s * (hd + 2) + hd]);
    float lsum = 0.f;
    for (int s = 0; s < S; ++s) {
        const float m = base[(int64_t)s * (hd + 2) + hd];
        if (m > -INFINITY) lsum += __expf(m - M) * base[(int64_t)s * (hd + 2) + hd + 1];
    }
    const float inv = lsum > 0.f ? 1.0f / lsum : 0.f;
    for (int d = threadIdx.x; d < hd; d += blockDim.x) {
        float o = 0.f;
        for (int s = 0; s < S; ++s) {
            const float m = base[(int64_t)s * (hd + 2) + hd];
            if (m > -INFINITY) o += __expf(m - M) * base[(int64_t)s * (hd + 2) + d];
        }
        out[(int64_t)h * hd + d] = f2h(o * inv);
    }
}

__global__ void advance_kernel(int32_t* tok, int32_t* pos, const int32_t* next, int32_t* hist, int32_t* count) {
    if (threadIdx.x == 0 && blockIdx.x == 0) {
        const int32_t n = *next;
        *tok = n;
        *pos = *pos + 1;
        if (hist) {
            const int32_t c = *count;
            hist[c] = n;
            *count = c + 1;
        }
    }
}

unsigned gemv_blocks(int64_t rows) {
    int64_t b = (rows + kWaves - 1) / kWaves;
    const int64_t cap = (int64_t)num_cus() * 8;
    if (b > cap) b = cap;
    return (unsigned)(b < 1 ? 1 : b);
}

size_t norm_lds(int K) { return (size_t)K * 2 + (size_t)(K / 16) * 4 + 64 * 4; }

bool quant_or_f16(int t) {
    return t == BX_TYPE_Q4_K || t == BX_TYPE_Q6_K || t == BX_TYPE_Q8_0 || t == BX_TYPE_F16;
}

int check_dims(const bx_decode_dims* d) {
    if (!d) return fail(BX_EINVAL, "decode: null dims");
    if (d->hidden <= 0 || d->hidden % 256 || d->intermediate <= 0 || d->intermediate % 256)
        return fail(BX_EUNSUPPORTED, "decode: hidden and intermediate must be multiples of 256");
    if (d->n_q <= 0 || d->n_kv <= 0 || d->n_q % d->n_kv || d->n_q / d->n_kv > kAttnMaxGroup)
        return fail(BX_EUNSUPPORTED, "decode: unsupported head counts");
    if (d->head_dim % 8 || d->head_dim > 256 || d->head_dim <= 0)
        return fail(BX_EUNSUPPORTED, "decode: head_dim must be a multiple of 8 and <= 256");
    if ((d->n_q * d->head_dim) % 256) return fail(BX_EUNSUPPORTED, "decode: n_q*head_dim must be a multiple of 256");
    if (d->cap <= 0 || d->vocab <= 0) return fail(BX_EINVAL, "decode: bad cap / vocab");
    const int ts[8] = {d->qkv_type_q, d->qkv_type_k, d->qkv_type_v, d->o_type,
                       d->gate_type, d->up_type, d->down_type, d->lm_type};
    for (int t : ts)
        if (!quant_or_f16(t)) return fail(BX_EUNSUPPORTED, "decode: unsupported weight type");
    if (norm_lds(d->intermediate) > 65536 || norm_lds(d->hidden) > 65536 ||
        norm_lds(d->n_q * d->head_dim) > 65536)
        return fail(BX_EUNSUPPORTED, "decode: activation too large for LDS staging");
    return BX_OK;
}

}  // namespace
}  // namespace bx

using namespace bx;

extern "C" {

size_t bx_decode_ws_bytes(const bx_decode_dims* d) {
    if (check_dims(d)) return 0;
    return ws_layout(*d).total;
}

int bx_decode_embed(const bx_decode_dims* d, const uint16_t* embed, const int32_t* tok_dev, void* ws, void* stream) {
    if (int rc = check_dims(d)) return rc;
    if (!embed || !tok_dev || !ws) return fail(BX_EINVAL, "decode_embed: null pointer");
    const WsLayout w = ws_layout(*d);
    float* h = reinterpret_cast<float*>(static_cast<char*>(ws) + w.h);
    embed_kernel<<<(d->hidden + 255) / 256, 256, 0, as_stream(stream)>>>(embed, tok_dev, d->hidden, h);
    return launch_check("decode_embed");
}

int bx_decode_layer_run(const bx_decode_dims* d, const bx_decode_layer* L, const int32_t* pos_dev,
                        const float* cos_tab, const float* sin_tab, void* ws, void* stream) {
    if (int rc = check_dims(d)) return rc;
    if (!L || !pos_dev || !cos_tab || !sin_tab || !ws) return fail(BX_EINVAL, "decode_layer: null pointer");
    const WsLayout w = ws_layout(*d);
    char* base = static_cast<char*>(ws);
    float* h = reinterpret_cast<float*>(base + w.h);
    float* qkv = reinterpret_cast<float*>(base + w.qkv);
    uint16_t* attn = reinterpret_cast<uint16_t*>(base + w.attn);
    uint16_t* act = reinterpret_cast<uint16_t*>(base + w.act);
    float* part = reinterpret_cast<float*>(base + w.part);
    const int H = d->hidden, F = d->intermediate, hd = d->head_dim;
    const int qd = d->n_q * hd, kvd = d->n_kv * hd;
    hipStream_t st = as_stream(stream);

    Seg3 seg{};
    seg.W[0] = L->Wq; seg.type[0] = d->qkv_type_q; seg.rows[0] = qd;
    seg.W[1] = L->Wk; seg.type[1] = d->qkv_type_k; seg.rows[1] = kvd;
    seg.W[2] = L->Wv; seg.type[2] = d->qkv_type_v; seg.rows[2] = kvd;
    norm_qkv_kernel<<<gemv_blocks(qd + 2 * kvd), kThreads, norm_lds(H), st>>>(
        h, static_cast<const uint16_t*>(L->in_ln), d->eps, H, seg, qkv);
    if (int rc = launch_check("decode norm_qkv")) return rc;

    const int G = d->n_q / d->n_kv;
    const size_t alds = (size_t)(G * hd + 2 * hd + G * 256 + 64) * sizeof(float);
    attn_kernel<<<dim3(w.S, d->n_kv), kThreads, alds, st>>>(
        qkv, static_cast<const uint16_t*>(L->q_norm), static_cast<const uint16_t*>(L->k_norm), d->eps, d->n_q,
        d->n_kv, hd, pos_dev, cos_tab, sin_tab, static_cast<uint16_t*>(L->Kc), static_cast<uint16_t*>(L->Vc), w.S,
        part);
    if (int rc = launch_check("decode attn")) return rc;
    combine_kernel<<<d->n_q, 128, 0, st>>>(part, w.S, hd, attn);
    if (int rc = launch_check("decode combine")) return rc;

    gemv_resid_kernel<<<gemv_blocks(H), kThreads, norm_lds(qd), st>>>(attn, qd, L->Wo, d->o_type, H, h);
    if (int rc = launch_check("decode o_proj")) return rc;

    norm_mlp_kernel<<<gemv_blocks(F), kThreads, norm_lds(H), st>>>(
        h, static_cast<const uint16_t*>(L->post_ln), d->eps, H, L->Wg, d->gate_type, L->Wu, d->up_type, F, act);
    if (int rc = launch_check("decode norm_mlp")) return rc;

    gemv_resid_kernel<<<gemv_blocks(H), kThreads, norm_lds(F), st>>>(act, F, L->Wd, d->down_type, H, h);
    return launch_check("decode down");
}

int bx_decode_head(const bx_decode_dims* d, const uint16_t* final_norm, const void* lm_head, uint16_t* logits,
                   void* ws, void* stream) {
    if (int rc = check_dims(d)) return rc;
    if (!final_norm || !lm_head || !logits || !ws) return fail(BX_EINVAL, "decode_head: null pointer");
    const WsLayout w = ws_layout(*d);
    const float* h = reinterpret_cast<const float*>(static_cast<char*>(ws) + w.h);
    norm_head_kernel<<<gemv_blocks(d->vocab), kThreads, norm_lds(d->hidden), as_stream(stream)>>>(
        h, final_norm, d->eps, d->hidden, lm_head, d->lm_type, d->vocab, logits);
    return launch_check("decode head");
}

int bx_decode_advance(int32_t* tok_dev, int32_t* pos_dev, const int32_t* next_dev, int32_t* hist, int32_t* count,
                      void* stream) {
    if (!tok_dev || !pos_dev || !next_dev || (hist == nullptr) != (count == nullptr))
        return fail(BX_EINVAL, "decode_advance: bad arguments");
    advance_kernel<<<1, 64, 0, as_stream(stream)>>>(tok_dev, pos_dev, next_dev, hist, count);
    return launch_check("decode_advance");
}

}  // extern "C"
