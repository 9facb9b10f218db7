// Fused single-token decode step: the captured graph body of
// src/detail/dense_decoder.cpp:439-496 (run_layers_ at L == 1, :526-681),
// restructured into six kernels per layer:
//
//   1 norm_qkv   rms_norm(h) in the prologue, GEMV over [Wq; Wk; Wv] (mixed
//                carrier formats by row segment), FP32 q/k/v out
//   2 attn       per (KV head, split): QK-norm + RoPE of q and k, KV-cache
//                write of position pos, split-K attention partials (K/V tiles
//                staged in LDS)
//   3 combine    merge splits -> FP16 attention output
//   4 o_proj     GEMV + residual add into the FP32 residual stream
//   5 norm_mlp   rms_norm(h) prologue, gate and up rows of the same index in
//                one wavefront, SwiGLU epilogue -> FP16 activation
//   6 down       GEMV + residual add
//
// GEMVs use the M = 1 core of gemv_core.h: activations staged once per block
// in LDS, then held in registers; each wavefront streams R weight rows at a
// time with all their 16-byte loads in flight.
//
// The token id and position are read from device memory (pos_dev, tok_dev),
// so one capture serves every step; the split count is fixed at capture time
// and the keys per split follow pos on the device.
#include <cmath>

#include "gemv_core.h"

namespace bx {

// One-row GEMV with K split over a workgroup's wavefronts (gemv.hip), here
// adding into the FP32 residual h.
int gemv_m1_ksplit(int wtype, const void* W, const uint16_t* X, const uint16_t* bias, uint16_t* Y, float* h, int N,
                   int K, hipStream_t st);

namespace {

constexpr int kThreads = 256;
constexpr int kWaves = kThreads / 64;
constexpr int kMinKeysPerSplit = 16;
constexpr int kMaxKeysPerSplit = 64;
constexpr int kMaxGroup = 8;

struct WsLayout {
    size_t h, qkv, attn, act, part, total;
    int S;
};

// Key splits per KV head: two workgroups per CU over the heads, at most the
// combine's 512.  The cache length does not enter: a split walks its keys in
// 64-key tiles.
int splits_for(const bx_decode_dims& d) {
    int S = (2 * num_cus()) / (d.n_kv > 0 ? d.n_kv : 1);
    return std::max(1, std::min(S, 512));
}

WsLayout ws_layout(const bx_decode_dims& d) {
    WsLayout w{};
    const int qd = d.n_q * d.head_dim, kvd = d.n_kv * d.head_dim;
    w.S = splits_for(d);
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
    w.part = take((size_t)d.n_q * w.S * (d.head_dim + 2) * 4);
    w.total = off;
    return w;
}

// ---- activation staging (swizzled FP16 pairs + 16-element sums in LDS) ----

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
    sums8_from_lds(xs, K, xsum);
    __syncthreads();
}

__device__ void stage_f16(const uint16_t* __restrict__ x, int K, uint32_t* xs, float* xsum) {
    for (int g = threadIdx.x; g < K / 4; g += kThreads) {
        const u2v v = *reinterpret_cast<const u2v*>(x + 4 * g);
        store_group<true>(xs, g, v.x & 0xffff, v.x >> 16, v.y & 0xffff, v.y >> 16);
    }
    __syncthreads();
    sums8_from_lds(xs, K, xsum);
    __syncthreads();
}

// Stream rows [0, N) of one matrix; epi(row, value) runs on lane 0.
template <int FMT, int UPL, class Epi>
__device__ __forceinline__ void stream_matrix(const void* W, int64_t N, int K, const uint32_t* xs, const float* xsum,
                                              int64_t task0, int64_t task_stride, Epi epi) {
    constexpr int R = RowsPer<UPL>::R;
    const int lane = threadIdx.x & 63;
    XCache<FMT, UPL> xu;
    xu.init(xs, xsum, K);
    const int64_t tasks = (N + R - 1) / R;
    for (int64_t t = task0; t < tasks; t += task_stride) {
        float o[R];
        rows_dot_m1<FMT, UPL, R>(W, N, K, t * R, xu, o);
        if (lane == 0) {
#pragma unroll
            for (int rr = 0; rr < R; ++rr)
                if (t * R + rr < N) epi(t * R + rr, o[rr]);
        }
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

// Each GEMV kernel is specialised on the weight format(s) and units per lane
// so the register budget is that of one path; waves_per_eu(4) caps it at 128.
#define BX_GEMV_BOUNDS __launch_bounds__(kThreads, 4)

// 1: rms_norm + [Wq; Wk; Wv] -> FP32 rows.  q and k share format FA, v has
// FB.  Wavefront tasks walk the segments in turn; a task streams R rows.
template <int FA, int FB, int UPL>
__global__ BX_GEMV_BOUNDS void norm_qkv_kernel(const float* __restrict__ h, const uint16_t* __restrict__ gamma,
                                               float eps, int K, Seg3 seg, float* __restrict__ out) {
    extern __shared__ __align__(16) uint32_t smem[];
    uint32_t* xs = smem;
    float* xsum = reinterpret_cast<float*>(smem + K / 2);
    float* red = xsum + K / 8;
    stage_norm(h, gamma, eps, K, xs, xsum, red);
    const int wave = threadIdx.x >> 6;
    const int64_t w0 = (int64_t)blockIdx.x * kWaves + wave, ws = (int64_t)gridDim.x * kWaves;
    constexpr int R = RowsPer<UPL>::R;
    int64_t base = 0, tbase = 0;
    for (int sg = 0; sg < 3; ++sg) {
        const int64_t N = seg.rows[sg];
        float* o = out + base;
        int64_t t0 = w0 - (tbase % ws);  // this wavefront's first task inside the segment
        if (t0 < 0) t0 += ws;
        if (sg < 2) stream_matrix<FA, UPL>(seg.W[sg], N, K, xs, xsum, t0, ws, [&](int64_t r, float v) { o[r] = v; });
        else stream_matrix<FB, UPL>(seg.W[sg], N, K, xs, xsum, t0, ws, [&](int64_t r, float v) { o[r] = v; });
        tbase += (N + R - 1) / R;
        base += N;
    }
}

// 4 / 6: FP16 activation x, GEMV, residual add into h.  The wide form (16
// units per lane, K up to 32768) gets 256 registers: its 80 KB of staged
// activations allow two workgroups per CU anyway.
template <int FMT, int UPL>
__global__ __launch_bounds__(kThreads, UPL > 6 ? 2 : 4) void gemv_resid_kernel(const uint16_t* __restrict__ x, int K, const void* W, int N,
                                                 float* __restrict__ h) {
    extern __shared__ __align__(16) uint32_t smem[];
    uint32_t* xs = smem;
    float* xsum = reinterpret_cast<float*>(smem + K / 2);
    stage_f16(x, K, xs, xsum);
    const int wave = threadIdx.x >> 6;
    const int64_t w0 = (int64_t)blockIdx.x * kWaves + wave, ws = (int64_t)gridDim.x * kWaves;
    stream_matrix<FMT, UPL>(W, N, K, xs, xsum, w0, ws, [&](int64_t r, float v) { h[r] += v; });
}

// 5: rms_norm + gate/up rows of index n -> act[n] = fp16(silu(g) * u).
template <int FMT, int UPL>
__global__ BX_GEMV_BOUNDS void norm_mlp_kernel(const float* __restrict__ h, const uint16_t* __restrict__ gamma,
                                               float eps, int K, const void* Wg, const void* Wu, int F,
                                               uint16_t* __restrict__ act) {
    extern __shared__ __align__(16) uint32_t smem[];
    uint32_t* xs = smem;
    float* xsum = reinterpret_cast<float*>(smem + K / 2);
    float* red = xsum + K / 8;
    stage_norm(h, gamma, eps, K, xs, xsum, red);
    constexpr int R = RowsPer<UPL>::R > 1 ? RowsPer<UPL>::R / 2 : 1;
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    const int64_t w0 = (int64_t)blockIdx.x * kWaves + wave, ws = (int64_t)gridDim.x * kWaves;
    XCache<FMT, UPL> xu;
    xu.init(xs, xsum, K);
    const int64_t tasks = (F + R - 1) / R;
    for (int64_t t = w0; t < tasks; t += ws) {
        float g[R], u[R];
        rows_dot_m1_pair<FMT, UPL, R>(Wg, Wu, F, K, t * R, xu, g, u);
        if (lane == 0) {
#pragma unroll
            for (int rr = 0; rr < R; ++rr) {
                const int64_t r = t * R + rr;
                if (r < F) act[r] = f2h(g[rr] / (1.0f + __expf(-g[rr])) * u[rr]);
            }
        }
    }
}

// Final: rms_norm + lm_head rows -> FP16 logits.
template <int FMT, int UPL>
__global__ BX_GEMV_BOUNDS void norm_head_kernel(const float* __restrict__ h, const uint16_t* __restrict__ gamma,
                                                float eps, int K, const void* W, int N,
                                                uint16_t* __restrict__ logits) {
    extern __shared__ __align__(16) uint32_t smem[];
    uint32_t* xs = smem;
    float* xsum = reinterpret_cast<float*>(smem + K / 2);
    float* red = xsum + K / 8;
    stage_norm(h, gamma, eps, K, xs, xsum, red);
    const int wave = threadIdx.x >> 6;
    const int64_t w0 = (int64_t)blockIdx.x * kWaves + wave, ws = (int64_t)gridDim.x * kWaves;
    stream_matrix<FMT, UPL>(W, N, K, xs, xsum, w0, ws, [&](int64_t r, float v) { logits[r] = f2h(v); });
}

// Per-head RMSNorm of an hd-long FP32 vector (one wavefront), RoPE at the
// table row, optional FP16 rounding (the value the cache will hold), scale.
// gamma == nullptr: no norm; the head is the projection output rounded to
// FP16 (the op path stores q and k in FP16 before RoPE).
__device__ void head_norm_rope(const float* src, const uint16_t* gamma, float eps, int hd, const float* cos_row,
                               const float* sin_row, float* dst, bool round16, float post_scale) {
    const int lane = threadIdx.x & 63;
    float inv = 1.0f;
    if (gamma) {
        float ss = 0.f;
        for (int d = lane; d < hd; d += 64) ss += src[d] * src[d];
        ss = wave_allsum(ss);
        inv = 1.0f / sqrtf(ss / (float)hd + eps);
    }
    for (int p = lane; p < hd / 2; p += 64) {
        float x0, x1;
        if (gamma) {
            x0 = src[2 * p] * inv * h2f(gamma[2 * p]);
            x1 = src[2 * p + 1] * inv * h2f(gamma[2 * p + 1]);
        } else {
            x0 = h2f(f2h(src[2 * p]));
            x1 = h2f(f2h(src[2 * p + 1]));
        }
        if (round16) { x0 = h2f(f2h(x0)); x1 = h2f(f2h(x1)); }
        const float c = cos_row[p], s = sin_row[p];
        float y0 = x0 * c - x1 * s, y1 = x0 * s + x1 * c;
        if (round16) { y0 = h2f(f2h(y0)); y1 = h2f(f2h(y1)); }
        dst[2 * p] = y0 * post_scale;
        dst[2 * p + 1] = y1 * post_scale;
    }
}

// 2: attention partials for (split s, KV head g) at position *pos.  The
// split's keys go through LDS in tiles of kMaxKeysPerSplit, with a running
// maximum and sum per query head (a tile's probabilities are taken against
// the running maximum, and what came before is rescaled when it grows), so
// the number of splits does not depend on the cache length.  A split of one
// tile computes exactly what a single pass would.
// LDS: q[G][hd] f32 | kt[64][hd+8] f16 | vt[64][hd] f16 | p[G][64] f32 |
// current k, v [hd] f32 each | rescale factors [G] f32.
template <int HD>
__global__ __launch_bounds__(kThreads) void attn_kernel(const float* __restrict__ qkv, const uint16_t* q_norm,
                                                        const uint16_t* k_norm, float eps, int n_q, int n_kv, int,
                                                        const int32_t* __restrict__ pos_dev,
                                                        const float* __restrict__ cos_t,
                                                        const float* __restrict__ sin_t, uint16_t* Kc, uint16_t* Vc,
                                                        int S, float* __restrict__ part) {
    extern __shared__ __align__(16) float sm[];
    constexpr int hd = HD;
    constexpr int kTileKeys = kMaxKeysPerSplit;
    constexpr int kHeadsPerWave = (kMaxGroup + kWaves - 1) / kWaves;
    constexpr int kPairsPerThread = (kMaxGroup * HD / 2 + kThreads - 1) / kThreads;
    const int s = blockIdx.x, g = blockIdx.y;
    const int G = n_q / n_kv;
    const int pos = *pos_dev;
    int kps = (pos + 1 + S - 1) / S;
    if (kps < kMinKeysPerSplit) kps = kMinKeysPerSplit;
    const int kb = (int)min((int64_t)s * kps, (int64_t)pos + 1), ke = min(pos + 1, kb + kps);
    const int nk = ke - kb;
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    const int qd = n_q * hd, kvd = n_kv * hd;
    if (nk <= 0) {  // empty split: a zero record the combine can read without branching
        for (int i = threadIdx.x; i < G * (hd + 2); i += kThreads) {
            const int h = i / (hd + 2), e = i % (hd + 2);
            part[((int64_t)(g * G + h) * S + s) * (hd + 2) + e] = e == hd ? -INFINITY : 0.f;
        }
        return;
    }
    const int kstride = hd + 8;  // halves per K row in LDS (padding against bank conflicts)
    float* qs = sm;
    uint16_t* kt = reinterpret_cast<uint16_t*>(qs + G * hd);
    uint16_t* vt = kt + kTileKeys * kstride;
    float* pr = reinterpret_cast<float*>(vt + kTileKeys * hd);
    float* ck = pr + G * kTileKeys;
    float* cv = ck + hd;
    float* alpha = cv + hd;

    // K/V of keys [c0, c0 + cn) of the split into registers (16 bytes per
    // thread per step)
    constexpr int kMaxChunks = kTileKeys * HD / 8 / kThreads;
    u4v kreg[kMaxChunks], vreg[kMaxChunks];
    auto load_tile = [&](int c0, int cn) {
#pragma unroll
        for (int i = 0; i < kMaxChunks; ++i) {
            const int c = threadIdx.x + i * kThreads;
            if (c < cn * (hd / 8)) {
                const int j = c / (hd / 8), d8 = c % (hd / 8);
                const int64_t off = (int64_t)(kb + c0 + j) * kvd + (int64_t)g * hd + 8 * d8;
                kreg[i] = ldg16(Kc + off);
                vreg[i] = ldg16(Vc + off);
            }
        }
    };
    auto store_tile = [&](int cn) {
#pragma unroll
        for (int i = 0; i < kMaxChunks; ++i) {
            const int c = threadIdx.x + i * kThreads;
            if (c < cn * (hd / 8)) {
                const int j = c / (hd / 8), d8 = c % (hd / 8);
                *reinterpret_cast<u4v*>(kt + j * kstride + 8 * d8) = kreg[i];
                *reinterpret_cast<u4v*>(vt + j * hd + 8 * d8) = vreg[i];
            }
        }
    };

    // the first tile's loads are in flight while q (and the current key) are formed
    load_tile(0, min(nk, kTileKeys));
    const float* cos_row = cos_t + (int64_t)pos * (hd / 2);
    const float* sin_row = sin_t + (int64_t)pos * (hd / 2);
    const float scale = 1.0f / sqrtf((float)hd);
    for (int i = wave; i < G; i += kWaves)
        head_norm_rope(qkv + (int64_t)(g * G + i) * hd, q_norm, eps, hd, cos_row, sin_row, qs + i * hd, false,
                       scale);
    const bool has_cur = pos < ke;  // key pos is the last key of this split
    if (has_cur && wave == kWaves - 1) {
        head_norm_rope(qkv + qd + (int64_t)g * hd, k_norm, eps, hd, cos_row, sin_row, ck, true, 1.0f);
        for (int d = lane; d < hd; d += 64) cv[d] = h2f(f2h(qkv[qd + kvd + (int64_t)g * hd + d]));
    }

    // running maximum and sum of the heads this wave scores (h = wave + kWaves i),
    // unnormalized outputs of the (head, dim pair)s this thread owns
    float m_run[kHeadsPerWave], l_run[kHeadsPerWave];
#pragma unroll
    for (int i = 0; i < kHeadsPerWave; ++i) {
        m_run[i] = -INFINITY;
        l_run[i] = 0.f;
    }
    float o0[kPairsPerThread], o1[kPairsPerThread];
#pragma unroll
    for (int k = 0; k < kPairsPerThread; ++k) o0[k] = o1[k] = 0.f;

    for (int c0 = 0; c0 < nk; c0 += kTileKeys) {
        const int cn = min(kTileKeys, nk - c0);
        if (c0 > 0) {
            load_tile(c0, cn);
            __syncthreads();  // the previous tile's readers are done
        }
        store_tile(cn);
        __syncthreads();
        if (has_cur && c0 + cn == nk) {
            // the current key/value replace the (stale) cache row in the tile and go to the cache
            for (int d = threadIdx.x; d < hd; d += kThreads) {
                const uint16_t kh = f2h(ck[d]), vh = f2h(cv[d]);
                kt[(cn - 1) * kstride + d] = kh;
                vt[(cn - 1) * hd + d] = vh;
                Kc[(int64_t)pos * kvd + (int64_t)g * hd + d] = kh;
                Vc[(int64_t)pos * kvd + (int64_t)g * hd + d] = vh;
            }
            __syncthreads();
        }
        // scores: wave h handles query head h, lane j handles key j
#pragma unroll
        for (int i = 0; i < kHeadsPerWave; ++i) {
            const int h = wave + kWaves * i;
            if (h >= G) break;
            float sc = -INFINITY;
            if (lane < cn) {
                const float* q = qs + h * hd;
                const uint16_t* kr = kt + lane * kstride;
                float a = 0.f;
                for (int d = 0; d < hd; d += 8) {
                    const u4v kv = *reinterpret_cast<const u4v*>(kr + d);
                    const float4 q0 = *reinterpret_cast<const float4*>(q + d);
                    const float4 q1 = *reinterpret_cast<const float4*>(q + d + 4);
                    a += q0.x * h2f(kv.x & 0xffff) + q0.y * h2f(kv.x >> 16) + q0.z * h2f(kv.y & 0xffff) +
                         q0.w * h2f(kv.y >> 16) + q1.x * h2f(kv.z & 0xffff) + q1.y * h2f(kv.z >> 16) +
                         q1.z * h2f(kv.w & 0xffff) + q1.w * h2f(kv.w >> 16);
                }
                sc = a;
            }
            const float m = fmaxf(m_run[i], wave_max(sc));
            const float al = m_run[i] == -INFINITY ? 0.f : __expf(m_run[i] - m);
            const float p = lane < cn ? __expf(sc - m) : 0.f;
            l_run[i] = l_run[i] * al + wave_allsum(p);
            m_run[i] = m;
            pr[h * kTileKeys + lane] = p;
            if (lane == 0) alpha[h] = al;
        }
        __syncthreads();
        // o[h][d] = alpha[h] o[h][d] + sum_j p[h][j] * V[j][d]; thread -> (h, dim pair)
#pragma unroll
        for (int k = 0; k < kPairsPerThread; ++k) {
            const int idx = threadIdx.x + k * kThreads;
            if (idx >= G * (hd / 2)) break;
            const int h = idx / (hd / 2), dp = idx % (hd / 2);
            const float* p = pr + h * kTileKeys;
            float a0 = 0.f, a1 = 0.f;
            for (int j = 0; j < cn; ++j) {
                const uint32_t v = *reinterpret_cast<const uint32_t*>(vt + j * hd + 2 * dp);
                a0 += p[j] * h2f(v & 0xffff);
                a1 += p[j] * h2f(v >> 16);
            }
            o0[k] = o0[k] * alpha[h] + a0;
            o1[k] = o1[k] * alpha[h] + a1;
        }
    }
    // the record of each head: o (unnormalized), m, l
#pragma unroll
    for (int k = 0; k < kPairsPerThread; ++k) {
        const int idx = threadIdx.x + k * kThreads;
        if (idx >= G * (hd / 2)) break;
        const int h = idx / (hd / 2), dp = idx % (hd / 2);
        float* rec = part + ((int64_t)(g * G + h) * S + s) * (hd + 2);
        rec[2 * dp] = o0[k];
        rec[2 * dp + 1] = o1[k];
    }
    if (lane == 0) {
#pragma unroll
        for (int i = 0; i < kHeadsPerWave; ++i) {
            const int h = wave + kWaves * i;
            if (h >= G) break;
            float* rec = part + ((int64_t)(g * G + h) * S + s) * (hd + 2);
            rec[hd] = m_run[i];
            rec[hd + 1] = l_run[i];
        }
    }
}

// 3: merge the S partials of each query head -> FP16 attention output.
__global__ __launch_bounds__(128) void combine_kernel(const float* __restrict__ part, int S, int hd,
                                                     uint16_t* __restrict__ out) {
    __shared__ float w[512];
    __shared__ float red[2];
    const int h = blockIdx.x;
    const float* base = part + (int64_t)h * S * (hd + 2);
    float mloc = -INFINITY;
    for (int s = threadIdx.x; s < S; s += blockDim.x) mloc = fmaxf(mloc, base[(int64_t)s * (hd + 2) + hd]);
    mloc = wave_max(mloc);
    if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = mloc;
    __syncthreads();
    const float M = fmaxf(red[0], red[1]);
    float lloc = 0.f;
    for (int s = threadIdx.x; s < S; s += blockDim.x) {
        const float m = base[(int64_t)s * (hd + 2) + hd];
        const float ws = m > -INFINITY ? __expf(m - M) : 0.f;
        w[s] = ws;
        lloc += ws * base[(int64_t)s * (hd + 2) + hd + 1];
    }
    lloc = wave_allsum(lloc);
    __syncthreads();
    if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = lloc;
    __syncthreads();
    const float lsum = red[0] + red[1];
    const float inv = lsum > 0.f ? 1.0f / lsum : 0.f;
    for (int d = threadIdx.x; d < hd; d += blockDim.x) {
        // branch-free so the loads of consecutive splits are issued back to back
        float o0 = 0.f, o1 = 0.f, o2 = 0.f, o3 = 0.f;
        int s = 0;
        for (; s + 4 <= S; s += 4) {
            const float v0 = base[(int64_t)s * (hd + 2) + d], v1 = base[(int64_t)(s + 1) * (hd + 2) + d];
            const float v2 = base[(int64_t)(s + 2) * (hd + 2) + d], v3 = base[(int64_t)(s + 3) * (hd + 2) + d];
            o0 += w[s] * v0;
            o1 += w[s + 1] * v1;
            o2 += w[s + 2] * v2;
            o3 += w[s + 3] * v3;
        }
        for (; s < S; ++s) o0 += w[s] * base[(int64_t)s * (hd + 2) + d];
        out[(int64_t)h * hd + d] = f2h((o0 + o1 + o2 + o3) * inv);
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

unsigned gemv_blocks(int64_t rows, int K) {
    const int upl = upl_for(K);
    const int R = upl == 1 ? 4 : (upl == 2 ? 2 : 1);
    int64_t b = (rows + (int64_t)kWaves * R - 1) / ((int64_t)kWaves * R);
    const int64_t cap = (int64_t)num_cus() * 8;
    if (b > cap) b = cap;
    return (unsigned)(b < 1 ? 1 : b);
}

// Workgroups of a kernel that normalizes its input itself (q / k / v and
// gate / up): every workgroup stages and normalizes the whole residual before
// its rows, so at most 4 workgroups per CU, each taking more rows (measured at
// H 4096 and 5120: +7 % and +8 % a step; at H 2048 the cap does not bind).
unsigned norm_blocks(int64_t rows, int K) {
    return std::min<unsigned>(gemv_blocks(rows, K), (unsigned)num_cus() * 4);
}

size_t norm_lds(int K) { return (size_t)K * 2 + (size_t)(K / 8) * 4 + 64 * 4; }

size_t attn_lds(int G, int hd) {
    return (size_t)G * hd * 4 + (size_t)kMaxKeysPerSplit * (hd + 8) * 2 + (size_t)kMaxKeysPerSplit * hd * 2 +
           (size_t)G * kMaxKeysPerSplit * 4 + (size_t)2 * hd * 4 + (size_t)G * 4 + 256;
}

bool known_type(int t) {
    return t == BX_TYPE_Q4_K || t == BX_TYPE_Q6_K || t == BX_TYPE_Q8_0 || t == BX_TYPE_F16;
}

int check_dims(const bx_decode_dims* d) {
    if (!d) return fail(BX_EINVAL, "decode: null dims");
    if (d->hidden <= 0 || d->hidden % 256 || d->intermediate <= 0 || d->intermediate % 256)
        return fail(BX_EUNSUPPORTED, "decode: hidden and intermediate must be multiples of 256");
    // the intermediate width is K only of the down projection (wide dispatch)
    if (d->hidden > 12288 || d->intermediate > 32768 || d->n_q * d->head_dim > 12288)
        return fail(BX_EUNSUPPORTED, "decode: hidden or n_q*head_dim above 12288, or intermediate above 32768");
    if (d->n_q <= 0 || d->n_kv <= 0 || d->n_q % d->n_kv || d->n_q / d->n_kv > kMaxGroup)
        return fail(BX_EUNSUPPORTED, "decode: unsupported head counts");
    if (d->head_dim % 8 || d->head_dim > 256 || d->head_dim <= 0)
        return fail(BX_EUNSUPPORTED, "decode: head_dim must be a multiple of 8 and <= 256");
    if ((d->n_q * d->head_dim) % 256) return fail(BX_EUNSUPPORTED, "decode: n_q*head_dim must be a multiple of 256");
    if (d->cap <= 0 || d->vocab <= 0) return fail(BX_EINVAL, "decode: bad cap / vocab");
    const int ts[8] = {d->qkv_type_q, d->qkv_type_k, d->qkv_type_v, d->o_type,
                       d->gate_type, d->up_type, d->down_type, d->lm_type};
    for (int t : ts)
        if (!known_type(t)) return fail(BX_EUNSUPPORTED, "decode: unsupported weight type");
    if (d->gate_type != d->up_type) return fail(BX_EUNSUPPORTED, "decode: gate and up must share a type");
    if (d->qkv_type_q != d->qkv_type_k) return fail(BX_EUNSUPPORTED, "decode: q and k must share a type");
    if (d->head_dim != 64 && d->head_dim != 128 && d->head_dim != 256)
        return fail(BX_EUNSUPPORTED, "decode: head_dim must be 64, 128 or 256");
    if (attn_lds(d->n_q / d->n_kv, d->head_dim) > 65536)
        return fail(BX_EUNSUPPORTED, "decode: attention tile too large for LDS");
    return BX_OK;
}

// ---- host-side specialisation dispatch ------------------------------------

template <int FA, int FB>
int launch_qkv_ab(int upl, unsigned blocks, size_t lds, hipStream_t st, const float* h, const uint16_t* g, float eps,
                  int K, Seg3 seg, float* out) {
    BX_DISPATCH_UPL(upl, (norm_qkv_kernel<FA, FB, UPL_><<<blocks, kThreads, lds, st>>>(h, g, eps, K, seg, out)));
    return launch_check("decode norm_qkv");
}
template <int FA>
int launch_qkv_a(int tb, int upl, unsigned blocks, size_t lds, hipStream_t st, const float* h, const uint16_t* g,
                 float eps, int K, Seg3 seg, float* out) {
    switch (tb) {
        case BX_TYPE_Q4_K: return launch_qkv_ab<FA, FMT_Q4_K>(upl, blocks, lds, st, h, g, eps, K, seg, out);
        case BX_TYPE_Q6_K: return launch_qkv_ab<FA, FMT_Q6_K>(upl, blocks, lds, st, h, g, eps, K, seg, out);
        case BX_TYPE_Q8_0: return launch_qkv_ab<FA, FMT_Q8_0>(upl, blocks, lds, st, h, g, eps, K, seg, out);
        default: return launch_qkv_ab<FA, FMT_F16>(upl, blocks, lds, st, h, g, eps, K, seg, out);
    }
}
int launch_qkv(int ta, int tb, int upl, unsigned blocks, size_t lds, hipStream_t st, const float* h,
               const uint16_t* g, float eps, int K, Seg3 seg, float* out) {
    switch (ta) {
        case BX_TYPE_Q4_K: return launch_qkv_a<FMT_Q4_K>(tb, upl, blocks, lds, st, h, g, eps, K, seg, out);
        case BX_TYPE_Q6_K: return launch_qkv_a<FMT_Q6_K>(tb, upl, blocks, lds, st, h, g, eps, K, seg, out);
        case BX_TYPE_Q8_0: return launch_qkv_a<FMT_Q8_0>(tb, upl, blocks, lds, st, h, g, eps, K, seg, out);
        default: return launch_qkv_a<FMT_F16>(tb, upl, blocks, lds, st, h, g, eps, K, seg, out);
    }
}
int launch_resid(int type, int upl, unsigned blocks, size_t lds, hipStream_t st, const uint16_t* x, int K,
                 const void* W, int N, float* h) {
    // FFN widths of 24576 / 32768: K split over each workgroup's wavefronts
    if (K % 8192 == 0 && K > 16384) return gemv_m1_ksplit(type, W, x, nullptr, nullptr, h, N, K, st);
    BX_DISPATCH_FMT(type, BX_DISPATCH_UPL_WIDE(upl, {
        const void* fn = reinterpret_cast<const void*>(&gemv_resid_kernel<FMT_, UPL_>);
        if (lds > 65536) {   // the down projection of FFN widths above 26112
            if (int rc = hip_check(hipFuncSetAttribute(fn, hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds),
                                   "decode gemv_resid: LDS attribute"))
                return rc;
        }
        // wide rows: one round of resident workgroups, each staging its
        // activations once for many rows (a fixed count: this launch is
        // recorded into the step graph)
        unsigned b = blocks;
        if (UPL_ > 6) b = (unsigned)std::min<int64_t>(b, (int64_t)num_cus() * BX_WIDE_WGS_PER_CU);
        gemv_resid_kernel<FMT_, UPL_><<<b, kThreads, lds, st>>>(x, K, W, N, h);
    }));
    return launch_check("decode gemv_resid");
}
int launch_mlp(int type, int upl, unsigned blocks, size_t lds, hipStream_t st, const float* h, const uint16_t* g,
               float eps, int K, const void* Wg, const void* Wu, int F, uint16_t* act) {
    BX_DISPATCH_FMT(type, BX_DISPATCH_UPL(upl, (norm_mlp_kernel<FMT_, UPL_><<<blocks, kThreads, lds, st>>>(
                                                   h, g, eps, K, Wg, Wu, F, act))));
    return launch_check("decode norm_mlp");
}
int launch_head(int type, int upl, unsigned blocks, size_t lds, hipStream_t st, const float* h, const uint16_t* g,
                float eps, int K, const void* W, int N, uint16_t* logits) {
    BX_DISPATCH_FMT(type, BX_DISPATCH_UPL(upl, (norm_head_kernel<FMT_, UPL_><<<blocks, kThreads, lds, st>>>(
                                                   h, g, eps, K, W, N, logits))));
    return launch_check("decode head");
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

    // this layer's own matrix types (a mixed file differs per layer)
    const int lts[7] = {L->type_q, L->type_k, L->type_v, L->type_o, L->type_gate, L->type_up, L->type_down};
    for (int t : lts)
        if (!known_type(t)) return fail(BX_EUNSUPPORTED, "decode_layer: unsupported weight type");
    if (L->type_q != L->type_k || L->type_gate != L->type_up)
        return fail(BX_EUNSUPPORTED, "decode_layer: q/k or gate/up types differ");
    Seg3 seg{};
    seg.W[0] = L->Wq; seg.type[0] = L->type_q; seg.rows[0] = qd;
    seg.W[1] = L->Wk; seg.type[1] = L->type_k; seg.rows[1] = kvd;
    seg.W[2] = L->Wv; seg.type[2] = L->type_v; seg.rows[2] = kvd;
    if (int rc = launch_qkv(L->type_q, L->type_v, upl_for(H), norm_blocks(qd + 2 * kvd, H), norm_lds(H), st,
                            h, static_cast<const uint16_t*>(L->in_ln), d->eps, H, seg, qkv))
        return rc;

    const int G = d->n_q / d->n_kv;
    const dim3 agrid(w.S, d->n_kv);
    const size_t alds = attn_lds(G, hd);
    const auto* qn = d->no_qk_norm ? nullptr : static_cast<const uint16_t*>(L->q_norm);
    const auto* kn = d->no_qk_norm ? nullptr : static_cast<const uint16_t*>(L->k_norm);
    auto* Kc = static_cast<uint16_t*>(L->Kc);
    auto* Vc = static_cast<uint16_t*>(L->Vc);
    if (hd == 64)
        attn_kernel<64><<<agrid, kThreads, alds, st>>>(qkv, qn, kn, d->eps, d->n_q, d->n_kv, hd, pos_dev, cos_tab,
                                                       sin_tab, Kc, Vc, w.S, part);
    else if (hd == 128)
        attn_kernel<128><<<agrid, kThreads, alds, st>>>(qkv, qn, kn, d->eps, d->n_q, d->n_kv, hd, pos_dev, cos_tab,
                                                        sin_tab, Kc, Vc, w.S, part);
    else
        attn_kernel<256><<<agrid, kThreads, alds, st>>>(qkv, qn, kn, d->eps, d->n_q, d->n_kv, hd, pos_dev, cos_tab,
                                                        sin_tab, Kc, Vc, w.S, part);
    if (int rc = launch_check("decode attn")) return rc;
    combine_kernel<<<d->n_q, 128, 0, st>>>(part, w.S, hd, attn);
    if (int rc = launch_check("decode combine")) return rc;

    if (int rc = launch_resid(L->type_o, upl_for(qd), gemv_blocks(H, qd), norm_lds(qd), st, attn, qd, L->Wo, H, h))
        return rc;
    if (int rc = launch_mlp(L->type_gate, upl_for(H), norm_blocks(2 * F, H), norm_lds(H), st, h,
                            static_cast<const uint16_t*>(L->post_ln), d->eps, H, L->Wg, L->Wu, F, act))
        return rc;
    return launch_resid(L->type_down, upl_for(F), gemv_blocks(H, F), norm_lds(F), st, act, F, L->Wd, H, h);
}

int bx_decode_head(const bx_decode_dims* d, const uint16_t* final_norm, const void* lm_head, uint16_t* logits,
                   void* ws, void* stream) {
    if (int rc = check_dims(d)) return rc;
    if (!final_norm || !lm_head || !logits || !ws) return fail(BX_EINVAL, "decode_head: null pointer");
    const WsLayout w = ws_layout(*d);
    const float* h = reinterpret_cast<const float*>(static_cast<char*>(ws) + w.h);
    return launch_head(d->lm_type, upl_for(d->hidden), gemv_blocks(d->vocab, d->hidden), norm_lds(d->hidden),
                       as_stream(stream), h, final_norm, d->eps, d->hidden, lm_head, d->vocab, logits);
}

int bx_decode_advance(int32_t* tok_dev, int32_t* pos_dev, const int32_t* next_dev, int32_t* hist, int32_t* count,
                      void* stream) {
    if (!tok_dev || !pos_dev || !next_dev || (hist == nullptr) != (count == nullptr))
        return fail(BX_EINVAL, "decode_advance: bad arguments");
    advance_kernel<<<1, 64, 0, as_stream(stream)>>>(tok_dev, pos_dev, next_dev, hist, count);
    return launch_check("decode_advance");
}

}  // extern "C"
