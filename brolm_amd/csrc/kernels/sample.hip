// Device top-k / top-p sampling over FP16 logits (reference
// src/detail/generate.cpp:68-142, sample_token).  The reference sorts all V
// probabilities on the host; here one workgroup finds the same thresholds by
// bisection on the probability value, so nothing is sorted and only the
// chosen id leaves the device (the bisection runs over the few candidates a
// histogram pass leaves when top-k or top-p cut the set, see below):
//   p_i   = fp32(exp(l_i / T - max)) * fp32(1 / sum)  (sum in FP64), as the reference;
//   M(v)  = sum of p_i >= v (FP64), C(v) = count of p_i >= v;
//   top-k level  v_k = largest v with C(v) >= k   (k-th largest p);
//   top-p level  v_p = largest v with M'(v) >= top_p, M' over p >= v_k
//                (the nucleus ends at the token whose running sum crosses top_p);
//   kept = p >= max(v_k, v_p); r = u * M(kept);
//   token = the lowest index whose p is the largest level w with M'(w) > r.
// The host draws u from the caller's std::mt19937_64 exactly as the reference
// does (one uniform_real_distribution<double>(0, 1) per sampled token).
// Ties: tokens of equal probability at a top-k boundary are all kept, and
// within a level the lowest index is chosen, where the reference's std::sort
// leaves the order of equal probabilities unspecified.
#include <cmath>

#include "common.h"

namespace bx {
namespace {

constexpr int kST = 1024;

__device__ double block_sum_d(double v, double* red) {
    const int t = threadIdx.x;
    red[t] = v;
    __syncthreads();
    for (int s = kST / 2; s > 0; s >>= 1) {
        if (t < s) red[t] += red[t + s];
        __syncthreads();
    }
    const double r = red[0];
    __syncthreads();
    return r;
}

__device__ float block_max_f(float v, float* red) {
    const int t = threadIdx.x;
    red[t] = v;
    __syncthreads();
    for (int s = kST / 2; s > 0; s >>= 1) {
        if (t < s) red[t] = fmaxf(red[t], red[t + s]);
        __syncthreads();
    }
    const float r = red[0];
    __syncthreads();
    return r;
}

__device__ __forceinline__ double wave_sum_d(double v) {
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o);
    return v;
}

// Both sums over the workgroup in a fixed order (lanes by butterfly, then
// the 16 wave partials by every wave alike): one barrier per pass.
__device__ void block_sum2(double& a, double& b, double* red) {
    a = wave_sum_d(a);
    b = wave_sum_d(b);
    const int w = threadIdx.x >> 6, l = threadIdx.x & 63;
    if (l == 0) {
        red[w] = a;
        red[kST / 64 + w] = b;
    }
    __syncthreads();
    double x = l < kST / 64 ? red[l] : 0.0, y = l < kST / 64 ? red[kST / 64 + l] : 0.0;
    a = wave_sum_d(x);
    b = wave_sum_d(y);
    __syncthreads();
}

// The FP64 sums of a pass: NT = kST, the whole workgroup (block_sum2); NT =
// 64, wavefront 0 alone (butterfly shuffles, no barrier).
template <int NT>
__device__ __forceinline__ void sum2(double& a, double& b, double* red) {
    if constexpr (NT == kST) {
        block_sum2(a, b, red);
    } else {
        a = wave_sum_d(a);
        b = wave_sum_d(b);
    }
}

// Mass (FP64) and count of p_i >= v among p_i >= floor_v, over n values.
template <int NT>
__device__ void mass_at(const float* p, int n, float v, float floor_v, double* red, double& mass, double& cnt) {
    double m = 0.0, c = 0.0;
    const float lo = fmaxf(v, floor_v);
    for (int i = threadIdx.x; i < n; i += NT) {
        const float x = p[i];
        if (x >= lo) {
            m += x;
            c += 1.0;
        }
    }
    sum2<NT>(m, c, red);
    mass = m;
    cnt = c;
}

// The id drawn from n probabilities pp (ic maps a position to its id, or null
// for the identity), NT threads taking part; -1 when no mass is kept.
template <int NT>
__device__ int select_token(const float* pp, const int* ic, int n, int V, int top_k, float top_p, double u,
                            double* red, int* cnt) {
    // bisection over the bit patterns of non-negative floats: lo satisfies the
    // predicate, hi does not
    auto search = [&](float floor_v, auto pred) {
        uint32_t lo = 0, hi = 0x3f800001u;   // p <= 1
        while (hi - lo > 1) {
            const uint32_t mid = lo + (hi - lo) / 2;
            double m, c;
            mass_at<NT>(pp, n, __uint_as_float(mid), floor_v, red, m, c);
            if (pred(m, c)) lo = mid;
            else hi = mid;
        }
        return __uint_as_float(lo);
    };
    auto above = [&](float v, double& m, double& c) {   // mass / count of p > v
        mass_at<NT>(pp, n, __uint_as_float(__float_as_uint(v) + 1u), 0.0f, red, m, c);
    };
    double m, c, mg, cg;
    // top-k: the k-th largest probability; the reference keeps exactly k ids,
    // so of the ids tied at that level only k - (ids above) count
    float vk = 0.0f;
    double take_k = -1.0;
    if (top_k > 0 && top_k < V) {
        vk = search(0.0f, [&](double, double cc) { return cc >= (double)top_k; });
        above(vk, mg, cg);
        take_k = (double)top_k - cg;
    }
    // kept mass before top-p: the ids above vk plus take_k of those at vk
    mass_at<NT>(pp, n, vk, vk, red, m, c);
    above(vk, mg, cg);
    const double kept_k = take_k < 0.0 ? m : mg + take_k * (double)vk;
    float vf = vk;          // the lowest kept level
    double take = take_k;   // ids kept at vf (-1: all of them)
    if (top_p < 1.0f && kept_k >= (double)top_p) {
        // the nucleus ends at the id whose running sum reaches top_p
        const float vp = search(vk, [&](double mm, double) { return mm >= (double)top_p; });
        above(vp, mg, cg);
        double nn = ceil(((double)top_p - mg) / (double)vp);
        mass_at<NT>(pp, n, vp, vp, red, m, c);
        const double group = c - cg;
        nn = fmin(fmax(nn, 1.0), group);
        if (vp == vk && take_k >= 0.0) nn = fmin(nn, take_k);
        vf = vp;
        take = nn;
    }
    above(vf, mg, cg);
    mass_at<NT>(pp, n, vf, vf, red, m, c);
    const double nf = take < 0.0 ? c - cg : take;
    const double kept = mg + nf * (double)vf;
    if (!(kept > 0.0)) return -1;
    const double r = u * kept;
    // the level holding the id where the running kept mass passes r, and the
    // position of that id among the level's ids (lowest index first)
    const float w = search(vf, [&](double mm, double) { return mm > r; });
    above(w, mg, cg);
    mass_at<NT>(pp, n, w, w, red, m, c);
    const double gw = w == vf ? nf : c - cg;
    double j = w > 0.0f ? floor((r - mg) / (double)w) : 0.0;
    j = fmin(fmax(j, 0.0), gw - 1.0);
    const int jj = (int)j;
    // j-th lowest index with p == w: per-thread counts over contiguous chunks
    // (positions are in index order), an exclusive scan, then the thread whose
    // chunk holds it walks the chunk
    const int t = threadIdx.x;
    const int ch = (n + NT - 1) / NT;
    const int q0 = t * ch, q1 = min(n, q0 + ch);
    int own = 0;
    for (int q = q0; q < q1; ++q) own += pp[q] == w;
    int before;
    if constexpr (NT == kST) {
        __syncthreads();
        cnt[t] = own;
        __syncthreads();
        if (t == 0) {
            int acc = 0;
            for (int i = 0; i < kST; ++i) {
                const int x = cnt[i];
                cnt[i] = acc;
                acc += x;
            }
        }
        __syncthreads();
        before = cnt[t];
    } else {
        int inc = own;   // inclusive scan over the wavefront
#pragma unroll
        for (int o = 1; o < 64; o <<= 1) {
            const int y = __shfl_up(inc, o);
            if (t >= o) inc += y;
        }
        before = inc - own;
    }
    int pick = -1;
    if (jj >= before && jj < before + own) {
        int seen = before;
        for (int q = q0; q < q1; ++q)
            if (pp[q] == w) {
                if (seen == jj) {
                    pick = ic ? ic[q] : q;
                    break;
                }
                ++seen;
            }
    }
    if constexpr (NT == kST) {
        __shared__ int pick_sh;
        if (t == 0) pick_sh = -1;
        __syncthreads();
        if (pick >= 0) pick_sh = pick;
        __syncthreads();
        return pick_sh;
    } else {
#pragma unroll
        for (int o = 32; o > 0; o >>= 1) pick = max(pick, __shfl_xor(pick, o));
        return pick;
    }
}

// Candidate compaction.  A histogram of the probabilities by the top 13 bits
// of their pattern (16 buckets per octave of (0, 1]) gives counts (integer) and
// masses (fixed point, 2^-44 units, integer adds: the same totals in any
// order) per bucket.  Walking down from the top bucket, the first bucket where
// the running count reaches top_k (or, without top_k, the bucket below the one
// where the running mass reaches top_p) bounds the final kept level from below,
// so every id the selection can keep or draw has p at or above that bucket's
// floor.  When at most kCand ids do, they are copied with their indices, in
// index order, and the selection runs over them alone.
constexpr int kBuckets = 2048;
constexpr int kCand = 4096;
constexpr double kFix = 17592186044416.0;   // 2^44

// p in [0, 1] maps to buckets 0 .. 2032; anything else (a NaN from bad logits)
// to the last bucket, so the histogram stays in bounds
__device__ __forceinline__ int bucket_of(float x) { return min((int)(__float_as_uint(x) >> 19), kBuckets - 1); }

// FEED: u is u_dev[count[0] - 1] and the id replaces the token and the last
// history entry of a fused decode step (out = its token slot), so sampled
// decoding continues on the device without a host round trip per token.
template <bool FEED>
__global__ __launch_bounds__(kST) void sample_kernel(const uint16_t* __restrict__ logits, int V, float inv_t,
                                                     int top_k, float top_p, double u, float* __restrict__ p,
                                                     int32_t* __restrict__ out, const double* __restrict__ u_dev,
                                                     const int32_t* __restrict__ count, int32_t* __restrict__ hist) {
    if constexpr (FEED) u = u_dev[count[0] - 1];
    __shared__ double red[kST];
    __shared__ int cnt[kST];
    __shared__ __align__(16) unsigned char pool[kCand * 8];   // histogram, then candidates
    __shared__ int sh_floor, sh_n;
    float* redf = reinterpret_cast<float*>(red);
    // passes over the vocabulary take eight elements per thread per step
    // (stride kST, so each of the eight loads is coalesced), all loads first
    constexpr int kU = 8;
    const int tid = threadIdx.x;
    float mx = -INFINITY;
    for (int i0 = 0; i0 < V; i0 += kU * kST) {
        float x[kU];
#pragma unroll
        for (int k = 0; k < kU; ++k) {
            const int i = i0 + k * kST + tid;
            x[k] = i < V ? h2f(logits[i]) * inv_t : -INFINITY;
        }
#pragma unroll
        for (int k = 0; k < kU; ++k) mx = fmaxf(mx, x[k]);
    }
    mx = block_max_f(mx, redf);
    // exponentials and their FP64 sum, in the same per-thread order as one
    // element per step (i = tid, tid + kST, ...)
    double s = 0.0;
    for (int i0 = 0; i0 < V; i0 += kU * kST) {
        float x[kU];
#pragma unroll
        for (int k = 0; k < kU; ++k) {
            const int i = i0 + k * kST + tid;
            x[k] = i < V ? h2f(logits[i]) : 0.f;
        }
#pragma unroll
        for (int k = 0; k < kU; ++k) {
            const int i = i0 + k * kST + tid;
            if (i < V) {
                const float e = expf(x[k] * inv_t - mx);
                p[i] = e;
                s += e;
            }
        }
    }
    s = block_sum_d(s, red);
    const float norm = s > 0.0 ? (float)(1.0 / s) : 0.0f;

    // ---- candidate floor from the histogram
    uint32_t* hcount = reinterpret_cast<uint32_t*>(pool);
    unsigned long long* hmass = reinterpret_cast<unsigned long long*>(pool + kBuckets * 4);
    for (int b = threadIdx.x; b < kBuckets; b += kST) {
        hcount[b] = 0u;
        hmass[b] = 0ull;
    }
    __syncthreads();
    // normalise (each thread its own elements) and, when top-k or top-p cut
    // the set, the histogram
    const bool want_hist = top_k > 0 || top_p < 1.0f;
    for (int i0 = 0; i0 < V; i0 += kU * kST) {
        float x[kU];
#pragma unroll
        for (int k = 0; k < kU; ++k) {
            const int i = i0 + k * kST + tid;
            x[k] = i < V ? p[i] : 0.f;
        }
#pragma unroll
        for (int k = 0; k < kU; ++k) {
            const int i = i0 + k * kST + tid;
            if (i < V) {
                const float v = x[k] * norm;
                p[i] = v;
                if (want_hist) {
                    const int b = bucket_of(v);
                    atomicAdd(&hcount[b], 1u);
                    atomicAdd(&hmass[b], (unsigned long long)((double)v * kFix));
                }
            }
        }
    }
    __syncthreads();
    if (threadIdx.x == 0) {
        int fb = -1;   // the floor bucket; -1: no useful floor
        if (top_k > 0 || top_p < 1.0f) {
            uint32_t c = 0;
            unsigned long long m = 0;
            const unsigned long long target = top_p < 1.0f ? (unsigned long long)((double)top_p * kFix) : ~0ull;
            for (int b = kBuckets - 1; b >= 0; --b) {
                c += hcount[b];
                m += hmass[b];
                if (top_k > 0 && c >= (uint32_t)top_k) { fb = b; break; }
                if (top_k <= 0 && m >= target) { fb = b > 0 ? b - 1 : 0; break; }
            }
        }
        sh_floor = fb;
    }
    __syncthreads();
    const int fb = sh_floor;
    // ids at or above the floor bucket, counted per contiguous chunk (index order)
    const int chunk = (V + kST - 1) / kST;
    const int b0 = threadIdx.x * chunk, b1 = min(V, b0 + chunk);
    int mine = 0;
    if (fb >= 0)
        for (int q0 = b0; q0 < b1; q0 += kU) {
            float x[kU];
#pragma unroll
            for (int k = 0; k < kU; ++k) x[k] = q0 + k < b1 ? p[q0 + k] : 0.f;
#pragma unroll
            for (int k = 0; k < kU; ++k) mine += (q0 + k < b1 && bucket_of(x[k]) >= fb) ? 1 : 0;
        }
    cnt[threadIdx.x] = mine;
    __syncthreads();
    if (threadIdx.x == 0) {
        int acc = 0;
        for (int t = 0; t < kST; ++t) {
            const int x = cnt[t];
            cnt[t] = acc;
            acc += x;
        }
        sh_n = acc;
    }
    __syncthreads();
    const bool compact = fb >= 0 && sh_n <= kCand;
    float* pc = reinterpret_cast<float*>(pool);
    int* ic = reinterpret_cast<int*>(pool + kCand * 4);
    if (compact && mine > 0) {
        int o = cnt[threadIdx.x];
        for (int q = b0; q < b1; ++q)
            if (bucket_of(p[q]) >= fb) {
                pc[o] = p[q];
                ic[o] = q;
                ++o;
            }
    }
    __syncthreads();
    int32_t chosen;
    if (compact) {
        // at most kCand candidates: wavefront 0 alone, no barriers
        __shared__ int chosen_sh;
        if (threadIdx.x < 64) {
            const int pk = select_token<64>(pc, ic, sh_n, V, top_k, top_p, u, red, cnt);
            if (threadIdx.x == 0) chosen_sh = pk;
        }
        __syncthreads();
        chosen = chosen_sh;
    } else {
        chosen = select_token<kST>(p, nullptr, V, V, top_k, top_p, u, red, cnt);
    }
    if (chosen < 0) {   // no mass: the most probable id (lowest index on ties)
        __shared__ int best2;
        if (threadIdx.x == 0) best2 = 0x7fffffff;
        __syncthreads();
        float pm = -1.0f;
        for (int q = threadIdx.x; q < V; q += kST) pm = fmaxf(pm, p[q]);
        pm = block_max_f(pm, redf);
        for (int q = threadIdx.x; q < V; q += kST)
            if (p[q] == pm) atomicMin(&best2, q);
        __syncthreads();
        chosen = best2 == 0x7fffffff ? 0 : best2;
    }
    if (threadIdx.x == 0) {
        out[0] = chosen;
        if constexpr (FEED) hist[count[0] - 1] = chosen;
    }
}

}  // namespace
}  // namespace bx

using namespace bx;

extern "C" {

size_t bx_sample_workspace_bytes(int vocab) { return vocab > 0 ? (size_t)vocab * sizeof(float) : 0; }

int bx_sample_f16(const uint16_t* logits, int vocab, float temperature, int top_k, float top_p, double u,
                  int32_t* out, void* workspace, void* stream) {
    if (!logits || !out || !workspace || vocab <= 0) return fail(BX_EINVAL, "sample: bad arguments");
    if (!(temperature > 0.0f)) return fail(BX_EINVAL, "sample: temperature must be positive (greedy uses argmax)");
    if (!(u >= 0.0 && u < 1.0)) return fail(BX_EINVAL, "sample: u must be in [0, 1)");
    sample_kernel<false><<<1, kST, 0, as_stream(stream)>>>(logits, vocab, 1.0f / temperature, top_k, top_p, u,
                                                           static_cast<float*>(workspace), out, nullptr, nullptr,
                                                           nullptr);
    return launch_check("sample");
}

int bx_sample_feed_f16(const uint16_t* logits, int vocab, float temperature, int top_k, float top_p,
                       const double* u_dev, int32_t* tok, int32_t* hist, const int32_t* count, void* workspace,
                       void* stream) {
    if (!logits || !u_dev || !tok || !hist || !count || !workspace || vocab <= 0)
        return fail(BX_EINVAL, "sample_feed: bad arguments");
    if (!(temperature > 0.0f)) return fail(BX_EINVAL, "sample_feed: temperature must be positive");
    sample_kernel<true><<<1, kST, 0, as_stream(stream)>>>(logits, vocab, 1.0f / temperature, top_k, top_p, 0.0,
                                                          static_cast<float*>(workspace), tok, u_dev, count, hist);
    return launch_check("sample_feed");
}

}  // extern "C"
