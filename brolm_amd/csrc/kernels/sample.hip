// Device top-k / top-p sampling over FP16 logits (reference
// src/detail/generate.cpp:68-142, sample_token).  The reference sorts all V
// probabilities on the host; here nothing is sorted and only the chosen id
// leaves the device.  Four launches, stream-ordered, no workgroup waits on
// another:
//   (1) per-segment maxima of l / T (segments of 1024 ids, one workgroup each);
//   (2) e_i = fp32(exp(l_i / T - max)), per-segment FP64 sums, and a histogram
//       of e over all segments (integer adds);
//   (3) every workgroup forms the same FP64 sum (segments in order) and the same
//       candidate floor, writes p_i = e_i * fp32(1 / sum) and its segment's
//       candidates (ids whose e reaches the floor) in index order;
//   (4) one workgroup gathers the candidates, sorts them by p (descending,
//       ids ascending among equal p) and follows the reference's steps over
//       them: the first k, the nucleus, the draw by running FP64 sums.  When
//       there is no floor or too many candidates, it finds the same thresholds
//       over all V ids by bisection on the probability value:
//   p_i   = fp32(exp(l_i / T - max)) * fp32(1 / sum)  (sum in FP64), as the reference;
//   M(v)  = sum of p_i >= v (FP64), C(v) = count of p_i >= v;
//   top-k level  v_k = largest v with C(v) >= k   (k-th largest p);
//   top-p level  v_p = largest v with M'(v) >= top_p, M' over p >= v_k
//                (the nucleus ends at the token whose running sum crosses top_p);
//   kept = p >= max(v_k, v_p); r = u * M(kept);
//   token = the lowest index whose p is the largest level w with M'(w) > r.
// The host draws u from the caller's std::mt19937_64 exactly as the reference
// does (one uniform_real_distribution<double>(0, 1) per sampled token).
// Ties: equal probabilities are ordered by ascending id.  A top-k cut keeps
// exactly k ids, as the reference does: of the ids tied at the cut level, the
// lowest-indexed ones that fit; the top-p cut likewise ends at one id.  The
// reference's std::sort leaves the order of equal probabilities unspecified,
// so ascending id is one of the orders it may produce.
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

// Mass (FP64) and count of p_i >= v among p_i >= floor_v, over n values.
__device__ void mass_at(const float* p, int n, float v, float floor_v, double* red, double& mass, double& cnt) {
    double m = 0.0, c = 0.0;
    const float lo = fmaxf(v, floor_v);
    for (int i = threadIdx.x; i < n; i += kST) {
        const float x = p[i];
        if (x >= lo) {
            m += x;
            c += 1.0;
        }
    }
    block_sum2(m, c, red);
    mass = m;
    cnt = c;
}

// The id drawn from all n = V probabilities pp by bisection on the value,
// the whole workgroup taking part; -1 when no mass is kept.
__device__ int select_token(const float* pp, int n, int V, int top_k, float top_p, double u, double* red, int* cnt) {
    // bisection over the bit patterns of non-negative floats: lo satisfies the
    // predicate, hi does not
    auto search = [&](float floor_v, auto pred) {
        uint32_t lo = 0, hi = 0x3f800001u;   // p <= 1
        while (hi - lo > 1) {
            const uint32_t mid = lo + (hi - lo) / 2;
            double m, c;
            mass_at(pp, n, __uint_as_float(mid), floor_v, red, m, c);
            if (pred(m, c)) lo = mid;
            else hi = mid;
        }
        return __uint_as_float(lo);
    };
    auto above = [&](float v, double& m, double& c) {   // mass / count of p > v
        mass_at(pp, n, __uint_as_float(__float_as_uint(v) + 1u), 0.0f, red, m, c);
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
    mass_at(pp, n, vk, vk, red, m, c);
    above(vk, mg, cg);
    const double kept_k = take_k < 0.0 ? m : mg + take_k * (double)vk;
    float vf = vk;          // the lowest kept level
    double take = take_k;   // ids kept at vf (-1: all of them)
    if (top_p < 1.0f && kept_k >= (double)top_p) {
        // the nucleus ends at the id whose running sum reaches top_p
        const float vp = search(vk, [&](double mm, double) { return mm >= (double)top_p; });
        above(vp, mg, cg);
        double nn = ceil(((double)top_p - mg) / (double)vp);
        mass_at(pp, n, vp, vp, red, m, c);
        const double group = c - cg;
        nn = fmin(fmax(nn, 1.0), group);
        if (vp == vk && take_k >= 0.0) nn = fmin(nn, take_k);
        vf = vp;
        take = nn;
    }
    above(vf, mg, cg);
    mass_at(pp, n, vf, vf, red, m, c);
    const double nf = take < 0.0 ? c - cg : take;
    const double kept = mg + nf * (double)vf;
    if (!(kept > 0.0)) return -1;
    const double r = u * kept;
    // the level holding the id where the running kept mass passes r, and the
    // position of that id among the level's ids (lowest index first)
    const float w = search(vf, [&](double mm, double) { return mm > r; });
    above(w, mg, cg);
    mass_at(pp, n, w, w, red, m, c);
    const double gw = w == vf ? nf : c - cg;
    double j = w > 0.0f ? floor((r - mg) / (double)w) : 0.0;
    j = fmin(fmax(j, 0.0), gw - 1.0);
    const int jj = (int)j;
    // j-th lowest index with p == w: per-thread counts over contiguous chunks
    // (positions are in index order), an exclusive scan, then the thread whose
    // chunk holds it walks the chunk
    const int t = threadIdx.x;
    const int ch = (n + kST - 1) / kST;
    const int q0 = t * ch, q1 = min(n, q0 + ch);
    int own = 0;
    for (int q = q0; q < q1; ++q) own += pp[q] == w;
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
    const int before = cnt[t];
    int pick = -1;
    if (jj >= before && jj < before + own) {
        int seen = before;
        for (int q = q0; q < q1; ++q)
            if (pp[q] == w) {
                if (seen == jj) {
                    pick = q;
                    break;
                }
                ++seen;
            }
    }
    __shared__ int pick_sh;
    if (t == 0) pick_sh = -1;
    __syncthreads();
    if (pick >= 0) pick_sh = pick;
    __syncthreads();
    return pick_sh;
}

// The draw over n candidates (1 <= n <= 4096) by the reference's own steps
// (generate.cpp:68-142): order by p descending, ids ascending among equal p
// (a bitonic sort of 64-bit keys: ~bits(p) above the id), keep the first k
// (k = 0: all n), then the nucleus up to the first running FP64 sum at or
// above top_p, then the first kept id whose running sum exceeds u * kept.
// Running sums: four consecutive positions a thread in order, thread totals
// scanned in thread order.  -1 when no mass is kept.  The whole workgroup
// takes part.
__device__ __forceinline__ unsigned long long cand_key(float p, int id) {
    return ((unsigned long long)(~__float_as_uint(p)) << 32) | (uint32_t)id;
}
__device__ __forceinline__ float key_p(unsigned long long k) { return __uint_as_float(~(uint32_t)(k >> 32)); }

__device__ int select_sorted(unsigned long long* key, int n, int k, float top_p, double u, double* red, int* sh) {
    const int t = threadIdx.x, l = t & 63, wv = t >> 6;
    int np = 1;
    while (np < n) np <<= 1;
    for (int i = n + t; i < np; i += kST) key[i] = ~0ull;
    __syncthreads();
    for (int size = 2; size <= np; size <<= 1)
        for (int stride = size >> 1; stride > 0; stride >>= 1) {
            for (int i = t; i < (np >> 1); i += kST) {
                const int a = ((i & ~(stride - 1)) << 1) | (i & (stride - 1));
                const int b = a + stride;
                const unsigned long long x = key[a], y = key[b];
                if ((x > y) == ((a & size) == 0)) {
                    key[a] = y;
                    key[b] = x;
                }
            }
            __syncthreads();
        }
    const int keep0 = k > 0 && k < n ? k : n;
    double c[4], run = 0.0;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        const int i = 4 * t + j;
        run += i < keep0 ? (double)key_p(key[i]) : 0.0;
        c[j] = run;
    }
    double inc = run;
#pragma unroll
    for (int o = 1; o < 64; o <<= 1) {
        const double y = __shfl_up(inc, o);
        if (l >= o) inc += y;
    }
    if (l == 63) red[wv] = inc;
    if (t == 0) {
        sh[0] = 0x7fffffff;
        sh[1] = 0x7fffffff;
    }
    __syncthreads();
    double before = 0.0;
    for (int i = 0; i < wv; ++i) before += red[i];
    before += inc - run;
#pragma unroll
    for (int j = 0; j < 4; ++j) c[j] += before;
    int keep = keep0;
    if (top_p < 1.0f) {
#pragma unroll
        for (int j = 0; j < 4; ++j)
            if (4 * t + j < keep0 && c[j] >= (double)top_p) {
                atomicMin(&sh[0], 4 * t + j);
                break;
            }
        __syncthreads();
        if (sh[0] != 0x7fffffff) keep = sh[0] + 1;
    }
    // kept mass: the running sum at keep - 1
    __syncthreads();
    if (t == (keep - 1) >> 2) red[kST / 64] = c[(keep - 1) & 3];
    __syncthreads();
    const double kept = red[kST / 64];
    if (!(kept > 0.0)) return -1;
    const double r = u * kept;
#pragma unroll
    for (int j = 0; j < 4; ++j)
        if (4 * t + j < keep && r < c[j]) {
            atomicMin(&sh[1], 4 * t + j);
            break;
        }
    __syncthreads();
    const int pos = sh[1] != 0x7fffffff ? sh[1] : keep - 1;
    return (int)(uint32_t)key[pos];
}

// Candidate compaction.  A histogram of the unnormalised exponentials e_i by
// the top 13 bits of their pattern (16 buckets per octave of (0, 1]) gives
// counts (integer) and masses (fixed point, 2^-44 units, integer adds: the same
// totals in any order) per bucket.  Walking down from the top bucket, the
// first bucket where the running count reaches top_k (without a top-k cut, the
// one where the running mass reaches top_p, scaled to e and raised by 2^-20 to
// cover the normalising product's rounding) is found, and the bucket below it
// is the floor: p = fp32(e * norm) is monotone in e, and a bucket spans far
// more than one rounding step, so every id the selection can keep or draw
// (ids tied in p with the last kept one included) has e at or above the
// floor's lower edge.  When at most kCand ids do, the selection runs over
// them alone.
constexpr int kBuckets = 2048;
constexpr int kCand = 4096;
// Fixed-point scale of the per-bucket mass: each e <= 1 adds at most 2^40,
// so even kMaxSegs * kSeg = 2^22 ids cannot carry a 64-bit total past 2^62.
// Truncating each e only lowers the running mass, which moves the floor down
// (more candidates), never up.
constexpr double kFix = 1099511627776.0;   // 2^40

// e in [0, 1] maps to buckets 0 .. 2032; anything else (a NaN from bad
// logits) to the last bucket, so the histogram stays in bounds
__device__ __forceinline__ int bucket_of(float x) { return min((int)(__float_as_uint(x) >> 19), kBuckets - 1); }

// The vocabulary is cut into segments of kSeg ids, one workgroup of kPT
// threads each, four consecutive ids a thread.
constexpr int kSeg = 1024;
constexpr int kPT = 256;
constexpr int kMaxSegs = 4096;   // vocabularies up to 4M ids

// Workspace carve-up (one allocation of bx_sample_workspace_bytes(V)).
struct SampleWs {
    float* p;                  // e, then p = e * norm (V)
    float* cv;                 // candidates' p, each segment's at its own offset (V)
    int* ci;                   // candidates' ids (V)
    float* pmax;               // per-segment max of l / T
    double* psum;              // per-segment FP64 sum of e
    int* ncand;                // per-segment candidate count
    uint32_t* hcnt;            // histogram counts (kBuckets)
    unsigned long long* hmass; // histogram masses (kBuckets)
    int* floor_b;              // the floor bucket, -1 without one
};

__host__ __device__ inline size_t ws_round(size_t x) { return (x + 255) & ~size_t(255); }

__host__ inline size_t ws_layout(void* base, int V, SampleWs* w) {
    const int nb = (V + kSeg - 1) / kSeg;
    char* c = static_cast<char*>(base);
    size_t o = 0;
    auto take = [&](size_t bytes) {
        char* q = c ? c + o : nullptr;
        o += ws_round(bytes);
        return q;
    };
    SampleWs t;
    t.p = reinterpret_cast<float*>(take((size_t)V * 4));
    t.cv = reinterpret_cast<float*>(take((size_t)V * 4));
    t.ci = reinterpret_cast<int*>(take((size_t)V * 4));
    t.pmax = reinterpret_cast<float*>(take((size_t)nb * 4));
    t.psum = reinterpret_cast<double*>(take((size_t)nb * 8));
    t.ncand = reinterpret_cast<int*>(take((size_t)nb * 4));
    t.hcnt = reinterpret_cast<uint32_t*>(take(kBuckets * 4));
    t.hmass = reinterpret_cast<unsigned long long*>(take(kBuckets * 8));
    t.floor_b = reinterpret_cast<int*>(take(4));
    if (w) *w = t;
    return o;
}

// Sum over a kPT-thread workgroup in a fixed order (lanes by butterfly, then
// the four wave totals in wave order), the result in every thread.
__device__ double seg_sum_d(double v, double* red4) {
    v = wave_sum_d(v);
    const int w = threadIdx.x >> 6;
    if ((threadIdx.x & 63) == 0) red4[w] = v;
    __syncthreads();
    const double r = ((red4[0] + red4[1]) + red4[2]) + red4[3];
    __syncthreads();
    return r;
}

__device__ float seg_max_f(float v, float* red4) {
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) v = fmaxf(v, __shfl_xor(v, o));
    const int w = threadIdx.x >> 6;
    if ((threadIdx.x & 63) == 0) red4[w] = v;
    __syncthreads();
    const float r = fmaxf(fmaxf(red4[0], red4[1]), fmaxf(red4[2], red4[3]));
    __syncthreads();
    return r;
}

// Exclusive prefix over a kPT-thread workgroup in thread order; *total gets
// the sum.  T is an integer type.
template <typename T>
__device__ T seg_scan_excl(T v, T* red4, T* total) {
    const int l = threadIdx.x & 63, w = threadIdx.x >> 6;
    T inc = v;
#pragma unroll
    for (int o = 1; o < 64; o <<= 1) {
        const T y = __shfl_up(inc, o);
        if (l >= o) inc += y;
    }
    if (l == 63) red4[w] = inc;
    __syncthreads();
    T before = 0;
    for (int i = 0; i < w; ++i) before += red4[i];
    *total = red4[0] + red4[1] + red4[2] + red4[3];
    __syncthreads();
    return before + inc - v;
}

// (1) per-segment max of l / T; the launch also clears the global histogram
// for (2)
__global__ __launch_bounds__(kPT) void sample_max_kernel(const uint16_t* __restrict__ logits, int V, float inv_t,
                                                         SampleWs w) {
    __shared__ float red4[4];
    for (int g = blockIdx.x * kPT + threadIdx.x; g < kBuckets; g += gridDim.x * kPT) {
        w.hcnt[g] = 0u;
        w.hmass[g] = 0ull;
    }
    const int i0 = blockIdx.x * kSeg + 4 * threadIdx.x;
    uint16_t x[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) x[j] = i0 + j < V ? logits[i0 + j] : (uint16_t)0;
    float mx = -INFINITY;
#pragma unroll
    for (int j = 0; j < 4; ++j)
        if (i0 + j < V) mx = fmaxf(mx, h2f(x[j]) * inv_t);
    mx = seg_max_f(mx, red4);
    if (threadIdx.x == 0) w.pmax[blockIdx.x] = mx;
}

// (2) e_i = fp32(exp(l_i / T - max)), the segment's FP64 sum of e, and (when
// top-k or top-p cut the set) the segment's histogram of e, added into the
// global one with integer device-scope atomics
__global__ __launch_bounds__(kPT) void sample_exp_kernel(const uint16_t* __restrict__ logits, int V, float inv_t,
                                                         SampleWs w, int want_hist, int want_mass) {
    __shared__ uint32_t hc[kBuckets];
    __shared__ unsigned long long hm[kBuckets];
    __shared__ float red4f[4];
    __shared__ double red4d[4];
    const int nb = gridDim.x;
    float mx = -INFINITY;
    for (int b = threadIdx.x; b < nb; b += kPT) mx = fmaxf(mx, w.pmax[b]);
    mx = seg_max_f(mx, red4f);
    if (want_hist)
        for (int b = threadIdx.x; b < kBuckets; b += kPT) {
            hc[b] = 0u;
            hm[b] = 0ull;
        }
    const int i0 = blockIdx.x * kSeg + 4 * threadIdx.x;
    uint16_t x[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) x[j] = i0 + j < V ? logits[i0 + j] : (uint16_t)0;
    __syncthreads();
    double s = 0.0;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        if (i0 + j < V) {
            const float e = expf(h2f(x[j]) * inv_t - mx);
            w.p[i0 + j] = e;
            s += e;
            if (want_hist) {
                const int b = bucket_of(e);
                atomicAdd(&hc[b], 1u);
                if (want_mass) atomicAdd(&hm[b], (unsigned long long)((double)e * kFix));
            }
        }
    }
    s = seg_sum_d(s, red4d);
    if (threadIdx.x == 0) w.psum[blockIdx.x] = s;
    if (want_hist) {
        __syncthreads();
        for (int b = threadIdx.x; b < kBuckets; b += kPT) {
            if (hc[b] == 0u) continue;
            __hip_atomic_fetch_add(&w.hcnt[b], hc[b], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            if (want_mass) __hip_atomic_fetch_add(&w.hmass[b], hm[b], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        }
    }
}

// (3) every workgroup forms the same sum (segments in order) and the same
// floor from the global histogram; then p = e * norm over its segment, and
// its candidates (e at or above the floor) written in index order at the
// segment's own offset, with their count
__global__ __launch_bounds__(kPT) void sample_compact_kernel(int V, int top_k, float top_p, SampleWs w, int want_hist,
                                                             int want_mass) {
    __shared__ double red4d[4];
    __shared__ uint32_t red4u[4];
    __shared__ unsigned long long red4m[4];
    __shared__ int fb_sh;
    const int nb = gridDim.x, t = threadIdx.x;
    double s = 0.0;
    for (int b = t; b < nb; b += kPT) s += w.psum[b];
    s = seg_sum_d(s, red4d);
    const float norm = s > 0.0 ? (float)(1.0 / s) : 0.0f;
    if (t == 0) fb_sh = -1;
    if (want_hist) {
        // thread t holds buckets 2047 - 8t .. 2040 - 8t, walked downwards
        constexpr int kPer = kBuckets / kPT;
        uint32_t c[kPer];
        unsigned long long m[kPer];
        uint32_t cs = 0u;
        unsigned long long ms = 0ull;
#pragma unroll
        for (int j = 0; j < kPer; ++j) {
            const int b = kBuckets - 1 - (kPer * t + j);
            c[j] = w.hcnt[b];
            m[j] = want_mass ? w.hmass[b] : 0ull;
            cs += c[j];
            ms += m[j];
        }
        uint32_t ctot;
        unsigned long long mtot;
        uint32_t cb = seg_scan_excl<uint32_t>(cs, red4u, &ctot);
        unsigned long long mb = seg_scan_excl<unsigned long long>(ms, red4m, &mtot);
        // the one bucket where the running total (from the top) first reaches
        // the target: k ids, or the top-p mass scaled to e (2^-20 above it)
        int hit = -1;
        if (!want_mass) {
            const uint32_t k = (uint32_t)top_k;
            for (int j = 0; j < kPer && hit < 0; ++j) {
                const uint32_t before = cb;
                cb += c[j];
                if (cb >= k && before < k) hit = kBuckets - 1 - (kPer * t + j);
            }
        } else {
            const double tgt = (double)top_p / (double)norm * (1.0 + 9.5367431640625e-07) * kFix;
            if (norm > 0.0f && tgt < 1.8e19) {
                const unsigned long long target = (unsigned long long)tgt + 1ull;
                for (int j = 0; j < kPer && hit < 0; ++j) {
                    const unsigned long long before = mb;
                    mb += m[j];
                    if (mb >= target && before < target) hit = kBuckets - 1 - (kPer * t + j);
                }
            }
        }
        __syncthreads();
        if (hit >= 0) fb_sh = hit > 0 ? hit - 1 : 0;
    }
    __syncthreads();
    const int fb = fb_sh;
    if (blockIdx.x == 0 && t == 0) w.floor_b[0] = fb;
    const int i0 = blockIdx.x * kSeg + 4 * t;
    float e[4], v[4];
    if (i0 + 3 < V) {
        const float4 q = *reinterpret_cast<const float4*>(w.p + i0);
        e[0] = q.x, e[1] = q.y, e[2] = q.z, e[3] = q.w;
    } else {
#pragma unroll
        for (int j = 0; j < 4; ++j) e[j] = i0 + j < V ? w.p[i0 + j] : 0.f;
    }
    int mine = 0;
    bool keep[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        v[j] = e[j] * norm;
        keep[j] = fb >= 0 && i0 + j < V && bucket_of(e[j]) >= fb;
        mine += keep[j] ? 1 : 0;
    }
    if (i0 + 3 < V) {
        *reinterpret_cast<float4*>(w.p + i0) = float4{v[0], v[1], v[2], v[3]};
    } else {
#pragma unroll
        for (int j = 0; j < 4; ++j)
            if (i0 + j < V) w.p[i0 + j] = v[j];
    }
    if (fb < 0) return;   // uniform across the grid
    int total;
    int o = blockIdx.x * kSeg + seg_scan_excl<int>(mine, reinterpret_cast<int*>(red4u), &total);
#pragma unroll
    for (int j = 0; j < 4; ++j)
        if (keep[j]) {
            w.cv[o] = v[j];
            w.ci[o] = i0 + j;
            ++o;
        }
    if (t == 0) w.ncand[blockIdx.x] = total;
}

// (4) one workgroup: the candidates gathered and drawn from in sorted order
// (or, without a floor or with more than kCand of them, the draw by bisection
// over all V probabilities).
// FEED: u is u_dev[count[0] - 1] and the id replaces the token and the last
// history entry of a fused decode step (out = its token slot), so sampled
// decoding continues on the device without a host round trip per token.
template <bool FEED>
__global__ __launch_bounds__(kST) void sample_select_kernel(int V, int top_k, float top_p, double u, SampleWs w,
                                                            int32_t* __restrict__ out,
                                                            const double* __restrict__ u_dev,
                                                            const int32_t* __restrict__ count,
                                                            int32_t* __restrict__ hist) {
    if constexpr (FEED) u = u_dev[count[0] - 1];
    __shared__ double red[kST];
    __shared__ int cnt[kST];
    __shared__ int pre[kMaxSegs + 1];
    __shared__ __align__(16) unsigned char pool[kCand * 8];
    float* redf = reinterpret_cast<float*>(red);
    const int t = threadIdx.x;
    const int nb = (V + kSeg - 1) / kSeg;
    const int fb = w.floor_b[0];
    int n = 0;
    if (fb >= 0) {
        // exclusive prefix of the segments' counts (4 segments a thread at most)
        constexpr int kPer = kMaxSegs / kST;
        int c[kPer], own = 0;
#pragma unroll
        for (int j = 0; j < kPer; ++j) {
            const int b = kPer * t + j;
            c[j] = b < nb ? w.ncand[b] : 0;
            own += c[j];
        }
        // wave-level inclusive scan of the per-thread sums, then the waves in order
        int inc = own;
        const int l = t & 63, wv = t >> 6;
#pragma unroll
        for (int o = 1; o < 64; o <<= 1) {
            const int y = __shfl_up(inc, o);
            if (l >= o) inc += y;
        }
        __syncthreads();
        if (l == 63) cnt[wv] = inc;
        __syncthreads();
        int before = 0;
        for (int i = 0; i < wv; ++i) before += cnt[i];
        int run = before + inc - own;
#pragma unroll
        for (int j = 0; j < kPer; ++j) {
            const int b = kPer * t + j;
            if (b < nb) pre[b] = run;
            run += c[j];
        }
        if (t == kST - 1) pre[nb] = run;
        __syncthreads();
        n = pre[nb];
    }
    const bool compact = fb >= 0 && n <= kCand;
    unsigned long long* key = reinterpret_cast<unsigned long long*>(pool);
    int32_t chosen;
    if (compact) {
        for (int j = t; j < n; j += kST) {
            // the segment holding candidate j: the last b with pre[b] <= j
            int lo = 0, hi = nb;   // pre[lo] <= j < pre[hi]
            while (hi - lo > 1) {
                const int mid = (lo + hi) >> 1;
                if (pre[mid] <= j) lo = mid;
                else hi = mid;
            }
            const int src = lo * kSeg + (j - pre[lo]);
            key[j] = cand_key(w.cv[src], w.ci[src]);
        }
        __syncthreads();
        chosen = select_sorted(key, n, top_k > 0 && top_k < V ? top_k : 0, top_p, u, red, cnt);
    } else {
        chosen = select_token(w.p, V, V, top_k, top_p, u, red, cnt);
    }
    if (chosen < 0) {   // no mass: the most probable id (lowest index on ties)
        __shared__ int best2;
        if (t == 0) best2 = 0x7fffffff;
        __syncthreads();
        float pm = -1.0f;
        for (int q = t; q < V; q += kST) pm = fmaxf(pm, w.p[q]);
        pm = block_max_f(pm, redf);
        for (int q = t; q < V; q += kST)
            if (w.p[q] == pm) atomicMin(&best2, q);
        __syncthreads();
        chosen = best2 == 0x7fffffff ? 0 : best2;
    }
    if (t == 0) {
        out[0] = chosen;
        if constexpr (FEED) hist[count[0] - 1] = chosen;
    }
}

template <bool FEED>
int sample_launch(const uint16_t* logits, int V, float temperature, int top_k, float top_p, double u, int32_t* out,
                  const double* u_dev, const int32_t* count, int32_t* hist, void* workspace, hipStream_t st) {
    SampleWs w;
    ws_layout(workspace, V, &w);
    const int nb = (V + kSeg - 1) / kSeg;
    const float inv_t = 1.0f / temperature;
    const bool cut_k = top_k > 0 && top_k < V;
    const int want_hist = cut_k || top_p < 1.0f;
    const int want_mass = !cut_k && top_p < 1.0f;
    sample_max_kernel<<<nb, kPT, 0, st>>>(logits, V, inv_t, w);
    sample_exp_kernel<<<nb, kPT, 0, st>>>(logits, V, inv_t, w, want_hist, want_mass);
    sample_compact_kernel<<<nb, kPT, 0, st>>>(V, top_k, top_p, w, want_hist, want_mass);
    sample_select_kernel<FEED><<<1, kST, 0, st>>>(V, top_k, top_p, u, w, out, u_dev, count, hist);
    return launch_check("sample");
}

}  // namespace
}  // namespace bx

using namespace bx;

extern "C" {

size_t bx_sample_workspace_bytes(int vocab) { return vocab > 0 ? ws_layout(nullptr, vocab, nullptr) : 0; }

int bx_sample_f16(const uint16_t* logits, int vocab, float temperature, int top_k, float top_p, double u,
                  int32_t* out, void* workspace, void* stream) {
    if (!logits || !out || !workspace || vocab <= 0) return fail(BX_EINVAL, "sample: bad arguments");
    if (vocab > kMaxSegs * kSeg) return fail(BX_EINVAL, "sample: vocabulary above 4194304 ids");
    if (!(temperature > 0.0f)) return fail(BX_EINVAL, "sample: temperature must be positive (greedy uses argmax)");
    if (!(u >= 0.0 && u < 1.0)) return fail(BX_EINVAL, "sample: u must be in [0, 1)");
    if (reinterpret_cast<uintptr_t>(workspace) & 255) return fail(BX_EINVAL, "sample: workspace not 256-byte aligned");
    return sample_launch<false>(logits, vocab, temperature, top_k, top_p, u, out, nullptr, nullptr, nullptr,
                                workspace, as_stream(stream));
}

int bx_sample_feed_f16(const uint16_t* logits, int vocab, float temperature, int top_k, float top_p,
                       const double* u_dev, int32_t* tok, int32_t* hist, const int32_t* count, void* workspace,
                       void* stream) {
    if (!logits || !u_dev || !tok || !hist || !count || !workspace || vocab <= 0)
        return fail(BX_EINVAL, "sample_feed: bad arguments");
    if (vocab > kMaxSegs * kSeg) return fail(BX_EINVAL, "sample_feed: vocabulary above 4194304 ids");
    if (!(temperature > 0.0f)) return fail(BX_EINVAL, "sample_feed: temperature must be positive");
    if (reinterpret_cast<uintptr_t>(workspace) & 255)
        return fail(BX_EINVAL, "sample_feed: workspace not 256-byte aligned");
    return sample_launch<true>(logits, vocab, temperature, top_k, top_p, 0.0, tok, u_dev, count, hist, workspace,
                               as_stream(stream));
}

}  // extern "C"
