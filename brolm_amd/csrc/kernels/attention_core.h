// Block-level attention over a key range with an online softmax (shared by the
// op-surface attention kernel and the fused decode step).
#pragma once

#include "common.h"

namespace bx {

constexpr int kAttnMaxGroup = 8;   // query heads per KV head
constexpr int kAttnPairsPerThread = 8;  // G * hd <= 256 * 8

struct AttnArgs {
    const uint16_t* q;
    const uint16_t* Kc;
    const uint16_t* Vc;
    const float* mask;  // optional: keys with mask[j] == 0 are skipped
    int L, valid_len, n_q, n_kv, hd;
    float softcap;
    int window;
    int kps, S;
    float* ws;  // partials [L][n_q][S][hd + 2]
    int bidir;  // 1: every row attends all valid_len keys (no causal limit)
    // per-row key ranges (batched decode of independent sequences): row r
    // attends cache rows rbase[r] .. rbase[r] + rlen[r] - 1; null otherwise
    const int32_t* rlen;
    const int64_t* rbase;
};

// Flash attention on MFMA for L >= 16 query rows (attention_mfma.hip): head
// dims 64 and 128, no softcap / window / key mask.
bool attn_mfma_supported(int L, int hd, float softcap, int window, const float* mask);
int attn_mfma(const uint16_t* q, const uint16_t* Kc, const uint16_t* Vc, int L, int valid_len, int n_q, int n_kv,
              int hd, int bidir, uint16_t* out, hipStream_t st);

struct AttnState {
    float o[kAttnPairsPerThread];
};

__device__ __forceinline__ void attn_state_init(AttnState& st) {
#pragma unroll
    for (int i = 0; i < kAttnPairsPerThread; ++i) st.o[i] = 0.f;
}

// Runs keys [kb, ke) of KV head g for the G = n_q/n_kv query heads whose
// scaled query vectors are in qs (LDS, G*hd floats).  sc: LDS G*256 floats;
// red: LDS >= 4*kAttnMaxGroup floats (holds running m, l at red[0..G),
// red[G..2G) on return).  cur_pos >= 0 substitutes key cur_pos with the LDS
// vectors cur_k / cur_v (FP32, hd each) instead of reading the cache.
__device__ inline void attn_range(const AttnArgs& a, int g, int kb, int ke, const float* qs, float* sc, float* red,
                                  AttnState& st, const float* cur_k, const float* cur_v, int cur_pos) {
    const int G = a.n_q / a.n_kv;
    const int hd = a.hd;
    const int64_t kvd = (int64_t)a.n_kv * hd;
    float* m_run = red;          // G
    float* l_run = red + G;      // G
    float* tmp = red + 2 * G;    // G (new running max)
    float* alph = red + 3 * G;   // G (rescale factor of the old partials)
    if (threadIdx.x < G) {
        m_run[threadIdx.x] = -INFINITY;
        l_run[threadIdx.x] = 0.f;
    }
    __syncthreads();
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    for (int c0 = kb; c0 < ke; c0 += 256) {
        // --- scores: one thread per key
        {
            const int j = c0 + threadIdx.x;
            float acc[kAttnMaxGroup];
#pragma unroll
            for (int h = 0; h < kAttnMaxGroup; ++h) acc[h] = 0.f;
            bool valid = j < ke;
            if (valid && a.mask) valid = a.mask[j] != 0.f;
            if (valid) {
                const uint16_t* krow = a.Kc + (int64_t)j * kvd + (int64_t)g * hd;
                for (int d0 = 0; d0 < hd; d0 += 8) {
                    float kf[8];
                    if (j == cur_pos) {
#pragma unroll
                        for (int e = 0; e < 8; ++e) kf[e] = cur_k[d0 + e];
                    } else {
                        const u4v kv = ldg16(krow + d0);
                        const uint32_t w[4] = {kv.x, kv.y, kv.z, kv.w};
#pragma unroll
                        for (int e = 0; e < 4; ++e) {
                            kf[2 * e] = h2f(w[e] & 0xffff);
                            kf[2 * e + 1] = h2f(w[e] >> 16);
                        }
                    }
#pragma unroll
                    for (int h = 0; h < kAttnMaxGroup; ++h) {
                        if (h < G) {
#pragma unroll
                            for (int e = 0; e < 8; ++e) acc[h] += qs[h * hd + d0 + e] * kf[e];
                        }
                    }
                }
            }
            for (int h = 0; h < G; ++h) {
                float s = acc[h];
                if (a.softcap > 0.f) s = a.softcap * tanhf(s / a.softcap);
                sc[h * 256 + threadIdx.x] = valid ? s : -INFINITY;
            }
        }
        __syncthreads();
        // --- chunk max per head (wave w handles heads w, w+4)
        for (int h = wave; h < G; h += 4) {
            float mx = -INFINITY;
            for (int i = lane; i < 256; i += 64) mx = fmaxf(mx, sc[h * 256 + i]);
            mx = wave_max(mx);
            if (lane == 0) tmp[h] = fmaxf(m_run[h], mx);
        }
        __syncthreads();
        // --- exponentiate against the new running max
        if (threadIdx.x < G) {
            const float mo = m_run[threadIdx.x];
            alph[threadIdx.x] = (mo == -INFINITY) ? 0.f : __expf(mo - tmp[threadIdx.x]);
        }
        for (int h = 0; h < G; ++h) {
            const float mn = tmp[h];
            const float s = sc[h * 256 + threadIdx.x];
            sc[h * 256 + threadIdx.x] = (s == -INFINITY) ? 0.f : __expf(s - mn);
        }
        __syncthreads();
        // --- rescale + accumulate V (thread owns pairs i = tid + 256*t)
        const int nkeys = min(256, ke - c0);
#pragma unroll
        for (int t = 0; t < kAttnPairsPerThread; ++t) {
            const int i = threadIdx.x + 256 * t;
            if (i < G * hd) {
                const int h = i / hd, d = i - h * hd;
                float o = st.o[t] * alph[h];
                const uint16_t* vcol = a.Vc + (int64_t)g * hd + d;
                const float* p = sc + h * 256;
                for (int jj = 0; jj < nkeys; ++jj) {
                    const int j = c0 + jj;
                    const float pv = p[jj];
                    const float v = (j == cur_pos) ? cur_v[d] : h2f(vcol[(int64_t)j * kvd]);
                    o += pv * v;
                }
                st.o[t] = o;
            }
        }
        // --- running sums
        for (int h = wave; h < G; h += 4) {
            float s = 0.f;
            for (int i = lane; i < 256; i += 64) s += sc[h * 256 + i];
            s = wave_sum(s);
            if (lane == 0) {
                l_run[h] = l_run[h] * alph[h] + s;
                m_run[h] = tmp[h];
            }
        }
        __syncthreads();
    }
}

// Partial record of (row r, query head h, split s): o[hd] (unnormalised), m, l.
__device__ inline void attn_write_partial(const AttnArgs& a, int r, int g, int s, const AttnState& st) {
    const int G = a.n_q / a.n_kv;
    const int hd = a.hd;
#pragma unroll
    for (int t = 0; t < kAttnPairsPerThread; ++t) {
        const int i = threadIdx.x + 256 * t;
        if (i < G * hd) {
            const int h = g * G + i / hd, d = i % hd;
            a.ws[(((int64_t)r * a.n_q + h) * a.S + s) * (hd + 2) + d] = st.o[t];
        }
    }
}

__device__ inline void attn_write_ml(const AttnArgs& a, int r, int g, int s, const float* red) {
    const int G = a.n_q / a.n_kv;
    const int hd = a.hd;
    if (threadIdx.x < G) {
        const int h = g * G + threadIdx.x;
        float* rec = a.ws + (((int64_t)r * a.n_q + h) * a.S + s) * (hd + 2);
        rec[hd] = red[threadIdx.x];
        rec[hd + 1] = red[G + threadIdx.x];
    }
}

}  // namespace bx
