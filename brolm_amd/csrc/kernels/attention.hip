// GQA attention over the FP16 KV cache (brotensor flash_attention_decode,
// called at src/detail/dense_decoder.cpp:606-607; Gemma form with softcap and
// window at src/gemma2.cpp:365-367; masked form at dense_decoder.cpp:476-478).
//
// L >= 16 rows with head_dim 64 / 128 and no softcap, window or mask run the
// MFMA flash-attention kernel (attention_mfma.hip); everything else runs
// split-K ("flash decoding"): block (split s, kv head g, query row r) streams
// its key range in chunks of 256 with an online softmax and writes an
// unnormalised partial (o[hd], m, l) per query head of the group; a combine
// kernel merges the splits.  Query head h reads KV head h / (n_q / n_kv).
#include <cmath>

#include "attention_core.h"

namespace bx {
namespace {

constexpr int kChunk = 128;   // keys per chunk: two per lane quad for the scores, 32 per wavefront for P.V

// One chunk's key and value rows in registers, requested together before any
// of them is used, so a chunk costs one memory round trip.  Scores: lane ql of
// quad q takes the 16-byte chunks ql, ql + 4, ... of keys q and q + 64.  P.V:
// wavefront w takes keys w, w + 4, ..., each lane 2 DP head dims of them.
template <int DP>
struct ChunkRows {
    static constexpr int CPL = 4 * DP;   // 16-byte chunks per lane per key: hd / 32 <= 4 DP
    u4v kr[2][CPL];
    uint32_t vv[kChunk / 4][DP];

    // Buffer loads: the key rows' offsets are per lane, the value rows' offsets
    // are uniform per wavefront (a scalar operand), so the 32 value loads need
    // no address registers.  rk / rv cover the keys below the block's end.
    __device__ __forceinline__ void issue(__amdgpu_buffer_rsrc_t rk, __amdgpu_buffer_rsrc_t rv, int kvd, int g,
                                          int hd, int c0, int nk) {
        const int tid = threadIdx.x, quad = tid >> 2, ql = tid & 3, nch = hd >> 3;
        const int wave = __builtin_amdgcn_readfirstlane(tid >> 6), lane = tid & 63, d0 = 2 * DP * lane;
#pragma unroll
        for (int b = 0; b < 2; ++b) {
            const int kl = 64 * b + quad;
            const int off = ((c0 + (kl < nk ? kl : nk - 1)) * kvd + g * hd) * 2 + 16 * ql;
#pragma unroll
            for (int c = 0; c < CPL; ++c) {
                const int ch = ql + 4 * c;
                kr[b][c] = (ch < nch && kl < nk) ? __builtin_bit_cast(u4v, __builtin_amdgcn_raw_buffer_load_b128(
                                                                            rk, off + 64 * c, 0, 0))
                                                 : u4v{0u, 0u, 0u, 0u};
            }
        }
        if (d0 < hd) {
            const int voff = (g * hd + d0) * 2;
#pragma unroll
            for (int u = 0; u < kChunk / 4; ++u) {
                const int t = min(wave + 4 * u, nk - 1);   // uniform
                const int soff = (c0 + t) * kvd * 2;
                if constexpr (DP == 1) {
                    vv[u][0] = __builtin_amdgcn_raw_buffer_load_b32(rv, voff, soff, 0);
                } else {
                    const auto x = __builtin_amdgcn_raw_buffer_load_b64(rv, voff, soff, 0);
                    vv[u][0] = x[0];
                    vv[u][1] = x[1];
                }
            }
        }
    }
};

// Block (split s, KV head g, query row r): keys [kb, ke) of row r in chunks of
// 128 with an online softmax per head; the group's G query heads are scaled
// into LDS.  The four wavefronts' P.V accumulators are added in LDS at the
// end, and the unnormalised partial (o[hd], m, l) of each query head goes to
// the split records; a combine kernel merges the splits.
template <int DP>   // head dims per lane / 2: hd <= 128 DP
__global__ __launch_bounds__(256) void attn_partial_kernel(AttnArgs a) {
    extern __shared__ __align__(16) float att_smem[];
    const int s = blockIdx.x, g = blockIdx.y, r = blockIdx.z;
    const int G = a.n_q / a.n_kv, hd = a.hd;
    const int64_t kvd = (int64_t)a.n_kv * hd;
    const uint16_t* Kc = a.Kc;
    const uint16_t* Vc = a.Vc;
    if (a.rlen) {  // this row's own sequence: its keys start at cache row rbase[r]
        Kc += a.rbase[r] * kvd;
        Vc += a.rbase[r] * kvd;
    }
    const int p = a.rlen ? a.rlen[r] - 1 : a.bidir ? a.valid_len - 1 : a.valid_len - a.L + r;  // last key
    const int lo = a.window > 0 ? max(0, p - a.window + 1) : 0;
    const int kb = max(lo, s * a.kps);
    const int ke = min(p + 1, (s + 1) * a.kps);
    float* qs = att_smem;                  // G * hd scaled query
    float* sc = qs + G * hd;               // G * kChunk scores, then probabilities
    float* m_run = sc + G * kChunk;        // G running max
    float* l_run = m_run + kAttnMaxGroup;  // G running sum
    float* m_new = l_run + kAttnMaxGroup;  // G
    float* alpha = m_new + kAttnMaxGroup;  // G rescale of the old partials
    float* accs = alpha + kAttnMaxGroup;   // 4 x G x hd wavefront accumulators
    const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
    const int quad = tid >> 2, ql = tid & 3, nch = hd >> 3;
    // the query values first, then the first chunk's rows, then the query to
    // LDS (its wait does not cover the rows issued after it)
    const float scale = 1.0f / sqrtf((float)hd);
    float qv[kAttnMaxGroup];   // G * hd <= 8 * 256 = 8 per thread
#pragma unroll
    for (int k = 0; k < kAttnMaxGroup; ++k) {
        const int i = tid + 256 * k;
        qv[k] = 0.f;
        if (i < G * hd) qv[k] = h2f(a.q[((int64_t)r * a.n_q + g * G + i / hd) * hd + i % hd]);
    }
    // byte ranges of the keys this block may read (the host keeps them below 2^31)
    const int span = ke > 0 ? (int)((int64_t)ke * kvd * 2) : 0;
    const __amdgpu_buffer_rsrc_t rk = __builtin_amdgcn_make_buffer_rsrc(const_cast<uint16_t*>(Kc), 0, span, 0x00020000);
    const __amdgpu_buffer_rsrc_t rv = __builtin_amdgcn_make_buffer_rsrc(const_cast<uint16_t*>(Vc), 0, span, 0x00020000);
    ChunkRows<DP> cr0, cr1;
    if (kb < ke) cr0.issue(rk, rv, (int)kvd, g, hd, kb, min(kChunk, ke - kb));
#pragma unroll
    for (int k = 0; k < kAttnMaxGroup; ++k) {
        const int i = tid + 256 * k;
        if (i < G * hd) qs[i] = qv[k] * scale;
    }
    if (tid < G) {
        m_run[tid] = -INFINITY;
        l_run[tid] = 0.f;
    }
    float acc[kAttnMaxGroup][2 * DP];
#pragma unroll
    for (int h = 0; h < kAttnMaxGroup; ++h)
#pragma unroll
        for (int e = 0; e < 2 * DP; ++e) acc[h][e] = 0.f;
    const int d0 = 2 * DP * lane;   // this lane's first head dim (P.V)
    const bool has_dims = d0 < hd;
    __syncthreads();
    // one chunk whose rows are in cr (the next chunk's rows are already in flight)
    auto chunk = [&](const ChunkRows<DP>& cr, int c0) {
        const int nk = min(kChunk, ke - c0);
        // ---- scores (the quad's partial dots added by DPP)
#pragma unroll
        for (int b = 0; b < 2; ++b) {
            float sv[kAttnMaxGroup];
#pragma unroll
            for (int h = 0; h < kAttnMaxGroup; ++h) sv[h] = 0.f;
#pragma unroll
            for (int c = 0; c < ChunkRows<DP>::CPL; ++c) {
                const int ch = ql + 4 * c;
                if (ch < nch) {
                    const uint32_t w[4] = {cr.kr[b][c].x, cr.kr[b][c].y, cr.kr[b][c].z, cr.kr[b][c].w};
                    float kf[8];
#pragma unroll
                    for (int e = 0; e < 4; ++e) {
                        kf[2 * e] = h2f(w[e] & 0xffff);
                        kf[2 * e + 1] = h2f(w[e] >> 16);
                    }
#pragma unroll
                    for (int h = 0; h < kAttnMaxGroup; ++h)
                        if (h < G) {
                            const float* qh = qs + h * hd + 8 * ch;
#pragma unroll
                            for (int e = 0; e < 8; ++e) sv[h] += qh[e] * kf[e];
                        }
                }
            }
            const int kl = 64 * b + quad;
            bool valid = kl < nk;
            if (valid && a.mask) valid = a.mask[c0 + kl] != 0.f;
#pragma unroll
            for (int h = 0; h < kAttnMaxGroup; ++h)
                if (h < G) {
                    float v = sv[h];
                    v += dpp_f<0xB1>(v, 0.f);   // quad_perm [1, 0, 3, 2]
                    v += dpp_f<0x4E>(v, 0.f);   // quad_perm [2, 3, 0, 1]
                    if (a.softcap > 0.f) v = a.softcap * tanhf(v / a.softcap);
                    if (ql == 0) sc[h * kChunk + kl] = valid ? v : -INFINITY;
                }
        }
        __syncthreads();
        // ---- new running max per head (wavefront w: heads w, w + 4)
        for (int h = wave; h < G; h += 4) {
            float mx = -INFINITY;
            for (int i = lane; i < kChunk; i += 64) mx = fmaxf(mx, sc[h * kChunk + i]);
            mx = wave_max(mx);
            if (lane == 0) {
                const float mo = m_run[h], mn = fmaxf(mo, mx);
                m_new[h] = mn;
                alpha[h] = mo == -INFINITY ? 0.f : __expf(mo - mn);
            }
        }
        __syncthreads();
        for (int i = tid; i < G * kChunk; i += 256) {
            const float v = sc[i];
            sc[i] = v == -INFINITY ? 0.f : __expf(v - m_new[i / kChunk]);
        }
        __syncthreads();
        // ---- P.V from the rows in registers
#pragma unroll
        for (int h = 0; h < kAttnMaxGroup; ++h)
            if (h < G) {
                const float al = alpha[h];
#pragma unroll
                for (int e = 0; e < 2 * DP; ++e) acc[h][e] *= al;
            }
        if (has_dims) {
#pragma unroll
            for (int u = 0; u < kChunk / 4; ++u) {
                const int t = wave + 4 * u;
                float vf[2 * DP];
#pragma unroll
                for (int e = 0; e < DP; ++e) {
                    vf[2 * e] = h2f(cr.vv[u][e] & 0xffff);
                    vf[2 * e + 1] = h2f(cr.vv[u][e] >> 16);
                }
#pragma unroll
                for (int h = 0; h < kAttnMaxGroup; ++h)
                    if (h < G) {
                        const float pr = sc[h * kChunk + t];   // 0 past nk
#pragma unroll
                        for (int e = 0; e < 2 * DP; ++e) acc[h][e] += pr * vf[e];
                    }
            }
        }
        // ---- running sums
        for (int h = wave; h < G; h += 4) {
            float sum = 0.f;
            for (int i = lane; i < kChunk; i += 64) sum += sc[h * kChunk + i];
            sum = wave_sum(sum);
            if (lane == 0) {
                l_run[h] = l_run[h] * alpha[h] + sum;
                m_run[h] = m_new[h];
            }
        }
        __syncthreads();
    };
    if constexpr (DP == 1) {
        // chunks alternate between the two row buffers; each chunk's successor
        // is requested before the chunk is computed
        for (int c0 = kb; c0 < ke;) {
            if (c0 + kChunk < ke) cr1.issue(rk, rv, (int)kvd, g, hd, c0 + kChunk, min(kChunk, ke - c0 - kChunk));
            chunk(cr0, c0);
            c0 += kChunk;
            if (c0 >= ke) break;
            if (c0 + kChunk < ke) cr0.issue(rk, rv, (int)kvd, g, hd, c0 + kChunk, min(kChunk, ke - c0 - kChunk));
            chunk(cr1, c0);
            c0 += kChunk;
        }
    } else {
        // head dims above 128: one buffer (two would not fit the registers)
        for (int c0 = kb; c0 < ke; c0 += kChunk) {
            chunk(cr0, c0);
            if (c0 + kChunk < ke) cr0.issue(rk, rv, (int)kvd, g, hd, c0 + kChunk, min(kChunk, ke - c0 - kChunk));
        }
    }
    // ---- the four wavefronts' accumulators -> one partial per head
    if (has_dims) {
#pragma unroll
        for (int h = 0; h < kAttnMaxGroup; ++h)
            if (h < G) {
#pragma unroll
                for (int e = 0; e < 2 * DP; ++e)
                    if (d0 + e < hd) accs[(wave * G + h) * hd + d0 + e] = acc[h][e];
            }
    }
    __syncthreads();
    for (int i = tid; i < G * hd; i += blockDim.x) {
        const int h = i / hd, d = i - h * hd;
        float o = 0.f;
        if (kb < ke)
            o = (accs[(0 * G + h) * hd + d] + accs[(1 * G + h) * hd + d]) +
                (accs[(2 * G + h) * hd + d] + accs[(3 * G + h) * hd + d]);
        a.ws[(((int64_t)r * a.n_q + g * G + h) * a.S + s) * (hd + 2) + d] = o;
    }
    if (tid < G) {
        float* rec = a.ws + (((int64_t)r * a.n_q + g * G + tid) * a.S + s) * (hd + 2);
        rec[hd] = m_run[tid];
        rec[hd + 1] = l_run[tid];
    }
}

// LDS bytes of attn_partial_kernel for a group of G heads of hd dims.
size_t attn_partial_lds(int G, int hd) {
    return (size_t)(G * hd + G * kChunk + 4 * kAttnMaxGroup + 4 * G * hd) * sizeof(float);
}

inline size_t combine_lds(int S) { return (size_t)(S + 4) * sizeof(float); }

// The split-K kernel addresses a row's keys by 32-bit byte offsets.
inline bool attn_span_ok(int keys, int n_kv, int hd) { return (int64_t)keys * n_kv * hd * 2 < ((int64_t)1 << 31); }

// Launch the split-K partials (the host has checked hd <= 256, G <= 8, and
// that max_keys rows of the cache span less than 2^31 bytes).
void attn_partial_launch(const AttnArgs& a, int rows, hipStream_t st) {
    const int G = a.n_q / a.n_kv;
    const size_t lds = attn_partial_lds(G, a.hd);
    if (a.hd <= 128)
        attn_partial_kernel<1><<<dim3(a.S, a.n_kv, rows), 256, lds, st>>>(a);
    else
        attn_partial_kernel<2><<<dim3(a.S, a.n_kv, rows), 256, lds, st>>>(a);
}

// Merge the S split records of (query head h, row r): the maxima and sums
// go to LDS once (sw: S weights exp(m_s - M)), then each thread adds its head
// dims over the splits with eight loads in flight.
__global__ __launch_bounds__(128) void attn_combine_kernel(const float* __restrict__ ws, int n_q, int hd, int S,
                                                          uint16_t* __restrict__ out) {
    extern __shared__ float sw[];   // S weights, then 4 reduction slots
    float* red = sw + S;
    const int h = blockIdx.x, r = blockIdx.y, tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int64_t rec = hd + 2;
    const float* base = ws + ((int64_t)r * n_q + h) * S * rec;
    float mx = -INFINITY;
    for (int s = tid; s < S; s += blockDim.x) {
        const float m = base[s * rec + hd];
        sw[s] = m;
        mx = fmaxf(mx, m);
    }
    mx = wave_max(mx);
    if (lane == 0) red[wave] = mx;
    __syncthreads();
    const float M = fmaxf(red[0], red[1]);
    float ls = 0.f;
    for (int s = tid; s < S; s += blockDim.x) {
        const float m = sw[s];
        const float w = m == -INFINITY ? 0.f : __expf(m - M);
        sw[s] = w;
        ls += w * base[s * rec + hd + 1];
    }
    ls = wave_sum(ls);
    __syncthreads();
    if (lane == 0) red[2 + wave] = ls;
    __syncthreads();
    const float lsum = red[2] + red[3];
    const float inv = lsum > 0.f ? 1.0f / lsum : 0.f;
    for (int d = tid; d < hd; d += blockDim.x) {
        float o = 0.f;
        int s = 0;
        for (; s + 8 <= S; s += 8) {
            float v[8];
#pragma unroll
            for (int u = 0; u < 8; ++u) v[u] = base[(s + u) * rec + d];
#pragma unroll
            for (int u = 0; u < 8; ++u) o += sw[s + u] * v[u];
        }
        for (; s < S; ++s) o += sw[s] * base[s * rec + d];
        out[((int64_t)r * n_q + h) * hd + d] = f2h(o * inv);
    }
}

}  // namespace

// Keys per split: about two blocks per CU (each block streams its keys in
// double-buffered chunks), at least 64 keys each; long prefills are their own
// blocks.
int attn_keys_per_split(int L, int n_kv, int valid_len) {
    const int target_blocks = 2 * num_cus();
    int splits = target_blocks / max(1, n_kv * L);
    if (splits < 1) splits = 1;
    int kps = (valid_len + splits - 1) / splits;
    if (kps < 64) kps = 64;
    return kps;
}

}  // namespace bx

using namespace bx;

extern "C" {

size_t bx_attention_workspace_bytes(int L, int n_q, int hd, int valid_len) {
    if (L <= 0 || n_q <= 0 || hd <= 0 || valid_len <= 0) return 0;
    // Worst case over n_kv >= 1 is n_kv = 1 (most splits).
    const int kps = attn_keys_per_split(L, 1, valid_len);
    const int S = (valid_len + kps - 1) / kps;
    return (size_t)L * n_q * S * (hd + 2) * sizeof(float);
}

int bx_attention_decode_f16(const uint16_t* q, const uint16_t* Kc, const uint16_t* Vc, int L, int valid_len, int n_q,
                            int n_kv, int hd, float softcap, int window, uint16_t* out, void* workspace,
                            void* stream) {
    if (!q || !Kc || !Vc || !out || !workspace) return fail(BX_EINVAL, "attention: null pointer");
    if (L <= 0 || n_q <= 0 || n_kv <= 0 || n_q % n_kv) return fail(BX_EINVAL, "attention: bad head counts");
    if (n_q / n_kv > kAttnMaxGroup) return fail(BX_EUNSUPPORTED, "attention: GQA group larger than 8");
    if (hd <= 0 || hd % 8 || hd > 256) return fail(BX_EUNSUPPORTED, "attention: head_dim must be a multiple of 8, <= 256");
    if (valid_len < L) return fail(BX_EINVAL, "attention: valid_len < L");
    if (attn_mfma_supported(L, hd, softcap, window, nullptr))
        return attn_mfma(q, Kc, Vc, L, valid_len, n_q, n_kv, hd, 0, out, as_stream(stream));
    if (!attn_span_ok(valid_len, n_kv, hd)) return fail(BX_EUNSUPPORTED, "attention: cache rows span 2 GiB or more");
    AttnArgs a{};
    a.q = q; a.Kc = Kc; a.Vc = Vc; a.mask = nullptr;
    a.L = L; a.valid_len = valid_len; a.n_q = n_q; a.n_kv = n_kv; a.hd = hd;
    a.softcap = softcap; a.window = window;
    a.kps = attn_keys_per_split(L, n_kv, valid_len);
    a.S = (valid_len + a.kps - 1) / a.kps;
    a.ws = static_cast<float*>(workspace);
    hipStream_t st = as_stream(stream);
    attn_partial_launch(a, L, st);
    if (int rc = launch_check("attention partial")) return rc;
    attn_combine_kernel<<<dim3(n_q, L), 128, combine_lds(a.S), st>>>(a.ws, n_q, hd, a.S, out);
    return launch_check("attention combine");
}

int bx_attention_gqa_f16(const uint16_t* q, const uint16_t* K, const uint16_t* V, int L, int n_keys, int n_q,
                         int n_kv, int hd, int causal, uint16_t* out, void* workspace, void* stream) {
    if (!q || !K || !V || !out || !workspace) return fail(BX_EINVAL, "attention_gqa: null pointer");
    if (L <= 0 || n_keys <= 0 || n_q <= 0 || n_kv <= 0 || n_q % n_kv)
        return fail(BX_EINVAL, "attention_gqa: bad shape");
    if (n_q / n_kv > kAttnMaxGroup) return fail(BX_EUNSUPPORTED, "attention_gqa: GQA group larger than 8");
    if (hd <= 0 || hd % 8 || hd > 256)
        return fail(BX_EUNSUPPORTED, "attention_gqa: head_dim must be a multiple of 8, <= 256");
    if (causal && n_keys < L) return fail(BX_EINVAL, "attention_gqa: causal with fewer keys than rows");
    if (attn_mfma_supported(L, hd, 0.f, 0, nullptr))
        return attn_mfma(q, K, V, L, n_keys, n_q, n_kv, hd, causal ? 0 : 1, out, as_stream(stream));
    if (!attn_span_ok(n_keys, n_kv, hd)) return fail(BX_EUNSUPPORTED, "attention_gqa: keys span 2 GiB or more");
    AttnArgs a{};
    a.q = q; a.Kc = K; a.Vc = V; a.mask = nullptr;
    a.L = L; a.valid_len = n_keys; a.n_q = n_q; a.n_kv = n_kv; a.hd = hd;
    a.softcap = 0.f; a.window = 0; a.bidir = causal ? 0 : 1;
    a.kps = attn_keys_per_split(L, n_kv, n_keys);
    a.S = (n_keys + a.kps - 1) / a.kps;
    a.ws = static_cast<float*>(workspace);
    hipStream_t st = as_stream(stream);
    attn_partial_launch(a, L, st);
    if (int rc = launch_check("attention_gqa partial")) return rc;
    attn_combine_kernel<<<dim3(n_q, L), 128, combine_lds(a.S), st>>>(a.ws, n_q, hd, a.S, out);
    return launch_check("attention_gqa combine");
}

int bx_attention_varlen_f16(const uint16_t* q, const uint16_t* Kc, const uint16_t* Vc, int rows,
                            const int32_t* lens_dev, const int64_t* base_rows_dev, int max_len, int n_q, int n_kv,
                            int hd, uint16_t* out, void* workspace, void* stream) {
    if (!q || !Kc || !Vc || !lens_dev || !base_rows_dev || !out || !workspace)
        return fail(BX_EINVAL, "attention_varlen: null pointer");
    if (rows <= 0 || max_len <= 0 || n_q <= 0 || n_kv <= 0 || n_q % n_kv)
        return fail(BX_EINVAL, "attention_varlen: bad shape");
    if (n_q / n_kv > kAttnMaxGroup) return fail(BX_EUNSUPPORTED, "attention_varlen: GQA group larger than 8");
    if (hd <= 0 || hd % 8 || hd > 256) return fail(BX_EUNSUPPORTED, "attention_varlen: bad head_dim");
    if (!attn_span_ok(max_len, n_kv, hd)) return fail(BX_EUNSUPPORTED, "attention_varlen: keys span 2 GiB or more");
    AttnArgs a{};
    a.q = q; a.Kc = Kc; a.Vc = Vc; a.mask = nullptr;
    a.L = rows; a.valid_len = max_len; a.n_q = n_q; a.n_kv = n_kv; a.hd = hd;
    a.softcap = 0.f; a.window = 0;
    a.rlen = lens_dev; a.rbase = base_rows_dev;
    a.kps = attn_keys_per_split(rows, n_kv, max_len);
    a.S = (max_len + a.kps - 1) / a.kps;
    a.ws = static_cast<float*>(workspace);
    hipStream_t st = as_stream(stream);
    attn_partial_launch(a, rows, st);
    if (int rc = launch_check("attention_varlen partial")) return rc;
    attn_combine_kernel<<<dim3(n_q, rows), 128, combine_lds(a.S), st>>>(a.ws, n_q, hd, a.S, out);
    return launch_check("attention_varlen combine");
}

int bx_attention_masked_f16(const uint16_t* q, const uint16_t* Kc, const uint16_t* Vc, const float* mask, int n_keys,
                            int n_q, int n_kv, int hd, uint16_t* out, void* workspace, void* stream) {
    if (!q || !Kc || !Vc || !mask || !out || !workspace) return fail(BX_EINVAL, "attention_masked: null pointer");
    if (n_keys <= 0 || n_q <= 0 || n_kv <= 0 || n_q % n_kv) return fail(BX_EINVAL, "attention_masked: bad shape");
    if (n_q / n_kv > kAttnMaxGroup) return fail(BX_EUNSUPPORTED, "attention_masked: GQA group larger than 8");
    if (hd <= 0 || hd % 8 || hd > 256) return fail(BX_EUNSUPPORTED, "attention_masked: bad head_dim");
    if (!attn_span_ok(n_keys, n_kv, hd)) return fail(BX_EUNSUPPORTED, "attention_masked: keys span 2 GiB or more");
    AttnArgs a{};
    a.q = q; a.Kc = Kc; a.Vc = Vc; a.mask = mask;
    a.L = 1; a.valid_len = n_keys; a.n_q = n_q; a.n_kv = n_kv; a.hd = hd;
    a.softcap = 0.f; a.window = 0;
    a.kps = attn_keys_per_split(1, n_kv, n_keys);
    a.S = (n_keys + a.kps - 1) / a.kps;
    a.ws = static_cast<float*>(workspace);
    hipStream_t st = as_stream(stream);
    attn_partial_launch(a, 1, st);
    if (int rc = launch_check("attention_masked partial")) return rc;
    attn_combine_kernel<<<dim3(n_q, 1), 128, combine_lds(a.S), st>>>(a.ws, n_q, hd, a.S, out);
    return launch_check("attention_masked combine");
}

}  // extern "C"
