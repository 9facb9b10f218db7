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

__global__ __launch_bounds__(256) void attn_partial_kernel(AttnArgs a) {
    extern __shared__ __align__(16) float att_smem[];
    const int s = blockIdx.x, g = blockIdx.y, r = blockIdx.z;
    const int G = a.n_q / a.n_kv;
    if (a.rlen) {  // this row's own sequence: its keys start at cache row rbase[r]
        const int64_t shift = a.rbase[r] * (int64_t)a.n_kv * a.hd;
        a.Kc += shift;
        a.Vc += shift;
    }
    const int p = a.rlen ? a.rlen[r] - 1 : a.bidir ? a.valid_len - 1 : a.valid_len - a.L + r;  // last key
    const int lo = a.window > 0 ? max(0, p - a.window + 1) : 0;
    const int kb = max(lo, s * a.kps);
    const int ke = min(p + 1, (s + 1) * a.kps);
    float* qs = att_smem;                    // G * hd (scaled query)
    float* sc = qs + G * a.hd;               // G * 256 scores
    float* red = sc + G * 256;               // scratch for reductions
    const float scale = 1.0f / sqrtf((float)a.hd);
    for (int i = threadIdx.x; i < G * a.hd; i += blockDim.x) {
        const int h = g * G + i / a.hd, d = i % a.hd;
        qs[i] = h2f(a.q[((int64_t)r * a.n_q + h) * a.hd + d]) * scale;
    }
    __syncthreads();
    AttnState st;
    attn_state_init(st);
    attn_range(a, g, kb, ke, qs, sc, red, st, nullptr, nullptr, -1);
    attn_write_partial(a, r, g, s, st);
    attn_write_ml(a, r, g, s, red);
}

__global__ __launch_bounds__(128) void attn_combine_kernel(const float* __restrict__ ws, int n_q, int hd, int S,
                                                          uint16_t* __restrict__ out) {
    const int h = blockIdx.x, r = blockIdx.y;
    const float* base = ws + ((int64_t)r * n_q + h) * S * (hd + 2);
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
        out[((int64_t)r * n_q + h) * hd + d] = f2h(o * inv);
    }
}

}  // namespace

// Keys per split: enough splits to spread one decode row over the chip, few
// for long prefills (each row is already its own set of blocks).
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
    AttnArgs a{};
    a.q = q; a.Kc = Kc; a.Vc = Vc; a.mask = nullptr;
    a.L = L; a.valid_len = valid_len; a.n_q = n_q; a.n_kv = n_kv; a.hd = hd;
    a.softcap = softcap; a.window = window;
    a.kps = attn_keys_per_split(L, n_kv, valid_len);
    a.S = (valid_len + a.kps - 1) / a.kps;
    a.ws = static_cast<float*>(workspace);
    const int G = n_q / n_kv;
    const size_t lds = (size_t)(G * hd + G * 256 + 64) * sizeof(float);
    hipStream_t st = as_stream(stream);
    attn_partial_kernel<<<dim3(a.S, n_kv, L), 256, lds, st>>>(a);
    if (int rc = launch_check("attention partial")) return rc;
    attn_combine_kernel<<<dim3(n_q, L), 128, 0, st>>>(a.ws, n_q, hd, a.S, out);
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
    AttnArgs a{};
    a.q = q; a.Kc = K; a.Vc = V; a.mask = nullptr;
    a.L = L; a.valid_len = n_keys; a.n_q = n_q; a.n_kv = n_kv; a.hd = hd;
    a.softcap = 0.f; a.window = 0; a.bidir = causal ? 0 : 1;
    a.kps = attn_keys_per_split(L, n_kv, n_keys);
    a.S = (n_keys + a.kps - 1) / a.kps;
    a.ws = static_cast<float*>(workspace);
    const int G = n_q / n_kv;
    const size_t lds = (size_t)(G * hd + G * 256 + 64) * sizeof(float);
    hipStream_t st = as_stream(stream);
    attn_partial_kernel<<<dim3(a.S, n_kv, L), 256, lds, st>>>(a);
    if (int rc = launch_check("attention_gqa partial")) return rc;
    attn_combine_kernel<<<dim3(n_q, L), 128, 0, st>>>(a.ws, n_q, hd, a.S, out);
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
    AttnArgs a{};
    a.q = q; a.Kc = Kc; a.Vc = Vc; a.mask = nullptr;
    a.L = rows; a.valid_len = max_len; a.n_q = n_q; a.n_kv = n_kv; a.hd = hd;
    a.softcap = 0.f; a.window = 0;
    a.rlen = lens_dev; a.rbase = base_rows_dev;
    a.kps = attn_keys_per_split(rows, n_kv, max_len);
    a.S = (max_len + a.kps - 1) / a.kps;
    a.ws = static_cast<float*>(workspace);
    const int G = n_q / n_kv;
    const size_t lds = (size_t)(G * hd + G * 256 + 64) * sizeof(float);
    hipStream_t st = as_stream(stream);
    attn_partial_kernel<<<dim3(a.S, n_kv, rows), 256, lds, st>>>(a);
    if (int rc = launch_check("attention_varlen partial")) return rc;
    attn_combine_kernel<<<dim3(n_q, rows), 128, 0, st>>>(a.ws, n_q, hd, a.S, out);
    return launch_check("attention_varlen combine");
}

int bx_attention_masked_f16(const uint16_t* q, const uint16_t* Kc, const uint16_t* Vc, const float* mask, int n_keys,
                            int n_q, int n_kv, int hd, uint16_t* out, void* workspace, void* stream) {
    if (!q || !Kc || !Vc || !mask || !out || !workspace) return fail(BX_EINVAL, "attention_masked: null pointer");
    if (n_keys <= 0 || n_q <= 0 || n_kv <= 0 || n_q % n_kv) return fail(BX_EINVAL, "attention_masked: bad shape");
    if (n_q / n_kv > kAttnMaxGroup) return fail(BX_EUNSUPPORTED, "attention_masked: GQA group larger than 8");
    if (hd <= 0 || hd % 8 || hd > 256) return fail(BX_EUNSUPPORTED, "attention_masked: bad head_dim");
    AttnArgs a{};
    a.q = q; a.Kc = Kc; a.Vc = Vc; a.mask = mask;
    a.L = 1; a.valid_len = n_keys; a.n_q = n_q; a.n_kv = n_kv; a.hd = hd;
    a.softcap = 0.f; a.window = 0;
    a.kps = attn_keys_per_split(1, n_kv, n_keys);
    a.S = (n_keys + a.kps - 1) / a.kps;
    a.ws = static_cast<float*>(workspace);
    const int G = n_q / n_kv;
    const size_t lds = (size_t)(G * hd + G * 256 + 64) * sizeof(float);
    hipStream_t st = as_stream(stream);
    attn_partial_kernel<<<dim3(a.S, n_kv, 1), 256, lds, st>>>(a);
    if (int rc = launch_check("attention_masked partial")) return rc;
    attn_combine_kernel<<<dim3(n_q, 1), 128, 0, st>>>(a.ws, n_q, hd, a.S, out);
    return launch_check("attention_masked combine");
}

}  // extern "C"
