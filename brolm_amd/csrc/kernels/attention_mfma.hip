// Prefill / encode attention on the matrix cores (flash attention), for
// L >= 16 query rows: the L > 1 form of brotensor flash_attention_decode
// (reference src/detail/dense_decoder.cpp:606-607, causal with the query rows
// at positions valid_len - L ...) and flash_attention_gqa_forward
// (dense_decoder.cpp:737-745, causal or bidirectional).
//
// Block = 64 query rows of one query head (4 wavefronts x 16 rows); it
// streams its visible keys in tiles of 64 through LDS (K as stored, V
// transposed so both MFMA operands are contiguous 8-byte reads), double
// buffered: the next tile's global loads are issued before this tile's
// MFMAs.  Per key tile and wavefront, on v_mfma_f32_16x16x32_f16:
//   S^T = K Q^T     (16 keys x 16 queries per fragment; the query fragments
//                    stay in registers for the whole key loop)
//   online softmax  (base-2 exponent, running max / sum per query in FP32)
//   O  += P V       (P converted to FP16 in registers: the S^T layout puts
//                    each lane's query in the row the A operand needs, with
//                    the 8 keys of a k-slot group in a fixed permutation that
//                    the V^T reads follow)
// Query tiles are issued latest-first (they see the most keys).  Results
// differ from the split-K kernel by FP16 rounding of P (relative 2^-11).
#include "attention_core.h"

namespace bx {
namespace {

typedef _Float16 fa_h8 __attribute__((ext_vector_type(8)));
typedef float fa_f4 __attribute__((ext_vector_type(4)));

constexpr int kFaRows = 64, kFaKeys = 64;

template <int HD>
struct FaShape {
    static constexpr int KROW = HD + 8;                  // K tile row stride (halves): rows 4 banks apart
    static constexpr int VROW = kFaKeys + 8;             // V^T row stride (halves)
    static constexpr int CH = HD / 8;                    // 16-byte chunks per key row
    static constexpr int KRPP = 256 / CH;                // key rows one loader pass covers
    static constexpr int KPASS = kFaKeys / KRPP;         // loader passes for K
    static constexpr int VKP = kFaKeys / (256 / CH);     // keys per thread in the V transpose (4 or 2)
};

template <int HD>
__global__ __launch_bounds__(256) void fa_kernel(const uint16_t* __restrict__ q, const uint16_t* __restrict__ Kc,
                                                 const uint16_t* __restrict__ Vc, int L, int valid_len, int n_q,
                                                 int n_kv, int bidir, uint16_t* __restrict__ out) {
    using S = FaShape<HD>;
    __shared__ __align__(16) uint16_t Ks[2][kFaKeys * S::KROW];
    __shared__ __align__(16) uint16_t Vt[2][HD * S::VROW];

    const int ntile = (L + kFaRows - 1) / kFaRows;
    const int qt = ntile - 1 - (int)blockIdx.x;
    const int h = (int)blockIdx.y, g = h / (n_q / n_kv);
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int lq = lane & 15, lg = lane >> 4;
    const int p0 = valid_len - L;  // position of query row 0
    const int64_t qstride = (int64_t)n_q * HD, kvstride = (int64_t)n_kv * HD;
    const int kend = bidir ? valid_len : min(valid_len, p0 + qt * kFaRows + kFaRows);
    const int nkb = (kend + kFaKeys - 1) / kFaKeys;

    // this lane's query (the column of its S^T fragments) and the last key it sees
    const int qi = qt * kFaRows + wave * 16 + lq;
    const int last = bidir ? valid_len - 1 : min(p0 + qi, valid_len - 1);
    const uint16_t* qrow = q + (int64_t)min(qi, L - 1) * qstride + (int64_t)h * HD;
    fa_h8 qf[HD / 32];
#pragma unroll
    for (int s = 0; s < HD / 32; ++s) qf[s] = *reinterpret_cast<const fa_h8*>(qrow + 32 * s + 8 * lg);

    // loaders: K rows kr0 + KRPP*i, chunk kc; V keys vq*VKP .. +VKP, chunk vc
    const int kr0 = tid / S::CH, kc = (tid % S::CH) * 8;
    const int vq = tid / S::CH, vc = (tid % S::CH) * 8;
    const uint16_t* kbase = Kc + (int64_t)g * HD;
    const uint16_t* vbase = Vc + (int64_t)g * HD;
    u4v kreg[S::KPASS], vreg[S::VKP];
    auto gload = [&](int kb) {
        const int k0 = kb * kFaKeys;
#pragma unroll
        for (int i = 0; i < S::KPASS; ++i) {
            const int key = min(k0 + kr0 + S::KRPP * i, valid_len - 1);
            kreg[i] = ldg16(kbase + (int64_t)key * kvstride + kc);
        }
#pragma unroll
        for (int i = 0; i < S::VKP; ++i) {
            const int key = min(k0 + vq * S::VKP + i, valid_len - 1);
            vreg[i] = ldg16(vbase + (int64_t)key * kvstride + vc);
        }
    };
    auto lstore = [&](int buf) {
#pragma unroll
        for (int i = 0; i < S::KPASS; ++i)
            *reinterpret_cast<u4v*>(&Ks[buf][(kr0 + S::KRPP * i) * S::KROW + kc]) = kreg[i];
        // V^T[d][key]: the VKP keys of this thread for each of its 8 d values
#pragma unroll
        for (int e = 0; e < 8; ++e) {
            uint32_t hv[S::VKP];
#pragma unroll
            for (int i = 0; i < S::VKP; ++i) hv[i] = (vreg[i][e >> 1] >> (16 * (e & 1))) & 0xffff;
            uint16_t* dst = &Vt[buf][(vc + e) * S::VROW + vq * S::VKP];
            if constexpr (S::VKP == 4) {
                u2v w;
                w.x = hv[0] | (hv[1] << 16);
                w.y = hv[2] | (hv[3] << 16);
                *reinterpret_cast<u2v*>(dst) = w;
            } else {
                *reinterpret_cast<uint32_t*>(dst) = hv[0] | (hv[1] << 16);
            }
        }
    };

    fa_f4 o[HD / 16];
#pragma unroll
    for (int j = 0; j < HD / 16; ++j) o[j] = (fa_f4){0.f, 0.f, 0.f, 0.f};
    float m = -INFINITY, l = 0.f;  // running max (base-2 units) and sum for query lq
    const float sl2 = 1.4426950408889634f / sqrtf((float)HD);

    gload(0);
    lstore(0);
    __syncthreads();
    for (int kb = 0; kb < nkb; ++kb) {
        const int cur = kb & 1;
        if (kb + 1 < nkb) gload(kb + 1);

        // S^T fragments: t-th holds keys 16t + 4*lg + r (r = 0..3) for query lq
        fa_f4 s[4];
#pragma unroll
        for (int t = 0; t < 4; ++t) {
            s[t] = (fa_f4){0.f, 0.f, 0.f, 0.f};
#pragma unroll
            for (int ds = 0; ds < HD / 32; ++ds) {
                const fa_h8 a = *reinterpret_cast<const fa_h8*>(&Ks[cur][(16 * t + lq) * S::KROW + 32 * ds + 8 * lg]);
                s[t] = __builtin_amdgcn_mfma_f32_16x16x32_f16(a, qf[ds], s[t], 0, 0, 0);
            }
        }
        const int key0 = kb * kFaKeys + 4 * lg;
        float mx = -INFINITY;
#pragma unroll
        for (int t = 0; t < 4; ++t)
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const float x = (key0 + 16 * t + r <= last) ? s[t][r] * sl2 : -INFINITY;
                s[t][r] = x;
                mx = fmaxf(mx, x);
            }
        mx = fmaxf(mx, __shfl_xor(mx, 16));
        mx = fmaxf(mx, __shfl_xor(mx, 32));
        const float mnew = fmaxf(m, mx);   // finite: key 0 is in the first tile of every query
        const float alpha = exp2f(m - mnew);
        float ls = 0.f;
#pragma unroll
        for (int t = 0; t < 4; ++t)
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const float p = exp2f(s[t][r] - mnew);
                s[t][r] = p;
                ls += p;
            }
        ls += __shfl_xor(ls, 16);
        ls += __shfl_xor(ls, 32);
        l = l * alpha + ls;
        m = mnew;

        // O rows are queries 4*lg + r: their rescale factors live in lanes 4*lg + r
        float ar[4];
#pragma unroll
        for (int r = 0; r < 4; ++r) ar[r] = __shfl(alpha, 4 * lg + r);
#pragma unroll
        for (int j = 0; j < HD / 16; ++j)
#pragma unroll
            for (int r = 0; r < 4; ++r) o[j][r] *= ar[r];

        // O += P V over two 32-key steps; k-slot 8*lg + e holds key
        // 32*ks + 4*lg + e (e < 4) or 32*ks + 16 + 4*lg + e - 4 (e >= 4)
#pragma unroll
        for (int ks = 0; ks < 2; ++ks) {
            fa_h8 pa;
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                pa[r] = (_Float16)s[2 * ks][r];
                pa[4 + r] = (_Float16)s[2 * ks + 1][r];
            }
#pragma unroll
            for (int j = 0; j < HD / 16; ++j) {
                const uint16_t* vr = &Vt[cur][(16 * j + lq) * S::VROW + 32 * ks + 4 * lg];
                const u2v lo = *reinterpret_cast<const u2v*>(vr);
                const u2v hi = *reinterpret_cast<const u2v*>(vr + 16);
                const u4v bv = {lo.x, lo.y, hi.x, hi.y};
                o[j] = __builtin_amdgcn_mfma_f32_16x16x32_f16(pa, __builtin_bit_cast(fa_h8, bv), o[j], 0, 0, 0);
            }
        }
        if (kb + 1 < nkb) lstore(cur ^ 1);
        __syncthreads();
    }

    // out rows: queries 4*lg + r of this wavefront, column 16j + lq
#pragma unroll
    for (int r = 0; r < 4; ++r) {
        const float lr = __shfl(l, 4 * lg + r);
        const int row = qt * kFaRows + wave * 16 + 4 * lg + r;
        if (row >= L) continue;
        const float inv = 1.0f / lr;
        uint16_t* orow = out + (int64_t)row * qstride + (int64_t)h * HD;
#pragma unroll
        for (int j = 0; j < HD / 16; ++j) orow[16 * j + lq] = f2h(o[j][r] * inv);
    }
}

}  // namespace

bool attn_mfma_supported(int L, int hd, float softcap, int window, const float* mask) {
    return L >= 16 && (hd == 64 || hd == 128) && softcap == 0.f && window <= 0 && mask == nullptr;
}

int attn_mfma(const uint16_t* q, const uint16_t* Kc, const uint16_t* Vc, int L, int valid_len, int n_q, int n_kv,
              int hd, int bidir, uint16_t* out, hipStream_t st) {
    const int ntile = (L + kFaRows - 1) / kFaRows;
    if (n_q > 65535) return fail(BX_EINVAL, "attention: too many heads");
    const dim3 grid((unsigned)ntile, (unsigned)n_q);
    if (hd == 128) fa_kernel<128><<<grid, 256, 0, st>>>(q, Kc, Vc, L, valid_len, n_q, n_kv, bidir, out);
    else fa_kernel<64><<<grid, 256, 0, st>>>(q, Kc, Vc, L, valid_len, n_q, n_kv, bidir, out);
    return launch_check("attention (mfma)");
}

}  // namespace bx
