// Prefill / encode attention on the matrix cores (flash attention), for
// L >= 16 query rows: the L > 1 form of brotensor flash_attention_decode
// (reference src/detail/dense_decoder.cpp:606-607, causal with the query rows
// at positions valid_len - L ...) and flash_attention_gqa_forward
// (dense_decoder.cpp:737-745, causal or bidirectional).
//
// Block = 4 wavefronts over one KV head: each wavefront holds NF = GB x R
// query fragments of 16 rows (GB query heads of the group, R row groups), so
// every K / V^T fragment it reads from LDS feeds NF MFMAs.  Keys stream in
// tiles of 64 through LDS (K as stored, V transposed so both MFMA operands
// are contiguous reads), double buffered: the next tile's global loads are
// issued before this tile's MFMAs.  Per key tile, on v_mfma_f32_16x16x32_f16:
//   S^T = K Q^T     (16 keys x 16 queries per fragment; the query fragments
//                    stay in registers for the whole key loop)
//   online softmax  (base-2 exponent, running max / sum per query in FP32;
//                    the four lanes holding a query combine by ds_bpermute;
//                    the running max moves lazily, only by more than 2^8,
//                    and tiles below the diagonal skip the causal mask)
//   O^T += V^T P^T  (P converted to FP16 in registers: the S^T layout is
//                    the B operand's, with the 8 keys of a k-slot group in a
//                    fixed permutation that the V^T reads follow; O^T keeps
//                    each query in one lane, so the rescale needs no shuffle)
// Row tiles are issued latest-first (they see the most keys).  Results
// differ from the split-K kernel by FP16 rounding of P (relative 2^-11).
#include "attention_core.h"

namespace bx {
namespace {

typedef _Float16 fa_h8 __attribute__((ext_vector_type(8)));
typedef float fa_f4 __attribute__((ext_vector_type(4)));

constexpr int kFaKeys = 64;

template <int HD>
struct FaShape {
    static constexpr int KROW = HD + 8;                  // K tile row stride (halves): rows 4 banks apart
    static constexpr int VROW = kFaKeys + 8;             // V^T row stride (halves)
    static constexpr int CH = HD / 8;                    // 16-byte chunks per key row
    static constexpr int KRPP = 256 / CH;                // key rows one loader pass covers
    static constexpr int KPASS = kFaKeys / KRPP;         // loader passes for K
    static constexpr int VKP = kFaKeys / (256 / CH);     // keys per thread in the V transpose (4 or 2)
    static constexpr int VNG = kFaKeys / VKP;            // key groups of the V transpose (16 or 32)
};

// Pairwise max / sum with the lanes 16 and 32 positions away (the other rows
// holding the same query).  v_permlane16/32_swap would keep this off the LDS
// path, but this compiler folds a swap whose two operands hold one value
// into a copy and drops the exchange, so ds_bpermute it is.
__device__ __forceinline__ float fa_max_rows(float v) {
    v = fmaxf(v, __shfl_xor(v, 16));
    return fmaxf(v, __shfl_xor(v, 32));
}
__device__ __forceinline__ float fa_sum_rows(float v) {
    v += __shfl_xor(v, 16);
    return v + __shfl_xor(v, 32);
}

// GB query heads of one KV group x R fragments of 16 rows per wavefront
// (NF = GB * R query fragments share every K / V^T fragment read from LDS);
// 4 wavefronts stack 4 * 16 * R rows.
template <int HD, int GB, int R>
__global__ __launch_bounds__(256, (HD == 128 && GB * R > 2) ? 1 : 2) void fa_kernel(const uint16_t* __restrict__ q, const uint16_t* __restrict__ Kc,
                                                 const uint16_t* __restrict__ Vc, int L, int valid_len, int n_q,
                                                 int n_kv, int bidir, uint16_t* __restrict__ out) {
    using S = FaShape<HD>;
    constexpr int NF = GB * R, BR = 64 * R;
    __shared__ __align__(16) uint16_t Ks[2][kFaKeys * S::KROW];
    __shared__ __align__(16) uint16_t Vt[2][HD * S::VROW];

    const int G = n_q / n_kv, splits = G / GB;
    const int ntile = (L + BR - 1) / BR;
    const int rt = ntile - 1 - (int)blockIdx.x;  // latest rows first: they see the most keys
    const int g = (int)blockIdx.y / splits, h0 = g * G + ((int)blockIdx.y % splits) * GB;
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int lq = lane & 15, lg = lane >> 4;
    const int p0 = valid_len - L;  // position of query row 0
    const int64_t qstride = (int64_t)n_q * HD, kvstride = (int64_t)n_kv * HD;
    const int kend = bidir ? valid_len : min(valid_len, p0 + rt * BR + BR);
    const int nkb = (kend + kFaKeys - 1) / kFaKeys;

    // fragment f: rows row0 + 16*(f / GB) + lq of head h0 + f % GB; this
    // lane holds query lq of each fragment (the column of S^T and O^T)
    const int row0 = rt * BR + wave * 16 * R;
    int last[NF];
    fa_h8 qf[NF][HD / 32];
#pragma unroll
    for (int f = 0; f < NF; ++f) {
        const int qi = row0 + 16 * (f / GB) + lq;
        last[f] = bidir ? valid_len - 1 : min(p0 + qi, valid_len - 1);
        const uint16_t* qrow = q + (int64_t)min(qi, L - 1) * qstride + (int64_t)(h0 + f % GB) * HD;
#pragma unroll
        for (int s = 0; s < HD / 32; ++s) qf[f][s] = *reinterpret_cast<const fa_h8*>(qrow + 32 * s + 8 * lg);
    }

    // loaders: K rows kr0 + KRPP*i, chunk kc (a row per CH lanes, coalesced);
    // V keys vq*VKP .. +VKP, chunk vc, consecutive lanes on consecutive key
    // groups so that the transposed LDS writes of a wavefront land on
    // consecutive banks (a lane per d-chunk instead puts 16 lanes 8 rows of
    // V^T apart, an 8-way bank conflict on every write)
    const int kr0 = tid / S::CH, kc = (tid % S::CH) * 8;
    const int vq = tid % S::VNG, vc = (tid / S::VNG) * 8;
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

    // O^T fragments: o[j][f] holds d = 16j + 4*lg + r (r = 0..3) for query lq of fragment f
    fa_f4 o[HD / 16][NF];
#pragma unroll
    for (int j = 0; j < HD / 16; ++j)
#pragma unroll
        for (int f = 0; f < NF; ++f) o[j][f] = (fa_f4){0.f, 0.f, 0.f, 0.f};
    float m[NF], l[NF];  // running max (base-2 units) and sum per fragment query
#pragma unroll
    for (int f = 0; f < NF; ++f) {
        m[f] = -INFINITY;
        l[f] = 0.f;
    }
    const float sl2 = 1.4426950408889634f / sqrtf((float)HD);
    // the smallest last-visible key over the block's rows (its first row)
    const int first_last = bidir ? valid_len - 1 : min(p0 + rt * BR, valid_len - 1);

    gload(0);
    lstore(0);
    __syncthreads();
    for (int kb = 0; kb < nkb; ++kb) {
        const int cur = kb & 1;
        if (kb + 1 < nkb) gload(kb + 1);

        // S^T: s[t][f] holds keys 16t + 4*lg + r for query lq of fragment f
        fa_f4 s[4][NF];
#pragma unroll
        for (int t = 0; t < 4; ++t) {
#pragma unroll
            for (int f = 0; f < NF; ++f) s[t][f] = (fa_f4){0.f, 0.f, 0.f, 0.f};
#pragma unroll
            for (int ds = 0; ds < HD / 32; ++ds) {
                const fa_h8 a = *reinterpret_cast<const fa_h8*>(&Ks[cur][(16 * t + lq) * S::KROW + 32 * ds + 8 * lg]);
#pragma unroll
                for (int f = 0; f < NF; ++f) s[t][f] = __builtin_amdgcn_mfma_f32_16x16x32_f16(a, qf[f][ds], s[t][f], 0, 0, 0);
            }
        }
        // a tile every query of the block sees in full needs no mask
        const bool full = kb * kFaKeys + kFaKeys - 1 <= first_last;
        const int key0 = kb * kFaKeys + 4 * lg;
#pragma unroll
        for (int f = 0; f < NF; ++f) {
            float mx = -INFINITY;
#pragma unroll
            for (int t = 0; t < 4; ++t)
#pragma unroll
                for (int r = 0; r < 4; ++r) {
                    if (!full && key0 + 16 * t + r > last[f]) s[t][f][r] = -INFINITY;
                    mx = fmaxf(mx, s[t][f][r]);
                }
            mx = fa_max_rows(mx) * sl2;  // the tile's max in base-2 units (sl2 > 0)
            // v_exp_f32 flushes results below 2^-126 to zero: weights that
            // small (scores 87 natural units under the row max) are zero in
            // any FP16 / FP32 sum here anyway
            // Lazy rescale: the running max moves only when some query's tile
            // max exceeds it by more than 8 (a factor 256; P stays <= 256,
            // well inside FP16).  Key 0 is in every query's first tile, so
            // that tile always moves it off -inf.
            if (__any(mx > m[f] + 8.f)) {
                const float mnew = fmaxf(m[f], mx);
                const float alpha = __builtin_amdgcn_exp2f(m[f] - mnew);
                l[f] *= alpha;
#pragma unroll
                for (int j = 0; j < HD / 16; ++j) o[j][f] *= alpha;
                m[f] = mnew;
            }
            const float nm = -m[f];
            float ls = 0.f;
#pragma unroll
            for (int t = 0; t < 4; ++t)
#pragma unroll
                for (int r = 0; r < 4; ++r) {
                    const float p = __builtin_amdgcn_exp2f(fmaf(s[t][f][r], sl2, nm));
                    s[t][f][r] = p;
                    ls += p;
                }
            l[f] += fa_sum_rows(ls);
        }

        // O^T += V^T P^T over two 32-key steps; k-slot 8*lg + e holds key
        // 32*ks + 4*lg + e (e < 4) or 32*ks + 16 + 4*lg + e - 4 (e >= 4)
#pragma unroll
        for (int ks = 0; ks < 2; ++ks) {
            fa_h8 pb[NF];
#pragma unroll
            for (int f = 0; f < NF; ++f)
#pragma unroll
                for (int r = 0; r < 4; ++r) {
                    pb[f][r] = (_Float16)s[2 * ks][f][r];
                    pb[f][4 + r] = (_Float16)s[2 * ks + 1][f][r];
                }
#pragma unroll
            for (int j = 0; j < HD / 16; ++j) {
                const uint16_t* vr = &Vt[cur][(16 * j + lq) * S::VROW + 32 * ks + 4 * lg];
                const u2v lo = *reinterpret_cast<const u2v*>(vr);
                const u2v hi = *reinterpret_cast<const u2v*>(vr + 16);
                const u4v av = {lo.x, lo.y, hi.x, hi.y};
                const fa_h8 a = __builtin_bit_cast(fa_h8, av);
#pragma unroll
                for (int f = 0; f < NF; ++f) o[j][f] = __builtin_amdgcn_mfma_f32_16x16x32_f16(a, pb[f], o[j][f], 0, 0, 0);
            }
        }
        if (kb + 1 < nkb) lstore(cur ^ 1);
        __syncthreads();
    }

    // out[row][head][16j + 4*lg .. +4]: four consecutive d per fragment tile
#pragma unroll
    for (int f = 0; f < NF; ++f) {
        const int row = row0 + 16 * (f / GB) + lq;
        if (row >= L) continue;
        const float inv = 1.0f / l[f];
        uint16_t* orow = out + (int64_t)row * qstride + (int64_t)(h0 + f % GB) * HD + 4 * lg;
#pragma unroll
        for (int j = 0; j < HD / 16; ++j) {
            u2v w;
            w.x = (uint32_t)f2h(o[j][f][0] * inv) | ((uint32_t)f2h(o[j][f][1] * inv) << 16);
            w.y = (uint32_t)f2h(o[j][f][2] * inv) | ((uint32_t)f2h(o[j][f][3] * inv) << 16);
            *reinterpret_cast<u2v*>(orow + 16 * j) = w;
        }
    }
}

template <int HD, int GB, int R>
int fa_launch(const uint16_t* q, const uint16_t* Kc, const uint16_t* Vc, int L, int valid_len, int n_q, int n_kv,
              int bidir, uint16_t* out, hipStream_t st) {
    const int ntile = (L + 64 * R - 1) / (64 * R);
    const int ny = n_kv * ((n_q / n_kv) / GB);
    if (ny > 65535) return fail(BX_EINVAL, "attention: too many heads");
    fa_kernel<HD, GB, R><<<dim3((unsigned)ntile, (unsigned)ny), 256, 0, st>>>(q, Kc, Vc, L, valid_len, n_q, n_kv,
                                                                              bidir, out);
    return launch_check("attention (mfma)");
}

// Fragments per wavefront: 2 for head_dim 128 (two blocks per CU fit in the
// register file, so one block's softmax runs under the other's MFMAs), 4 for
// head_dim 64.  Heads per block: the largest of those, 2, 1 dividing the
// group; the rest are 16-row fragments, halved while the grid would leave
// CUs idle.
template <int HD>
int fa_dispatch(const uint16_t* q, const uint16_t* Kc, const uint16_t* Vc, int L, int valid_len, int n_q, int n_kv,
                int bidir, uint16_t* out, hipStream_t st) {
    const int G = n_q / n_kv;
    const int nf = HD == 128 ? 2 : 4;
    int gb = (G % 4 == 0 && nf == 4) ? 4 : G % 2 == 0 ? 2 : 1;
    auto blocks = [&](int r, int b) { return (int64_t)((L + 64 * r - 1) / (64 * r)) * n_kv * (G / b); };
    int r = nf / gb;
    while (r > 1 && blocks(r, gb) < num_cus()) r /= 2;
    while (gb > 1 && blocks(r, gb) < num_cus()) gb /= 2;  // fewer heads per block: more blocks
    if (gb == 4) return fa_launch<HD, 4, 1>(q, Kc, Vc, L, valid_len, n_q, n_kv, bidir, out, st);
    if (gb == 2) {
        if (r == 2) return fa_launch<HD, 2, 2>(q, Kc, Vc, L, valid_len, n_q, n_kv, bidir, out, st);
        return fa_launch<HD, 2, 1>(q, Kc, Vc, L, valid_len, n_q, n_kv, bidir, out, st);
    }
    if (r == 4) return fa_launch<HD, 1, 4>(q, Kc, Vc, L, valid_len, n_q, n_kv, bidir, out, st);
    if (r == 2) return fa_launch<HD, 1, 2>(q, Kc, Vc, L, valid_len, n_q, n_kv, bidir, out, st);
    return fa_launch<HD, 1, 1>(q, Kc, Vc, L, valid_len, n_q, n_kv, bidir, out, st);
}

}  // namespace

bool attn_mfma_supported(int L, int hd, float softcap, int window, const float* mask) {
    return L >= 16 && (hd == 64 || hd == 128) && softcap == 0.f && window <= 0 && mask == nullptr;
}

int attn_mfma(const uint16_t* q, const uint16_t* Kc, const uint16_t* Vc, int L, int valid_len, int n_q, int n_kv,
              int hd, int bidir, uint16_t* out, hipStream_t st) {
    if (hd == 128) return fa_dispatch<128>(q, Kc, Vc, L, valid_len, n_q, n_kv, bidir, out, st);
    return fa_dispatch<64>(q, Kc, Vc, L, valid_len, n_q, n_kv, bidir, out, st);
}

}  // namespace bx
