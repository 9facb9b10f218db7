// Quant-carrier GEMV core: one lane dots one 32-element "unit" of a weight row
// against FP16 activations staged in LDS, with FP32 accumulation.
//
// Weights are expanded in registers to FP16 pairs with the magic-exponent
// trick (0x6400 | q is the binary16 value 1024+q) followed by one packed FP16
// subtract, which yields the small integer q - offset exactly; v_dot2_f32_f16
// then forms x0*w0 + x1*w1 + acc with exact products.  Per-unit scales are
// applied once in FP32, so the result is the factored form
//     sum_k x_k * (d*sc*q_k - dmin*m) = d*sc*sum_k x_k q_k - dmin*m*sum_k x_k.
//
// LDS activation layout (dwords = FP16 pairs), per activation row m:
//   swizzled (quant formats): group g of 4 elements x[4g..4g+3] is stored as
//     pair 2g = (x[4g], x[4g+2]), pair 2g+1 = (x[4g+1], x[4g+3]); this matches
//     the pairs a 16-bit-lane mask pulls out of a dword of packed bytes/nibbles.
//   natural (FP16 weights): pair p = (x[2p], x[2p+1]).
// xsum16[m][j] = sum of x[16j .. 16j+15] (needed for the Q4_K min term).
#pragma once

#include "carrier_layout.h"
#include "common.h"

namespace bx {

enum { FMT_F16 = BX_TYPE_F16, FMT_Q8_0 = BX_TYPE_Q8_0, FMT_Q4_K = BX_TYPE_Q4_K, FMT_Q6_K = BX_TYPE_Q6_K };

__device__ __forceinline__ uint32_t magic_pair(uint32_t v) { return v | 0x64006400u; }
// (1024 + a, 1024 + b) - (off, off), exact for small integers.
__device__ __forceinline__ uint32_t centre(uint32_t magic, float off) {
    const _Float16 o = (_Float16)(-off);
    return as_u32(as_h2(magic) + (h2){o, o});
}

// ---- weight unit loads (raw register images) -------------------------------

struct RawQ4K { u4v q; u4v h; };
struct RawQ6K { u4v ql; u2v qh; u4v sc; uint32_t d; };
struct RawQ8 { u4v q0, q1; uint32_t d; };
struct RawF16 { u4v w0, w1, w2, w3; };

template <int FMT> struct RawOf;
template <> struct RawOf<FMT_Q4_K> { using T = RawQ4K; };
template <> struct RawOf<FMT_Q6_K> { using T = RawQ6K; };
template <> struct RawOf<FMT_Q8_0> { using T = RawQ8; };
template <> struct RawOf<FMT_F16> { using T = RawF16; };

// Unit u of row n (K elements; units are 32 elements).
template <int FMT>
__device__ __forceinline__ typename RawOf<FMT>::T load_unit(const void* W, int64_t N, int64_t K, int64_t n, int u);

template <>
__device__ __forceinline__ RawQ4K load_unit<FMT_Q4_K>(const void* W, int64_t N, int64_t K, int64_t n, int u) {
    const CarrierQ4K c = carrier_q4k(W, N, K);
    const int64_t s = n * (K / 256) + (u >> 3);
    RawQ4K r;
    r.q = ldg_nt16(c.qs + s * 128 + 16 * (u & 7));
    r.h = ldg16(c.hdr + s * 16);
    return r;
}

template <>
__device__ __forceinline__ RawQ6K load_unit<FMT_Q6_K>(const void* W, int64_t N, int64_t K, int64_t n, int u) {
    const CarrierQ6K c = carrier_q6k(W, N, K);
    const int64_t s = n * (K / 256) + (u >> 3);
    const int t = u & 7;
    RawQ6K r;
    r.ql = ldg_nt16(c.ql + s * 128 + 16 * t);
    r.qh = ldg_nt8(c.qh + s * 64 + 8 * t);
    r.sc = ldg16(c.sc + s * 16);
    r.d = ldg_u16(c.d + s * 2);
    return r;
}

template <>
__device__ __forceinline__ RawQ8 load_unit<FMT_Q8_0>(const void* W, int64_t N, int64_t K, int64_t n, int u) {
    const CarrierQ8 c = carrier_q8(W, N, K);
    const int64_t s = n * (K / 32) + u;
    RawQ8 r;
    r.q0 = ldg_nt16(c.qs + s * 32);
    r.q1 = ldg_nt16(c.qs + s * 32 + 16);
    r.d = ldg_u16(c.d + s * 2);
    return r;
}

template <>
__device__ __forceinline__ RawF16 load_unit<FMT_F16>(const void* W, int64_t N, int64_t K, int64_t n, int u) {
    const uint8_t* p = static_cast<const uint8_t*>(W) + (n * K + (int64_t)u * 32) * 2;
    RawF16 r;
    r.w0 = ldg_nt16(p);
    r.w1 = ldg_nt16(p + 16);
    r.w2 = ldg_nt16(p + 32);
    r.w3 = ldg_nt16(p + 48);
    return r;
}

// ---- unit dot products -------------------------------------------------------
// xs: LDS pairs of activation row 0; row m at xs + m * xstride (dwords).
// xsum: LDS 16-element sums of row 0; row m at xsum + m * sstride.

template <int M>
__device__ __forceinline__ void dot_unit(const RawQ4K& r, int u, const uint32_t* xs, int xstride, const float* xsum,
                                         int sstride, float (&acc)[M]) {
    const int b = u >> 3, t = u & 7, c = t >> 1;
    const int e_lo = 256 * b + 64 * c + 16 * (t & 1);
    const int e_hi = e_lo + 32;
    const float d = h2f(r.h.x & 0xffff), dmin = h2f(r.h.x >> 16);
    int sc0, m0, sc1, m1;
    q4k_pair_scales(r.h.y, r.h.z, r.h.w, c, sc0, m0, sc1, m1);
    const float s_lo = d * (float)sc0, s_hi = d * (float)sc1;
    // sum x*(d*sc*q - dmin*m) with q = (q-8) + 8: s*acc + (8s - dmin*m) * X
    const float c_lo = 8.f * s_lo - dmin * (float)m0;
    const float c_hi = 8.f * s_hi - dmin * (float)m1;
    uint32_t wl[8], wh[8];
    const uint32_t qw[4] = {r.q.x, r.q.y, r.q.z, r.q.w};
#pragma unroll
    for (int k = 0; k < 4; ++k) {
        const uint32_t w = qw[k];
        wl[2 * k] = centre(magic_pair(w & 0x000F000Fu), 1032.f);
        wl[2 * k + 1] = centre(magic_pair((w >> 8) & 0x000F000Fu), 1032.f);
        wh[2 * k] = centre(magic_pair((w >> 4) & 0x000F000Fu), 1032.f);
        wh[2 * k + 1] = centre(magic_pair((w >> 12) & 0x000F000Fu), 1032.f);
    }
#pragma unroll
    for (int m = 0; m < M; ++m) {
        const uint32_t* xl = xs + m * xstride + (e_lo >> 1);
        const uint32_t* xh = xs + m * xstride + (e_hi >> 1);
        const u4v xl0 = *reinterpret_cast<const u4v*>(xl), xl1 = *reinterpret_cast<const u4v*>(xl + 4);
        const u4v xh0 = *reinterpret_cast<const u4v*>(xh), xh1 = *reinterpret_cast<const u4v*>(xh + 4);
        float al = 0.f, ah = 0.f;
        al = dot2(xl0.x, wl[0], al); al = dot2(xl0.y, wl[1], al); al = dot2(xl0.z, wl[2], al); al = dot2(xl0.w, wl[3], al);
        al = dot2(xl1.x, wl[4], al); al = dot2(xl1.y, wl[5], al); al = dot2(xl1.z, wl[6], al); al = dot2(xl1.w, wl[7], al);
        ah = dot2(xh0.x, wh[0], ah); ah = dot2(xh0.y, wh[1], ah); ah = dot2(xh0.z, wh[2], ah); ah = dot2(xh0.w, wh[3], ah);
        ah = dot2(xh1.x, wh[4], ah); ah = dot2(xh1.y, wh[5], ah); ah = dot2(xh1.z, wh[6], ah); ah = dot2(xh1.w, wh[7], ah);
        const float Xl = xsum[m * sstride + (e_lo >> 4)];
        const float Xh = xsum[m * sstride + (e_hi >> 4)];
        acc[m] += s_lo * al + c_lo * Xl + s_hi * ah + c_hi * Xh;
    }
}

template <int M>
__device__ __forceinline__ void dot_unit(const RawQ6K& r, int u, const uint32_t* xs, int xstride, const float*, int,
                                         float (&acc)[M]) {
    const int b = u >> 3, t = u & 7, h = t >> 2, l0 = 8 * (t & 3);
    const float d = h2f(r.d & 0xffff);
    // scales is0 + {0,2,4,6} with is0 = 8h + (l0 >= 16): bytes of dwords (x,y) or (z,w)
    const uint32_t slo = h ? r.sc.z : r.sc.x, shi = h ? r.sc.w : r.sc.y;
    const int sb = (l0 >= 16) ? 8 : 0;
    const float s0 = d * (float)(int8_t)((slo >> sb) & 0xff), s1 = d * (float)(int8_t)((slo >> (16 + sb)) & 0xff);
    const float s2 = d * (float)(int8_t)((shi >> sb) & 0xff), s3 = d * (float)(int8_t)((shi >> (16 + sb)) & 0xff);
    // w[j][p]: group j (0..3), pair p (0..3): p = 2k + {0: elems (4k,4k+2), 1: (4k+1,4k+3)}
    uint32_t w[4][4];
    const uint32_t A[2] = {r.ql.x, r.ql.y}, B[2] = {r.ql.z, r.ql.w}, Hq[2] = {r.qh.x, r.qh.y};
#pragma unroll
    for (int k = 0; k < 2; ++k) {
        const uint32_t a = A[k], bb = B[k], q = Hq[k];
        w[0][2 * k] = (a & 0x000F000Fu) | ((q & 0x00030003u) << 4);
        w[0][2 * k + 1] = ((a >> 8) & 0x000F000Fu) | (((q >> 8) & 0x00030003u) << 4);
        w[1][2 * k] = (bb & 0x000F000Fu) | (((q >> 2) & 0x00030003u) << 4);
        w[1][2 * k + 1] = ((bb >> 8) & 0x000F000Fu) | (((q >> 10) & 0x00030003u) << 4);
        w[2][2 * k] = ((a >> 4) & 0x000F000Fu) | (((q >> 4) & 0x00030003u) << 4);
        w[2][2 * k + 1] = ((a >> 12) & 0x000F000Fu) | (((q >> 12) & 0x00030003u) << 4);
        w[3][2 * k] = ((bb >> 4) & 0x000F000Fu) | (((q >> 6) & 0x00030003u) << 4);
        w[3][2 * k + 1] = ((bb >> 12) & 0x000F000Fu) | (((q >> 14) & 0x00030003u) << 4);
    }
#pragma unroll
    for (int j = 0; j < 4; ++j)
#pragma unroll
        for (int p = 0; p < 4; ++p) w[j][p] = centre(magic_pair(w[j][p]), 1056.f);
    const int e0 = 256 * b + 128 * h + l0;
#pragma unroll
    for (int m = 0; m < M; ++m) {
        const uint32_t* x = xs + m * xstride + (e0 >> 1);
        float a[4];
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const u4v xv = *reinterpret_cast<const u4v*>(x + 16 * j);
            float s = 0.f;
            s = dot2(xv.x, w[j][0], s);
            s = dot2(xv.y, w[j][1], s);
            s = dot2(xv.z, w[j][2], s);
            s = dot2(xv.w, w[j][3], s);
            a[j] = s;
        }
        acc[m] += s0 * a[0] + s1 * a[1] + s2 * a[2] + s3 * a[3];
    }
}

template <int M>
__device__ __forceinline__ void dot_unit(const RawQ8& r, int u, const uint32_t* xs, int xstride, const float*, int,
                                         float (&acc)[M]) {
    const float d = h2f(r.d & 0xffff);
    uint32_t w[16];
    const uint32_t qw[8] = {r.q0.x, r.q0.y, r.q0.z, r.q0.w, r.q1.x, r.q1.y, r.q1.z, r.q1.w};
#pragma unroll
    for (int k = 0; k < 8; ++k) {
        w[2 * k] = centre(magic_pair((qw[k] & 0x00FF00FFu) ^ 0x00800080u), 1152.f);
        w[2 * k + 1] = centre(magic_pair(((qw[k] >> 8) & 0x00FF00FFu) ^ 0x00800080u), 1152.f);
    }
    const int e0 = 32 * u;
#pragma unroll
    for (int m = 0; m < M; ++m) {
        const uint32_t* x = xs + m * xstride + (e0 >> 1);
        float s = 0.f;
#pragma unroll
        for (int q = 0; q < 4; ++q) {
            const u4v xv = *reinterpret_cast<const u4v*>(x + 4 * q);
            s = dot2(xv.x, w[4 * q + 0], s);
            s = dot2(xv.y, w[4 * q + 1], s);
            s = dot2(xv.z, w[4 * q + 2], s);
            s = dot2(xv.w, w[4 * q + 3], s);
        }
        acc[m] += d * s;
    }
}

template <int M>
__device__ __forceinline__ void dot_unit(const RawF16& r, int u, const uint32_t* xs, int xstride, const float*, int,
                                         float (&acc)[M]) {
    const uint32_t w[16] = {r.w0.x, r.w0.y, r.w0.z, r.w0.w, r.w1.x, r.w1.y, r.w1.z, r.w1.w,
                            r.w2.x, r.w2.y, r.w2.z, r.w2.w, r.w3.x, r.w3.y, r.w3.z, r.w3.w};
    const int e0 = 32 * u;
#pragma unroll
    for (int m = 0; m < M; ++m) {
        const uint32_t* x = xs + m * xstride + (e0 >> 1);
        float s = 0.f;
#pragma unroll
        for (int q = 0; q < 4; ++q) {
            const u4v xv = *reinterpret_cast<const u4v*>(x + 4 * q);
            s = dot2(xv.x, w[4 * q + 0], s);
            s = dot2(xv.y, w[4 * q + 1], s);
            s = dot2(xv.z, w[4 * q + 2], s);
            s = dot2(xv.w, w[4 * q + 3], s);
        }
        acc[m] += s;
    }
}

// ---- activation staging --------------------------------------------------------

template <int FMT>
struct XLayout {
    static constexpr bool swizzled = FMT != FMT_F16;
    static constexpr bool needs_sums = FMT == FMT_Q4_K;
};

// Store 4 consecutive FP16 values (x0..x3 bit patterns) of group g into row xs.
template <bool SWZ>
__device__ __forceinline__ void store_group(uint32_t* xs, int g, uint32_t x0, uint32_t x1, uint32_t x2, uint32_t x3) {
    if (SWZ) {
        xs[2 * g] = x0 | (x2 << 16);
        xs[2 * g + 1] = x1 | (x3 << 16);
    } else {
        xs[2 * g] = x0 | (x1 << 16);
        xs[2 * g + 1] = x2 | (x3 << 16);
    }
}

// Stage M rows of FP16 X (row stride ldx elements) into LDS; K % 16 == 0.
template <bool SWZ, bool SUMS>
__device__ void stage_x_f16(const uint16_t* __restrict__ X, int64_t ldx, int M, int K, uint32_t* xs, int xstride,
                            float* xsum, int sstride) {
    const int G = K / 4;
    for (int i = threadIdx.x; i < M * G; i += blockDim.x) {
        const int m = i / G, g = i - m * G;
        const u2v v = *reinterpret_cast<const u2v*>(X + m * ldx + 4 * g);
        store_group<SWZ>(xs + m * xstride, g, v.x & 0xffff, v.x >> 16, v.y & 0xffff, v.y >> 16);
    }
    if (SUMS) {
        const int S = K / 16;
        for (int i = threadIdx.x; i < M * S; i += blockDim.x) {
            const int m = i / S, j = i - m * S;
            const uint16_t* p = X + m * ldx + 16 * j;
            float s = 0.f;
#pragma unroll
            for (int e = 0; e < 16; ++e) s += h2f(p[e]);
            xsum[m * sstride + j] = s;
        }
    }
}

}  // namespace bx

namespace bx {

// FP16 weights against swizzled activations (pairs (x0,x2),(x1,x3) per group of
// 4): the weight dwords (w0,w1),(w2,w3) are re-paired with v_perm.
template <int M>
__device__ __forceinline__ void dot_unit_f16_swz(const RawF16& r, int u, const uint32_t* xs, int xstride,
                                                 float (&acc)[M]) {
    const uint32_t w[16] = {r.w0.x, r.w0.y, r.w0.z, r.w0.w, r.w1.x, r.w1.y, r.w1.z, r.w1.w,
                            r.w2.x, r.w2.y, r.w2.z, r.w2.w, r.w3.x, r.w3.y, r.w3.z, r.w3.w};
    uint32_t p[16];
#pragma unroll
    for (int g = 0; g < 8; ++g) {
        const uint32_t a = w[2 * g], b = w[2 * g + 1];
        p[2 * g] = __builtin_amdgcn_perm(b, a, 0x05040100u);      // (a.lo, b.lo)
        p[2 * g + 1] = __builtin_amdgcn_perm(b, a, 0x07060302u);  // (a.hi, b.hi)
    }
    const int e0 = 32 * u;
#pragma unroll
    for (int m = 0; m < M; ++m) {
        const uint32_t* x = xs + m * xstride + (e0 >> 1);
        float s = 0.f;
#pragma unroll
        for (int q = 0; q < 4; ++q) {
            const u4v xv = *reinterpret_cast<const u4v*>(x + 4 * q);
            s = dot2(xv.x, p[4 * q + 0], s);
            s = dot2(xv.y, p[4 * q + 1], s);
            s = dot2(xv.z, p[4 * q + 2], s);
            s = dot2(xv.w, p[4 * q + 3], s);
        }
        acc[m] += s;
    }
}

}  // namespace bx

namespace bx {

// ---- M = 1 decode core: activations held in registers ------------------------
//
// Each lane owns the units u = lane + 64*i (i < UPL) of every row, so its 32
// activation values per unit are loaded from LDS once and reused for all rows
// the wavefront streams.  R rows are loaded before any math so R*UPL 16-byte
// weight loads are in flight per lane.
//
// The M = 1 dots leave the magic-exponent offset in the weights: a pair is
// built by one v_and_or_b32 per field, (w & mask) | 0x64006400, giving
// 1024 + q (nibble at bits 0-3) or 1024 + 16 q (nibble at bits 4-7), and the
// offsets come off once per segment as offset * sum(x) from 8-element sums of
// the staged activations (xsum8[j] = x[8j] + ... + x[8j+7], FP32).  Products
// stay exact; the FP32 accumulator carries the offset's magnitude, which adds
// about 2^-24 * 1040 * |x| per accumulation, an order below the FP16 rounding
// of x itself.

struct XU {
    uint32_t p[16];   // activation pairs in the unit's weight-pair order
    float s[4];       // sums of the unit's x segments (Q4_K: low / high 16, Q6_K: four 8s)
};

// 8-element sums of an LDS-staged row (any layout: the pairs of an 8-aligned
// segment are a permutation of its elements).
__device__ __forceinline__ void sums8_from_lds(const uint32_t* xs, int K, float* xsum8) {
    for (int j = threadIdx.x; j < K / 8; j += blockDim.x) {
        const u4v v = *reinterpret_cast<const u4v*>(xs + 4 * j);
        xsum8[j] = ((h2f(v.x & 0xffff) + h2f(v.x >> 16)) + (h2f(v.y & 0xffff) + h2f(v.y >> 16))) +
                   ((h2f(v.z & 0xffff) + h2f(v.z >> 16)) + (h2f(v.w & 0xffff) + h2f(v.w >> 16)));
    }
}

template <int FMT>
__device__ __forceinline__ XU load_xu(const uint32_t* xs, const float* xsum8, int u) {
    XU x;
    if constexpr (FMT == FMT_Q4_K) {
        const int b = u >> 3, t = u & 7, c = t >> 1;
        const int e_lo = 256 * b + 64 * c + 16 * (t & 1), e_hi = e_lo + 32;
        const u4v a0 = *reinterpret_cast<const u4v*>(xs + (e_lo >> 1));
        const u4v a1 = *reinterpret_cast<const u4v*>(xs + (e_lo >> 1) + 4);
        const u4v b0 = *reinterpret_cast<const u4v*>(xs + (e_hi >> 1));
        const u4v b1 = *reinterpret_cast<const u4v*>(xs + (e_hi >> 1) + 4);
        x.p[0] = a0.x; x.p[1] = a0.y; x.p[2] = a0.z; x.p[3] = a0.w;
        x.p[4] = a1.x; x.p[5] = a1.y; x.p[6] = a1.z; x.p[7] = a1.w;
        x.p[8] = b0.x; x.p[9] = b0.y; x.p[10] = b0.z; x.p[11] = b0.w;
        x.p[12] = b1.x; x.p[13] = b1.y; x.p[14] = b1.z; x.p[15] = b1.w;
        const f2v sl = *reinterpret_cast<const f2v*>(xsum8 + (e_lo >> 3));
        const f2v sh = *reinterpret_cast<const f2v*>(xsum8 + (e_hi >> 3));
        x.s[0] = sl.x + sl.y;
        x.s[1] = sh.x + sh.y;
        x.s[2] = x.s[3] = 0.f;
    } else if constexpr (FMT == FMT_Q6_K) {
        const int b = u >> 3, t = u & 7, h = t >> 2, l0 = 8 * (t & 3);
        const int e0 = 256 * b + 128 * h + l0;
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const u4v v = *reinterpret_cast<const u4v*>(xs + ((e0 + 32 * j) >> 1));
            x.p[4 * j] = v.x; x.p[4 * j + 1] = v.y; x.p[4 * j + 2] = v.z; x.p[4 * j + 3] = v.w;
            x.s[j] = xsum8[(e0 + 32 * j) >> 3];
        }
    } else {
        const int e0 = 32 * u;
#pragma unroll
        for (int q = 0; q < 4; ++q) {
            const u4v v = *reinterpret_cast<const u4v*>(xs + (e0 >> 1) + 4 * q);
            x.p[4 * q] = v.x; x.p[4 * q + 1] = v.y; x.p[4 * q + 2] = v.z; x.p[4 * q + 3] = v.w;
        }
        x.s[0] = x.s[1] = x.s[2] = x.s[3] = 0.f;
    }
    return x;
}

// 0x64006400 in a VGPR: v_and_or_b32 on gfx9 reads at most one scalar operand
// and no literal, so the masks go in SGPRs and the magic pair in a register.
__device__ __forceinline__ uint32_t magic_vgpr() {
    uint32_t r;
    asm("v_mov_b32 %0, 0x64006400" : "=v"(r));
    return r;
}
// (x & m) | c as one v_and_or_b32, the mask in an SGPR (on gfx9 a VOP3
// instruction reads at most one scalar operand and no literal).  Written out:
// for two nested and-ors (Q6_K's low nibble, then its two high bits) the
// instruction selector emits two ANDs and a three-input OR, three
// instructions where two do.
__device__ __forceinline__ uint32_t and_or(uint32_t x, uint32_t m, uint32_t c) {
    uint32_t r;
    asm("v_and_or_b32 %0, %1, %2, %3" : "=v"(r) : "v"(x), "s"(m), "v"(c));
    return r;
}

// Q4_K unit: low nibbles (bits 0-3 of each byte) give 1024 + q, high nibbles
// masked in place (bits 4-7) give 1024 + 16 q, so
//   sum x w = s_lo (al - 1024 X_lo) - dmin m_lo X_lo
//           + s_hi / 16 (ah - 1024 X_hi) - dmin m_hi X_hi.
__device__ __forceinline__ float dot_reg(const RawQ4K& r, int u, const XU& x) {
    const int c = (u & 7) >> 1;
    const float d = h2f(r.h.x & 0xffff), dmin = h2f(r.h.x >> 16);
    int sc0, m0, sc1, m1;
    q4k_pair_scales(r.h.y, r.h.z, r.h.w, c, sc0, m0, sc1, m1);
    const uint32_t mg = magic_vgpr();
    const uint32_t qw[4] = {r.q.x, r.q.y, r.q.z, r.q.w};
    float al = 0.f, ah = 0.f;
#pragma unroll
    for (int k = 0; k < 4; ++k) {
        const uint32_t w = qw[k], w8 = w >> 8;
        al = dot2(x.p[2 * k], and_or(w, 0x000F000Fu, mg), al);
        al = dot2(x.p[2 * k + 1], and_or(w8, 0x000F000Fu, mg), al);
        ah = dot2(x.p[8 + 2 * k], and_or(w, 0x00F000F0u, mg), ah);
        ah = dot2(x.p[8 + 2 * k + 1], and_or(w8, 0x00F000F0u, mg), ah);
    }
    const float s_lo = d * (float)sc0, s_hi = d * (float)sc1;
    return s_lo * __builtin_fmaf(-1024.f, x.s[0], al) - dmin * (float)m0 * x.s[0] +
           (s_hi * 0.0625f) * __builtin_fmaf(-1024.f, x.s[1], ah) - dmin * (float)m1 * x.s[1];
}

// Q6_K unit: groups 0 and 1 place the 6-bit q at bits 0-5 (1024 + q), groups
// 2 and 3 take the high nibble in place and the two high bits at 8-9
// (1024 + 16 q); with q centred on 32,
//   group 0/1: s_j (a_j - 1056 X_j),  group 2/3: s_j / 16 (a_j - 1536 X_j).
__device__ __forceinline__ float dot_reg(const RawQ6K& r, int u, const XU& x) {
    const int t = u & 7, h = t >> 2, l0 = 8 * (t & 3);
    const float d = h2f(r.d & 0xffff);
    const uint32_t slo = h ? r.sc.z : r.sc.x, shi = h ? r.sc.w : r.sc.y;
    const int sb = (l0 >= 16) ? 8 : 0;
    const uint32_t mg = magic_vgpr();
    const uint32_t A[2] = {r.ql.x, r.ql.y}, B[2] = {r.ql.z, r.ql.w}, Hq[2] = {r.qh.x, r.qh.y};
    float a0 = 0.f, a1 = 0.f, a2 = 0.f, a3 = 0.f;
#pragma unroll
    for (int k = 0; k < 2; ++k) {
        const uint32_t a = A[k], bb = B[k], q = Hq[k];
        const uint32_t a8 = a >> 8, b8 = bb >> 8;
        const uint32_t ql4 = q << 4, qr4 = q >> 4, ql2 = q << 2, qr6 = q >> 6;
        a0 = dot2(x.p[2 * k], and_or(ql4, 0x00300030u, and_or(a, 0x000F000Fu, mg)), a0);
        a0 = dot2(x.p[2 * k + 1], and_or(qr4, 0x00300030u, and_or(a8, 0x000F000Fu, mg)), a0);
        a1 = dot2(x.p[4 + 2 * k], and_or(ql2, 0x00300030u, and_or(bb, 0x000F000Fu, mg)), a1);
        a1 = dot2(x.p[4 + 2 * k + 1], and_or(qr6, 0x00300030u, and_or(b8, 0x000F000Fu, mg)), a1);
        a2 = dot2(x.p[8 + 2 * k], and_or(ql4, 0x03000300u, and_or(a, 0x00F000F0u, mg)), a2);
        a2 = dot2(x.p[8 + 2 * k + 1], and_or(qr4, 0x03000300u, and_or(a8, 0x00F000F0u, mg)), a2);
        a3 = dot2(x.p[12 + 2 * k], and_or(ql2, 0x03000300u, and_or(bb, 0x00F000F0u, mg)), a3);
        a3 = dot2(x.p[12 + 2 * k + 1], and_or(qr6, 0x03000300u, and_or(b8, 0x00F000F0u, mg)), a3);
    }
    const float s0 = d * (float)(int8_t)((slo >> sb) & 0xff), s1 = d * (float)(int8_t)((slo >> (16 + sb)) & 0xff);
    const float s2 = d * (float)(int8_t)((shi >> sb) & 0xff), s3 = d * (float)(int8_t)((shi >> (16 + sb)) & 0xff);
    return s0 * __builtin_fmaf(-1056.f, x.s[0], a0) + s1 * __builtin_fmaf(-1056.f, x.s[1], a1) +
           (s2 * 0.0625f) * __builtin_fmaf(-1536.f, x.s[2], a2) + (s3 * 0.0625f) * __builtin_fmaf(-1536.f, x.s[3], a3);
}

__device__ __forceinline__ float dot_reg(const RawQ8& r, int, const XU& x) {
    const float d = h2f(r.d & 0xffff);
    const uint32_t qw[8] = {r.q0.x, r.q0.y, r.q0.z, r.q0.w, r.q1.x, r.q1.y, r.q1.z, r.q1.w};
    float s = 0.f;
#pragma unroll
    for (int k = 0; k < 8; ++k) {
        s = dot2(x.p[2 * k], centre(magic_pair((qw[k] & 0x00FF00FFu) ^ 0x00800080u), 1152.f), s);
        s = dot2(x.p[2 * k + 1], centre(magic_pair(((qw[k] >> 8) & 0x00FF00FFu) ^ 0x00800080u), 1152.f), s);
    }
    return d * s;
}

// FP16 weights against swizzled activations: re-pair (w0,w1),(w2,w3) -> (w0,w2),(w1,w3).
__device__ __forceinline__ float dot_reg(const RawF16& r, int, const XU& x) {
    const uint32_t w[16] = {r.w0.x, r.w0.y, r.w0.z, r.w0.w, r.w1.x, r.w1.y, r.w1.z, r.w1.w,
                            r.w2.x, r.w2.y, r.w2.z, r.w2.w, r.w3.x, r.w3.y, r.w3.z, r.w3.w};
    float s = 0.f;
#pragma unroll
    for (int g = 0; g < 8; ++g) {
        const uint32_t a = w[2 * g], b = w[2 * g + 1];
        s = dot2(x.p[2 * g], __builtin_amdgcn_perm(b, a, 0x05040100u), s);
        s = dot2(x.p[2 * g + 1], __builtin_amdgcn_perm(b, a, 0x07060302u), s);
    }
    return s;
}

// 64-lane all-reduce (DPP only).
__device__ __forceinline__ float wave_allsum(float v) { return wave_sum(v); }

// Dot products of rows row0 .. row0+R-1 (clamped to N-1 for loads) with the
// activation held in xu; every lane returns the R sums.
// Activation source for rows_dot_m1: registers when a lane owns at most two
// units (K <= 4096), otherwise re-read from LDS per unit to stay in budget
// (REGS overrides the choice: the several-row GEMV keeps at most four units
// of all its rows in registers).
template <int FMT, int UPL, bool REGS = (UPL <= 2)>
struct XCache {
    static constexpr bool kRegs = REGS;
    XU x[kRegs ? UPL : 1];
    const uint32_t* xs;
    const float* xsum;
    __device__ __forceinline__ void init(const uint32_t* xs_, const float* xsum_, int K);
    __device__ __forceinline__ XU get(int i, int u) const;
};

// Rows per wavefront task for a given units-per-lane count.
template <int UPL>
struct RowsPer {
    static constexpr int R = UPL == 1 ? 4 : (UPL == 2 ? 2 : 1);
};

// A Q6_K lane owning more than 8 units (K above 16384) loads them in batches
// of 4, each batch's math before the next batch's loads (measured at K 32768:
// 51 us against 83 us for one batch); every other case issues all its loads
// before any math.
template <int FMT, int UPL, int R>
__device__ __forceinline__ void rows_dot_m1(const void* W, int64_t N, int K, int64_t row0,
                                            const XCache<FMT, UPL>& xu, float (&out)[R]) {
    constexpr int kB = (UPL > 8 && FMT == FMT_Q6_K) ? 4 : UPL;
    static_assert(UPL % kB == 0, "units per lane must be a whole number of batches");
    const int lane = threadIdx.x & 63;
    const int U = K / 32;
    float a[R];
#pragma unroll
    for (int rr = 0; rr < R; ++rr) a[rr] = 0.f;
#pragma unroll
    for (int b0 = 0; b0 < UPL; b0 += kB) {
        typename RawOf<FMT>::T raw[R][kB];
#pragma unroll
        for (int rr = 0; rr < R; ++rr) {
            const int64_t row = row0 + rr < N ? row0 + rr : N - 1;
#pragma unroll
            for (int i = 0; i < kB; ++i) {
                const int u = lane + 64 * (b0 + i);
                if (u < U) raw[rr][i] = load_unit<FMT>(W, N, K, row, u);
            }
        }
#pragma unroll
        for (int rr = 0; rr < R; ++rr) {
#pragma unroll
            for (int i = 0; i < kB; ++i) {
                const int u = lane + 64 * (b0 + i);
                if (u < U) a[rr] += dot_reg(raw[rr][i], u, xu.get(b0 + i, u));
            }
        }
        // keep the next batch's loads behind this batch's math
        if constexpr (kB < UPL) asm volatile("" ::: "memory");
    }
#pragma unroll
    for (int rr = 0; rr < R; ++rr) out[rr] = wave_allsum(a[rr]);
}

// rows_dot_m1 for MR activation rows: every weight unit is loaded once and
// dotted against each row; out[rr][m] is formed exactly as rows_dot_m1 forms
// the one-row sum of activation row m (same units, same order, same lane
// reduction), so each row's result equals a one-row launch's bit for bit.
template <int FMT, int UPL, int R, int MR, bool XR>
__device__ __forceinline__ void rows_dot_mr(const void* W, int64_t N, int K, int64_t row0,
                                            const XCache<FMT, UPL, XR> (&xu)[MR], float (&out)[R][MR]) {
    constexpr int kB = (UPL > 8 && FMT == FMT_Q6_K) ? 4 : UPL;
    static_assert(UPL % kB == 0, "units per lane must be a whole number of batches");
    const int lane = threadIdx.x & 63;
    const int U = K / 32;
    float a[R][MR];
#pragma unroll
    for (int rr = 0; rr < R; ++rr)
#pragma unroll
        for (int m = 0; m < MR; ++m) a[rr][m] = 0.f;
#pragma unroll
    for (int b0 = 0; b0 < UPL; b0 += kB) {
        typename RawOf<FMT>::T raw[R][kB];
#pragma unroll
        for (int rr = 0; rr < R; ++rr) {
            const int64_t row = row0 + rr < N ? row0 + rr : N - 1;
#pragma unroll
            for (int i = 0; i < kB; ++i) {
                const int u = lane + 64 * (b0 + i);
                if (u < U) raw[rr][i] = load_unit<FMT>(W, N, K, row, u);
            }
        }
#pragma unroll
        for (int rr = 0; rr < R; ++rr) {
#pragma unroll
            for (int i = 0; i < kB; ++i) {
                const int u = lane + 64 * (b0 + i);
                if (u < U) {
#pragma unroll
                    for (int m = 0; m < MR; ++m) a[rr][m] += dot_reg(raw[rr][i], u, xu[m].get(b0 + i, u));
                }
            }
        }
        if constexpr (kB < UPL) asm volatile("" ::: "memory");
    }
#pragma unroll
    for (int rr = 0; rr < R; ++rr)
#pragma unroll
        for (int m = 0; m < MR; ++m) out[rr][m] = wave_allsum(a[rr][m]);
}

template <int FMT, int UPL, bool REGS>
__device__ __forceinline__ void XCache<FMT, UPL, REGS>::init(const uint32_t* xs_, const float* xsum_, int K) {
    xs = xs_;
    xsum = xsum_;
    if constexpr (kRegs) load_xu_all<FMT, UPL>(xs_, xsum_, K, x);
}

template <int FMT, int UPL, bool REGS>
__device__ __forceinline__ XU XCache<FMT, UPL, REGS>::get(int i, int u) const {
    if constexpr (kRegs) return x[i];
    else return load_xu<FMT>(xs, xsum, u);
}

template <int FMT, int UPL>
__device__ __forceinline__ void load_xu_all(const uint32_t* xs, const float* xsum, int K, XU (&xu)[UPL]) {
    const int lane = threadIdx.x & 63;
    const int U = K / 32;
#pragma unroll
    for (int i = 0; i < UPL; ++i) {
        const int u = lane + 64 * i;
        if (u < U) xu[i] = load_xu<FMT>(xs, xsum, u);
    }
    // keep the LDS reads issued together, ahead of their first use (the
    // scheduler would otherwise pair each read with its use)
    asm volatile("" ::: "memory");
}

}  // namespace bx

namespace bx {

// Same as rows_dot_m1 for two matrices of one format and shape (gate / up):
// all 2*R rows are in flight before the math.
template <int FMT, int UPL, int R>
__device__ __forceinline__ void rows_dot_m1_pair(const void* Wa, const void* Wb, int64_t N, int K, int64_t row0,
                                                 const XCache<FMT, UPL>& xu, float (&oa)[R], float (&ob)[R]) {
    const int lane = threadIdx.x & 63;
    const int U = K / 32;
    typename RawOf<FMT>::T ra[R][UPL], rb[R][UPL];
#pragma unroll
    for (int rr = 0; rr < R; ++rr) {
        const int64_t row = row0 + rr < N ? row0 + rr : N - 1;
#pragma unroll
        for (int i = 0; i < UPL; ++i) {
            const int u = lane + 64 * i;
            if (u < U) {
                ra[rr][i] = load_unit<FMT>(Wa, N, K, row, u);
                rb[rr][i] = load_unit<FMT>(Wb, N, K, row, u);
            }
        }
    }
#pragma unroll
    for (int rr = 0; rr < R; ++rr) {
        float a = 0.f, b = 0.f;
#pragma unroll
        for (int i = 0; i < UPL; ++i) {
            const int u = lane + 64 * i;
            if (u < U) {
                a += dot_reg(ra[rr][i], u, xu.get(i, u));
                b += dot_reg(rb[rr][i], u, xu.get(i, u));
            }
        }
        oa[rr] = wave_allsum(a);
        ob[rr] = wave_allsum(b);
    }
}

// Units per lane for K (32-element units spread over 64 lanes).
__host__ __device__ constexpr int upl_for(int K) { return (K / 32 + 63) / 64; }

}  // namespace bx

// Dispatch `BODY` with constexpr FMT_ (from a runtime ggml type) and UPL_ (from
// a runtime units-per-lane count in {1,2,3,4,6}).
#define BX_DISPATCH_UPL(upl, ...)                                  \
    switch (upl) {                                                 \
        case 1: { constexpr int UPL_ = 1; __VA_ARGS__; } break;    \
        case 2: { constexpr int UPL_ = 2; __VA_ARGS__; } break;    \
        case 3: { constexpr int UPL_ = 3; __VA_ARGS__; } break;    \
        case 4: { constexpr int UPL_ = 4; __VA_ARGS__; } break;    \
        default: { constexpr int UPL_ = 6; __VA_ARGS__; } break;   \
    }
// As BX_DISPATCH_UPL, with 7..16 units per lane (K up to 32768) run as 16:
// for the GEMVs whose K is an FFN width (down projection, M = 1 linear).
#define BX_DISPATCH_UPL_WIDE(upl, ...)                             \
    switch (upl) {                                                 \
        case 1: { constexpr int UPL_ = 1; __VA_ARGS__; } break;    \
        case 2: { constexpr int UPL_ = 2; __VA_ARGS__; } break;    \
        case 3: { constexpr int UPL_ = 3; __VA_ARGS__; } break;    \
        case 4: { constexpr int UPL_ = 4; __VA_ARGS__; } break;    \
        case 5:                                                    \
        case 6: { constexpr int UPL_ = 6; __VA_ARGS__; } break;    \
        default: { constexpr int UPL_ = 16; __VA_ARGS__; } break;  \
    }
#define BX_DISPATCH_FMT(type, ...)                                                 \
    switch (type) {                                                                \
        case BX_TYPE_Q4_K: { constexpr int FMT_ = bx::FMT_Q4_K; __VA_ARGS__; } break; \
        case BX_TYPE_Q6_K: { constexpr int FMT_ = bx::FMT_Q6_K; __VA_ARGS__; } break; \
        case BX_TYPE_Q8_0: { constexpr int FMT_ = bx::FMT_Q8_0; __VA_ARGS__; } break; \
        default: { constexpr int FMT_ = bx::FMT_F16; __VA_ARGS__; } break;         \
    }
