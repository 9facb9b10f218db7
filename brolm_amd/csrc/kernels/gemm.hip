// Prefill contraction (M > 16) on MFMA: Y[M,N] = X[M,K] deq(W)[N,K]^T + bias.
// Weight tiles are dequantized to FP16 in LDS with the exact GGUF formula
// (same values as bx_dequant_to_f16), activations are FP16, products
// accumulate in FP32.
//
// Two kernels:
//  - gemm_tile_kernel<FMT, BM, BN, NW> (M >= 128, K a multiple of 64): a
//    BM x BN block tile (256x128 with 8 wavefronts as 4x2, or 128x128 with 4
//    as 2x2), each wavefront owning a 64x64 tile of 32x32
//    v_mfma_f32_32x32x16_f16 fragments.  K
//    advances 64 per stage through two LDS buffers: the global loads of
//    stage k+1 (activation rows, raw quant bytes) are issued before the
//    MFMAs of stage k, the weights are dequantized after them and written to
//    the other buffer, one barrier per stage.  Blocks map to tiles so that
//    each XCD (blocks are dispatched round-robin over the 8) works a
//    contiguous run of tiles that share weight columns in its own L2.
//  - gemm_kernel<FMT> (other shapes): 64x64 block tile, K step 32, 4
//    wavefronts each a 32x32 quadrant of 16x16x16 MFMAs.
#include "carrier_layout.h"
#include "common.h"

namespace bx {
namespace {

typedef _Float16 h4 __attribute__((ext_vector_type(4)));
typedef float f4 __attribute__((ext_vector_type(4)));

constexpr int BM = 64, BN = 64, BK = 32;
constexpr int LDSROW = BK + 8;  // halves per LDS row (padding against bank conflicts)

#pragma clang fp contract(off)
// Dequantize 8 consecutive weights [k0, k0+8) of row n into out[8] (FP16 bits).
template <int FMT>
__device__ __forceinline__ void deq8(const void* W, int64_t N, int64_t K, int64_t n, int64_t k0, uint16_t* out);

template <>
__device__ __forceinline__ void deq8<BX_TYPE_F16>(const void* W, int64_t, int64_t K, int64_t n, int64_t k0,
                                                   uint16_t* out) {
    const u4v v = ldg16(static_cast<const uint16_t*>(W) + n * K + k0);
    const uint32_t a[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        out[2 * i] = a[i] & 0xffff;
        out[2 * i + 1] = a[i] >> 16;
    }
}

template <>
__device__ __forceinline__ void deq8<BX_TYPE_Q8_0>(const void* W, int64_t N, int64_t K, int64_t n, int64_t k0,
                                                    uint16_t* out) {
    const CarrierQ8 c = carrier_q8(W, N, K);
    const int64_t s = n * (K / 32) + k0 / 32;
    const float d = h2f(*reinterpret_cast<const uint16_t*>(c.d + s * 2));
    const u2v q = *reinterpret_cast<const u2v*>(c.qs + n * K + k0);
    const uint32_t a[2] = {q.x, q.y};
#pragma unroll
    for (int i = 0; i < 8; ++i) out[i] = f2h(d * (float)(int8_t)((a[i >> 2] >> (8 * (i & 3))) & 0xff));
}

template <>
__device__ __forceinline__ void deq8<BX_TYPE_Q4_K>(const void* W, int64_t N, int64_t K, int64_t n, int64_t k0,
                                                    uint16_t* out) {
    const CarrierQ4K c = carrier_q4k(W, N, K);
    const int64_t s = n * (K / 256) + k0 / 256;
    const int o = (int)(k0 % 256);
    const int j = o / 32, cc = j >> 1, shift = (j & 1) * 4;
    const u4v h = ldg16(c.hdr + s * 16);
    const float d = h2f(h.x & 0xffff), dmin = h2f(h.x >> 16);
    int sc, m;
    q4k_scale_min_regs(h.y, h.z, h.w, j, sc, m);
    const float d1 = d * (float)sc, m1 = dmin * (float)m;
    const u2v q = *reinterpret_cast<const u2v*>(c.qs + s * 128 + 32 * cc + (o % 32));
    const uint32_t a[2] = {q.x, q.y};
#pragma unroll
    for (int i = 0; i < 8; ++i) out[i] = f2h(d1 * (float)((a[i >> 2] >> (8 * (i & 3) + shift)) & 0x0f) - m1);
}

template <>
__device__ __forceinline__ void deq8<BX_TYPE_Q6_K>(const void* W, int64_t N, int64_t K, int64_t n, int64_t k0,
                                                    uint16_t* out) {
    const CarrierQ6K c = carrier_q6k(W, N, K);
    const int64_t s = n * (K / 256) + k0 / 256;
    const int o = (int)(k0 % 256);
    const int h = o / 128, j = (o % 128) / 32, l0 = o % 32;  // l0 in {0, 8, 16, 24}
    const int t = 4 * h + l0 / 8;
    const u2v qa = *reinterpret_cast<const u2v*>(c.ql + s * 128 + 16 * t + ((j & 1) ? 8 : 0));
    const u2v qh = *reinterpret_cast<const u2v*>(c.qh + s * 64 + 8 * t);
    const int8_t scv = (int8_t)c.sc[s * 16 + 8 * h + 2 * j + (l0 >= 16 ? 1 : 0)];
    const float d = h2f(*reinterpret_cast<const uint16_t*>(c.d + s * 2));
    const float d1 = d * (float)scv;
    const uint32_t a[2] = {qa.x, qa.y}, hb[2] = {qh.x, qh.y};
    const int nshift = (j >> 1) * 4;  // groups 2,3 use the high nibble
#pragma unroll
    for (int i = 0; i < 8; ++i) {
        const uint32_t lo = (a[i >> 2] >> (8 * (i & 3) + nshift)) & 0x0f;
        const uint32_t hi = (hb[i >> 2] >> (8 * (i & 3) + 2 * j)) & 0x03;
        out[i] = f2h(d1 * (float)((int)(lo | (hi << 4)) - 32));
    }
}
#pragma clang fp contract(on)

template <int FMT>
__global__ __launch_bounds__(256) void gemm_kernel(const void* __restrict__ W, const uint16_t* __restrict__ X,
                                                  const uint16_t* __restrict__ bias, uint16_t* __restrict__ Y, int M,
                                                  int N, int K) {
    __shared__ __align__(16) uint16_t As[BM * LDSROW];
    __shared__ __align__(16) uint16_t Bs[BN * LDSROW];
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int64_t m_base = (int64_t)blockIdx.y * BM, n_base = (int64_t)blockIdx.x * BN;
    const int wm = (wave >> 1) * 32, wn = (wave & 1) * 32;
    f4 acc[2][2];
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int j = 0; j < 2; ++j) acc[i][j] = (f4){0.f, 0.f, 0.f, 0.f};

    // loader mapping: row = tid / 4 (0..63), 8-element segment = tid % 4
    const int lr = tid >> 2, ls = (tid & 3) * 8;
    const int64_t am = m_base + lr < M ? m_base + lr : M - 1;
    const int64_t bn = n_base + lr < N ? n_base + lr : N - 1;

    for (int k0 = 0; k0 < K; k0 += BK) {
        const u4v xa = ldg16(X + am * K + k0 + ls);
        uint16_t wv[8];
        deq8<FMT>(W, N, K, bn, k0 + ls, wv);
        __syncthreads();
        *reinterpret_cast<u4v*>(&As[lr * LDSROW + ls]) = xa;
        u4v wpk;
        wpk.x = wv[0] | ((uint32_t)wv[1] << 16);
        wpk.y = wv[2] | ((uint32_t)wv[3] << 16);
        wpk.z = wv[4] | ((uint32_t)wv[5] << 16);
        wpk.w = wv[6] | ((uint32_t)wv[7] << 16);
        *reinterpret_cast<u4v*>(&Bs[lr * LDSROW + ls]) = wpk;
        __syncthreads();
#pragma unroll
        for (int kk = 0; kk < BK; kk += 16) {
            h4 a[2], b[2];
            const int kq = kk + 4 * (lane >> 4);
#pragma unroll
            for (int i = 0; i < 2; ++i) {
                a[i] = *reinterpret_cast<const h4*>(&As[(wm + 16 * i + (lane & 15)) * LDSROW + kq]);
                b[i] = *reinterpret_cast<const h4*>(&Bs[(wn + 16 * i + (lane & 15)) * LDSROW + kq]);
            }
#pragma unroll
            for (int i = 0; i < 2; ++i)
#pragma unroll
                for (int j = 0; j < 2; ++j) acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x16f16(a[i], b[j], acc[i][j], 0, 0, 0);
        }
    }
    // C layout: lane holds rows 4*(lane/16)+r, column lane%16 of each 16x16 tile
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int j = 0; j < 2; ++j) {
            const int64_t n = n_base + wn + 16 * j + (lane & 15);
            if (n >= N) continue;
            const float bv = bias ? h2f(bias[n]) : 0.f;
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const int64_t m = m_base + wm + 16 * i + 4 * (lane >> 4) + r;
                if (m < M) Y[m * N + n] = f2h(acc[i][j][r] + bv);
            }
        }
}


// ---------------------------------------------------------------- big tiles

typedef _Float16 h8 __attribute__((ext_vector_type(8)));
typedef float f16v __attribute__((ext_vector_type(16)));

constexpr int TK = 64;         // K per LDS stage
constexpr int TROW = TK + 8;   // halves per LDS row: 144 bytes, rows start 4 banks apart

// The raw bytes behind 8 consecutive weights [k0, k0+8) of one row, loaded
// ahead of the MFMAs that hide their latency, and their FP16 values.
template <int FMT>
struct RawW;
template <>
struct RawW<BX_TYPE_F16> {
    u4v v;
};
template <>
struct RawW<BX_TYPE_Q8_0> {
    u2v q;
    uint32_t d;
};
template <>
struct RawW<BX_TYPE_Q4_K> {
    u4v hdr;
    u2v q;
};
template <>
struct RawW<BX_TYPE_Q6_K> {
    u2v ql, qh;
    uint32_t sc, d;
};

template <int FMT>
__device__ __forceinline__ RawW<FMT> load_w(const void* W, int64_t N, int64_t K, int64_t n, int64_t k0);
template <>
__device__ __forceinline__ RawW<BX_TYPE_F16> load_w<BX_TYPE_F16>(const void* W, int64_t, int64_t K, int64_t n,
                                                                  int64_t k0) {
    return {ldg16(static_cast<const uint16_t*>(W) + n * K + k0)};
}
template <>
__device__ __forceinline__ RawW<BX_TYPE_Q8_0> load_w<BX_TYPE_Q8_0>(const void* W, int64_t N, int64_t K, int64_t n,
                                                                    int64_t k0) {
    const CarrierQ8 c = carrier_q8(W, N, K);
    RawW<BX_TYPE_Q8_0> r;
    r.q = *gptr<u2v>(c.qs + n * K + k0);
    r.d = ldg_u16(c.d + (n * (K / 32) + k0 / 32) * 2);
    return r;
}
template <>
__device__ __forceinline__ RawW<BX_TYPE_Q4_K> load_w<BX_TYPE_Q4_K>(const void* W, int64_t N, int64_t K, int64_t n,
                                                                    int64_t k0) {
    const CarrierQ4K c = carrier_q4k(W, N, K);
    const int64_t s = n * (K / 256) + k0 / 256;
    const int o = (int)(k0 % 256);
    RawW<BX_TYPE_Q4_K> r;
    r.hdr = ldg16(c.hdr + s * 16);
    r.q = *gptr<u2v>(c.qs + s * 128 + 32 * (o / 64) + (o % 32));
    return r;
}
template <>
__device__ __forceinline__ RawW<BX_TYPE_Q6_K> load_w<BX_TYPE_Q6_K>(const void* W, int64_t N, int64_t K, int64_t n,
                                                                    int64_t k0) {
    const CarrierQ6K c = carrier_q6k(W, N, K);
    const int64_t s = n * (K / 256) + k0 / 256;
    const int o = (int)(k0 % 256);
    const int h = o / 128, j = (o % 128) / 32, l0 = o % 32;
    const int t = 4 * h + l0 / 8;
    RawW<BX_TYPE_Q6_K> r;
    r.ql = *gptr<u2v>(c.ql + s * 128 + 16 * t + ((j & 1) ? 8 : 0));
    r.qh = *gptr<u2v>(c.qh + s * 64 + 8 * t);
    r.sc = *gptr<uint8_t>(c.sc + s * 16 + 8 * h + 2 * j + (l0 >= 16 ? 1 : 0));
    r.d = ldg_u16(c.d + s * 2);
    return r;
}

__device__ __forceinline__ u4v pack8(const uint16_t (&v)[8]) {
    u4v p;
    p.x = v[0] | ((uint32_t)v[1] << 16);
    p.y = v[2] | ((uint32_t)v[3] << 16);
    p.z = v[4] | ((uint32_t)v[5] << 16);
    p.w = v[6] | ((uint32_t)v[7] << 16);
    return p;
}

#pragma clang fp contract(off)
// FP16 values of the 8 weights, the same formulas as deq8 / bx_dequant_to_f16.
template <int FMT>
__device__ __forceinline__ u4v decode_w(const RawW<FMT>& r, int k0);
template <>
__device__ __forceinline__ u4v decode_w<BX_TYPE_F16>(const RawW<BX_TYPE_F16>& r, int) {
    return r.v;
}
template <>
__device__ __forceinline__ u4v decode_w<BX_TYPE_Q8_0>(const RawW<BX_TYPE_Q8_0>& r, int) {
    const float d = h2f((uint16_t)r.d);
    const uint32_t a[2] = {r.q.x, r.q.y};
    uint16_t out[8];
#pragma unroll
    for (int i = 0; i < 8; ++i) out[i] = f2h(d * (float)(int8_t)((a[i >> 2] >> (8 * (i & 3))) & 0xff));
    return pack8(out);
}
template <>
__device__ __forceinline__ u4v decode_w<BX_TYPE_Q4_K>(const RawW<BX_TYPE_Q4_K>& r, int k0) {
    const int j = (k0 % 256) / 32, shift = (j & 1) * 4;
    const float d = h2f(r.hdr.x & 0xffff), dmin = h2f(r.hdr.x >> 16);
    int sc, m;
    q4k_scale_min_regs(r.hdr.y, r.hdr.z, r.hdr.w, j, sc, m);
    const float d1 = d * (float)sc, m1 = dmin * (float)m;
    const uint32_t a[2] = {r.q.x, r.q.y};
    uint16_t out[8];
#pragma unroll
    for (int i = 0; i < 8; ++i) out[i] = f2h(d1 * (float)((a[i >> 2] >> (8 * (i & 3) + shift)) & 0x0f) - m1);
    return pack8(out);
}
template <>
__device__ __forceinline__ u4v decode_w<BX_TYPE_Q6_K>(const RawW<BX_TYPE_Q6_K>& r, int k0) {
    const int j = ((k0 % 256) % 128) / 32;
    const float d1 = h2f((uint16_t)r.d) * (float)(int8_t)r.sc;
    const uint32_t a[2] = {r.ql.x, r.ql.y}, hb[2] = {r.qh.x, r.qh.y};
    const int nshift = (j >> 1) * 4;
    uint16_t out[8];
#pragma unroll
    for (int i = 0; i < 8; ++i) {
        const uint32_t lo = (a[i >> 2] >> (8 * (i & 3) + nshift)) & 0x0f;
        const uint32_t hi = (hb[i >> 2] >> (8 * (i & 3) + 2 * j)) & 0x03;
        out[i] = f2h(d1 * (float)((int)(lo | (hi << 4)) - 32));
    }
    return pack8(out);
}
#pragma clang fp contract(on)

// Tile t of T (tiles of M fastest within a weight column) for block b: the
// dispatcher deals blocks to the 8 XCDs round-robin, so XCD x receives
// blocks x, x+8, ...; those are given the x-th contiguous run of tiles.
__device__ __forceinline__ int xcd_tile(int b, int T) {
    const int x = b & 7, i = b >> 3, per = T >> 3, rem = T & 7;
    return (x < rem ? x * (per + 1) : rem * (per + 1) + (x - rem) * per) + i;
}

// What a tile launch computes.  Up to three weights share the activation
// rows X (q / k / v): member i has N[i] output columns in Y[i], tiles_n[i]
// column tiles; a block's tile index runs over the members' column tiles in
// order.  EPI_STORE writes Y = f16(acc + bias); EPI_RESID adds f16(acc) to
// the FP32 residual H[M, N[0]]; EPI_SWIGLU computes gate (W[0]) and up (W[1])
// columns of the same tile and writes Y[0] = f16(f16(silu(f16(gate))) *
// f16(up)), the values the separate linear, silu and mul kernels give.
enum : int { EPI_STORE = 0, EPI_RESID = 1, EPI_SWIGLU = 2 };
struct TileJob {
    const void* W[3];
    uint16_t* Y[3];
    int N[3];
    int tiles_n[3];
    int members;
    int tiles_m;
    float* H;
};

// NW wavefronts (4 or 8) as (NW/2) x 2 over the block tile.
template <int FMT, int TBM, int TBN, int NW, int EPI>
__global__ __launch_bounds__(64 * NW) void gemm_tile_kernel(TileJob job, const uint16_t* __restrict__ X,
                                                           const uint16_t* __restrict__ bias, int M, int K) {
    constexpr int NT = 64 * NW, ROWS = NT / 8;  // threads; rows one loader pass covers
    constexpr int WM = TBM / (NW / 2), WN = TBN / 2;  // wave tile
    constexpr int FM = WM / 32, FN = WN / 32;         // 32x32 fragments per wave
    constexpr int RA = TBM / ROWS, RB = TBN / ROWS;   // loader rows per thread
    // SwiGLU: B rows [0, TBN/2) are gate rows, [TBN/2, TBN) the same up rows
    constexpr int CN = EPI == EPI_SWIGLU ? TBN / 2 : TBN;  // output columns per tile
    static_assert(EPI != EPI_SWIGLU || RB == 2, "SwiGLU tiles take one gate and one up row per loader thread");
    __shared__ __align__(16) uint16_t As[2][TBM * TROW];
    __shared__ __align__(16) uint16_t Bs[2][TBN * TROW];

    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    int tiles = 0;
    for (int i = 0; i < job.members; ++i) tiles += job.tiles_n[i];
    const int t = xcd_tile((int)blockIdx.x, job.tiles_m * tiles);
    int tn = t / job.tiles_m, mem = 0;
    while (tn >= job.tiles_n[mem]) tn -= job.tiles_n[mem++];
    const int N = job.N[mem];
    const int64_t m0 = (int64_t)(t % job.tiles_m) * TBM, n0 = (int64_t)tn * CN;

    // loaders: 8 lanes per row, 8 halves each; rows past M / N read the last
    // row (their results are not stored)
    const int lrow = tid >> 3, lcol = (tid & 7) * 8;
    const uint16_t* xrow[RA];
#pragma unroll
    for (int i = 0; i < RA; ++i) {
        const int64_t m = m0 + lrow + ROWS * i;
        xrow[i] = X + (m < M ? m : M - 1) * (int64_t)K;
    }
    int64_t wrow[RB];
    const void* wsrc[RB];
#pragma unroll
    for (int i = 0; i < RB; ++i) {
        const int r = lrow + ROWS * i;
        const int64_t n = n0 + (EPI == EPI_SWIGLU ? r % CN : r);
        wrow[i] = n < N ? n : N - 1;
        wsrc[i] = EPI == EPI_SWIGLU ? job.W[i] : job.W[mem];
    }
    u4v ra[RA];
    RawW<FMT> rb[RB];
    auto gload = [&](int kt) {
        const int64_t k0 = (int64_t)kt * TK + lcol;
#pragma unroll
        for (int i = 0; i < RA; ++i) ra[i] = ldg16(xrow[i] + k0);
#pragma unroll
        for (int i = 0; i < RB; ++i) rb[i] = load_w<FMT>(wsrc[i], N, K, wrow[i], k0);
    };
    auto lstore = [&](int buf, int kt) {
        const int k0 = (int)(((int64_t)kt * TK + lcol) % 256);
#pragma unroll
        for (int i = 0; i < RA; ++i) *reinterpret_cast<u4v*>(&As[buf][(lrow + ROWS * i) * TROW + lcol]) = ra[i];
#pragma unroll
        for (int i = 0; i < RB; ++i)
            *reinterpret_cast<u4v*>(&Bs[buf][(lrow + ROWS * i) * TROW + lcol]) = decode_w<FMT>(rb[i], k0);
    };

    f16v acc[FM][FN];
#pragma unroll
    for (int f = 0; f < FM; ++f)
#pragma unroll
        for (int g = 0; g < FN; ++g)
#pragma unroll
            for (int r = 0; r < 16; ++r) acc[f][g][r] = 0.f;

    const int nk = K / TK;
    gload(0);
    lstore(0, 0);
    __syncthreads();
    // fragment reads: lane l holds row l%32, k [8*(l/32), +8) of a 32x16 slice
    const int wm0 = (wave >> 1) * WM, wn0 = (wave & 1) * WN;
    const int fr = lane & 31, fk = 8 * (lane >> 5);
    for (int kt = 0; kt < nk; ++kt) {
        const int cur = kt & 1;
        if (kt + 1 < nk) gload(kt + 1);
#pragma unroll
        for (int kk = 0; kk < TK; kk += 16) {
            h8 a[FM], b[FN];
#pragma unroll
            for (int f = 0; f < FM; ++f)
                a[f] = *reinterpret_cast<const h8*>(&As[cur][(wm0 + 32 * f + fr) * TROW + kk + fk]);
#pragma unroll
            for (int g = 0; g < FN; ++g)
                b[g] = *reinterpret_cast<const h8*>(&Bs[cur][(wn0 + 32 * g + fr) * TROW + kk + fk]);
#pragma unroll
            for (int f = 0; f < FM; ++f)
#pragma unroll
                for (int g = 0; g < FN; ++g)
                    acc[f][g] = __builtin_amdgcn_mfma_f32_32x32x16_f16(a[f], b[g], acc[f][g], 0, 0, 0);
        }
        if (kt + 1 < nk) lstore(cur ^ 1, kt + 1);
        __syncthreads();
    }

    // D layout: lane l, register r holds row 8*(r/4) + 4*(l/32) + r%4, column l%32
    if constexpr (EPI == EPI_SWIGLU) {
        // the up wavefront (right half of the tile) hands its accumulators to
        // the gate wavefront of the same rows through LDS (the loop's buffers
        // are free after its last barrier)
        float* xs = reinterpret_cast<float*>(&As[0][0]);
        const int wm = wave >> 1;
        if (wave & 1) {
#pragma unroll
            for (int f = 0; f < FM; ++f)
#pragma unroll
                for (int g = 0; g < FN; ++g)
#pragma unroll
                    for (int r = 0; r < 16; ++r) xs[(((wm * FM + f) * FN + g) * 16 + r) * 64 + lane] = acc[f][g][r];
        }
        __syncthreads();
        if (!(wave & 1)) {
            uint16_t* Y = job.Y[0];
#pragma unroll
            for (int g = 0; g < FN; ++g) {
                const int64_t n = n0 + 32 * g + (lane & 31);
                if (n >= N) continue;
#pragma unroll
                for (int f = 0; f < FM; ++f)
#pragma unroll
                    for (int r = 0; r < 16; ++r) {
                        const int64_t m = m0 + wm0 + 32 * f + 8 * (r >> 2) + 4 * (lane >> 5) + (r & 3);
                        if (m >= M) continue;
                        const float up = h2f(f2h(xs[(((wm * FM + f) * FN + g) * 16 + r) * 64 + lane]));
                        const float act = h2f(f2h(silu_f32(h2f(f2h(acc[f][g][r])))));
                        Y[m * N + n] = f2h(act * up);
                    }
            }
        }
    } else {
#pragma unroll
        for (int g = 0; g < FN; ++g) {
            const int64_t n = n0 + wn0 + 32 * g + (lane & 31);
            if (n >= N) continue;
            const float bv = (EPI == EPI_STORE && bias) ? h2f(bias[n]) : 0.f;
#pragma unroll
            for (int f = 0; f < FM; ++f)
#pragma unroll
                for (int r = 0; r < 16; ++r) {
                    const int64_t m = m0 + wm0 + 32 * f + 8 * (r >> 2) + 4 * (lane >> 5) + (r & 3);
                    if (m >= M) continue;
                    if constexpr (EPI == EPI_RESID) job.H[m * N + n] += h2f(f2h(acc[f][g][r]));
                    else job.Y[mem][m * N + n] = f2h(acc[f][g][r] + bv);
                }
        }
    }
}

template <int FMT, int TBM, int TBN, int NW, int EPI>
int launch_tiles(TileJob job, const uint16_t* bias, const uint16_t* X, int M, int K, hipStream_t st) {
    constexpr int CN = EPI == EPI_SWIGLU ? TBN / 2 : TBN;
    job.tiles_m = (M + TBM - 1) / TBM;
    int64_t tiles = 0;
    for (int i = 0; i < job.members; ++i) {
        job.tiles_n[i] = (job.N[i] + CN - 1) / CN;
        tiles += job.tiles_n[i];
    }
    tiles *= job.tiles_m;
    if (tiles > (1 << 30)) return fail(BX_EINVAL, "gemm: too many tiles");
    gemm_tile_kernel<FMT, TBM, TBN, NW, EPI><<<dim3((unsigned)tiles), 64 * NW, 0, st>>>(job, X, bias, M, K);
    return launch_check("gemm_tile");
}

template <int FMT, int EPI>
int gemm_tiles(const TileJob& job, const uint16_t* bias, const uint16_t* X, int M, int K, hipStream_t st) {
    // 256x128 tiles (eight wavefronts, two per SIMD: one wave's
    // dequantization overlaps the other's MFMAs) when they still give every
    // CU a block, else 128x128; SwiGLU tiles always take 256 rows x 64 gate
    // and 64 up columns
    // ... and 64x64 tiles (four wavefronts of one 32x32 fragment) where
    // 128x128 would leave CUs without a block.  Every tile shape runs the same
    // 32x32x16 MFMA over the same K order, so an output element gets the same
    // bits whichever tile computes it.
    int64_t cols = 0, cols64 = 0;
    for (int i = 0; i < job.members; ++i) {
        cols += (job.N[i] + 127) / 128;
        cols64 += (job.N[i] + (EPI == EPI_SWIGLU ? 31 : 63)) / (EPI == EPI_SWIGLU ? 32 : 64);
    }
    const int64_t big = (int64_t)((M + 255) / 256) * cols;
    const int64_t mid = (int64_t)((M + 127) / 128) * cols;
    if constexpr (EPI == EPI_SWIGLU) {
        if (big >= num_cus() || (int64_t)((M + 63) / 64) * cols64 <= big)
            return launch_tiles<FMT, 256, 128, 8, EPI>(job, bias, X, M, K, st);
        return launch_tiles<FMT, 64, 64, 4, EPI>(job, bias, X, M, K, st);
    } else {
        if (big >= num_cus()) return launch_tiles<FMT, 256, 128, 8, EPI>(job, bias, X, M, K, st);
        if (mid >= num_cus()) return launch_tiles<FMT, 128, 128, 4, EPI>(job, bias, X, M, K, st);
        return launch_tiles<FMT, 64, 64, 4, EPI>(job, bias, X, M, K, st);
    }
}

template <int EPI>
int gemm_tiles_typed(int wtype, const TileJob& job, const uint16_t* bias, const uint16_t* X, int M, int K,
                     hipStream_t st) {
    switch (wtype) {
        case BX_TYPE_Q4_K: return gemm_tiles<BX_TYPE_Q4_K, EPI>(job, bias, X, M, K, st);
        case BX_TYPE_Q6_K: return gemm_tiles<BX_TYPE_Q6_K, EPI>(job, bias, X, M, K, st);
        case BX_TYPE_Q8_0: return gemm_tiles<BX_TYPE_Q8_0, EPI>(job, bias, X, M, K, st);
        case BX_TYPE_F16: return gemm_tiles<BX_TYPE_F16, EPI>(job, bias, X, M, K, st);
        default: return fail(BX_EUNSUPPORTED, "gemm: unsupported type");
    }
}

}  // namespace

bool gemm_tiles_ok(int M, int K);

int gemm_f16(int wtype, const void* W, const uint16_t* bias, const uint16_t* X, uint16_t* Y, int M, int N, int K,
             hipStream_t st) {
    if (gemm_tiles_ok(M, K)) {
        TileJob job{};
        job.W[0] = W;
        job.Y[0] = Y;
        job.N[0] = N;
        job.members = 1;
        return gemm_tiles_typed<EPI_STORE>(wtype, job, bias, X, M, K, st);
    }
    const dim3 grid((unsigned)((N + BN - 1) / BN), (unsigned)((M + BM - 1) / BM));
    if (grid.y > 65535) return fail(BX_EINVAL, "gemm: M too large");
    switch (wtype) {
        case BX_TYPE_Q4_K: gemm_kernel<BX_TYPE_Q4_K><<<grid, 256, 0, st>>>(W, X, bias, Y, M, N, K); break;
        case BX_TYPE_Q6_K: gemm_kernel<BX_TYPE_Q6_K><<<grid, 256, 0, st>>>(W, X, bias, Y, M, N, K); break;
        case BX_TYPE_Q8_0: gemm_kernel<BX_TYPE_Q8_0><<<grid, 256, 0, st>>>(W, X, bias, Y, M, N, K); break;
        case BX_TYPE_F16: gemm_kernel<BX_TYPE_F16><<<grid, 256, 0, st>>>(W, X, bias, Y, M, N, K); break;
        default: return fail(BX_EUNSUPPORTED, "gemm: unsupported type");
    }
    return launch_check("gemm");
}

bool gemm_tiles_ok(int M, int K) { return M >= 128 && K % TK == 0; }

int gemm_group_f16(int wtype, int members, const void* const* W, uint16_t* const* Y, const int* N,
                   const uint16_t* X, int M, int K, hipStream_t st) {
    TileJob job{};
    job.members = members;
    for (int i = 0; i < members; ++i) {
        job.W[i] = W[i];
        job.Y[i] = Y[i];
        job.N[i] = N[i];
    }
    return gemm_tiles_typed<EPI_STORE>(wtype, job, nullptr, X, M, K, st);
}

int gemm_resid_f16(int wtype, const void* W, const uint16_t* X, float* H, int M, int N, int K, hipStream_t st) {
    TileJob job{};
    job.W[0] = W;
    job.N[0] = N;
    job.members = 1;
    job.H = H;
    return gemm_tiles_typed<EPI_RESID>(wtype, job, nullptr, X, M, K, st);
}

int gemm_swiglu_f16(int wtype, const void* Wg, const void* Wu, const uint16_t* X, uint16_t* Y, int M, int F, int K,
                    hipStream_t st) {
    TileJob job{};
    job.W[0] = Wg;
    job.W[1] = Wu;
    job.Y[0] = Y;
    job.N[0] = F;
    job.members = 1;
    return gemm_tiles_typed<EPI_SWIGLU>(wtype, job, nullptr, X, M, K, st);
}

}  // namespace bx
