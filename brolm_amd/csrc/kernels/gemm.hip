// Prefill contraction (M > 16) on MFMA: Y[M,N] = X[M,K] deq(W)[N,K]^T + bias.
// Weight tiles are dequantized to FP16 in LDS with the exact GGUF formula
// (same values as bx_dequant_to_f16), activations are FP16, products
// accumulate in FP32 on v_mfma_f32_16x16x16_f16.
//
// Block tile 64 (M) x 64 (N), K step 32; 4 wavefronts each own a 32x32
// quadrant as 2x2 MFMA tiles of 16x16.
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

}  // namespace

int gemm_f16(int wtype, const void* W, const uint16_t* bias, const uint16_t* X, uint16_t* Y, int M, int N, int K,
             hipStream_t st) {
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

}  // namespace bx
