// Quant-carrier / FP16 batched linear (brotensor linear_forward_batched_*_fp16,
// dispatched at include/brolm/detail/compute.h:54-86): Y[M,N] = X[M,K] W[N,K]^T.
// M = 1: GEMV kernels (lanes across K, rows per wavefront); 2 <= M <= 4 over
// lm_head-sized matrices: the same kernel with the rows' activations held per
// lane (gemv_mr_kernel).
// 3 <= M <= 16 with K % 256 == 0: the matrix-core GEMV (gemv_mfma.hip), except
// M = 2 and 4 (see gemv_f16) and other K, which take the per-row GEMV kernel.
// M > 16: the prefill GEMM (gemm.hip).
#include <type_traits>

#include "gemv_core.h"

namespace bx {

bool gemm_tiles_ok(int M, int K);
int gemm_group_f16(int wtype, int members, const void* const* W, uint16_t* const* Y, const int* N,
                   const uint16_t* X, int M, int K, hipStream_t st);
int gemm_resid_f16(int wtype, const void* W, const uint16_t* X, float* H, int M, int N, int K, hipStream_t st);
int gemm_swiglu_f16(int wtype, const void* Wg, const void* Wu, const uint16_t* X, uint16_t* Y, int M, int F, int K,
                    hipStream_t st);
int gemm_f16(int wtype, const void* W, const uint16_t* bias, const uint16_t* X, uint16_t* Y, int M, int N, int K,
             hipStream_t st);
int gemv_mfma(int wtype, const void* W, const uint16_t* bias, const uint16_t* X, uint16_t* Y, int M, int N, int K,
              void* ws, size_t wsb, hipStream_t st);
// One-row GEMV with K split over a workgroup's wavefronts (K 24576 or 32768):
// FP16 out (+ bias), or with h non-null added into the FP32 residual h.
int gemv_m1_ksplit(int wtype, const void* W, const uint16_t* X, const uint16_t* bias, uint16_t* Y, float* h, int N,
                   int K, hipStream_t st);
int gemv_mfma_split(int wtype, const void* W, const uint16_t* bias, const uint16_t* X, uint16_t* Y, int M, int N, int K,
                    void* ws, size_t wsb, hipStream_t st);
int gemv_mfma_group(int wtype, int n, const void* const* W, uint16_t* const* Y, const int* N, const uint16_t* X,
                    int M, int K, void* ws, size_t wsb, hipStream_t st);
int gemv_mfma_resid(int wtype, const void* W, const uint16_t* X, float* H, int M, int N, int K, void* ws, size_t wsb, hipStream_t st);
int gemv_mfma_swiglu(int wtype, const void* Wg, const void* Wu, const uint16_t* X, uint16_t* Y, int M, int F, int K,
                     void* ws, size_t wsb, hipStream_t st);
int gemv_mfma_resid_ss(int wtype, const void* W, const uint16_t* X, float* H, float* ss_out, int M, int N, int K,
                       void* ws, size_t wsb, hipStream_t st);
int gemv_mfma_group_norm(int wtype, int n, const void* const* W, uint16_t* const* Y, const int* N, const float* H,
                         const uint16_t* gamma, float eps, const float* ss_in, int M, int K, void* ws, size_t wsb, hipStream_t st);
int gemv_mfma_swiglu_norm(int wtype, const void* Wg, const void* Wu, const float* H, const uint16_t* gamma, float eps,
                          const float* ss_in, uint16_t* Y, int M, int F, int K, void* ws, size_t wsb, hipStream_t st);
int gemv_mfma_group2(int wtype, int wtype2, int n, int n1, const void* const* W, uint16_t* const* Y, const int* N,
                     const uint16_t* X, const float* H, const uint16_t* gamma, float eps, const float* ss_in, int M,
                     int K, void* ws, size_t wsb, hipStream_t st);

// The fused linear forms run on the MFMA tile GEMM (M >= 128, K % 64 == 0)
// and, for decode batches, on the MFMA GEMV (3 <= M <= 16, K % 256 == 0).
inline bool fused_gemv_ok(int M, int K) { return M >= 3 && M <= 16 && K % 256 == 0; }

namespace {

constexpr int kThreads = 256;
constexpr int kWaves = kThreads / 64;

template <int FMT, int M, int RB>
__global__ __launch_bounds__(kThreads) void gemv_kernel(const void* __restrict__ W, const uint16_t* __restrict__ X,
                                                       int64_t ldx, const uint16_t* __restrict__ bias,
                                                       uint16_t* __restrict__ Y, int64_t ldy, int N, int K) {
    extern __shared__ __align__(16) uint32_t smem[];
    const int xstride = K / 2;
    const int sstride = K / 16;
    uint32_t* xs = smem;
    float* xsum = reinterpret_cast<float*>(smem + M * xstride);
    stage_x_f16<XLayout<FMT>::swizzled, XLayout<FMT>::needs_sums>(X, ldx, M, K, xs, xstride, xsum, sstride);
    __syncthreads();
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int U = K / 32;
    for (int64_t r0 = ((int64_t)blockIdx.x * kWaves + wave) * RB; r0 < N; r0 += (int64_t)gridDim.x * kWaves * RB) {
        float acc[RB][M];
#pragma unroll
        for (int rb = 0; rb < RB; ++rb)
#pragma unroll
            for (int m = 0; m < M; ++m) acc[rb][m] = 0.f;
        for (int u = lane; u < U; u += 64) {
            typename RawOf<FMT>::T raw[RB];
#pragma unroll
            for (int rb = 0; rb < RB; ++rb) {
                const int64_t row = r0 + rb < N ? r0 + rb : N - 1;
                raw[rb] = load_unit<FMT>(W, N, K, row, u);
            }
#pragma unroll
            for (int rb = 0; rb < RB; ++rb) dot_unit<M>(raw[rb], u, xs, xstride, xsum, sstride, acc[rb]);
        }
#pragma unroll
        for (int rb = 0; rb < RB; ++rb) {
            const int64_t row = r0 + rb;
            const float b = (bias && row < N) ? h2f(bias[row]) : 0.f;
#pragma unroll
            for (int m = 0; m < M; ++m) {
                const float v = wave_sum(acc[rb][m]);
                if (lane == 0 && row < N) Y[m * ldy + row] = f2h(v + b);
            }
        }
    }
}

// M = 1: activations staged swizzled for every format, then held in
// registers; each wavefront streams R rows per task (gemv_core.h).
template <int FMT, int UPL>
__global__ __launch_bounds__(kThreads) void gemv_m1_kernel(const void* __restrict__ W,
                                                          const uint16_t* __restrict__ X,
                                                          const uint16_t* __restrict__ bias,
                                                          uint16_t* __restrict__ Y, int N, int K) {
    extern __shared__ __align__(16) uint32_t smem[];
    uint32_t* xs = smem;
    float* xsum = reinterpret_cast<float*>(smem + K / 2);
    stage_x_f16<true, false>(X, K, 1, K, xs, K / 2, xsum, K / 16);
    __syncthreads();
    sums8_from_lds(xs, K, xsum);
    __syncthreads();
    constexpr int R = RowsPer<UPL>::R;
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    XCache<FMT, UPL> xu;
    xu.init(xs, xsum, K);
    const int64_t tasks = ((int64_t)N + R - 1) / R;
    for (int64_t t = (int64_t)blockIdx.x * kWaves + wave; t < tasks; t += (int64_t)gridDim.x * kWaves) {
        float o[R];
        rows_dot_m1<FMT, UPL, R>(W, N, K, t * R, xu, o);
        if (lane == 0) {
#pragma unroll
            for (int rr = 0; rr < R; ++rr) {
                const int64_t row = t * R + rr;
                if (row < N) Y[row] = f2h(o[rr] + (bias ? h2f(bias[row]) : 0.f));
            }
        }
    }
}

// MR <= 4 activation rows with one unit per lane (K <= 2048): each wavefront
// double-buffers its weight-row blocks (the next block's loads go out before
// the current block's math) and keeps its sums in LDS until its last block,
// because a global store inside the loop would make every later wait for
// weights a wait for all loads in flight.  Each weight unit is loaded once for
// the MR rows, and every sum is formed as gemv_m1_kernel forms a one-row sum,
// so row m of Y equals a one-row launch on row m of X bit for bit.
constexpr int kM1pRows = 4;       // rows per block
constexpr int kM1pMaxBlocks = 32; // blocks per wavefront at most (the grid grows past that)
template <int FMT, int MR>
__global__ __launch_bounds__(kThreads) void gemv_m1p_kernel(const void* __restrict__ W,
                                                           const uint16_t* __restrict__ X,
                                                           const uint16_t* __restrict__ bias,
                                                           uint16_t* __restrict__ Y, int N, int K) {
    extern __shared__ __align__(16) uint32_t smem[];
    uint32_t* xs = smem;                                           // MR rows of K / 2 pairs
    float* xsum = reinterpret_cast<float*>(smem + MR * (K / 2));   // MR rows of K / 8 sums
    float* sums = xsum + MR * (K / 8);   // [kWaves][kM1pMaxBlocks * kM1pRows * MR]
    stage_x_f16<true, false>(X, K, MR, K, xs, K / 2, xsum, K / 8);
    __syncthreads();
#pragma unroll
    for (int m = 0; m < MR; ++m) sums8_from_lds(xs + m * (K / 2), K, xsum + m * (K / 8));
    __syncthreads();
    constexpr int R = kM1pRows;
    using Raw = typename RawOf<FMT>::T;
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int U = K / 32;
    const int uc = lane < U ? lane : U - 1;
    XU xu[MR];
#pragma unroll
    for (int m = 0; m < MR; ++m) xu[m] = load_xu<FMT>(xs + m * (K / 2), xsum + m * (K / 8), uc);
    const int64_t tasks = ((int64_t)N + R - 1) / R;
    const int64_t stride = (int64_t)gridDim.x * kWaves;
    const int64_t t0 = (int64_t)blockIdx.x * kWaves + wave;
    float* ws = sums + wave * (kM1pMaxBlocks * R * MR);
    Raw b0[R], b1[R];
    auto load = [&](Raw (&b)[R], int64_t t) {
#pragma unroll
        for (int rr = 0; rr < R; ++rr) {
            const int64_t row = t * R + rr < N ? t * R + rr : N - 1;
            b[rr] = load_unit<FMT>(W, N, K, row, uc);
        }
    };
    int k = 0;
    auto dot = [&](const Raw (&b)[R]) {
        float a[R][MR];
#pragma unroll
        for (int rr = 0; rr < R; ++rr)
#pragma unroll
            for (int m = 0; m < MR; ++m) {
                const float c = dot_reg(b[rr], uc, xu[m]);
                a[rr][m] = lane < U ? c : 0.f;
            }
#pragma unroll
        for (int rr = 0; rr < R; ++rr)
#pragma unroll
            for (int m = 0; m < MR; ++m) a[rr][m] = wave_allsum(a[rr][m]);
        if (lane == 0) {
#pragma unroll
            for (int rr = 0; rr < R; ++rr)
#pragma unroll
                for (int m = 0; m < MR; ++m) ws[(k * R + rr) * MR + m] = a[rr][m];
        }
        ++k;
    };
    // requests are unconditional (past the wave's last block they re-read its
    // current one): a request on one branch only would widen the other
    // buffer's wait to every load in flight
    if (t0 + stride >= tasks) {   // at most one block: nothing to overlap
        if (t0 < tasks) {
            load(b0, t0);
            dot(b0);
        }
    } else {
        load(b0, t0);
        for (int64_t t = t0; t < tasks; t += 2 * stride) {
            const int64_t t1 = t + stride;
            load(b1, t1 < tasks ? t1 : t);
            __builtin_amdgcn_sched_barrier(0);
            dot(b0);
            if (t1 >= tasks) break;
            load(b0, t1 + stride < tasks ? t1 + stride : t1);
            __builtin_amdgcn_sched_barrier(0);
            dot(b1);
        }
    }
    for (int e = lane; e < k * R; e += 64) {
        const int j = e / R, rr = e - j * R;
        const int64_t row = (t0 + (int64_t)j * stride) * R + rr;
        if (row < N) {
            const float bv = bias ? h2f(bias[row]) : 0.f;
#pragma unroll
            for (int m = 0; m < MR; ++m) Y[(int64_t)m * N + row] = f2h(ws[e * MR + m] + bv);
        }
    }
}

// 2 <= M <= 4 (MR rows): gemv_m1_kernel with MR activation rows staged and
// held per lane (in registers while MR x UPL <= 4 units, otherwise re-read
// from LDS): each weight unit is loaded once for all the rows, so a launch
// reads the weight bytes of a one-row launch, and row m of Y equals a one-row
// launch on row m of X bit for bit (rows_dot_mr).
template <int FMT, int UPL, int MR>
__global__ __launch_bounds__(kThreads) void gemv_mr_kernel(const void* __restrict__ W,
                                                          const uint16_t* __restrict__ X,
                                                          const uint16_t* __restrict__ bias,
                                                          uint16_t* __restrict__ Y, int N, int K) {
    extern __shared__ __align__(16) uint32_t smem[];
    uint32_t* xs = smem;                                           // MR rows of K / 2 pairs
    float* xsum = reinterpret_cast<float*>(smem + MR * (K / 2));   // MR rows of K / 8 sums
    stage_x_f16<true, false>(X, K, MR, K, xs, K / 2, xsum, K / 8);
    __syncthreads();
#pragma unroll
    for (int m = 0; m < MR; ++m) sums8_from_lds(xs + m * (K / 2), K, xsum + m * (K / 8));
    __syncthreads();
    constexpr int R = RowsPer<UPL>::R;
    constexpr bool XR = UPL * MR <= 4;
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    XCache<FMT, UPL, XR> xu[MR];
#pragma unroll
    for (int m = 0; m < MR; ++m) xu[m].init(xs + m * (K / 2), xsum + m * (K / 8), K);
    const int64_t tasks = ((int64_t)N + R - 1) / R;
    for (int64_t t = (int64_t)blockIdx.x * kWaves + wave; t < tasks; t += (int64_t)gridDim.x * kWaves) {
        float o[R][MR];
        rows_dot_mr<FMT, UPL, R, MR, XR>(W, N, K, t * R, xu, o);
        if (lane == 0) {
#pragma unroll
            for (int rr = 0; rr < R; ++rr) {
                const int64_t row = t * R + rr;
                if (row < N) {
                    const float b = bias ? h2f(bias[row]) : 0.f;
#pragma unroll
                    for (int m = 0; m < MR; ++m) Y[(int64_t)m * N + row] = f2h(o[rr][m] + b);
                }
            }
        }
    }
}

// M = 1 at K of 24576 or 32768 (U = K / 32 a multiple of 256): the four
// wavefronts of a workgroup split K in quarters, so a lane owns UPW = U / 256
// units of each row (a Q6_K row at K 32768: 4 units, where one wavefront per
// row holds 16 and streams them in four dependent batches).  Each wavefront
// keeps its quarter of the activation in registers for all its rows, requests
// the next row's units before the current row's math (two blocks in turn; the
// request past a chunk's last row repeats that row, so every path issues the
// same loads and the waits stay exact), and parks its quarter sums in LDS; the
// workgroup then adds the four quarters of each row in quarter order and
// stores FP16 (+ bias), or with RESID adds the sum into the FP32 residual h.
constexpr int kKsMaxRows = 64;   // rows of one workgroup chunk (LDS quarter sums)

template <int FMT, int UPW, bool RESID>
__global__ __launch_bounds__(kThreads) void gemv_m1_ksplit_kernel(const void* __restrict__ W,
                                                                 const uint16_t* __restrict__ X,
                                                                 const uint16_t* __restrict__ bias,
                                                                 uint16_t* __restrict__ Y, float* __restrict__ h,
                                                                 int N, int K, int rows) {
    extern __shared__ __align__(16) uint32_t smem[];
    uint32_t* xs = smem;
    float* xsum = reinterpret_cast<float*>(smem + K / 2);
    float* part = xsum + K / 8;
    stage_x_f16<true, false>(X, K, 1, K, xs, K / 2, xsum, K / 16);
    __syncthreads();
    sums8_from_lds(xs, K, xsum);
    __syncthreads();
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int ub = wave * 64 * UPW + lane;   // this lane's first unit
    XU xu[UPW];
#pragma unroll
    for (int i = 0; i < UPW; ++i) xu[i] = load_xu<FMT>(xs, xsum, ub + 64 * i);
    using Raw = typename RawOf<FMT>::T;
    auto load = [&](Raw(&b)[UPW], int64_t row) {
#pragma unroll
        for (int i = 0; i < UPW; ++i) b[i] = load_unit<FMT>(W, N, K, row, ub + 64 * i);
    };
    auto dot = [&](const Raw(&b)[UPW]) {
        float a = 0.f;
#pragma unroll
        for (int i = 0; i < UPW; ++i) a += dot_reg(b[i], ub + 64 * i, xu[i]);
        return wave_allsum(a);
    };
    for (int64_t c0 = (int64_t)blockIdx.x * rows; c0 < N; c0 += (int64_t)gridDim.x * rows) {
        const int nr = (int)(N - c0 < rows ? N - c0 : rows);
        Raw b0[UPW], b1[UPW];
        load(b0, c0);
        for (int j = 0; j < nr; j += 2) {
            load(b1, c0 + min(j + 1, nr - 1));
            const float s0 = dot(b0);
            if (lane == 0) part[4 * j + wave] = s0;
            if (j + 1 >= nr) break;
            load(b0, c0 + min(j + 2, nr - 1));
            const float s1 = dot(b1);
            if (lane == 0) part[4 * (j + 1) + wave] = s1;
        }
        __syncthreads();
        for (int r = threadIdx.x; r < nr; r += kThreads) {
            const float v = ((part[4 * r] + part[4 * r + 1]) + part[4 * r + 2]) + part[4 * r + 3];
            if constexpr (RESID) h[c0 + r] += v;
            else Y[c0 + r] = f2h(v + (bias ? h2f(bias[c0 + r]) : 0.f));
        }
        __syncthreads();
    }
}

// gemv_m1p_kernel for M (1..4) rows at K <= 2048: one round of resident
// workgroups, more where a wavefront would own more than kM1pMaxBlocks blocks.
int launch_gemv_m1p(int wtype, const void* W, const uint16_t* X, const uint16_t* bias, uint16_t* Y, int M, int N,
                    int K, hipStream_t st) {
    const int64_t tasks = ((int64_t)N + kM1pRows - 1) / kM1pRows;
    const size_t lds = (size_t)M * ((size_t)K * 2 + (size_t)(K / 8) * 4) +
                       (size_t)kWaves * kM1pMaxBlocks * kM1pRows * M * 4;
    auto go = [&](auto fn_kernel) -> int {
        const void* fn = reinterpret_cast<const void*>(fn_kernel);
        // resident workgroups per CU, asked once per kernel and LDS size
        struct Occ {
            const void* fn;
            size_t lds;
            int occ;
        };
        thread_local Occ cache[32];
        thread_local int ncache = 0;
        int occ = 0;
        for (int i = 0; i < ncache; ++i)
            if (cache[i].fn == fn && cache[i].lds == lds) occ = cache[i].occ;
        if (occ == 0) {
            if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&occ, fn, kThreads, lds) != hipSuccess || occ < 1) occ = 1;
            cache[ncache < 32 ? ncache++ : 31] = Occ{fn, lds, occ};
        }
        int64_t blocks = std::max<int64_t>((int64_t)num_cus() * occ, (tasks + (int64_t)kWaves * kM1pMaxBlocks - 1) /
                                                                         ((int64_t)kWaves * kM1pMaxBlocks));
        blocks = std::min<int64_t>(blocks, (tasks + kWaves - 1) / kWaves);
        hipLaunchKernelGGL(fn_kernel, dim3((unsigned)blocks), dim3(kThreads), lds, st, W, X, bias, Y, N, K);
        return 0;
    };
    BX_DISPATCH_FMT(wtype, {
        if (M == 1) go(gemv_m1p_kernel<FMT_, 1>);
        else if (M == 2) go(gemv_m1p_kernel<FMT_, 2>);
        else if (M == 3) go(gemv_m1p_kernel<FMT_, 3>);
        else go(gemv_m1p_kernel<FMT_, 4>);
    })
    return launch_check("gemv m1p");
}

int launch_gemv_m1(int wtype, const void* W, const uint16_t* X, const uint16_t* bias, uint16_t* Y, int N, int K,
                   hipStream_t st) {
    const int upl = upl_for(K);
    if (upl > 16) return fail(BX_EUNSUPPORTED, "gemv: K above 32768 at M = 1");
    if (K % 8192 == 0 && K > 16384) return gemv_m1_ksplit(wtype, W, X, bias, Y, nullptr, N, K, st);
    if (upl == 1) return launch_gemv_m1p(wtype, W, X, bias, Y, 1, N, K, st);
    const int R = upl == 1 ? 4 : (upl == 2 ? 2 : 1);
    int64_t blocks = ((int64_t)N + (int64_t)kWaves * R - 1) / ((int64_t)kWaves * R);
    const int64_t cap = (int64_t)num_cus() * 8;
    if (blocks > cap) blocks = cap;
    const size_t lds = (size_t)K * 2 + (size_t)(K / 8) * 4;
    BX_DISPATCH_FMT(wtype, BX_DISPATCH_UPL_WIDE(upl, {
        const void* fn = reinterpret_cast<const void*>(&gemv_m1_kernel<FMT_, UPL_>);
        if (lds > 65536) {   // K above 26214: more than the default 64 KB of dynamic LDS
            if (int rc = hip_check(hipFuncSetAttribute(fn, hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds),
                                   "gemv m1: LDS attribute"))
                return rc;
        }
        // wide rows: one round of resident workgroups (activations staged once each)
        if (UPL_ > 6) blocks = std::min<int64_t>(blocks, (int64_t)num_cus() * BX_WIDE_WGS_PER_CU);
        gemv_m1_kernel<FMT_, UPL_><<<(unsigned)blocks, kThreads, lds, st>>>(W, X, bias, Y, N, K);
    }))
    return launch_check("gemv m1");
}

// Staged activations of the several-row GEMV: M rows of K FP16 values and
// K / 8 sums each.
size_t gemv_mr_lds_bytes(int M, int K) { return (size_t)M * ((size_t)K * 2 + (size_t)(K / 8) * 4); }
bool gemv_mr_ok(int M, int K) { return M >= 2 && M <= 4 && upl_for(K) <= 6 && gemv_mr_lds_bytes(M, K) <= 65536; }

int launch_gemv_mr(int wtype, const void* W, const uint16_t* X, const uint16_t* bias, uint16_t* Y, int M, int N,
                   int K, hipStream_t st) {
    if (!gemv_mr_ok(M, K)) return fail(BX_EUNSUPPORTED, "gemv: several-row kernel shape");
    const int upl = upl_for(K);
    if (upl == 1) return launch_gemv_m1p(wtype, W, X, bias, Y, M, N, K, st);
    const int R = upl == 1 ? 4 : (upl == 2 ? 2 : 1);
    int64_t blocks = ((int64_t)N + (int64_t)kWaves * R - 1) / ((int64_t)kWaves * R);
    const int64_t cap = (int64_t)num_cus() * 8;
    if (blocks > cap) blocks = cap;
    const size_t lds = gemv_mr_lds_bytes(M, K);
    BX_DISPATCH_FMT(wtype, BX_DISPATCH_UPL(upl, {
        if (M == 2) gemv_mr_kernel<FMT_, UPL_, 2><<<(unsigned)blocks, kThreads, lds, st>>>(W, X, bias, Y, N, K);
        else if (M == 3) gemv_mr_kernel<FMT_, UPL_, 3><<<(unsigned)blocks, kThreads, lds, st>>>(W, X, bias, Y, N, K);
        else gemv_mr_kernel<FMT_, UPL_, 4><<<(unsigned)blocks, kThreads, lds, st>>>(W, X, bias, Y, N, K);
    }))
    return launch_check("gemv mr");
}

size_t gemv_lds_bytes(int fmt, int M, int K) {
    size_t b = (size_t)M * K * 2;
    if (fmt == FMT_Q4_K) b += (size_t)M * (K / 16) * 4;
    return b;
}

template <int FMT, int M>
int launch_gemv(const void* W, const uint16_t* X, int64_t ldx, const uint16_t* bias, uint16_t* Y, int64_t ldy, int N,
                int K, hipStream_t st) {
    constexpr int RB = M <= 2 ? 2 : 1;
    const int64_t rows_per_block = (int64_t)kWaves * RB;
    int64_t blocks = ((int64_t)N + rows_per_block - 1) / rows_per_block;
    const int64_t cap = (int64_t)num_cus() * 16;
    if (blocks > cap) blocks = cap;
    const size_t lds = gemv_lds_bytes(FMT, M, K);
    gemv_kernel<FMT, M, RB><<<(unsigned)blocks, kThreads, lds, st>>>(W, X, ldx, bias, Y, ldy, N, K);
    return launch_check("gemv");
}

template <int FMT>
int gemv_dispatch(int M, const void* W, const uint16_t* X, const uint16_t* bias, uint16_t* Y, int N, int K,
                  hipStream_t st) {
    // Largest row chunk whose staged activations fit in 64 KB of LDS.
    int m0 = 0;
    while (m0 < M) {
        const int rem = M - m0;
        int mc = 16;
        while (mc > 1 && (mc > rem || gemv_lds_bytes(FMT, mc, K) > 65536)) mc >>= 1;
        if (gemv_lds_bytes(FMT, mc, K) > 65536) return fail(BX_EUNSUPPORTED, "gemv: K too large for LDS staging");
        const uint16_t* Xc = X + (int64_t)m0 * K;
        uint16_t* Yc = Y + (int64_t)m0 * N;
        int rc;
        switch (mc) {
            case 16: rc = launch_gemv<FMT, 16>(W, Xc, K, bias, Yc, N, N, K, st); break;
            case 8: rc = launch_gemv<FMT, 8>(W, Xc, K, bias, Yc, N, N, K, st); break;
            case 4: rc = launch_gemv<FMT, 4>(W, Xc, K, bias, Yc, N, N, K, st); break;
            case 2: rc = launch_gemv<FMT, 2>(W, Xc, K, bias, Yc, N, N, K, st); break;
            default: rc = launch_gemv<FMT, 1>(W, Xc, K, bias, Yc, N, N, K, st); break;
        }
        if (rc) return rc;
        m0 += mc;
    }
    return BX_OK;
}

}  // namespace

int check_linear_shape(int wtype, int M, int N, int K) {
    if (M <= 0 || N <= 0 || K <= 0) return fail(BX_EINVAL, "linear: non-positive shape");
    const int64_t be = type_block_elems(wtype);
    if (wtype != BX_TYPE_F16 && wtype != BX_TYPE_Q8_0 && wtype != BX_TYPE_Q4_K && wtype != BX_TYPE_Q6_K)
        return fail(BX_EUNSUPPORTED, "linear: unsupported weight type " + std::to_string(wtype));
    if (K % 32 != 0 || K % be != 0)
        return fail(BX_EINVAL, "linear: K=" + std::to_string(K) + " must be a multiple of 32 and of the block size");
    return BX_OK;
}

int gemv_m1_ksplit(int wtype, const void* W, const uint16_t* X, const uint16_t* bias, uint16_t* Y, float* h, int N,
                   int K, hipStream_t st) {
    if (K % 8192 != 0 || K <= 16384 || K > 32768) return fail(BX_EUNSUPPORTED, "gemv ksplit: K must be 24576 or 32768");
    // one chunk of rows per CU where N allows, at most kKsMaxRows rows a chunk
    const int cus = num_cus();
    int rows = (int)std::min<int64_t>(kKsMaxRows, ((int64_t)N + cus - 1) / cus);
    if (rows < 1) rows = 1;
    const int64_t blocks = std::min<int64_t>(((int64_t)N + rows - 1) / rows, cus);
    const size_t lds = (size_t)K * 2 + (size_t)(K / 8) * 4 + (size_t)kKsMaxRows * 4 * sizeof(float);
    auto go = [&](auto fmt_c, auto upw_c, auto resid_c) -> int {
        constexpr int F = decltype(fmt_c)::value, P = decltype(upw_c)::value;
        constexpr bool R = decltype(resid_c)::value;
        const void* fn = reinterpret_cast<const void*>(&gemv_m1_ksplit_kernel<F, P, R>);
        if (int rc = hip_check(hipFuncSetAttribute(fn, hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds),
                               "gemv ksplit: LDS attribute"))
            return rc;
        gemv_m1_ksplit_kernel<F, P, R><<<(unsigned)blocks, kThreads, lds, st>>>(W, X, bias, Y, h, N, K, rows);
        return 0;
    };
    using I3 = std::integral_constant<int, 3>;
    using I4 = std::integral_constant<int, 4>;
    using RT = std::true_type;
    using RF = std::false_type;
    int rc = 0;
    BX_DISPATCH_FMT(wtype, {
        const std::integral_constant<int, FMT_> f{};
        if (K == 24576) rc = h ? go(f, I3{}, RT{}) : go(f, I3{}, RF{});
        else rc = h ? go(f, I4{}, RT{}) : go(f, I4{}, RF{});
    })
    if (rc) return rc;
    return launch_check("gemv ksplit");
}

int gemv_f16(int wtype, const void* W, const uint16_t* bias, const uint16_t* X, uint16_t* Y, int M, int N, int K,
             void* ws, size_t wsb, hipStream_t st) {
    if (M == 1 && upl_for(K) <= 16) return launch_gemv_m1(wtype, W, X, bias, Y, N, K, st);
    // measured (GEMV sweep, 151936 x 2048): the several-row kernel takes M = 2
    // in every quant format (Q4_K 69.6 -> 54.0 us) and M = 3 / 4 in Q6_K and
    // Q8_0 (Q8_0 at 3: 102.4 -> 73.3 us), where the matrix-core and per-row
    // kernels pay more per weight (Q4_K at 3 / 4 stays on the matrix cores:
    // 55 against 58-66 us on the pipelined several-row kernel); layer-sized
    // matrices are launch-bound either way and keep their kernels
    const bool big = (int64_t)N * K >= ((int64_t)32 << 20);
    if (big && wtype != BX_TYPE_F16 && gemv_mr_ok(M, K) && (M == 2 || wtype != BX_TYPE_Q4_K))
        return launch_gemv_mr(wtype, W, X, bias, Y, M, N, K, st);
    // measured crossover (GEMV sweep): the per-row kernel is one launch at
    // M = 2 and 4 and faster there, except Q4_K at 4 with N >= 4096; Q8_0
    // below 8 M weights keeps it up to M = 8
    const bool small_q8 = wtype == BX_TYPE_Q8_0 && M < 16 && (int64_t)N * K < (8 << 20);
    const bool mfma = K % 256 == 0 && M >= 3 && (M != 4 || (wtype == BX_TYPE_Q4_K && N >= 4096)) &&
                      !(small_q8 && (M == 8 || M <= 4));
    if (mfma) return gemv_mfma(wtype, W, bias, X, Y, M, N, K, ws, wsb, st);
    switch (wtype) {
        case BX_TYPE_Q4_K: return gemv_dispatch<FMT_Q4_K>(M, W, X, bias, Y, N, K, st);
        case BX_TYPE_Q6_K: return gemv_dispatch<FMT_Q6_K>(M, W, X, bias, Y, N, K, st);
        case BX_TYPE_Q8_0: return gemv_dispatch<FMT_Q8_0>(M, W, X, bias, Y, N, K, st);
        case BX_TYPE_F16: return gemv_dispatch<FMT_F16>(M, W, X, bias, Y, N, K, st);
        default: return fail(BX_EUNSUPPORTED, "gemv: unsupported type");
    }
}

}  // namespace bx

extern "C" int bx_linear_f16(int wtype, const void* W, const uint16_t* bias, const uint16_t* X, uint16_t* Y, int M,
                             int N, int K, void* ws, size_t ws_bytes, void* stream) {
    if (int rc = bx::check_linear_shape(wtype, M, N, K)) return rc;
    if (!W || !X || !Y) return bx::fail(BX_EINVAL, "linear: null pointer");
    hipStream_t st = bx::as_stream(stream);
    // K beyond 12288 (an FFN width such as 32768) at 2..16 rows: the per-row
    // kernels' staged activations outgrow LDS; the split MFMA GEMV stages only
    // a K slice (3..16 rows, shapes it takes), else the tiled GEMM
    if (M == 1 || (M <= 16 && K <= 12288)) return bx::gemv_f16(wtype, W, bias, X, Y, M, N, K, ws, ws_bytes, st);
    if (bx::fused_gemv_ok(M, K)) {
        const int rc = bx::gemv_mfma_split(wtype, W, bias, X, Y, M, N, K, ws, ws_bytes, st);
        if (rc != BX_EUNSUPPORTED) return rc;
    }
    return bx::gemm_f16(wtype, W, bias, X, Y, M, N, K, st);
}

extern "C" int bx_linear_tiles_ok(int M, int K) { return (bx::gemm_tiles_ok(M, K) || bx::fused_gemv_ok(M, K)) ? 1 : 0; }

extern "C" int bx_linear_group_f16(int wtype, int n, const void* const* W, uint16_t* const* Y, const int* N,
                                   const uint16_t* X, int M, int K, void* ws, size_t ws_bytes, void* stream) {
    if (n < 1 || n > 3 || !W || !Y || !N || !X) return bx::fail(BX_EINVAL, "linear_group: bad arguments");
    for (int i = 0; i < n; ++i) {
        if (int rc = bx::check_linear_shape(wtype, M, N[i], K)) return rc;
        if (!W[i] || !Y[i]) return bx::fail(BX_EINVAL, "linear_group: null pointer");
    }
    if (bx::fused_gemv_ok(M, K))
        return bx::gemv_mfma_group(wtype, n, W, Y, N, X, M, K, ws, ws_bytes, bx::as_stream(stream));
    if (!bx::gemm_tiles_ok(M, K))
        return bx::fail(BX_EUNSUPPORTED, "linear_group: needs 3 <= M <= 16 with K % 256 == 0, or M >= 128 with K % 64 == 0");
    return bx::gemm_group_f16(wtype, n, W, Y, N, X, M, K, bx::as_stream(stream));
}

extern "C" int bx_linear_residual_f16(int wtype, const void* W, const uint16_t* X, float* H, int M, int N, int K,
                                      void* ws, size_t ws_bytes, void* stream) {
    if (int rc = bx::check_linear_shape(wtype, M, N, K)) return rc;
    if (!W || !X || !H) return bx::fail(BX_EINVAL, "linear_residual: null pointer");
    if (bx::fused_gemv_ok(M, K)) return bx::gemv_mfma_resid(wtype, W, X, H, M, N, K, ws, ws_bytes, bx::as_stream(stream));
    if (!bx::gemm_tiles_ok(M, K))
        return bx::fail(BX_EUNSUPPORTED, "linear_residual: needs 3 <= M <= 16 with K % 256 == 0, or M >= 128 with K % 64 == 0");
    return bx::gemm_resid_f16(wtype, W, X, H, M, N, K, bx::as_stream(stream));
}

extern "C" int bx_linear_swiglu_f16(int wtype, const void* Wg, const void* Wu, const uint16_t* X, uint16_t* Y, int M,
                                    int F, int K, void* ws, size_t ws_bytes, void* stream) {
    if (int rc = bx::check_linear_shape(wtype, M, F, K)) return rc;
    if (!Wg || !Wu || !X || !Y) return bx::fail(BX_EINVAL, "linear_swiglu: null pointer");
    if (bx::fused_gemv_ok(M, K))
        return bx::gemv_mfma_swiglu(wtype, Wg, Wu, X, Y, M, F, K, ws, ws_bytes, bx::as_stream(stream));
    if (!bx::gemm_tiles_ok(M, K))
        return bx::fail(BX_EUNSUPPORTED, "linear_swiglu: needs 3 <= M <= 16 with K % 256 == 0, or M >= 128 with K % 64 == 0");
    return bx::gemm_swiglu_f16(wtype, Wg, Wu, X, Y, M, F, K, bx::as_stream(stream));
}

// Decode-batch forms with the residual RMSNorm carried between launches (3 <=
// M <= 16, K % 256 == 0, matrices the split batched GEMV takes; otherwise
// BX_EUNSUPPORTED and nothing launched, and the caller runs the separate norm).
extern "C" size_t bx_linear_ss_floats(int N) { return N > 0 ? (size_t)(N + 63) / 64 * 16 : 0; }

extern "C" int bx_linear_residual_ss_f16(int wtype, const void* W, const uint16_t* X, float* H, float* ss_out, int M,
                                         int N, int K, void* ws, size_t ws_bytes, void* stream) {
    if (int rc = bx::check_linear_shape(wtype, M, N, K)) return rc;
    if (!W || !X || !H || !ss_out) return bx::fail(BX_EINVAL, "linear_residual_ss: null pointer");
    if (!bx::fused_gemv_ok(M, K)) return bx::fail(BX_EUNSUPPORTED, "linear_residual_ss: needs 3 <= M <= 16, K % 256 == 0");
    return bx::gemv_mfma_resid_ss(wtype, W, X, H, ss_out, M, N, K, ws, ws_bytes, bx::as_stream(stream));
}

extern "C" int bx_linear_group_norm_f16(int wtype, int n, const void* const* W, uint16_t* const* Y, const int* N,
                                        const float* H, const uint16_t* gamma, float eps, const float* ss_in, int M,
                                        int K, void* ws, size_t ws_bytes, void* stream) {
    if (n < 1 || n > 3 || !W || !Y || !N || !H || !gamma || !ss_in)
        return bx::fail(BX_EINVAL, "linear_group_norm: bad arguments");
    for (int i = 0; i < n; ++i) {
        if (int rc = bx::check_linear_shape(wtype, M, N[i], K)) return rc;
        if (!W[i] || !Y[i]) return bx::fail(BX_EINVAL, "linear_group_norm: null pointer");
    }
    if (!bx::fused_gemv_ok(M, K)) return bx::fail(BX_EUNSUPPORTED, "linear_group_norm: needs 3 <= M <= 16, K % 256 == 0");
    return bx::gemv_mfma_group_norm(wtype, n, W, Y, N, H, gamma, eps, ss_in, M, K, ws, ws_bytes,
                                    bx::as_stream(stream));
}

extern "C" int bx_linear_swiglu_norm_f16(int wtype, const void* Wg, const void* Wu, const float* H,
                                         const uint16_t* gamma, float eps, const float* ss_in, uint16_t* Y, int M,
                                         int F, int K, void* ws, size_t ws_bytes, void* stream) {
    if (int rc = bx::check_linear_shape(wtype, M, F, K)) return rc;
    if (!Wg || !Wu || !H || !gamma || !ss_in || !Y) return bx::fail(BX_EINVAL, "linear_swiglu_norm: null pointer");
    if (!bx::fused_gemv_ok(M, K)) return bx::fail(BX_EUNSUPPORTED, "linear_swiglu_norm: needs 3 <= M <= 16, K % 256 == 0");
    return bx::gemv_mfma_swiglu_norm(wtype, Wg, Wu, H, gamma, eps, ss_in, Y, M, F, K, ws, ws_bytes,
                                     bx::as_stream(stream));
}

// q / k / v in one launch when v's weight type differs (members [0, n1) of
// type wtype, [n1, n) of type wtype2; Q4_K then Q6_K), from FP16 X or, with
// H non-null, from RMSNorm(H) with the residual launch's row sums.
static int group2_checks(int wtype, int wtype2, int n, int n1, const void* const* W, uint16_t* const* Y, const int* N,
                         int M, int K) {
    if (n < 2 || n > 3 || n1 < 1 || n1 >= n || !W || !Y || !N) return bx::fail(BX_EINVAL, "linear_group2: bad arguments");
    for (int i = 0; i < n; ++i) {
        if (int rc = bx::check_linear_shape(i < n1 ? wtype : wtype2, M, N[i], K)) return rc;
        if (!W[i] || !Y[i]) return bx::fail(BX_EINVAL, "linear_group2: null pointer");
    }
    if (!bx::fused_gemv_ok(M, K)) return bx::fail(BX_EUNSUPPORTED, "linear_group2: needs 3 <= M <= 16, K % 256 == 0");
    return BX_OK;
}

extern "C" int bx_linear_group2_f16(int wtype, int wtype2, int n, int n1, const void* const* W, uint16_t* const* Y,
                                    const int* N, const uint16_t* X, int M, int K, void* ws, size_t ws_bytes,
                                    void* stream) {
    if (int rc = group2_checks(wtype, wtype2, n, n1, W, Y, N, M, K)) return rc;
    if (!X) return bx::fail(BX_EINVAL, "linear_group2: null X");
    return bx::gemv_mfma_group2(wtype, wtype2, n, n1, W, Y, N, X, nullptr, nullptr, 0.f, nullptr, M, K, ws, ws_bytes,
                                bx::as_stream(stream));
}

extern "C" int bx_linear_group2_norm_f16(int wtype, int wtype2, int n, int n1, const void* const* W, uint16_t* const* Y,
                                         const int* N, const float* H, const uint16_t* gamma, float eps,
                                         const float* ss_in, int M, int K, void* ws, size_t ws_bytes, void* stream) {
    if (int rc = group2_checks(wtype, wtype2, n, n1, W, Y, N, M, K)) return rc;
    if (!H || !gamma || !ss_in) return bx::fail(BX_EINVAL, "linear_group2_norm: null pointer");
    return bx::gemv_mfma_group2(wtype, wtype2, n, n1, W, Y, N, nullptr, H, gamma, eps, ss_in, M, K, ws, ws_bytes,
                                bx::as_stream(stream));
}
