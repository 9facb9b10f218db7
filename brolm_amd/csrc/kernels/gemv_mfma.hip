// Batched quant-carrier linear on the matrix cores, 3 <= M <= 16 rows of
// activations (brotensor linear_forward_batched_*_fp16 at the decode batch
// sizes, dispatched at include/brolm/detail/compute.h:54-86):
// Y[M,N] = X[M,K] W[N,K]^T.
//
// A wavefront owns a tile of 16 weight rows and streams it along K in chunks
// of 256 elements.  Each v_mfma_f32_16x16x32_f16 (v_mfma_f32_16x16x16_f16 for
// Q6_K) multiplies the activations (A: 16 rows of X, zero past M) by one
// scale group of the tile's weights (B: the 16 rows' quantized values of one
// sub-block), so the group's scale applies to the instruction's result,
//     acc[m][n] += s[n] * D[m][n].
// Q4_K folds its 6-bit sub-block scales into the values instead (sc * q <= 945
// is an exact FP16 integer), so one accumulation chain covers a 256-element
// block and d applies once; the min term sum_sb dmin m_sb X_sb takes one more
// instruction on the 32-element sums of X, split into two FP16 halves.
// The weight values enter the matrix core as small exact integers (the
// magic-exponent FP16 pairs of gemv_core.h), so every product is exact and the
// result has the GEMV path's numerics: FP32 accumulation, no FP16 rounding of
// dequantized weights.
//
// Lane l of a wavefront feeds row (l mod 16) of both operands and k-group
// l / 16 (8 consecutive k slots; 4 for 16x16x16); its four results are
// D[4 (l / 16) + j][l mod 16].  The activations sit in LDS in the swizzled
// pair order of gemv_core.h, which is the order the byte masks pull weight
// values out of a dword, so a lane's A fragment is one aligned 16-byte read;
// rows past M read a zeroed row.
//
// Loads are software-pipelined: the next slice of SB chunks is requested
// before the current one is multiplied.  Wide matrices give each wavefront
// whole tiles; narrow ones split K over the 8 wavefronts of a workgroup and
// add the partial tiles in LDS.
#include <map>
#include <type_traits>
#include <mutex>
#include <utility>

#include "gemv_core.h"

namespace bx {
namespace {

typedef _Float16 h8v __attribute__((ext_vector_type(8)));
typedef _Float16 h4v __attribute__((ext_vector_type(4)));
typedef float f4v __attribute__((ext_vector_type(4)));

constexpr int kThr = 512;
constexpr int kWav = kThr / 64;

__device__ __forceinline__ f4v mfma_k32(u4v a, u4v b, f4v c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(h8v, a), __builtin_bit_cast(h8v, b), c, 0, 0, 0);
}
__device__ __forceinline__ f4v mfma_k16(u2v a, u2v b, f4v c) {
    return __builtin_amdgcn_mfma_f32_16x16x16f16(__builtin_bit_cast(h4v, a), __builtin_bit_cast(h4v, b), c, 0, 0, 0);
}
__device__ __forceinline__ uint32_t ldg_u32(const void* p) { return *gptr<uint32_t>(p); }
// Weight loads are plain (cached): a load instruction covers 32 bytes of each
// of 16 rows, and the next instructions finish the lines it touched, so L2
// must keep them meanwhile (streaming loads measured 10-20 % slower here).
__device__ __forceinline__ u2v ldw8(const void* p) { return *gptr<u2v>(p); }
__device__ __forceinline__ u4v ldw16(const void* p) { return *gptr<u4v>(p); }

// Staged activations: Mr rows of K elements (swizzled pairs, natural for FP16
// weights) and a zero row Mr, row stride xstride dwords; a lane reads row
// min(l mod 16, Mr) (xrow: its first dword).  Q4_K also keeps
// xs2[j * 16 + m] = the sum of x[m][32 j .. 32 j + 31] as an FP16 pair
// (high part, remainder), zero for m >= Mr.
struct XStage {
    const uint32_t* xs;
    const uint32_t* xs2;
    int xrow;
    __device__ __forceinline__ u4v a8(int e) const { return *reinterpret_cast<const u4v*>(xs + xrow + (e >> 1)); }
    __device__ __forceinline__ u2v a4(int e) const { return *reinterpret_cast<const u2v*>(xs + xrow + (e >> 1)); }
};

// Q4_K: 32-element sums of the Mr staged rows of K elements (16 dwords hold a
// permutation of a group's elements), kept as FP16 high part + remainder in
// xs2[j * 16 + m]; zero for m >= Mr.
__device__ __forceinline__ void q4k_xsums(const uint32_t* smem, int xstride, uint32_t* xs2, int Mr, int K) {
    for (int i = threadIdx.x; i < (K / 32) * 16; i += blockDim.x) {
        const int j = i >> 4, m = i & 15;
        float s = 0.f;
        if (m < Mr) {
            const u4v* p = reinterpret_cast<const u4v*>(smem + m * xstride + 16 * j);
#pragma unroll
            for (int q = 0; q < 4; ++q) {
                const u4v v = p[q];
                s += (h2f(v.x & 0xffff) + h2f(v.x >> 16)) + (h2f(v.y & 0xffff) + h2f(v.y >> 16)) +
                     (h2f(v.z & 0xffff) + h2f(v.z >> 16)) + (h2f(v.w & 0xffff) + h2f(v.w >> 16));
            }
        }
        const _Float16 hi = (_Float16)s;
        const _Float16 lo = (_Float16)(s - (float)hi);
        xs2[i] = (uint32_t)__builtin_bit_cast(uint16_t, hi) | ((uint32_t)__builtin_bit_cast(uint16_t, lo) << 16);
    }
}

// ---- per-format chunk: 256 K elements of one 16-row tile, per lane ---------

template <int FMT>
struct Chunk;

// Q4_K: block b of row n; lane group g takes the 32 qs bytes 32g .. 32g + 31
// (low nibbles: sub-block 2g, high: 2g + 1), eight k-slot groups of 8.
template <>
struct Chunk<FMT_Q4_K> {
    u4v hdr;
    u4v q0, q1;
    __device__ __forceinline__ void load(const void* W, int64_t N, int K, int64_t n, int b, int g) {
        const CarrierQ4K c = carrier_q4k(W, N, K);
        const int64_t s = n * (K / 256) + b;
        hdr = ldg16(c.hdr + s * 16);
        q0 = ldw16(c.qs + s * 128 + 32 * g);
        q1 = ldw16(c.qs + s * 128 + 32 * g + 16);
    }
    __device__ __forceinline__ void mul(const XStage& x, int e0, int r, int g, f4v& acc) const {
        u4v a[8];
#pragma unroll
        for (int k = 0; k < 8; ++k) a[k] = x.a8(e0 + 64 * g + 32 * (k >> 2) + 8 * (k & 3));
        const uint32_t xm = x.xs2[(e0 >> 5) * 16 + 2 * g * 16 + r];
        const uint32_t xm1 = x.xs2[(e0 >> 5) * 16 + (2 * g + 1) * 16 + r];
        const float d = h2f(hdr.x & 0xffff), dmin = h2f(hdr.x >> 16);
        int sc0, m0, sc1, m1;
        q4k_pair_scales(hdr.y, hdr.z, hdr.w, g, sc0, m0, sc1, m1);
        // (1024 + q) * sc - 1024 sc = sc q, one rounding of an exact integer
        const h2 s_lo = {(_Float16)sc0, (_Float16)sc0}, c_lo = {(_Float16)(-1024 * sc0), (_Float16)(-1024 * sc0)};
        const h2 s_hi = {(_Float16)sc1, (_Float16)sc1}, c_hi = {(_Float16)(-1024 * sc1), (_Float16)(-1024 * sc1)};
        const uint32_t mg = magic_vgpr();
        const uint32_t w[8] = {q0.x, q0.y, q0.z, q0.w, q1.x, q1.y, q1.z, q1.w};
        f4v d1 = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int k = 0; k < 8; ++k) {
            const int hi = k >> 2;
            const uint32_t wa = hi ? w[2 * (k & 3)] >> 4 : w[2 * (k & 3)];
            const uint32_t wb = hi ? w[2 * (k & 3) + 1] >> 4 : w[2 * (k & 3) + 1];
            const h2 sv = hi ? s_hi : s_lo, cv = hi ? c_hi : c_lo;
            const u4v bw = {as_u32(__builtin_elementwise_fma(as_h2(and_or(wa, 0x000F000Fu, mg)), sv, cv)),
                            as_u32(__builtin_elementwise_fma(as_h2(and_or(wa >> 8, 0x000F000Fu, mg)), sv, cv)),
                            as_u32(__builtin_elementwise_fma(as_h2(and_or(wb, 0x000F000Fu, mg)), sv, cv)),
                            as_u32(__builtin_elementwise_fma(as_h2(and_or(wb >> 8, 0x000F000Fu, mg)), sv, cv))};
            d1 = mfma_k32(a[k], bw, d1);
        }
        // min term: slots (X_hi, X_lo) of sub-blocks 2g and 2g + 1 against (m, m)
        const h2 mp0 = {(_Float16)m0, (_Float16)m0}, mp1 = {(_Float16)m1, (_Float16)m1};
        const u4v am = {xm, xm1, 0u, 0u};
        const u4v bm = {as_u32(mp0), as_u32(mp1), 0u, 0u};
        const f4v d2 = mfma_k32(am, bm, f4v{0.f, 0.f, 0.f, 0.f});
#pragma unroll
        for (int j = 0; j < 4; ++j) acc[j] += d * d1[j] - dmin * d2[j];
    }
};

// Q6_K: block b of row n; sub-block (h, p, hl) = elements 128h + 32p + 16hl
// + 0..15 (scale index 8h + 2p + hl); lane group g takes 16hl + 4g .. +3.
template <>
struct Chunk<FMT_Q6_K> {
    u4v sc;
    uint32_t d;
    u4v ql[4];
    uint32_t qh[4];
    __device__ __forceinline__ void load(const void* W, int64_t N, int K, int64_t n, int b, int g) {
        const CarrierQ6K c = carrier_q6k(W, N, K);
        const int64_t s = n * (K / 256) + b;
        sc = ldg16(c.sc + s * 16);
        d = ldg_u16(c.d + s * 2);
#pragma unroll
        for (int k = 0; k < 4; ++k) {
            const int t = 4 * (k >> 1) + 2 * (k & 1) + (g >> 1);
            ql[k] = ldw16(c.ql + s * 128 + 16 * t);
            qh[k] = ldg_u32(c.qh + s * 64 + 8 * t + 4 * (g & 1));
        }
    }
    __device__ __forceinline__ void mul(const XStage& x, int e0, int r, int g, f4v& acc) const {
        const float dd = h2f(d & 0xffff);
        const uint32_t mg = magic_vgpr();
        const uint32_t scw[4] = {sc.x, sc.y, sc.z, sc.w};
        const f4v z = {0.f, 0.f, 0.f, 0.f};
        u2v av[4][4];
#pragma unroll
        for (int k = 0; k < 4; ++k)
#pragma unroll
            for (int p = 0; p < 4; ++p) av[k][p] = x.a4(e0 + 128 * (k >> 1) + 32 * p + 16 * (k & 1) + 4 * g);
#pragma unroll
        for (int k = 0; k < 4; ++k) {
            const int h = k >> 1, hl = k & 1;
            const uint32_t a = (g & 1) ? ql[k].y : ql[k].x, bq = (g & 1) ? ql[k].w : ql[k].z, q = qh[k];
            const uint32_t a8 = a >> 8, b8 = bq >> 8;
            const uint32_t ql4 = q << 4, qr4 = q >> 4, ql2 = q << 2, qr6 = q >> 6;
            // (low nibble | 2 high bits) -> 1024 + q; (high nibble in place | 2 bits at 8-9) -> 1024 + 16 q
            const uint32_t v[4][2] = {
                {and_or(ql4, 0x00300030u, and_or(a, 0x000F000Fu, mg)), and_or(qr4, 0x00300030u, and_or(a8, 0x000F000Fu, mg))},
                {and_or(ql2, 0x00300030u, and_or(bq, 0x000F000Fu, mg)), and_or(qr6, 0x00300030u, and_or(b8, 0x000F000Fu, mg))},
                {and_or(ql4, 0x03000300u, and_or(a, 0x00F000F0u, mg)), and_or(qr4, 0x03000300u, and_or(a8, 0x00F000F0u, mg))},
                {and_or(ql2, 0x03000300u, and_or(bq, 0x00F000F0u, mg)), and_or(qr6, 0x03000300u, and_or(b8, 0x00F000F0u, mg))}};
#pragma unroll
            for (int p = 0; p < 4; ++p) {
                const float off = p < 2 ? 1056.f : 1536.f;   // centre: q - 32, or 16 (q - 32)
                const u2v bw = {centre(v[p][0], off), centre(v[p][1], off)};
                const f4v dv = mfma_k16(av[k][p], bw, z);
                const int sb = 8 * h + 2 * p + hl;
                const float s = dd * (float)(int8_t)((scw[sb >> 2] >> (8 * (sb & 3))) & 0xff) * (p < 2 ? 1.f : 0.0625f);
#pragma unroll
                for (int j = 0; j < 4; ++j) acc[j] += s * dv[j];
            }
        }
    }
};

// Q8_0: the 8 blocks of 32 of a chunk; lane group g takes qs bytes 8g .. +7.
template <>
struct Chunk<FMT_Q8_0> {
    u4v dv;
    u2v q[8];
    __device__ __forceinline__ void load(const void* W, int64_t N, int K, int64_t n, int b, int g) {
        const CarrierQ8 c = carrier_q8(W, N, K);
        const int64_t s = n * (K / 32) + 8 * b;
        dv = ldg16(c.d + s * 2);
#pragma unroll
        for (int j = 0; j < 8; ++j) q[j] = ldw8(c.qs + (s + j) * 32 + 8 * g);
    }
    __device__ __forceinline__ void mul(const XStage& x, int e0, int r, int g, f4v& acc) const {
        const uint32_t dw[4] = {dv.x, dv.y, dv.z, dv.w};
        const f4v z = {0.f, 0.f, 0.f, 0.f};
        u4v a[8];
#pragma unroll
        for (int j = 0; j < 8; ++j) a[j] = x.a8(e0 + 32 * j + 8 * g);
#pragma unroll
        for (int j = 0; j < 8; ++j) {
            const uint32_t w0 = q[j].x, w1 = q[j].y;
            const u4v bw = {centre(magic_pair((w0 & 0x00FF00FFu) ^ 0x00800080u), 1152.f),
                            centre(magic_pair(((w0 >> 8) & 0x00FF00FFu) ^ 0x00800080u), 1152.f),
                            centre(magic_pair((w1 & 0x00FF00FFu) ^ 0x00800080u), 1152.f),
                            centre(magic_pair(((w1 >> 8) & 0x00FF00FFu) ^ 0x00800080u), 1152.f)};
            const f4v dvv = mfma_k32(a[j], bw, z);
            const float s = h2f((dw[j >> 1] >> (16 * (j & 1))) & 0xffff);
#pragma unroll
            for (int i = 0; i < 4; ++i) acc[i] += s * dvv[i];
        }
    }
};

// FP16 weights (natural activation layout): 8 consecutive weights per lane.
template <>
struct Chunk<FMT_F16> {
    u4v w[8];
    __device__ __forceinline__ void load(const void* W, int64_t, int K, int64_t n, int b, int g) {
        const uint8_t* p = static_cast<const uint8_t*>(W) + (n * K + 256 * (int64_t)b + 8 * g) * 2;
#pragma unroll
        for (int j = 0; j < 8; ++j) w[j] = ldw16(p + 64 * j);
    }
    __device__ __forceinline__ void mul(const XStage& x, int e0, int r, int g, f4v& acc) const {
#pragma unroll
        for (int j = 0; j < 8; ++j) acc = mfma_k32(x.a8(e0 + 32 * j + 8 * g), w[j], acc);
    }
};

// chunks per slice (per buffer): two, one for Q6_K (register budget)
template <int FMT> struct SliceLen { static constexpr int SB = FMT == FMT_Q6_K ? 1 : 2; };

// A wavefront's walk over slices: tiles tile0, tile0 + tstride, ... below
// tiles; in each tile the chunks [c0, c1) in slices of SB.
struct Walk {
    int64_t tile;
    int cb;
    int64_t tstride, tiles;
    int c0, c1;
    __device__ __forceinline__ bool valid() const { return tile < tiles && c0 < c1; }
    __device__ __forceinline__ bool last_of_tile(int SB) const { return cb + SB >= c1; }
    __device__ __forceinline__ Walk next(int SB) const {
        Walk w = *this;
        w.cb += SB;
        if (w.cb >= c1) {
            w.cb = c0;
            w.tile += tstride;
        }
        return w;
    }
};

template <int FMT>
struct SliceBuf {
    static constexpr int SB = SliceLen<FMT>::SB;
    Chunk<FMT> c[SB];
    uint32_t bias;   // bias of the lane's row, loaded with a tile's first slice
    __device__ __forceinline__ void load(const void* W, const uint16_t* bias_p, int64_t N, int K, const Walk& w, int r,
                                         int g) {
        int64_t n = w.tile * 16 + r;
        if (n >= N) n = N - 1;
        // unconditional (a dummy in-bounds address without bias): a load under
        // a branch would make the compiler wait for every load before it
        bias = ldg_u16(bias_p ? bias_p + n : static_cast<const uint16_t*>(W));
#pragma unroll
        for (int i = 0; i < SB; ++i) {
            const int b = w.cb + i < w.c1 ? w.cb + i : w.c1 - 1;   // clamped: every load is issued
            c[i].load(W, N, K, n, b, g);
        }
    }
    __device__ __forceinline__ void mul(const XStage& x, const Walk& w, int r, int g, f4v& acc) const {
#pragma unroll
        for (int i = 0; i < SB; ++i)
            if (w.cb + i < w.c1) c[i].mul(x, 256 * (w.cb + i), r, g, acc);
    }
};

// What one launch computes.  STORE: Y[0] = f16(X W[0]^T + bias) (one weight)
// or up to three weights sharing X, each into its own Y[i] (q / k / v): the
// tile index runs over the members' row tiles in order.  RESID: the FP32
// residual H (Mr, N[0]) += f16(X W[0]^T).  SWIGLU: gate W[0] and up W[1] rows
// of the same tile, Y[0] = f16(f16(silu(f16(gate))) * f16(up)), the values the
// separate linear, silu and mul kernels give.
enum : int { MEPI_STORE = 0, MEPI_RESID = 1, MEPI_SWIGLU = 2 };
struct MfmaJob {
    const void* W[3];
    uint16_t* Y[3];
    float* H;
    const uint16_t* bias;   // STORE with one member only
    int N[3];
    int64_t tiles_n[3];
    int members;
    int64_t tiles;          // total tiles of the launch
    // norm-input split launches: X is the RMSNorm (gamma, eps) of the FP32
    // rows Hn, row m's sum of squares the sum of ss_in[q * 16 + m], q < ss_groups
    const float* Hn;
    const uint16_t* gamma;
    const float* ss_in;
    int ss_groups;
    float eps;
    // residual split launches: row sums of squares of the updated residual,
    // ss_out[group * 16 + m] for the 64 columns of each tile group (or null)
    float* ss_out;
    // two-format groups: members from mem2 on have the second weight type
    int mem2;
    // split launches: the caller's workspace (counters, then FP32 partials)
    // and the launch's tag (nonzero, new for every launch the host makes)
    uint64_t* cnt;
    float* part;
    uint32_t tag;
};

// Tile t of the launch -> (member, row tile within the member).
__device__ __forceinline__ void member_of(const MfmaJob& job, int64_t t, int& mem, int64_t& lt) {
    mem = 0;
    lt = t;
    while (mem + 1 < job.members && lt >= job.tiles_n[mem]) lt -= job.tiles_n[mem++];
}

// kpart: waves per tile.  1: every wave walks whole tiles (grid-stride);
// 2, 4, 8: the workgroup takes 8 / kpart tiles, each split along K over kpart
// waves whose partial tiles are added in LDS.
template <int FMT, int EPI>
__global__ __launch_bounds__(kThr) void gemv_mfma_kernel(MfmaJob job, const uint16_t* __restrict__ X, int Mr, int K,
                                                        int kpart) {
    extern __shared__ __align__(16) uint32_t smem[];
    constexpr bool kSwz = FMT != FMT_F16;
    constexpr bool kTwo = EPI == MEPI_SWIGLU;   // gate and up rows per tile
    const int xstride = K / 2 + 4;
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int r = lane & 15, g = lane >> 4;
    XStage xst;
    xst.xs = smem;
    xst.xrow = (r < Mr ? r : Mr) * xstride;
    uint32_t* xs2 = smem + (Mr + 1) * xstride;
    xst.xs2 = xs2;
    float* red = reinterpret_cast<float*>(xs2 + (FMT == FMT_Q4_K ? (K / 32) * 16 : 0));
    const int nch = K / 256;
    const int64_t tiles = job.tiles;
    Walk w;
    w.tiles = tiles;
    if (kpart == 1) {
        w.tile = (int64_t)blockIdx.x * kWav + wave;
        w.tstride = (int64_t)gridDim.x * kWav;
        w.c0 = 0;
        w.c1 = nch;
    } else {
        const int part = wave % kpart;
        w.tile = (int64_t)blockIdx.x * (kWav / kpart) + wave / kpart;
        w.tstride = tiles;   // one tile per wave
        w.c0 = part * nch / kpart;
        w.c1 = (part + 1) * nch / kpart;
    }
    w.cb = w.c0;
    const int64_t w0tile = w.tile;
    // the slice loads of a walk position: its member's weight (and the up
    // weight for SwiGLU) at the member's own row tile
    auto load = [&](SliceBuf<FMT>& bg, SliceBuf<FMT>& bu, const Walk& at) {
        int mem;
        Walk lw = at;
        member_of(job, at.tile, mem, lw.tile);
        const int N = job.N[mem];
        bg.load(job.W[mem], EPI == MEPI_STORE ? job.bias : nullptr, N, K, lw, r, g);
        if constexpr (kTwo) bu.load(job.W[1], nullptr, N, K, lw, r, g);
    };

    // the first slice's weights stream while the activations are staged
    SliceBuf<FMT> b0, b1, u0, u1;
    if (w.valid()) load(b0, u0, w);
    stage_x_f16<kSwz, false>(X, K, Mr, K, smem, xstride, nullptr, 0);
    for (int i = threadIdx.x; i < xstride; i += kThr) smem[Mr * xstride + i] = 0u;
    __syncthreads();
    if constexpr (FMT == FMT_Q4_K) {
        q4k_xsums(smem, xstride, xs2, Mr, K);
        __syncthreads();
    }

    f4v acc = {0.f, 0.f, 0.f, 0.f}, accu = {0.f, 0.f, 0.f, 0.f};
    // the epilogue of tile `tile` from lane values a (and u for SwiGLU)
    auto store = [&](int64_t tile, const f4v& a, const f4v& u, float bv) {
        int mem;
        int64_t lt;
        member_of(job, tile, mem, lt);
        const int N = job.N[mem];
        const int64_t n = lt * 16 + r;
        if (n >= N) return;
        if constexpr (EPI == MEPI_RESID) {
            float hv[4];
#pragma unroll
            for (int j = 0; j < 4; ++j)
                if (4 * g + j < Mr) hv[j] = job.H[(int64_t)(4 * g + j) * N + n];
#pragma unroll
            for (int j = 0; j < 4; ++j)
                if (4 * g + j < Mr) job.H[(int64_t)(4 * g + j) * N + n] = hv[j] + h2f(f2h(a[j]));
            return;
        }
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const int m = 4 * g + j;
            if (m >= Mr) continue;
            if constexpr (EPI == MEPI_SWIGLU) {
                const float act = h2f(f2h(silu_f32(h2f(f2h(a[j])))));
                job.Y[0][(int64_t)m * N + n] = f2h(act * h2f(f2h(u[j])));
            } else {
                job.Y[mem][(int64_t)m * N + n] = f2h(a[j] + bv);
            }
        }
    };
    auto finish = [&](int64_t tile, float bv) {
        store(tile, acc, accu, bv);
        acc = f4v{0.f, 0.f, 0.f, 0.f};
        accu = f4v{0.f, 0.f, 0.f, 0.f};
    };
    // The next slice's loads are issued before the current slice's math and
    // unconditionally (past the end they repeat the current slice), so the
    // compiler's in-order wait for a slice never covers its successor.
    float bv = 0.f;
    if (w.valid()) {
        for (;;) {
            Walk nx = w.next(SliceLen<FMT>::SB);
            load(b1, u1, nx.valid() ? nx : w);
            if (w.cb == w.c0) bv = (EPI == MEPI_STORE && job.bias) ? h2f(b0.bias & 0xffff) : 0.f;
            b0.mul(xst, w, r, g, acc);
            if constexpr (kTwo) u0.mul(xst, w, r, g, accu);
            if (kpart == 1 && w.last_of_tile(SliceLen<FMT>::SB)) finish(w.tile, bv);
            w = nx;
            if (!w.valid()) break;
            nx = w.next(SliceLen<FMT>::SB);
            load(b0, u0, nx.valid() ? nx : w);
            if (w.cb == w.c0) bv = (EPI == MEPI_STORE && job.bias) ? h2f(b1.bias & 0xffff) : 0.f;
            b1.mul(xst, w, r, g, acc);
            if constexpr (kTwo) u1.mul(xst, w, r, g, accu);
            if (kpart == 1 && w.last_of_tile(SliceLen<FMT>::SB)) finish(w.tile, bv);
            w = nx;
            if (!w.valid()) break;
        }
    }
    if (kpart > 1) {
        // partial tiles -> LDS -> the first wave of each tile adds and writes
        *reinterpret_cast<f4v*>(red + (wave * 64 + lane) * 4) = acc;
        if constexpr (kTwo) *reinterpret_cast<f4v*>(red + ((kWav + wave) * 64 + lane) * 4) = accu;
        __syncthreads();
        if (wave % kpart == 0 && w0tile < tiles) {
            f4v s = {0.f, 0.f, 0.f, 0.f}, su = {0.f, 0.f, 0.f, 0.f};
            for (int v = wave; v < wave + kpart; ++v) {
                s += *reinterpret_cast<const f4v*>(red + (v * 64 + lane) * 4);
                if constexpr (kTwo) su += *reinterpret_cast<const f4v*>(red + ((kWav + v) * 64 + lane) * 4);
            }
            int mem;
            int64_t lt;
            member_of(job, w0tile, mem, lt);
            const int64_t n = lt * 16 + r;
            store(w0tile, s, su, (EPI == MEPI_STORE && job.bias && n < job.N[mem]) ? h2f(job.bias[n]) : 0.f);
        }
    }
}

// ---- split-K launches for matrices of decoder-layer size --------------------
//
// Grid (tile groups, S): workgroup (x, s) runs the 16-row tiles 4x .. 4x + 3,
// one per wavefront, over K slice s (chunks [s nch / S, (s + 1) nch / S) of
// 256 elements) and stages only that slice of X, so a layer's matrix spreads
// over the whole chip at any M and the LDS holds 16 rows at any K.  With
// S > 1 every wavefront writes its partial tile (FP32, rows below Mr) to the
// split workspace; the workgroup that completes a tile group last (a counter
// per group) adds the S partials in slice order, so the sum does not depend on
// which workgroup arrives when, applies the epilogue, and sets the counter back
// to zero for the next launch.  The slice plan depends on K alone, so a member
// of a q / k / v group gets the same sums as alone, and the fused epilogues the
// same as the separate ops.
constexpr int kSplThr = 256;
constexpr int kSplWav = kSplThr / 64;
constexpr int kSplMaxCps = 3;                    // chunks per slice
constexpr int kSplMaxSlices = 64;                // K up to 49152
constexpr int64_t kSplFloats = 16ll << 20;       // partials: 64 MB
constexpr int kSplGroups = 4096;                 // tile groups of one launch

constexpr size_t kSplCntBytes = (size_t)kSplGroups * 8;

}  // namespace
}  // namespace bx

namespace bx {
namespace {

// Cache policy of the partials' buffer stores and loads: sc1, device scope.
constexpr int kSc1 = 16;

// Workgroup barrier for LDS data only: loads of global memory still in flight
// stay in flight (__syncthreads() would wait for every one of them).
__device__ __forceinline__ void lds_barrier() {
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup", "local");
    __builtin_amdgcn_s_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup", "local");
}

__global__ void split_clear_kernel(uint64_t* cnt) {
    for (int i = blockIdx.x * blockDim.x + threadIdx.x; i < kSplGroups; i += gridDim.x * blockDim.x) cnt[i] = 0ull;
}


// The residual values of the lane's rows 4 g + j (< Mr) at its column of the
// tile, read together (the residual epilogue's input, requested early).
__device__ __forceinline__ void resid_rows(const MfmaJob& job, int64_t tile, int r, int g, int Mr, float (&hv)[4]) {
    int mem;
    int64_t lt;
    member_of(job, tile, mem, lt);
    const int N = job.N[mem];
    const int64_t n = lt * 16 + r;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        hv[j] = 0.f;
        if (n < N && 4 * g + j < Mr) hv[j] = job.H[(int64_t)(4 * g + j) * N + n];
    }
}

// The epilogue of one tile from lane values a (and u for SwiGLU); for the
// residual, hv holds the rows' residuals (resid_rows) and sq[j] is the square
// of the lane's updated value of row 4 g + j (0 where there is none).
template <int EPI>
__device__ __forceinline__ void tile_epilogue(const MfmaJob& job, int64_t tile, int r, int g, int Mr, const f4v& a,
                                              const f4v& u, const float (&hv)[4], f4v& sq) {
    sq = f4v{0.f, 0.f, 0.f, 0.f};
    int mem;
    int64_t lt;
    member_of(job, tile, mem, lt);
    const int N = job.N[mem];
    const int64_t n = lt * 16 + r;
    if (n >= N) return;
    const float bv = (EPI == MEPI_STORE && job.bias) ? h2f(job.bias[n]) : 0.f;
    if constexpr (EPI == MEPI_RESID) {
#pragma unroll
        for (int j = 0; j < 4; ++j)
            if (4 * g + j < Mr) {
                const float y = hv[j] + h2f(f2h(a[j]));
                job.H[(int64_t)(4 * g + j) * N + n] = y;
                sq[j] = y * y;
            }
        return;
    }
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        const int m = 4 * g + j;
        if (m >= Mr) continue;
        if constexpr (EPI == MEPI_SWIGLU) {
            const float act = h2f(f2h(silu_f32(h2f(f2h(a[j])))));
            job.Y[0][(int64_t)m * N + n] = f2h(act * h2f(f2h(u[j])));
        } else {
            job.Y[mem][(int64_t)m * N + n] = f2h(a[j] + bv);
        }
    }
}

// Row sums of squares of a residual tile group (its 4 tiles x 16 columns):
// over the 16 lanes of a row group by DPP, then the 4 wavefronts in order, to
// ss_out[blockIdx.x * 16 + m].  Every thread of the workgroup calls it.
__device__ __forceinline__ void group_row_ss(const MfmaJob& job, int Mr, int wave, int r, int g, const f4v& sq,
                                             float (*wss)[16]) {
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        float v = sq[j];
        v += dpp_f<0xB1>(v, 0.f);
        v += dpp_f<0x4E>(v, 0.f);
        v += dpp_f<0x141>(v, 0.f);
        v += dpp_f<0x140>(v, 0.f);
        if (r == 0) wss[wave][4 * g + j] = v;
    }
    __syncthreads();
    if ((int)threadIdx.x < Mr) {
        const int m = threadIdx.x;
        job.ss_out[blockIdx.x * 16 + m] = ((wss[0][m] + wss[1][m]) + wss[2][m]) + wss[3][m];
    }
}

// FMT2 >= 0: a group whose members from job.mem2 on have weight type FMT2
// (q and k in FMT, v in FMT2); a wavefront's tile belongs to one member, so
// it takes that member's load and multiply path (a wave-uniform branch).
template <int FMT, int EPI, int CPS, bool NIN, int FMT2 = -1>
__global__ __launch_bounds__(kSplThr) void gemv_split_kernel(MfmaJob job, const uint16_t* __restrict__ X, int Mr,
                                                            int K, int S) {
    extern __shared__ __align__(16) uint32_t smem[];
    __shared__ uint32_t last;
    __shared__ float wss[kSplWav][16];   // per-row partials: residual sums of squares, norm-input row sums
    constexpr bool kSwz = FMT != FMT_F16;
    constexpr bool kTwo = EPI == MEPI_SWIGLU;
    constexpr int kParts = kTwo ? 2 : 1;
    const int nch = K / 256;
    const int s = blockIdx.y;
    const int c0 = s * nch / S, nc = (s + 1) * nch / S - c0;   // 1 <= nc <= CPS
    const int Ks = 256 * nc;
    const int xstride = Ks / 2 + 4;
    // the wavefront index as a scalar: the tile's member, row count and
    // weight pointer then come from the kernel arguments by scalar loads,
    // which the waits for the activations below do not count
    const int lane = threadIdx.x & 63, wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int r = lane & 15, g = lane >> 4;
    const int64_t tile = (int64_t)blockIdx.x * kSplWav + wave;
    const bool live = tile < job.tiles;
    // The slice's activations are requested first and this wavefront's
    // weights right behind them: loads complete in issue order, so the
    // staging below waits only for the activations and runs while the weights
    // stream (its barriers wait for LDS only).  A wavefront past the last tile
    // re-reads it, chunk slots past the slice repeat its last chunk, groups
    // past the slice repeat its last group (all in bounds).
    constexpr int kXG = 4 * CPS;    // 4-element groups of the slice per thread (Mr <= 16)
    constexpr int kSsL = 8;         // row-sum partials per thread requested up front (K <= 8192)
    const int G4 = Ks / 4, total = Mr * G4;
    f4v hv[NIN ? kXG : 1];
    u2v gv[NIN ? kXG : 1];
    u2v xv[NIN ? 1 : kXG];
    float ssv[NIN ? kSsL : 1];
    if constexpr (NIN) {
        // unconditional loads at clamped indices (no branch to wait at);
        // only the partials in range are added
        const int m = min((int)threadIdx.x & 15, Mr - 1), q0 = threadIdx.x >> 4;
#pragma unroll
        for (int e = 0; e < kSsL; ++e) ssv[e] = job.ss_in[min(q0 + 16 * e, job.ss_groups - 1) * 16 + m];
#pragma unroll
        for (int j = 0; j < kXG; ++j) {
            const int i = min((int)threadIdx.x + kSplThr * j, total - 1);
            const int mm = i / G4, k = 256 * c0 + 4 * (i - mm * G4);
            hv[j] = *reinterpret_cast<const f4v*>(job.Hn + (int64_t)mm * K + k);
            gv[j] = *reinterpret_cast<const u2v*>(job.gamma + k);
        }
    } else {
#pragma unroll
        for (int j = 0; j < kXG; ++j) {
            const int i = min((int)threadIdx.x + kSplThr * j, total - 1);
            const int mm = i / G4, gg = i - mm * G4;
            xv[j] = *reinterpret_cast<const u2v*>(X + (int64_t)mm * K + 256 * c0 + 4 * gg);
        }
    }
    int mem;
    int64_t lt;
    member_of(job, live ? tile : job.tiles - 1, mem, lt);
    const int N = job.N[mem];
    const int64_t n = lt * 16 + r < N ? lt * 16 + r : N - 1;
    constexpr bool kMix = FMT2 >= 0;
    const bool second = kMix && mem >= job.mem2;
    Chunk<FMT> cw[CPS];
    Chunk<FMT> cu[kTwo ? CPS : 1];
    Chunk<kMix ? FMT2 : FMT> c2[kMix ? CPS : 1];
    if (!second) {
#pragma unroll
        for (int i = 0; i < CPS; ++i) {
            const int b = c0 + (i < nc ? i : nc - 1);
            cw[i].load(job.W[mem], N, K, n, b, g);
            if constexpr (kTwo) cu[i].load(job.W[1], N, K, n, b, g);
        }
    } else if constexpr (kMix) {
#pragma unroll
        for (int i = 0; i < CPS; ++i) c2[i].load(job.W[mem], N, K, n, c0 + (i < nc ? i : nc - 1), g);
    }
    XStage xst;
    xst.xs = smem;
    xst.xrow = (r < Mr ? r : Mr) * xstride;
    uint32_t* xs2 = smem + (Mr + 1) * xstride;
    xst.xs2 = xs2;
    if constexpr (NIN) {
        // each row's 1 / rms from the producer's per-group sums of squares:
        // thread (q0, m) adds groups q0, q0 + 16, ..., then row m adds the 16
        // part sums in order
        __shared__ float qsum[16][16];
        __shared__ float row_inv[16];
        {
            const int m = threadIdx.x & 15, q0 = threadIdx.x >> 4;
            float v = 0.f;
            if (m < Mr) {
#pragma unroll
                for (int e = 0; e < kSsL; ++e)
                    if (q0 + 16 * e < job.ss_groups) v += ssv[e];
                for (int q = q0 + 16 * kSsL; q < job.ss_groups; q += 16) v += job.ss_in[q * 16 + m];
            }
            qsum[q0][m] = v;
        }
        lds_barrier();
        if ((int)threadIdx.x < Mr) {
            const int m = threadIdx.x;
            float ssum = 0.f;
#pragma unroll
            for (int q0 = 0; q0 < 16; ++q0) ssum += qsum[q0][m];
            row_inv[m] = 1.0f / sqrtf(ssum / (float)K + job.eps);
        }
        lds_barrier();
        // the slice of the normalised rows, FP16, into LDS
#pragma unroll
        for (int j = 0; j < kXG; ++j) {
            const int i = threadIdx.x + kSplThr * j;
            if (i < total) {
                const int mm = i / G4, gg = i - mm * G4;
                const float inv = row_inv[mm];
                const f4v& h4 = hv[j];
                const u2v& g4 = gv[j];
                store_group<kSwz>(smem + mm * xstride, gg, norm_f16(h4.x, inv, h2f(g4.x & 0xffff)),
                                  norm_f16(h4.y, inv, h2f(g4.x >> 16)), norm_f16(h4.z, inv, h2f(g4.y & 0xffff)),
                                  norm_f16(h4.w, inv, h2f(g4.y >> 16)));
            }
        }
    } else {
#pragma unroll
        for (int j = 0; j < kXG; ++j) {
            const int i = threadIdx.x + kSplThr * j;
            if (i < total) {
                const int mm = i / G4, gg = i - mm * G4;
                const u2v v = xv[j];
                store_group<kSwz>(smem + mm * xstride, gg, v.x & 0xffff, v.x >> 16, v.y & 0xffff, v.y >> 16);
            }
        }
    }
    for (int i = threadIdx.x; i < xstride; i += kSplThr) smem[Mr * xstride + i] = 0u;
    lds_barrier();
    if constexpr (FMT == FMT_Q4_K || FMT2 == FMT_Q4_K) {
        q4k_xsums(smem, xstride, xs2, Mr, Ks);
        lds_barrier();
    }
    f4v acc = {0.f, 0.f, 0.f, 0.f}, accu = {0.f, 0.f, 0.f, 0.f};
    if (!second) {
#pragma unroll
        for (int i = 0; i < CPS; ++i) {
            if (i < nc) {
                cw[i].mul(xst, 256 * i, r, g, acc);
                if constexpr (kTwo) cu[i].mul(xst, 256 * i, r, g, accu);
            }
        }
    } else if constexpr (kMix) {
#pragma unroll
        for (int i = 0; i < CPS; ++i)
            if (i < nc) c2[i].mul(xst, 256 * i, r, g, acc);
    }
    f4v sq;
    if (S == 1) {
        if (live) {
            float hv[4] = {0.f, 0.f, 0.f, 0.f};
            if constexpr (EPI == MEPI_RESID) resid_rows(job, tile, r, g, Mr, hv);
            tile_epilogue<EPI>(job, tile, r, g, Mr, acc, accu, hv, sq);
        } else {
            sq = f4v{0.f, 0.f, 0.f, 0.f};
        }
        if (EPI == MEPI_RESID && job.ss_out) group_row_ss(job, Mr, wave, r, g, sq, wss);
        return;
    }
    // Partial tile (tile, s): kParts blocks of the lane values of the lanes
    // holding rows below Mr (4 floats a lane, lanes 0 .. 4 Mr4 - 1 with Mr4 =
    // Mr rounded up to 4).  The partials travel by device-scope (sc1) buffer
    // stores and loads, which write through and read past the per-XCD L2s,
    // and every wavefront waits for its stores to complete before the
    // workgroup counts itself in: the counter never runs ahead of the data it
    // announces, without the L2 write-back a device-scope fence would cost.
    const int Mr4 = (Mr + 3) & ~3;
    const int pl = 4 * Mr4;                             // lanes with partials
    const int64_t pstride = (int64_t)kParts * pl * 4;   // floats per (tile, slice)
    const __amdgpu_buffer_rsrc_t rs = __builtin_amdgcn_make_buffer_rsrc(job.part, 0, 0x7fffffff, 0x00020000);
    const int64_t tbase = live ? tile * S * pstride : 0;
    if (live && lane < pl) {
        const int o = (int)((tbase + s * pstride) * 4) + lane * 16;
        __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(u4v, acc), rs, o, 0, kSc1);
        if constexpr (kTwo) __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(u4v, accu), rs, o + pl * 16, 0, kSc1);
    }
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    __syncthreads();
    // the group's arrival count (a word left by a launch that never finished
    // is not counted; the last arrival puts the word back to zero)
    if (threadIdx.x == 0) last = tagged_arrive(&job.cnt[blockIdx.x], job.tag) == (uint32_t)S ? 1u : 0u;
    __syncthreads();
    if (!last) return;
    if (live && lane < pl) {
        // the residual rows and all S partials requested before any partial
        // is added; added in slice order
        float hv[4] = {0.f, 0.f, 0.f, 0.f};
        if constexpr (EPI == MEPI_RESID) resid_rows(job, tile, r, g, Mr, hv);
        f4v a = {0.f, 0.f, 0.f, 0.f}, u = {0.f, 0.f, 0.f, 0.f};
        for (int q0 = 0; q0 < S; q0 += 8) {
            u4v va[8], vu[kTwo ? 8 : 1];
#pragma unroll
            for (int i = 0; i < 8; ++i) {
                const int q = q0 + i < S ? q0 + i : S - 1;
                const int o = (int)((tbase + q * pstride) * 4) + lane * 16;
                va[i] = __builtin_amdgcn_raw_buffer_load_b128(rs, o, 0, kSc1);
                if constexpr (kTwo) vu[i] = __builtin_amdgcn_raw_buffer_load_b128(rs, o + pl * 16, 0, kSc1);
            }
#pragma unroll
            for (int i = 0; i < 8; ++i) {
                if (q0 + i < S) {
                    a += __builtin_bit_cast(f4v, va[i]);
                    if constexpr (kTwo) u += __builtin_bit_cast(f4v, vu[i]);
                }
            }
        }
        tile_epilogue<EPI>(job, tile, r, g, Mr, a, u, hv, sq);
    } else {
        sq = f4v{0.f, 0.f, 0.f, 0.f};
    }
    if (EPI == MEPI_RESID && job.ss_out) group_row_ss(job, Mr, wave, r, g, sq, wss);
    if (threadIdx.x == 0) __hip_atomic_store(&job.cnt[blockIdx.x], 0ull, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// Slices of K for the split launch: up to 16 slices of as few chunks as that
// allows, then slices of kSplMaxCps chunks, at most kSplMaxSlices (cps
// returned); 0 when K needs more.  A function of K alone.
int split_plan(int K, int& cps) {
    const int nch = K / 256;
    cps = min(kSplMaxCps, (nch + 15) / 16);
    const int S = (nch + cps - 1) / cps;
    return S <= kSplMaxSlices ? S : 0;
}

size_t mfma_lds_bytes(int fmt, int Mr, int K, bool two = false) {
    size_t b = (size_t)(Mr + 1) * (K / 2 + 4) * 4;
    if (fmt == FMT_Q4_K) b += (size_t)(K / 32) * 16 * 4;
    return b + (size_t)(two ? 2 : 1) * kWav * 64 * 4 * 4;
}

constexpr size_t kMaxLds = 160 * 1024;
// Above this many row tiles (the lm_head) the whole-tile launch streams at
// full rate and the split partials would only add traffic.
constexpr int64_t kSplitTiles = 2048;

// Launch a job for M rows of X, in row chunks whose staging fits the LDS.
// nin: X is the RMSNorm of job.Hn (the split form only); split_only: fail
// with BX_EUNSUPPORTED, launching nothing, when the split form does not apply
// (norm-input launches, and residual launches that must report row sums).
// wtype2 >= 0: a two-format group (members from job.mem2 on), Q4_K then
// Q6_K only, split form only.
template <int EPI>
int mfma_launch(int wtype, MfmaJob job, const uint16_t* X, int M, int K, void* ws, size_t wsb, hipStream_t st,
                bool nin = false, bool split_only = false, int wtype2 = -1) {
    if (wtype2 >= 0 && (EPI != MEPI_STORE || wtype != BX_TYPE_Q4_K || wtype2 != BX_TYPE_Q6_K))
        return fail(BX_EUNSUPPORTED, "gemv: two-format groups are Q4_K then Q6_K");
    if (wtype2 < 0) job.mem2 = job.members;
    int fmt;
    switch (wtype) {
        case BX_TYPE_Q4_K: fmt = FMT_Q4_K; break;
        case BX_TYPE_Q6_K: fmt = FMT_Q6_K; break;
        case BX_TYPE_Q8_0: fmt = FMT_Q8_0; break;
        case BX_TYPE_F16: fmt = FMT_F16; break;
        default: return fail(BX_EUNSUPPORTED, "gemv mfma: unsupported type");
    }
    if (K % 256 != 0) return fail(BX_EUNSUPPORTED, "gemv mfma: K must be a multiple of 256");
    const bool two = EPI == MEPI_SWIGLU;
    int mc = M;
    while (mc > 1 && mfma_lds_bytes(fmt, mc, K, two) > kMaxLds) mc = (mc + 1) / 2;
    if (mfma_lds_bytes(fmt, mc, K, two) > kMaxLds) return fail(BX_EUNSUPPORTED, "gemv mfma: K too large for LDS staging");
    job.tiles = 0;
    for (int i = 0; i < job.members; ++i) {
        job.tiles_n[i] = ((int64_t)job.N[i] + 15) / 16;
        job.tiles += job.tiles_n[i];
    }
    const int64_t tiles = job.tiles;
    const int nch = K / 256;
    const int cus = num_cus();
    // layer-sized matrices: the split launch (one launch for all M rows)
    int cps = 0;
    const int S = split_plan(K, cps);
    const int64_t groups = (tiles + kSplWav - 1) / kSplWav;
    const bool fits = S > 0 && M <= 16 && tiles <= kSplitTiles && groups <= kSplGroups &&
                      groups * kSplWav * S * (two ? 2 : 1) * M * 16 <= kSplFloats;
    // the split form needs the caller's workspace (counters zero at entry,
    // zero again at exit); without one the shape takes the plain launch
    const bool split = fits && ws != nullptr && wsb >= kSplCntBytes + (size_t)kSplFloats * 4;
    if (fits && (split_only || nin || wtype2 >= 0) && !split)
        return fail(BX_EINVAL, "gemv: the fused-norm and two-format forms need a linear workspace "
                               "(bx_linear_workspace_bytes)");
    if (split) {
        job.cnt = static_cast<uint64_t*>(ws);
        job.tag = next_launch_tag();
        job.part = reinterpret_cast<float*>(static_cast<unsigned char*>(ws) + kSplCntBytes);
        const size_t lds = (size_t)(M + 1) * (128 * cps + 4) * 4 + (fmt == FMT_Q4_K ? (size_t)8 * cps * 16 * 4 : 0);
        const dim3 grid((unsigned)groups, (unsigned)S);
        if (wtype2 >= 0) {
            if constexpr (EPI == MEPI_STORE) {
                auto go = [&](auto nin_c) {
                    constexpr bool kN = decltype(nin_c)::value;
                    if (cps == 1)
                        gemv_split_kernel<FMT_Q4_K, EPI, 1, kN, FMT_Q6_K><<<grid, kSplThr, lds, st>>>(job, X, M, K, S);
                    else if (cps == 2)
                        gemv_split_kernel<FMT_Q4_K, EPI, 2, kN, FMT_Q6_K><<<grid, kSplThr, lds, st>>>(job, X, M, K, S);
                    else
                        gemv_split_kernel<FMT_Q4_K, EPI, 3, kN, FMT_Q6_K><<<grid, kSplThr, lds, st>>>(job, X, M, K, S);
                };
                if (nin) go(std::true_type{});
                else go(std::false_type{});
            }
        } else if (nin) {
            if constexpr (EPI != MEPI_RESID) {
                BX_DISPATCH_FMT(wtype, {
                    if (cps == 1) gemv_split_kernel<FMT_, EPI, 1, true><<<grid, kSplThr, lds, st>>>(job, X, M, K, S);
                    else if (cps == 2) gemv_split_kernel<FMT_, EPI, 2, true><<<grid, kSplThr, lds, st>>>(job, X, M, K, S);
                    else gemv_split_kernel<FMT_, EPI, 3, true><<<grid, kSplThr, lds, st>>>(job, X, M, K, S);
                })
            }
        } else {
            BX_DISPATCH_FMT(wtype, {
                if (cps == 1) gemv_split_kernel<FMT_, EPI, 1, false><<<grid, kSplThr, lds, st>>>(job, X, M, K, S);
                else if (cps == 2) gemv_split_kernel<FMT_, EPI, 2, false><<<grid, kSplThr, lds, st>>>(job, X, M, K, S);
                else gemv_split_kernel<FMT_, EPI, 3, false><<<grid, kSplThr, lds, st>>>(job, X, M, K, S);
            })
        }
        return launch_check("gemv split");
    }
    if (split_only || nin || wtype2 >= 0)
        return fail(BX_EUNSUPPORTED, "gemv: the fused-norm and two-format forms need the split launch");
    for (int m0 = 0; m0 < M; m0 += mc) {
        const int mr = M - m0 < mc ? M - m0 : mc;
        const size_t lds = mfma_lds_bytes(fmt, mr, K, two);
        MfmaJob jc = job;
        for (int i = 0; i < job.members; ++i)
            if (jc.Y[i]) jc.Y[i] += (int64_t)m0 * job.N[i];
        if (jc.H) jc.H += (int64_t)m0 * job.N[0];
        const uint16_t* Xc = X + (int64_t)m0 * K;
        BX_DISPATCH_FMT(wtype, {
            const void* fn = reinterpret_cast<const void*>(&gemv_mfma_kernel<FMT_, EPI>);
            if (lds > 64 * 1024) {
                const hipError_t e = hipFuncSetAttribute(fn, hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds);
                if (e != hipSuccess) return hip_check(e, "gemv mfma: LDS attribute");
            }
            // resident workgroups per CU (registers and LDS), asked once per
            // format and staging size
            const int occ = resident_wgs(fn, kThr, lds);
            const int64_t slots = (int64_t)cus * occ;
            // the most waves per tile (K split) whose workgroups still fit in
            // one round of resident slots; 1: whole tiles, grid-stride
            int kpart = 1;
            while (kpart * 2 <= kWav && kpart * 2 <= nch && (tiles * kpart * 2 + kWav - 1) / kWav <= slots) kpart *= 2;
            int64_t grid = (tiles * kpart + kWav - 1) / kWav;
            if (kpart == 1 && grid > slots) grid = slots;
            gemv_mfma_kernel<FMT_, EPI><<<(unsigned)grid, kThr, lds, st>>>(jc, Xc, mr, K, kpart);
        })
        if (int rc = launch_check("gemv mfma")) return rc;
    }
    return BX_OK;
}

}  // namespace

// 1 <= M <= 16, K % 256 == 0 (the linear entry point sends 3 <= M <= 16).
int gemv_mfma(int wtype, const void* W, const uint16_t* bias, const uint16_t* X, uint16_t* Y, int M, int N, int K,
              void* ws, size_t wsb, hipStream_t st) {
    MfmaJob job{};
    job.W[0] = W;
    job.Y[0] = Y;
    job.N[0] = N;
    job.bias = bias;
    job.members = 1;
    return mfma_launch<MEPI_STORE>(wtype, job, X, M, K, ws, wsb, st);
}

// The split launch only (BX_EUNSUPPORTED, nothing launched, when it does not
// take the shape): rows beyond the whole-K kernel's LDS staging.
int gemv_mfma_split(int wtype, const void* W, const uint16_t* bias, const uint16_t* X, uint16_t* Y, int M, int N, int K,
                    void* ws, size_t wsb, hipStream_t st) {
    MfmaJob job{};
    job.W[0] = W;
    job.Y[0] = Y;
    job.N[0] = N;
    job.bias = bias;
    job.members = 1;
    return mfma_launch<MEPI_STORE>(wtype, job, X, M, K, ws, wsb, st, false, true);
}

int gemv_mfma_group(int wtype, int n, const void* const* W, uint16_t* const* Y, const int* N, const uint16_t* X,
                    int M, int K, void* ws, size_t wsb, hipStream_t st) {
    MfmaJob job{};
    for (int i = 0; i < n; ++i) {
        job.W[i] = W[i];
        job.Y[i] = Y[i];
        job.N[i] = N[i];
    }
    job.members = n;
    return mfma_launch<MEPI_STORE>(wtype, job, X, M, K, ws, wsb, st);
}

int gemv_mfma_resid(int wtype, const void* W, const uint16_t* X, float* H, int M, int N, int K, void* ws, size_t wsb, hipStream_t st) {
    MfmaJob job{};
    job.W[0] = W;
    job.N[0] = N;
    job.H = H;
    job.members = 1;
    return mfma_launch<MEPI_RESID>(wtype, job, X, M, K, ws, wsb, st);
}

int gemv_mfma_resid_ss(int wtype, const void* W, const uint16_t* X, float* H, float* ss_out, int M, int N, int K,
                       void* ws, size_t wsb, hipStream_t st) {
    MfmaJob job{};
    job.W[0] = W;
    job.N[0] = N;
    job.H = H;
    job.ss_out = ss_out;
    job.members = 1;
    return mfma_launch<MEPI_RESID>(wtype, job, X, M, K, ws, wsb, st, false, true);
}

int gemv_mfma_group_norm(int wtype, int n, const void* const* W, uint16_t* const* Y, const int* N, const float* H,
                         const uint16_t* gamma, float eps, const float* ss_in, int M, int K, void* ws, size_t wsb, hipStream_t st) {
    MfmaJob job{};
    for (int i = 0; i < n; ++i) {
        job.W[i] = W[i];
        job.Y[i] = Y[i];
        job.N[i] = N[i];
    }
    job.members = n;
    job.Hn = H;
    job.gamma = gamma;
    job.eps = eps;
    job.ss_in = ss_in;
    job.ss_groups = (K + 63) / 64;
    return mfma_launch<MEPI_STORE>(wtype, job, nullptr, M, K, ws, wsb, st, true);
}

int gemv_mfma_group2(int wtype, int wtype2, int n, int n1, const void* const* W, uint16_t* const* Y, const int* N,
                     const uint16_t* X, const float* H, const uint16_t* gamma, float eps, const float* ss_in, int M,
                     int K, void* ws, size_t wsb, hipStream_t st) {
    MfmaJob job{};
    for (int i = 0; i < n; ++i) {
        job.W[i] = W[i];
        job.Y[i] = Y[i];
        job.N[i] = N[i];
    }
    job.members = n;
    job.mem2 = n1;
    const bool nin = H != nullptr;
    if (nin) {
        job.Hn = H;
        job.gamma = gamma;
        job.eps = eps;
        job.ss_in = ss_in;
        job.ss_groups = (K + 63) / 64;
    }
    return mfma_launch<MEPI_STORE>(wtype, job, X, M, K, ws, wsb, st, nin, true, wtype2);
}

int gemv_mfma_swiglu_norm(int wtype, const void* Wg, const void* Wu, const float* H, const uint16_t* gamma, float eps,
                          const float* ss_in, uint16_t* Y, int M, int F, int K, void* ws, size_t wsb, hipStream_t st) {
    MfmaJob job{};
    job.W[0] = Wg;
    job.W[1] = Wu;
    job.Y[0] = Y;
    job.N[0] = F;
    job.members = 1;
    job.Hn = H;
    job.gamma = gamma;
    job.eps = eps;
    job.ss_in = ss_in;
    job.ss_groups = (K + 63) / 64;
    return mfma_launch<MEPI_SWIGLU>(wtype, job, nullptr, M, K, ws, wsb, st, true);
}

int gemv_mfma_swiglu(int wtype, const void* Wg, const void* Wu, const uint16_t* X, uint16_t* Y, int M, int F, int K,
                     void* ws, size_t wsb, hipStream_t st) {
    MfmaJob job{};
    job.W[0] = Wg;
    job.W[1] = Wu;
    job.Y[0] = Y;
    job.N[0] = F;
    job.members = 1;   // one tile space; each tile takes the same rows of both
    return mfma_launch<MEPI_SWIGLU>(wtype, job, X, M, K, ws, wsb, st);
}

}  // namespace bx

extern "C" size_t bx_linear_workspace_bytes(void) { return bx::kSplCntBytes + (size_t)bx::kSplFloats * 4; }

extern "C" int bx_linear_workspace_init(void* ws, size_t ws_bytes, void* stream) {
    if (!ws || ws_bytes < bx_linear_workspace_bytes())
        return bx::fail(BX_EINVAL, "linear_workspace_init: workspace smaller than bx_linear_workspace_bytes()");
    bx::split_clear_kernel<<<16, 256, 0, bx::as_stream(stream)>>>(static_cast<uint64_t*>(ws));
    return bx::launch_check("linear workspace init");
}
