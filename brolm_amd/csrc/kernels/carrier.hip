// GGUF block repack into device carriers, the inverse, and bit-exact dequant
// (brotensor::dequant_{q8_0,q4k,q6k}_to_fp16, called at
// include/brolm/detail/weights.h:325-339).
//
// Block formats follow the published ggml k-quants (llama.cpp ggml-quants.c,
// block_q8_0 / block_q4_K / block_q6_K).  Dequant arithmetic: every product
// d*sc, dmin*m, (d*sc)*q is exact in FP32 (at most 23 significant bits), and
// Q4_K's single subtraction is correctly rounded with or without FMA, so the
// FP32 values do not depend on operation order.  FP32 -> FP16 is RNE with
// FP16 denormals kept.
#include "carrier_layout.h"
#include "common.h"

namespace bx {
namespace {

// One thread per GGUF block.  gguf: source bytes (row-major blocks);
// to_carrier selects the direction.
template <bool TO_CARRIER>
__global__ void q8_repack_kernel(const uint8_t* __restrict__ src, uint8_t* __restrict__ dst, int64_t N, int64_t K) {
    const int64_t nb32 = K / 32;
    const int64_t s = blockIdx.x * (int64_t)blockDim.x + threadIdx.x;
    if (s >= N * nb32) return;
    const CarrierQ8 c = carrier_q8(TO_CARRIER ? dst : src, N, K);
    uint8_t* cqs = const_cast<uint8_t*>(c.qs) + s * 32;
    uint8_t* cd = const_cast<uint8_t*>(c.d) + s * 2;
    if (TO_CARRIER) {
        const uint8_t* g = src + s * 34;
        cd[0] = g[0];
        cd[1] = g[1];
        for (int i = 0; i < 32; ++i) cqs[i] = g[2 + i];
    } else {
        uint8_t* g = dst + s * 34;
        g[0] = cd[0];
        g[1] = cd[1];
        for (int i = 0; i < 32; ++i) g[2 + i] = cqs[i];
    }
}

template <bool TO_CARRIER>
__global__ void q4k_repack_kernel(const uint8_t* __restrict__ src, uint8_t* __restrict__ dst, int64_t N, int64_t K) {
    const int64_t nb = K / 256;
    const int64_t s = blockIdx.x * (int64_t)blockDim.x + threadIdx.x;
    if (s >= N * nb) return;
    const CarrierQ4K c = carrier_q4k(TO_CARRIER ? dst : src, N, K);
    uint8_t* cqs = const_cast<uint8_t*>(c.qs) + s * 128;
    uint8_t* ch = const_cast<uint8_t*>(c.hdr) + s * 16;
    if (TO_CARRIER) {
        const uint8_t* g = src + s * 144;
        for (int i = 0; i < 16; ++i) ch[i] = g[i];
        for (int i = 0; i < 128; ++i) cqs[i] = g[16 + i];
    } else {
        uint8_t* g = dst + s * 144;
        for (int i = 0; i < 16; ++i) g[i] = ch[i];
        for (int i = 0; i < 128; ++i) g[16 + i] = cqs[i];
    }
}

// GGUF block_q6_K: ql[128] @0, qh[64] @128, scales[16] @192, d @208.
template <bool TO_CARRIER>
__global__ void q6k_repack_kernel(const uint8_t* __restrict__ src, uint8_t* __restrict__ dst, int64_t N, int64_t K) {
    const int64_t nb = K / 256;
    const int64_t s = blockIdx.x * (int64_t)blockDim.x + threadIdx.x;
    if (s >= N * nb) return;
    const CarrierQ6K c = carrier_q6k(TO_CARRIER ? dst : src, N, K);
    uint8_t* cql = const_cast<uint8_t*>(c.ql) + s * 128;
    uint8_t* cqh = const_cast<uint8_t*>(c.qh) + s * 64;
    uint8_t* csc = const_cast<uint8_t*>(c.sc) + s * 16;
    uint8_t* cd = const_cast<uint8_t*>(c.d) + s * 2;
    uint8_t* g = TO_CARRIER ? const_cast<uint8_t*>(src) + s * 210 : dst + s * 210;
    for (int t = 0; t < 8; ++t) {
        const int h = t >> 2, l0 = 8 * (t & 3);
        for (int i = 0; i < 8; ++i) {
            uint8_t* a = &cql[16 * t + i];
            uint8_t* b = &cql[16 * t + 8 + i];
            uint8_t* q = &cqh[8 * t + i];
            uint8_t* ga = &g[64 * h + l0 + i];
            uint8_t* gb = &g[64 * h + 32 + l0 + i];
            uint8_t* gq = &g[128 + 32 * h + l0 + i];
            if (TO_CARRIER) { *a = *ga; *b = *gb; *q = *gq; } else { *ga = *a; *gb = *b; *gq = *q; }
        }
    }
    for (int i = 0; i < 16; ++i) {
        if (TO_CARRIER) csc[i] = g[192 + i]; else g[192 + i] = csc[i];
    }
    if (TO_CARRIER) { cd[0] = g[208]; cd[1] = g[209]; } else { g[208] = cd[0]; g[209] = cd[1]; }
}

#pragma clang fp contract(off)

// Dequant: one thread per 32 output elements (one Q8_0 block, or one Q4_K
// sub-block, or two Q6_K sub-blocks of 16).
template <typename OutT>
__device__ __forceinline__ void store_out(OutT* p, float v);
template <>
__device__ __forceinline__ void store_out<float>(float* p, float v) { *p = v; }
template <>
__device__ __forceinline__ void store_out<uint16_t>(uint16_t* p, float v) { *p = f2h(v); }

template <typename OutT>
__global__ void dequant_q8_kernel(const uint8_t* __restrict__ base, OutT* __restrict__ out, int64_t N, int64_t K) {
    const int64_t nb32 = K / 32;
    const int64_t s = blockIdx.x * (int64_t)blockDim.x + threadIdx.x;
    if (s >= N * nb32) return;
    const CarrierQ8 c = carrier_q8(base, N, K);
    const float d = h2f(*reinterpret_cast<const uint16_t*>(c.d + s * 2));
    const int8_t* q = reinterpret_cast<const int8_t*>(c.qs + s * 32);
    for (int i = 0; i < 32; ++i) store_out(out + s * 32 + i, d * (float)q[i]);
}

template <typename OutT>
__global__ void dequant_q4k_kernel(const uint8_t* __restrict__ base, OutT* __restrict__ out, int64_t N, int64_t K) {
    const int64_t nb = K / 256;
    const int64_t t = blockIdx.x * (int64_t)blockDim.x + threadIdx.x;  // sub-block index
    if (t >= N * nb * 8) return;
    const int64_t s = t >> 3;
    const int j = (int)(t & 7);
    const CarrierQ4K c = carrier_q4k(base, N, K);
    const uint8_t* h = c.hdr + s * 16;
    const float d = h2f(*reinterpret_cast<const uint16_t*>(h));
    const float dmin = h2f(*reinterpret_cast<const uint16_t*>(h + 2));
    int sc, m;
    q4k_scale_min(j, h + 4, sc, m);
    const float d1 = d * (float)sc;
    const float m1 = dmin * (float)m;
    const uint8_t* q = c.qs + s * 128 + 32 * (j >> 1);
    const int shift = (j & 1) * 4;
    OutT* o = out + s * 256 + 32 * j;
    for (int l = 0; l < 32; ++l) store_out(o + l, d1 * (float)((q[l] >> shift) & 0x0f) - m1);
}

template <typename OutT>
__global__ void dequant_q6k_kernel(const uint8_t* __restrict__ base, OutT* __restrict__ out, int64_t N, int64_t K) {
    const int64_t nb = K / 256;
    const int64_t t = blockIdx.x * (int64_t)blockDim.x + threadIdx.x;  // carrier unit (32 elems)
    if (t >= N * nb * 8) return;
    const int64_t s = t >> 3;
    const int u = (int)(t & 7);
    const int h = u >> 2, l0 = 8 * (u & 3);
    const CarrierQ6K c = carrier_q6k(base, N, K);
    const uint8_t* ql = c.ql + s * 128 + 16 * u;
    const uint8_t* qh = c.qh + s * 64 + 8 * u;
    const int8_t* sc = reinterpret_cast<const int8_t*>(c.sc + s * 16);
    const float d = h2f(*reinterpret_cast<const uint16_t*>(c.d + s * 2));
    OutT* o = out + s * 256 + 128 * h + l0;
    for (int i = 0; i < 8; ++i) {
        const int l = l0 + i;
        const int is = l / 16;
        const int q1 = (int)((ql[i] & 0x0f) | (((qh[i] >> 0) & 3) << 4)) - 32;
        const int q2 = (int)((ql[8 + i] & 0x0f) | (((qh[i] >> 2) & 3) << 4)) - 32;
        const int q3 = (int)((ql[i] >> 4) | (((qh[i] >> 4) & 3) << 4)) - 32;
        const int q4 = (int)((ql[8 + i] >> 4) | (((qh[i] >> 6) & 3) << 4)) - 32;
        store_out(o + i, d * (float)sc[8 * h + is + 0] * (float)q1);
        store_out(o + 32 + i, d * (float)sc[8 * h + is + 2] * (float)q2);
        store_out(o + 64 + i, d * (float)sc[8 * h + is + 4] * (float)q3);
        store_out(o + 96 + i, d * (float)sc[8 * h + is + 6] * (float)q4);
    }
}

template <typename OutT>
__global__ void dense_copy_kernel(const uint16_t* __restrict__ in, OutT* __restrict__ out, int64_t n) {
    const int64_t i = blockIdx.x * (int64_t)blockDim.x + threadIdx.x;
    if (i < n) store_out(out + i, h2f(in[i]));
}

#pragma clang fp contract(on)

int check_shape(int type, int64_t rows, int64_t cols) {
    const int64_t be = type_block_elems(type);
    if (be == 0) return fail(BX_EUNSUPPORTED, "unsupported carrier type " + std::to_string(type));
    if (rows < 0 || cols <= 0 || cols % be != 0)
        return fail(BX_EINVAL, "carrier shape (" + std::to_string(rows) + ", " + std::to_string(cols) +
                                   ") not a multiple of the block size " + std::to_string(be));
    return BX_OK;
}

inline unsigned grid_for(int64_t n, int bs) { return (unsigned)((n + bs - 1) / bs); }

template <typename OutT>
int dequant_impl(int type, const void* carrier, OutT* dst, int64_t rows, int64_t cols, void* stream) {
    if (int rc = check_shape(type, rows, cols)) return rc;
    if (!carrier || !dst) return fail(BX_EINVAL, "dequant: null pointer");
    if (rows == 0) return BX_OK;
    hipStream_t st = as_stream(stream);
    const uint8_t* b = static_cast<const uint8_t*>(carrier);
    switch (type) {
        case BX_TYPE_Q8_0: {
            const int64_t n = rows * (cols / 32);
            dequant_q8_kernel<OutT><<<grid_for(n, 256), 256, 0, st>>>(b, dst, rows, cols);
            break;
        }
        case BX_TYPE_Q4_K: {
            const int64_t n = rows * (cols / 256) * 8;
            dequant_q4k_kernel<OutT><<<grid_for(n, 256), 256, 0, st>>>(b, dst, rows, cols);
            break;
        }
        case BX_TYPE_Q6_K: {
            const int64_t n = rows * (cols / 256) * 8;
            dequant_q6k_kernel<OutT><<<grid_for(n, 256), 256, 0, st>>>(b, dst, rows, cols);
            break;
        }
        case BX_TYPE_F16: {
            const int64_t n = rows * cols;
            dense_copy_kernel<OutT><<<grid_for(n, 256), 256, 0, st>>>(static_cast<const uint16_t*>(carrier), dst, n);
            break;
        }
        default: return fail(BX_EUNSUPPORTED, "dequant: unsupported type");
    }
    return launch_check("dequant");
}

template <bool TO_CARRIER>
int repack_impl(int type, const void* src, void* dst, int64_t rows, int64_t cols, void* stream) {
    if (int rc = check_shape(type, rows, cols)) return rc;
    if (!src || !dst) return fail(BX_EINVAL, "repack: null pointer");
    if (src == dst) return fail(BX_EINVAL, "repack: src and dst must not alias");
    if (rows == 0) return BX_OK;
    hipStream_t st = as_stream(stream);
    const uint8_t* s = static_cast<const uint8_t*>(src);
    uint8_t* d = static_cast<uint8_t*>(dst);
    switch (type) {
        case BX_TYPE_Q8_0:
            q8_repack_kernel<TO_CARRIER><<<grid_for(rows * (cols / 32), 256), 256, 0, st>>>(s, d, rows, cols);
            break;
        case BX_TYPE_Q4_K:
            q4k_repack_kernel<TO_CARRIER><<<grid_for(rows * (cols / 256), 256), 256, 0, st>>>(s, d, rows, cols);
            break;
        case BX_TYPE_Q6_K:
            q6k_repack_kernel<TO_CARRIER><<<grid_for(rows * (cols / 256), 256), 256, 0, st>>>(s, d, rows, cols);
            break;
        case BX_TYPE_F16:
        case BX_TYPE_F32:
            return hip_check(hipMemcpyAsync(dst, src, (size_t)(rows * cols * type_block_bytes(type)),
                                            hipMemcpyDeviceToDevice, st),
                             "repack copy");
        default: return fail(BX_EUNSUPPORTED, "repack: unsupported type");
    }
    return launch_check("repack");
}

}  // namespace
}  // namespace bx

extern "C" {

int64_t bx_carrier_bytes(int type, int64_t rows, int64_t cols) {
    const int64_t be = bx::type_block_elems(type);
    if (be == 0 || cols <= 0 || rows < 0 || cols % be) return -1;
    return rows * (cols / be) * bx::type_block_bytes(type);
}

int bx_repack_gguf_rows(int type, const void* src, void* dst, int64_t rows, int64_t cols, void* stream) {
    return bx::repack_impl<true>(type, src, dst, rows, cols, stream);
}

int bx_unpack_carrier_rows(int type, const void* src, void* dst, int64_t rows, int64_t cols, void* stream) {
    return bx::repack_impl<false>(type, src, dst, rows, cols, stream);
}

int bx_dequant_to_f16(int type, const void* carrier, uint16_t* dst, int64_t rows, int64_t cols, void* stream) {
    return bx::dequant_impl<uint16_t>(type, carrier, dst, rows, cols, stream);
}

int bx_dequant_to_f32(int type, const void* carrier, float* dst, int64_t rows, int64_t cols, void* stream) {
    return bx::dequant_impl<float>(type, carrier, dst, rows, cols, stream);
}

}  // extern "C"
