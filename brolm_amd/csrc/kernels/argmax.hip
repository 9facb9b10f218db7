// Device greedy sampling: argmax over FP16 logits with the reference's tie
// rule (strict '>' scan, so the lowest index wins; src/detail/generate.cpp:38-48).
#include <cmath>
#include <mutex>

#include "common.h"

// Partials of bx_argmax_f16_noalloc, the entry point that allocates nothing:
// one float value and one int index per partial block.  Each GPU the library
// runs on holds its own copy until the process ends.  Host code never uses
// this name as an address: the per-device address comes from
// hipGetSymbolAddress (scratch_device_ptr below).
static __device__ __align__(256) unsigned char scratch[256 * (sizeof(float) + sizeof(int))];

namespace bx {
namespace {

constexpr int kArgThreads = 256;
constexpr int kArgBlocks = 256;

struct VI {
    float v;
    int i;
};

// Preferred of two candidates: larger value, or the lower index on equal
// values; index -1 marks "no candidate"; a NaN loses to any number.
__device__ __forceinline__ VI better(VI a, VI b) {
    if (b.i < 0) return a;
    if (a.i < 0) return b;
    if (a.v > b.v) return a;
    if (b.v > a.v) return b;
    const bool an = a.v != a.v, bn = b.v != b.v;
    if (an != bn) return an ? b : a;
    return a.i < b.i ? a : b;
}

__device__ VI block_best(VI x, float* sv, int* si) {
#pragma unroll
    for (int off = 32; off >= 1; off >>= 1) {
        VI o{__shfl_xor(x.v, off, 64), __shfl_xor(x.i, off, 64)};
        x = better(x, o);
    }
    const int w = threadIdx.x >> 6, l = threadIdx.x & 63;
    if (l == 0) { sv[w] = x.v; si[w] = x.i; }
    __syncthreads();
    VI r{sv[0], si[0]};
    for (int k = 1; k < kArgThreads / 64; ++k) r = better(r, VI{sv[k], si[k]});
    return r;
}

__global__ __launch_bounds__(kArgThreads) void argmax_partial(const uint16_t* __restrict__ x, int64_t n,
                                                              float* __restrict__ pv, int* __restrict__ pi) {
    __shared__ float sv[kArgThreads / 64];
    __shared__ int si[kArgThreads / 64];
    VI best{-INFINITY, -1};
    for (int64_t i = blockIdx.x * (int64_t)kArgThreads + threadIdx.x; i < n; i += (int64_t)gridDim.x * kArgThreads) {
        const VI c{h2f(x[i]), (int)i};
        best = better(best, c);
    }
    best = block_best(best, sv, si);
    if (threadIdx.x == 0) { pv[blockIdx.x] = best.v; pi[blockIdx.x] = best.i; }
}

__global__ __launch_bounds__(kArgThreads) void argmax_final(const float* __restrict__ pv, const int* __restrict__ pi,
                                                            int nb, int32_t* __restrict__ out) {
    __shared__ float sv[kArgThreads / 64];
    __shared__ int si[kArgThreads / 64];
    VI best{-INFINITY, -1};
    for (int k = threadIdx.x; k < nb; k += kArgThreads) {
        const VI c{pv[k], pi[k]};
        best = better(best, c);
    }
    best = block_best(best, sv, si);
    if (threadIdx.x == 0) *out = best.i < 0 ? 0 : best.i;
}

static_assert(sizeof(scratch) == (size_t)kArgBlocks * (sizeof(float) + sizeof(int)),
              "scratch holds exactly one round of partials");

// Launch the two argmax kernels with the partials at pv / pi.
int argmax_launch(const uint16_t* logits, int64_t n, int32_t* out, float* pv, int* pi, hipStream_t st) {
    int64_t nb = (n + kArgThreads - 1) / kArgThreads;
    if (nb > kArgBlocks) nb = kArgBlocks;
    argmax_partial<<<(unsigned)nb, kArgThreads, 0, st>>>(logits, n, pv, pi);
    if (int rc = launch_check("argmax partial")) return rc;
    argmax_final<<<1, kArgThreads, 0, st>>>(pv, pi, (int)nb, out);
    return launch_check("argmax final");
}

// Device address of `scratch` on the current device: looked up once per
// device (with that device current) and kept.
constexpr int kMaxDevices = 64;
std::mutex g_scratch_mu;
void* g_scratch_ptr[kMaxDevices] = {};

int scratch_device_ptr(void** out) {
    int dev = 0;
    if (int rc = hip_check(hipGetDevice(&dev), "argmax_noalloc: hipGetDevice")) return rc;
    if (dev < 0 || dev >= kMaxDevices) return fail(BX_EUNSUPPORTED, "argmax_noalloc: device index above 63");
    std::lock_guard<std::mutex> lock(g_scratch_mu);
    if (!g_scratch_ptr[dev]) {
        void* p = nullptr;
        if (int rc = hip_check(hipGetSymbolAddress(&p, HIP_SYMBOL(scratch)), "argmax_noalloc: hipGetSymbolAddress"))
            return rc;
        if (!p) return fail(BX_ELAUNCH, "argmax_noalloc: scratch has no device address");
        g_scratch_ptr[dev] = p;
    }
    *out = g_scratch_ptr[dev];
    return BX_OK;
}

}  // namespace
}  // namespace bx

using namespace bx;

extern "C" {

size_t bx_argmax_workspace_bytes(int64_t n) {
    (void)n;
    return (size_t)kArgBlocks * (sizeof(float) + sizeof(int));
}

int bx_argmax_f16(const uint16_t* logits, int64_t n, int32_t* out, void* workspace, void* stream) {
    if (!logits || !out || !workspace || n <= 0 || n > 0x7fffffff) return fail(BX_EINVAL, "argmax: bad arguments");
    float* pv = static_cast<float*>(workspace);
    int* pi = reinterpret_cast<int*>(pv + kArgBlocks);
    return argmax_launch(logits, n, out, pv, pi, as_stream(stream));
}

int bx_argmax_f16_noalloc(const uint16_t* logits, int64_t n, int32_t* out, void* stream) {
    if (!logits || !out || n <= 0) return fail(BX_EINVAL, "argmax_noalloc: bad arguments");
    if (n > 0x7fffffff) return fail(BX_EUNSUPPORTED, "argmax_noalloc: n above 2^31 - 1 elements");
    if (bx_argmax_workspace_bytes(n) > sizeof(scratch))
        return fail(BX_EUNSUPPORTED, "argmax_noalloc: partials exceed the 2048-byte scratch");
    void* p = nullptr;
    if (int rc = scratch_device_ptr(&p)) return rc;
    // every partial argmax_final reads is written by argmax_partial in the
    // same call: nothing carries over from an earlier call
    float* pv = static_cast<float*>(p);
    int* pi = reinterpret_cast<int*>(pv + kArgBlocks);
    return argmax_launch(logits, n, out, pv, pi, as_stream(stream));
}

}  // extern "C"
