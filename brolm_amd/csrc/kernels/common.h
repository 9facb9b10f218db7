// Shared device helpers and host-side launch plumbing for the gfx950 kernels.
#pragma once

#include <hip/hip_runtime.h>

#include <cstddef>
#include <cstdint>
#include <string>

#include "../../../include/brolm_hip.h"

namespace bx {

// ---------------------------------------------------------------- host side

// Thread-local error message behind bx_last_error().
void set_error(const std::string& msg);
int fail(int code, const std::string& msg);
// Check a HIP status; on error record it and return BX_ELAUNCH.
int hip_check(hipError_t e, const char* what);
// Check the launch that was just issued.
int launch_check(const char* what);

inline hipStream_t as_stream(void* s) { return reinterpret_cast<hipStream_t>(s); }

// Number of compute units on the current device (cached per device).
int num_cus();
// true when a rocprofiler-sdk tool (rocprofv3) is loaded into the process
bool profiler_attached();

// A new nonzero 32-bit tag per call (1, 2, ..., wrapping past 0), for
// kernels whose workgroups count arrivals in caller memory (tagged_arrive).
uint32_t next_launch_tag();
// Workgroups of `threads` threads and `lds` dynamic LDS bytes that one CU
// holds at once for kernel `fn` (registers and LDS); asked of the runtime once
// per (kernel, threads, LDS) and cached; at least 1.
int resident_wgs(const void* fn, int threads, size_t lds);

// Workgroups per CU launched for the wide-row GEMVs (K above 12288), one
// round of residents: a lane's 128+ registers and up to 80 KB of staged
// activations leave room for two.
#ifndef BX_WIDE_WGS_PER_CU
#define BX_WIDE_WGS_PER_CU 2
#endif

// ------------------------------------------------------------- device side

typedef _Float16 h2 __attribute__((ext_vector_type(2)));
typedef unsigned u4v __attribute__((ext_vector_type(4)));
typedef unsigned u2v __attribute__((ext_vector_type(2)));
typedef float f2v __attribute__((ext_vector_type(2)));

__device__ __forceinline__ float h2f(uint16_t b) { return (float)__builtin_bit_cast(_Float16, b); }
// FP32 -> FP16 with round-to-nearest-even (v_cvt_f16_f32 under the default
// mode; FP16 denormals are kept by the default gfx950 float mode).
__device__ __forceinline__ uint16_t f2h(float f) { return __builtin_bit_cast(uint16_t, (_Float16)f); }

// SiLU as the elementwise kernels compute it (x / (1 + e^-x), fast exp).
__device__ __forceinline__ float silu_f32(float x) { return x / (1.0f + __expf(-x)); }

// An FP32 value the compiler cannot fuse into the instruction that consumes
// it.  The backend otherwise turns an FP32 multiply followed by an FP16
// conversion into one mixed-precision multiply (v_fma_mixlo_f16, a single
// rounding straight to FP16) in some kernels and not in others, so the same
// expression could round differently from one kernel to the next.
__device__ __forceinline__ float f32_fence(float x) {
    float y;
    asm("v_mov_b32 %0, %1" : "=v"(y) : "v"(x));
    return y;
}

// An RMSNorm output element: x * inv * gain rounded to FP32, then to FP16,
// the same bits in every kernel that applies a norm this way.
__device__ __forceinline__ uint16_t norm_f16(float x, float inv, float gain) {
    return f2h(f32_fence(x * inv * gain));
}

__device__ __forceinline__ h2 as_h2(uint32_t v) { return __builtin_bit_cast(h2, v); }
__device__ __forceinline__ uint32_t as_u32(h2 v) { return __builtin_bit_cast(uint32_t, v); }

__device__ __forceinline__ float dot2(uint32_t a, uint32_t b, float c) {
    return __builtin_amdgcn_fdot2(as_h2(a), as_h2(b), c, false);
}

// Global-memory views of generic pointers.  A pointer the compiler cannot
// trace to a kernel argument (e.g. one read from a device-side table of
// layers) is generic, and generic accesses become flat instructions, which
// count against lgkmcnt as well as vmcnt: every later wait for an LDS access
// would then also wait for them.  An explicit address-space cast keeps weight
// streams on global_load and out of the LDS counter.
#define BX_GLOBAL __attribute__((address_space(1)))
template <class T>
__device__ __forceinline__ const BX_GLOBAL T* gptr(const void* p) {
    return (const BX_GLOBAL T*)p;
}
template <class T>
__device__ __forceinline__ BX_GLOBAL T* gptr_w(void* p) {
    return (BX_GLOBAL T*)p;
}

// Streaming (read-once) loads: the `nt` hint keeps weight streams from
// thrashing L2/MALL; measured 7.1 TB/s vs 6.3 TB/s for plain loads.
__device__ __forceinline__ u4v ldg_nt16(const void* p) { return __builtin_nontemporal_load(gptr<u4v>(p)); }
__device__ __forceinline__ u2v ldg_nt8(const void* p) { return __builtin_nontemporal_load(gptr<u2v>(p)); }
__device__ __forceinline__ u4v ldg16(const void* p) { return *gptr<u4v>(p); }
__device__ __forceinline__ uint16_t ldg_u16(const void* p) { return *gptr<uint16_t>(p); }

// Cross-lane value by DPP (no LDS traffic): CTRL selects the source lane
// (quad_perm within 4 lanes, row_half_mirror 0x141 / row_mirror 0x140 within
// a row of 16, row_bcast:15 0x142 / row_bcast:31 0x143 from lane 15 / 31 into
// later rows); rows outside ROWS take `ident`.
template <int CTRL, int ROWS = 0xF>
__device__ __forceinline__ float dpp_f(float v, float ident) {
    return __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(__builtin_bit_cast(int, ident),
                                                                 __builtin_bit_cast(int, v), CTRL, ROWS, 0xF, false));
}
__device__ __forceinline__ float lane63(float v) {
    return __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), 63));
}

// Full 64-lane wavefront sum / max, returned in every lane: four steps give
// every lane its row's result, the two broadcasts fold the rows into lane 63.
__device__ __forceinline__ float wave_sum(float v) {
    v += dpp_f<0xB1>(v, 0.f);
    v += dpp_f<0x4E>(v, 0.f);
    v += dpp_f<0x141>(v, 0.f);
    v += dpp_f<0x140>(v, 0.f);
    v += dpp_f<0x142, 0xA>(v, 0.f);
    v += dpp_f<0x143, 0xC>(v, 0.f);
    return lane63(v);
}
__device__ __forceinline__ float wave_max(float v) {
    v = fmaxf(v, dpp_f<0xB1>(v, -INFINITY));
    v = fmaxf(v, dpp_f<0x4E>(v, -INFINITY));
    v = fmaxf(v, dpp_f<0x141>(v, -INFINITY));
    v = fmaxf(v, dpp_f<0x140>(v, -INFINITY));
    v = fmaxf(v, dpp_f<0x142, 0xA>(v, -INFINITY));
    v = fmaxf(v, dpp_f<0x143, 0xC>(v, -INFINITY));
    return lane63(v);
}
// R independent sums reduced step by step together, so the steps of
// different rows overlap instead of waiting on each other.
template <int R>
__device__ __forceinline__ void wave_sum_n(float (&v)[R]) {
#pragma unroll
    for (int r = 0; r < R; ++r) v[r] += dpp_f<0xB1>(v[r], 0.f);
#pragma unroll
    for (int r = 0; r < R; ++r) v[r] += dpp_f<0x4E>(v[r], 0.f);
#pragma unroll
    for (int r = 0; r < R; ++r) v[r] += dpp_f<0x141>(v[r], 0.f);
#pragma unroll
    for (int r = 0; r < R; ++r) v[r] += dpp_f<0x140>(v[r], 0.f);
#pragma unroll
    for (int r = 0; r < R; ++r) v[r] += dpp_f<0x142, 0xA>(v[r], 0.f);
#pragma unroll
    for (int r = 0; r < R; ++r) v[r] += dpp_f<0x143, 0xC>(v[r], 0.f);
#pragma unroll
    for (int r = 0; r < R; ++r) v[r] = lane63(v[r]);
}

// Block-wide sum for blockDim.x == NT (multiple of 64); `red` is >= NT/64 floats of LDS.
template <int NT>
__device__ __forceinline__ float block_sum(float v, float* red) {
    v = wave_sum(v);
    const int w = threadIdx.x >> 6, l = threadIdx.x & 63;
    __syncthreads();
    if (l == 0) red[w] = v;
    __syncthreads();
    float s = 0.f;
#pragma unroll
    for (int i = 0; i < NT / 64; ++i) s += red[i];
    return s;
}

// Q4_K 6-bit scale/min of sub-block j from the 12 packed bytes (ggml get_scale_min_k4).
__device__ __forceinline__ void q4k_scale_min(int j, const uint8_t* q, int& sc, int& m) {
    if (j < 4) {
        sc = q[j] & 63;
        m = q[j + 4] & 63;
    } else {
        sc = (q[j + 4] & 0x0f) | ((q[j - 4] >> 6) << 4);
        m = (q[j + 4] >> 4) | ((q[j] >> 6) << 4);
    }
}

// Q4_K scale/min of sub-block j from the scales dwords y (bytes 0-3),
// z (bytes 4-7), w (bytes 8-11); same bit layout as q4k_scale_min.
__device__ __forceinline__ void q4k_scale_min_regs(uint32_t y, uint32_t z, uint32_t w, int j, int& sc, int& m) {
    const int sh = 8 * (j & 3);
    const uint32_t by = (y >> sh) & 0xff, bz = (z >> sh) & 0xff, bw = (w >> sh) & 0xff;
    if (j < 4) {
        sc = (int)(by & 63);
        m = (int)(bz & 63);
    } else {
        sc = (int)((bw & 0x0f) | ((by >> 6) << 4));
        m = (int)((bw >> 4) | ((bz >> 6) << 4));
    }
}


// One workgroup's arrival at a counter word in caller memory that the last
// arrival of a launch puts back to zero; returns the arrival's number (1 for
// the first).  The word is {sum of the arrivals' tags mod 2^32 (high half),
// arrivals (low half)}, "clean" for tag T when high == low * T.  An arrival
// adds (T, 1) in one atomic; when the word it added to was not clean for T
// (left by a launch that never finished, or never cleared), the arrival
// restarts the count at (T, 1) by compare-and-swap, or joins a count another
// arrival of the same launch already restarted: a clean word stays clean, so
// no other launch's arrivals are ever counted.  Replays of a captured launch
// reuse one tag; each finds the word at zero.
__device__ __forceinline__ uint32_t tagged_arrive(uint64_t* word, uint32_t tag) {
    const uint64_t add = ((uint64_t)tag << 32) | 1u;
    auto clean = [tag](uint64_t v) { return (uint32_t)(v >> 32) == (uint32_t)v * tag; };
    const uint64_t old = __hip_atomic_fetch_add(word, add, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    if (clean(old)) return (uint32_t)old + 1u;
    uint64_t cur = __hip_atomic_load(word, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT), nw;
    do {
        nw = clean(cur) ? cur + add : add;
    } while (!__hip_atomic_compare_exchange_weak(word, &cur, nw, __ATOMIC_RELAXED, __ATOMIC_RELAXED,
                                                 __HIP_MEMORY_SCOPE_AGENT));
    return (uint32_t)nw;
}

// Scales and mins of sub-blocks 2c and 2c+1 (c = 0..3) of a Q4_K block from
// its scale dwords y (bytes 0-3), z (bytes 4-7), w (bytes 8-11): the same
// values as q4k_scale_min_regs, as eight bit-field extracts whichever half c
// falls in.  Sub-blocks 0-3 keep 6 bits in bytes j (scale) and j+4 (min);
// sub-blocks 4-7 keep the low 4 bits in the nibbles of byte j+4 and the high
// 2 bits in the top bits of bytes j-4 (scale) and j (min).  A width-0 field
// reads as 0, which drops the high part for the first half.
__device__ __forceinline__ void q4k_pair_scales(uint32_t y, uint32_t z, uint32_t w, int c, int& sc0, int& m0,
                                                int& sc1, int& m1) {
    const bool lo = c < 2;
    const uint32_t o = 16u * (uint32_t)(c & 1);
    const uint32_t as = lo ? y : w, am = lo ? z : w;
    const uint32_t wl = lo ? 6u : 4u, wh = lo ? 0u : 2u, om = lo ? o : o + 4u;
    sc0 = (int)(__builtin_amdgcn_ubfe(as, o, wl) | (__builtin_amdgcn_ubfe(y, o + 6u, wh) << 4));
    sc1 = (int)(__builtin_amdgcn_ubfe(as, o + 8u, wl) | (__builtin_amdgcn_ubfe(y, o + 14u, wh) << 4));
    m0 = (int)(__builtin_amdgcn_ubfe(am, om, wl) | (__builtin_amdgcn_ubfe(z, o + 6u, wh) << 4));
    m1 = (int)(__builtin_amdgcn_ubfe(am, om + 8u, wl) | (__builtin_amdgcn_ubfe(z, o + 14u, wh) << 4));
}

}  // namespace bx
