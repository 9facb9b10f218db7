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

// ------------------------------------------------------------- device side

typedef _Float16 h2 __attribute__((ext_vector_type(2)));
typedef unsigned u4v __attribute__((ext_vector_type(4)));
typedef unsigned u2v __attribute__((ext_vector_type(2)));

__device__ __forceinline__ float h2f(uint16_t b) { return (float)__builtin_bit_cast(_Float16, b); }
// FP32 -> FP16 with round-to-nearest-even (v_cvt_f16_f32 under the default
// mode; FP16 denormals are kept by the default gfx950 float mode).
__device__ __forceinline__ uint16_t f2h(float f) { return __builtin_bit_cast(uint16_t, (_Float16)f); }

__device__ __forceinline__ h2 as_h2(uint32_t v) { return __builtin_bit_cast(h2, v); }
__device__ __forceinline__ uint32_t as_u32(h2 v) { return __builtin_bit_cast(uint32_t, v); }

__device__ __forceinline__ float dot2(uint32_t a, uint32_t b, float c) {
    return __builtin_amdgcn_fdot2(as_h2(a), as_h2(b), c, false);
}

// Streaming (read-once) loads: the `nt` hint keeps weight streams from
// thrashing L2/MALL; measured 7.1 TB/s vs 6.3 TB/s for plain loads.
__device__ __forceinline__ u4v ldg_nt16(const void* p) {
    return __builtin_nontemporal_load(reinterpret_cast<const u4v*>(p));
}
__device__ __forceinline__ u2v ldg_nt8(const void* p) {
    return __builtin_nontemporal_load(reinterpret_cast<const u2v*>(p));
}
__device__ __forceinline__ u4v ldg16(const void* p) { return *reinterpret_cast<const u4v*>(p); }

// Full 64-lane wavefront sum.
__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
    for (int off = 32; off >= 1; off >>= 1) v += __shfl_xor(v, off, 64);
    return v;
}
__device__ __forceinline__ float wave_max(float v) {
#pragma unroll
    for (int off = 32; off >= 1; off >>= 1) v = fmaxf(v, __shfl_xor(v, off, 64));
    return v;
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

}  // namespace bx
