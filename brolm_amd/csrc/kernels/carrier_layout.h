// Device carrier layouts for GGUF quant blocks (host + device).
//
// A carrier is a byte permutation of a tensor's GGUF blocks: same byte count,
// regrouped into separate aligned streams so a wavefront reads each stream
// with coalesced 16-byte loads.  For a (N, K) weight with nb = K/256
// super-blocks (Q4_K, Q6_K) or nb32 = K/32 blocks (Q8_0), super-block s = n*nb+b:
//
//   Q8_0 : QS[N*K]            int8 values, row-major (32 per block)
//          D [N*nb32]         fp16 block scale
//   Q4_K : QS[N*nb*128]       the block's qs[128] verbatim
//          HDR[N*nb*16]       d, dmin, scales[12] verbatim
//   Q6_K : QL[N*nb*128]       unit t=0..7 (h=t/4, l0=8*(t%4)) holds
//                             ql[64h+l0 .. +8] ++ ql[64h+32+l0 .. +8]
//          QH[N*nb*64]        unit t holds qh[32h+l0 .. +8]
//          SC[N*nb*16]        scales[16] verbatim
//          D [N*nb]           fp16 d
//
// Every stream offset is a multiple of 16 bytes (128, 144, 192, 208 and 34*32
// are), so 16-byte loads are aligned whenever the base is.
#pragma once

#include <cstdint>

#include "../../../include/brolm_hip.h"

namespace bx {

struct CarrierQ8 {
    const uint8_t* qs;
    const uint8_t* d;
};
struct CarrierQ4K {
    const uint8_t* qs;
    const uint8_t* hdr;
};
struct CarrierQ6K {
    const uint8_t* ql;
    const uint8_t* qh;
    const uint8_t* sc;
    const uint8_t* d;
};

__host__ __device__ inline CarrierQ8 carrier_q8(const void* base, int64_t N, int64_t K) {
    const uint8_t* p = static_cast<const uint8_t*>(base);
    return CarrierQ8{p, p + N * K};
}
__host__ __device__ inline CarrierQ4K carrier_q4k(const void* base, int64_t N, int64_t K) {
    const uint8_t* p = static_cast<const uint8_t*>(base);
    const int64_t nb = K / 256;
    return CarrierQ4K{p, p + N * nb * 128};
}
__host__ __device__ inline CarrierQ6K carrier_q6k(const void* base, int64_t N, int64_t K) {
    const uint8_t* p = static_cast<const uint8_t*>(base);
    const int64_t nb = K / 256;
    return CarrierQ6K{p, p + N * nb * 128, p + N * nb * 192, p + N * nb * 208};
}

inline int64_t type_block_elems(int type) {
    switch (type) {
        case BX_TYPE_Q8_0: return 32;
        case BX_TYPE_Q4_K:
        case BX_TYPE_Q6_K: return 256;
        case BX_TYPE_F16: return 1;
        case BX_TYPE_F32: return 1;
        default: return 0;
    }
}
inline int64_t type_block_bytes(int type) {
    switch (type) {
        case BX_TYPE_Q8_0: return 34;
        case BX_TYPE_Q4_K: return 144;
        case BX_TYPE_Q6_K: return 210;
        case BX_TYPE_F16: return 2;
        case BX_TYPE_F32: return 4;
        default: return 0;
    }
}

}  // namespace bx
