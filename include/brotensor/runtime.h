#pragma once

// brotensor runtime registration, ROCm edition (brolm calls init(),
// default_device(), compute_dtype(), sync_all(): tools/bench_decode.cpp:187,
// include/brolm/detail/compute.h:29-31, include/brolm/detail/profile.h:12-13).
//
// init() registers the first gfx950 device and creates the one stream every
// op is ordered on.  This build has no CPU compute backend: init() throws when
// no ROCm device is present, and ops refuse CPU tensors, so nothing silently
// falls back to host math.

#include "brotensor/tensor.h"

namespace brotensor {

void init();
bool initialized();
Device default_device();        // Device::ROCm after init()
Dtype compute_dtype();          // FP16 (the GPU compute dtype)
void sync_all();                // waits for every op issued so far
void* stream();                 // the hipStream_t every op is issued on
int device_ordinal();

}  // namespace brotensor
