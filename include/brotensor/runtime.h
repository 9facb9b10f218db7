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

// Releases what the runtime itself holds on the device, after the queued
// work has finished: every hook registered with on_shutdown (latest first:
// the ops' scratch and RoPE tables, the sampler's buffers, the stage
// profiler's events), then the op stream.  Tensors and models the caller
// still owns stay valid to destroy afterwards.  init() may be called again.
// The Python package calls this from an atexit hook, so nothing the library
// allocated is left for the process's exit handlers to free.
void shutdown();
void on_shutdown(void (*release)());

}  // namespace brotensor
