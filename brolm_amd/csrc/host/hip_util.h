// Host helpers around the HIP runtime and the bx_* status codes.
#pragma once

#include <hip/hip_runtime_api.h>

#include <cstddef>
#include <stdexcept>
#include <string>

#include "brolm_hip.h"

namespace hipx {

inline void check(hipError_t e, const char* what) {
    if (e != hipSuccess) throw std::runtime_error(std::string("HIP ") + what + ": " + hipGetErrorString(e));
}

// Turn a bx_* status into a std::runtime_error carrying the library message.
inline void bx(int rc, const char* what) {
    if (rc != BX_OK) throw std::runtime_error(std::string(what) + ": " + bx_last_error());
}

hipStream_t stream();
void sync();
// The linear entry points' workspace for the op stream (bx_linear_workspace_bytes).
void* linear_ws();
std::size_t linear_ws_bytes();
// Stream-ordered copies; the host side waits (synchronous semantics).
void h2d(void* dst, const void* src, std::size_t n);
void d2h(void* dst, const void* src, std::size_t n);

}  // namespace hipx
