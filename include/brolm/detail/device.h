#pragma once

// resize_like (reference include/brolm/detail/device.h:21-27): pin an
// unallocated tensor to `dev` before sizing it.

#include "brotensor/tensor.h"

namespace brolm::detail {

inline void resize_like(brotensor::Tensor& t, int r, int c, brotensor::Dtype dt, brotensor::Device dev) {
    if (t.data == nullptr) t.device = dev;
    t.resize(r, c, dt);
}

}  // namespace brolm::detail
