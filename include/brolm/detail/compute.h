#pragma once

// Compute-precision policy and the dtype-dispatched linear
// (reference include/brolm/detail/compute.h:29-86).  On this build the compute
// dtype is FP16 (ROCm device); quantized weight dtypes route to the
// quant-carrier kernels of libbrolm_hip.

#include <cstdint>
#include <vector>

#include "brotensor/ops.h"
#include "brotensor/runtime.h"
#include "brotensor/tensor.h"

namespace brolm {

inline brotensor::Dtype compute_dtype() { return brotensor::compute_dtype(); }

namespace detail {

// Upload host FP32 values at the compute dtype on the default device.
inline brotensor::Tensor upload_host(const float* src, int rows, int cols) {
    if (compute_dtype() == brotensor::Dtype::FP16) {
        std::vector<std::uint16_t> bits(static_cast<std::size_t>(rows) * static_cast<std::size_t>(cols));
        for (std::size_t i = 0; i < bits.size(); ++i) bits[i] = brotensor::fp32_to_fp16_bits(src[i]);
        return brotensor::Tensor::from_host_fp16(bits.data(), rows, cols);
    }
    return brotensor::Tensor::from_host(src, rows, cols);
}

// Batched linear dispatched on the weight dtype (compute.h:54-86).
void linear_batched(const brotensor::Tensor& W, const brotensor::Tensor* bias, const brotensor::Tensor& X,
                    brotensor::Tensor& Y);

}  // namespace detail
}  // namespace brolm
