// linear_batched dtype dispatch (reference include/brolm/detail/compute.h:54-86).
#include "brolm/detail/compute.h"

#include <stdexcept>
#include <string>

namespace brolm::detail {

void linear_batched(const brotensor::Tensor& W, const brotensor::Tensor* bias, const brotensor::Tensor& X,
                    brotensor::Tensor& Y) {
    switch (W.dtype) {
        case brotensor::Dtype::FP16: brotensor::linear_forward_batched_fp16(W, bias, X, Y); return;
        case brotensor::Dtype::Q4_K: brotensor::linear_forward_batched_q4k_fp16(W, bias, X, Y); return;
        case brotensor::Dtype::Q6_K: brotensor::linear_forward_batched_q6k_fp16(W, bias, X, Y); return;
        case brotensor::Dtype::Q8_0: brotensor::linear_forward_batched_q8_0_fp16(W, bias, X, Y); return;
        default: break;
    }
    throw std::runtime_error(std::string("linear_batched: no ROCm kernel for weight dtype ") +
                             brotensor::dtype_name(W.dtype));
}

}  // namespace brolm::detail
