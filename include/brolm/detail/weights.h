#pragma once

// Weight-source adapter over GGUF checkpoints (reference
// include/brolm/detail/weights.h:50-98 interface, :277-519 GgufSource).
//
//   upload_compute_checked  quant tensors keep their dtype (device carrier);
//                           dense F16/F32/BF16 land at the compute dtype.
//   upload_compute_dequant  for ops without a quant path (embedding, norm
//                           gammas): quant sources are dequantized to FP16 on
//                           the device, bit-exact to the GGUF formula.
//   upload_compute_rope_permuted  row permute within each head so the
//                           interleaved-pair RoPE reproduces HF rotate_half:
//                           dst rows (2i, 2i+1) <- src rows (i, i + hd/2);
//                           byte-level for quant rows, FP32 for dense.

#include <cstddef>
#include <cstdint>
#include <functional>
#include <string>
#include <string_view>
#include <vector>

#include "brotensor/gguf.h"
#include "brotensor/tensor.h"

namespace brolm::detail::weights {

class Source {
public:
    virtual ~Source() = default;
    virtual bool has(const std::string& name) const = 0;
    virtual void upload_compute_checked(const std::string& name, int rows, int cols, brotensor::Tensor& dst,
                                        const std::string& label) const = 0;
    virtual void upload_compute_dequant(const std::string& name, int rows, int cols, brotensor::Tensor& dst,
                                        const std::string& label) const = 0;
    virtual void upload_compute_rope_permuted(const std::string& name, int rows, int cols, int num_heads,
                                              int head_dim, brotensor::Tensor& dst,
                                              const std::string& label) const = 0;
    virtual void download_host_fp16(const std::string& name, int rows, int cols, std::vector<std::uint16_t>& out,
                                    const std::string& label) const = 0;
};

namespace detail_ {
// FP32 host row permute, interleaved <- HF (weights.h:106-127).
std::vector<float> permute_rope_fp32(const std::vector<float>& src, int num_heads, int head_dim, int cols);
// Byte-level row permute for any row-contiguous layout (weights.h:132-148).
void permute_rope_bytes(const std::uint8_t* src, std::uint8_t* dst, int num_heads, int head_dim,
                        std::size_t bytes_per_row);
}  // namespace detail_

class GgufSource final : public Source {
public:
    using NameMap = std::function<std::string(std::string_view)>;
    GgufSource(std::vector<const brotensor::gguf::File*> shards, NameMap mapper);

    bool has(const std::string& name) const override;
    void upload_compute_checked(const std::string& name, int rows, int cols, brotensor::Tensor& dst,
                                const std::string& label) const override;
    void upload_compute_dequant(const std::string& name, int rows, int cols, brotensor::Tensor& dst,
                                const std::string& label) const override;
    void upload_compute_rope_permuted(const std::string& name, int rows, int cols, int num_heads, int head_dim,
                                      brotensor::Tensor& dst, const std::string& label) const override;
    void download_host_fp16(const std::string& name, int rows, int cols, std::vector<std::uint16_t>& out,
                            const std::string& label) const override;

private:
    // A tensor resolved for one request: its GGUF record and the text that
    // names it in errors ("label ('ggml name')").
    struct Resolved {
        const brotensor::gguf::TensorInfo* info;
        std::string where;
    };
    // The record of a ggml name in the first shard that holds it, or null.
    const brotensor::gguf::TensorInfo* lookup_ggml_(const std::string& ggml_name) const;
    // Maps an HF name, finds it and checks that it holds rows x cols elements;
    // throws std::runtime_error otherwise.
    Resolved resolve_(const std::string& hf_name, int rows, int cols, const std::string& label) const;

    std::vector<const brotensor::gguf::File*> shards_;
    NameMap mapper_;
};

}  // namespace brolm::detail::weights
