// GgufSource (reference include/brolm/detail/weights.h:277-519).
#include "brolm/detail/weights.h"

#include <cstring>
#include <stdexcept>

#include "brolm/detail/compute.h"
#include "brotensor/ops.h"
#include "brotensor/runtime.h"

namespace brolm::detail::weights {

namespace bt = ::brotensor;

namespace detail_ {

std::vector<float> permute_rope_fp32(const std::vector<float>& src, int num_heads, int head_dim, int cols) {
    const int half = head_dim / 2;
    std::vector<float> dst(src.size());
    const std::size_t c = static_cast<std::size_t>(cols);
    for (int h = 0; h < num_heads; ++h) {
        const std::size_t base = static_cast<std::size_t>(h) * head_dim * c;
        for (int i = 0; i < half; ++i) {
            std::memcpy(&dst[base + (2 * i) * c], &src[base + i * c], c * sizeof(float));
            std::memcpy(&dst[base + (2 * i + 1) * c], &src[base + (i + half) * c], c * sizeof(float));
        }
    }
    return dst;
}

void permute_rope_bytes(const std::uint8_t* src, std::uint8_t* dst, int num_heads, int head_dim,
                        std::size_t bytes_per_row) {
    const int half = head_dim / 2;
    for (int h = 0; h < num_heads; ++h) {
        const std::size_t base = static_cast<std::size_t>(h) * head_dim * bytes_per_row;
        for (int i = 0; i < half; ++i) {
            std::memcpy(dst + base + (2 * i) * bytes_per_row, src + base + i * bytes_per_row, bytes_per_row);
            std::memcpy(dst + base + (2 * i + 1) * bytes_per_row, src + base + (i + half) * bytes_per_row,
                        bytes_per_row);
        }
    }
}

}  // namespace detail_

namespace {

std::vector<float> host_fp32(const bt::gguf::TensorInfo& info) {
    const std::size_t n = static_cast<std::size_t>(info.numel);
    std::vector<float> out(n);
    if (info.dtype == bt::Dtype::FP32) {
        std::memcpy(out.data(), info.data, n * 4);
    } else {
        const auto* s = reinterpret_cast<const std::uint16_t*>(info.data);
        for (std::size_t i = 0; i < n; ++i)
            out[i] = info.dtype == bt::Dtype::FP16 ? bt::fp16_bits_to_fp32(s[i]) : bt::bf16_bits_to_fp32(s[i]);
    }
    return out;
}

}  // namespace

GgufSource::GgufSource(std::vector<const bt::gguf::File*> shards, NameMap mapper)
    : shards_(std::move(shards)), mapper_(std::move(mapper)) {}

bool GgufSource::has(const std::string& name) const {
    const std::string g = mapper_(name);
    return !g.empty() && find_(g) != nullptr;
}

const bt::gguf::TensorInfo* GgufSource::find_(const std::string& ggml_name) const {
    for (const auto* f : shards_)
        if (const auto* v = f->find_tensor(ggml_name)) return v;
    return nullptr;
}

const bt::gguf::TensorInfo& GgufSource::need_(const std::string& hf_name, const std::string& label) const {
    const std::string g = mapper_(hf_name);
    if (g.empty()) throw std::runtime_error(label + ": no ggml mapping for HF name '" + hf_name + "'");
    if (const auto* v = find_(g)) return *v;
    throw std::runtime_error(label + ": missing tensor '" + g + "' (mapped from HF name '" + hf_name + "')");
}

void GgufSource::check_shape_(const bt::gguf::TensorInfo& info, int rows, int cols, const std::string& label) {
    const std::int64_t expected = static_cast<std::int64_t>(rows) * cols;
    if (info.numel != expected)
        throw std::runtime_error(label + " ('" + info.name + "'): shape mismatch (expected " + std::to_string(rows) +
                                 "x" + std::to_string(cols) + " = " + std::to_string(expected) + " elements, got " +
                                 std::to_string(info.numel) + ")");
}

void GgufSource::upload_dense_(const bt::gguf::TensorInfo& info, int rows, int cols, bt::Tensor& dst,
                               const std::string& label) {
    if (info.dtype != bt::Dtype::FP32 && info.dtype != bt::Dtype::FP16 && info.dtype != bt::Dtype::BF16)
        throw std::runtime_error(label + " ('" + info.name + "'): unsupported dense gguf dtype (expected FP32/FP16/BF16)");
    if (info.dtype == bt::Dtype::FP16) {
        dst = bt::Tensor::from_host_fp16(reinterpret_cast<const std::uint16_t*>(info.data), rows, cols);
        return;
    }
    const std::vector<float> f = host_fp32(info);
    dst = brolm::detail::upload_host(f.data(), rows, cols);
}

void GgufSource::upload_compute_checked(const std::string& name, int rows, int cols, bt::Tensor& dst,
                                        const std::string& label) const {
    const auto& info = need_(name, label);
    check_shape_(info, rows, cols, label);
    if (bt::dtype_is_quant(info.dtype)) {
        bt::gguf::upload_raw(info, rows, cols, dst);
        return;
    }
    upload_dense_(info, rows, cols, dst, label);
}

void GgufSource::upload_compute_dequant(const std::string& name, int rows, int cols, bt::Tensor& dst,
                                        const std::string& label) const {
    const auto& info = need_(name, label);
    check_shape_(info, rows, cols, label);
    if (!bt::dtype_is_quant(info.dtype)) {
        upload_dense_(info, rows, cols, dst, label);
        return;
    }
    if (brolm::compute_dtype() != bt::Dtype::FP16)
        throw std::runtime_error(label + " ('" + info.name + "'): quant source requires FP16 compute");
    // A quant gamma of shape (H, 1) is stored as one row of H elements.
    const bool column = cols == 1 && rows > 1;
    const int rr = column ? 1 : rows, cc = column ? rows : cols;
    bt::Tensor raw;
    bt::gguf::upload_raw(info, rr, cc, raw);
    switch (info.dtype) {
        case bt::Dtype::Q8_0: bt::dequant_q8_0_to_fp16(raw, dst); break;
        case bt::Dtype::Q4_K: bt::dequant_q4k_to_fp16(raw, dst); break;
        case bt::Dtype::Q6_K: bt::dequant_q6k_to_fp16(raw, dst); break;
        default:
            throw std::runtime_error(label + " ('" + info.name +
                                     "'): unsupported quant dtype for upload_compute_dequant");
    }
    dst.rows = rows;
    dst.cols = cols;
}

void GgufSource::upload_compute_rope_permuted(const std::string& name, int rows, int cols, int num_heads,
                                              int head_dim, bt::Tensor& dst, const std::string& label) const {
    const auto& info = need_(name, label);
    check_shape_(info, rows, cols, label);
    if (rows != num_heads * head_dim)
        throw std::runtime_error(label + " ('" + info.name + "'): rope-permuted rows (" + std::to_string(rows) +
                                 ") != num_heads*head_dim (" + std::to_string(num_heads * head_dim) + ")");
    if (bt::dtype_is_quant(info.dtype)) {
        const int bs = bt::dtype_block_size(info.dtype);
        if (cols % bs != 0)
            throw std::runtime_error(label + " ('" + info.name + "'): cols (" + std::to_string(cols) +
                                     ") not a multiple of quant block size " + std::to_string(bs));
        const std::size_t bpr = static_cast<std::size_t>(bt::dtype_storage_bytes(info.dtype, cols));
        std::vector<std::uint8_t> permuted(info.nbytes);
        detail_::permute_rope_bytes(info.data, permuted.data(), num_heads, head_dim, bpr);
        bt::gguf::upload_raw_bytes(permuted.data(), permuted.size(), info.dtype, rows, cols, dst);
        return;
    }
    const std::vector<float> host = host_fp32(info);
    const std::vector<float> perm = detail_::permute_rope_fp32(host, num_heads, head_dim, cols);
    dst = brolm::detail::upload_host(perm.data(), rows, cols);
}

void GgufSource::download_host_fp16(const std::string& name, int rows, int cols, std::vector<std::uint16_t>& out,
                                    const std::string& label) const {
    const auto& info = need_(name, label);
    check_shape_(info, rows, cols, label);
    if (info.dtype != bt::Dtype::FP16 && info.dtype != bt::Dtype::FP32 && info.dtype != bt::Dtype::BF16)
        throw std::runtime_error(label + " ('" + info.name + "'): unsupported source dtype for download_host_fp16");
    const std::size_t n = static_cast<std::size_t>(rows) * cols;
    out.resize(n);
    if (info.dtype == bt::Dtype::FP16) {
        std::memcpy(out.data(), info.data, n * 2);
        return;
    }
    const std::vector<float> f = host_fp32(info);
    for (std::size_t i = 0; i < n; ++i) out[i] = bt::fp32_to_fp16_bits(f[i]);
}

}  // namespace brolm::detail::weights
