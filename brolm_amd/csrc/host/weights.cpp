// GgufSource: the weight-source contract of reference
// include/brolm/detail/weights.h:50-98 (interface) and :277-519 (GGUF),
// over this build's device carriers.  Every request resolves its tensor
// once (name map, shard lookup, element count) and then lands it in one of
// three ways: as stored (quant carrier or dense at the compute dtype),
// dequantized to FP16 on the device, or row-permuted within each head.
#include "brolm/detail/weights.h"

#include <cstring>
#include <stdexcept>

#include "brolm/detail/compute.h"
#include "brotensor/ops.h"
#include "brotensor/runtime.h"

namespace brolm::detail::weights {

namespace bt = ::brotensor;

namespace detail_ {

// Rows (2i, 2i + 1) of each head take source rows (i, i + hd / 2): the
// interleaved-pair RoPE of the decoder then computes HF's rotate_half
// (reference weights.h:106-148 states the same permutation).
std::vector<float> permute_rope_fp32(const std::vector<float>& src, int num_heads, int head_dim, int cols) {
    std::vector<float> dst(src.size());
    permute_rope_bytes(reinterpret_cast<const std::uint8_t*>(src.data()), reinterpret_cast<std::uint8_t*>(dst.data()),
                       num_heads, head_dim, static_cast<std::size_t>(cols) * sizeof(float));
    return dst;
}

void permute_rope_bytes(const std::uint8_t* src, std::uint8_t* dst, int num_heads, int head_dim,
                        std::size_t bytes_per_row) {
    const std::size_t half = static_cast<std::size_t>(head_dim / 2);
    const std::size_t head_bytes = static_cast<std::size_t>(head_dim) * bytes_per_row;
    for (int h = 0; h < num_heads; ++h) {
        const std::uint8_t* s = src + static_cast<std::size_t>(h) * head_bytes;
        std::uint8_t* d = dst + static_cast<std::size_t>(h) * head_bytes;
        for (std::size_t r = 0; r < static_cast<std::size_t>(head_dim); ++r) {
            // destination row r: pair r / 2, first or second half by parity
            const std::size_t from = (r & 1) ? r / 2 + half : r / 2;
            std::memcpy(d + r * bytes_per_row, s + from * bytes_per_row, bytes_per_row);
        }
    }
}

}  // namespace detail_

namespace {

bool is_dense(bt::Dtype t) { return t == bt::Dtype::FP32 || t == bt::Dtype::FP16 || t == bt::Dtype::BF16; }

// A dense GGUF tensor as FP32 on the host.
std::vector<float> dense_as_fp32(const bt::gguf::TensorInfo& info) {
    const std::size_t n = static_cast<std::size_t>(info.numel);
    std::vector<float> out(n);
    if (info.dtype == bt::Dtype::FP32) {
        std::memcpy(out.data(), info.data, n * sizeof(float));
        return out;
    }
    const auto* h = reinterpret_cast<const std::uint16_t*>(info.data);
    const bool fp16 = info.dtype == bt::Dtype::FP16;
    for (std::size_t i = 0; i < n; ++i) out[i] = fp16 ? bt::fp16_bits_to_fp32(h[i]) : bt::bf16_bits_to_fp32(h[i]);
    return out;
}

// A dense tensor on the device at the compute dtype (FP16 sources verbatim).
bt::Tensor dense_to_device(const bt::gguf::TensorInfo& info, int rows, int cols, const std::string& where) {
    if (!is_dense(info.dtype))
        throw std::runtime_error(where + ": unsupported dense gguf dtype (expected FP32/FP16/BF16)");
    if (info.dtype == bt::Dtype::FP16)
        return bt::Tensor::from_host_fp16(reinterpret_cast<const std::uint16_t*>(info.data), rows, cols);
    const std::vector<float> f = dense_as_fp32(info);
    return brolm::detail::upload_host(f.data(), rows, cols);
}

}  // namespace

GgufSource::GgufSource(std::vector<const bt::gguf::File*> shards, NameMap mapper)
    : shards_(std::move(shards)), mapper_(std::move(mapper)) {}

const bt::gguf::TensorInfo* GgufSource::lookup_ggml_(const std::string& ggml_name) const {
    for (const bt::gguf::File* shard : shards_)
        if (const bt::gguf::TensorInfo* t = shard->find_tensor(ggml_name)) return t;
    return nullptr;
}

GgufSource::Resolved GgufSource::resolve_(const std::string& hf_name, int rows, int cols,
                                          const std::string& label) const {
    const std::string ggml = mapper_(hf_name);
    if (ggml.empty()) throw std::runtime_error(label + ": no ggml mapping for HF name '" + hf_name + "'");
    const bt::gguf::TensorInfo* t = lookup_ggml_(ggml);
    if (!t) throw std::runtime_error(label + ": missing tensor '" + ggml + "' (mapped from HF name '" + hf_name + "')");
    Resolved r{t, label + " ('" + t->name + "')"};
    const std::int64_t want = static_cast<std::int64_t>(rows) * cols;
    if (t->numel != want)
        throw std::runtime_error(r.where + ": shape mismatch (expected " + std::to_string(rows) + "x" +
                                 std::to_string(cols) + " = " + std::to_string(want) + " elements, got " +
                                 std::to_string(t->numel) + ")");
    return r;
}

bool GgufSource::has(const std::string& name) const {
    const std::string ggml = mapper_(name);
    return !ggml.empty() && lookup_ggml_(ggml) != nullptr;
}

void GgufSource::upload_compute_checked(const std::string& name, int rows, int cols, bt::Tensor& dst,
                                        const std::string& label) const {
    const Resolved r = resolve_(name, rows, cols, label);
    if (bt::dtype_is_quant(r.info->dtype)) bt::gguf::upload_raw(*r.info, rows, cols, dst);   // device carrier
    else dst = dense_to_device(*r.info, rows, cols, r.where);
}

void GgufSource::upload_compute_dequant(const std::string& name, int rows, int cols, bt::Tensor& dst,
                                        const std::string& label) const {
    const Resolved r = resolve_(name, rows, cols, label);
    const bt::Dtype t = r.info->dtype;
    if (!bt::dtype_is_quant(t)) {
        dst = dense_to_device(*r.info, rows, cols, r.where);
        return;
    }
    if (brolm::compute_dtype() != bt::Dtype::FP16)
        throw std::runtime_error(r.where + ": quant source requires FP16 compute");
    // quant blocks run along a row: an (H, 1) gamma is one row of H values
    const bool column = cols == 1 && rows > 1;
    bt::Tensor carrier;
    bt::gguf::upload_raw(*r.info, column ? 1 : rows, column ? rows : cols, carrier);
    if (t == bt::Dtype::Q8_0) bt::dequant_q8_0_to_fp16(carrier, dst);
    else if (t == bt::Dtype::Q4_K) bt::dequant_q4k_to_fp16(carrier, dst);
    else if (t == bt::Dtype::Q6_K) bt::dequant_q6k_to_fp16(carrier, dst);
    else throw std::runtime_error(r.where + ": unsupported quant dtype for upload_compute_dequant");
    dst.rows = rows;
    dst.cols = cols;
}

void GgufSource::upload_compute_rope_permuted(const std::string& name, int rows, int cols, int num_heads,
                                              int head_dim, bt::Tensor& dst, const std::string& label) const {
    const Resolved r = resolve_(name, rows, cols, label);
    const bt::gguf::TensorInfo& t = *r.info;
    if (rows != num_heads * head_dim)
        throw std::runtime_error(r.where + ": rope-permuted rows (" + std::to_string(rows) +
                                 ") != num_heads*head_dim (" + std::to_string(num_heads * head_dim) + ")");
    if (!bt::dtype_is_quant(t.dtype)) {
        const std::vector<float> perm = detail_::permute_rope_fp32(dense_as_fp32(t), num_heads, head_dim, cols);
        dst = brolm::detail::upload_host(perm.data(), rows, cols);
        return;
    }
    // quant rows move whole: a row's blocks stay together, so the permuted
    // bytes are again a valid GGUF tensor of the same type
    const int block = bt::dtype_block_size(t.dtype);
    if (cols % block != 0)
        throw std::runtime_error(r.where + ": cols (" + std::to_string(cols) + ") not a multiple of quant block size " +
                                 std::to_string(block));
    std::vector<std::uint8_t> bytes(t.nbytes);
    detail_::permute_rope_bytes(t.data, bytes.data(), num_heads, head_dim,
                                static_cast<std::size_t>(bt::dtype_storage_bytes(t.dtype, cols)));
    bt::gguf::upload_raw_bytes(bytes.data(), bytes.size(), t.dtype, rows, cols, dst);
}

void GgufSource::download_host_fp16(const std::string& name, int rows, int cols, std::vector<std::uint16_t>& out,
                                    const std::string& label) const {
    const Resolved r = resolve_(name, rows, cols, label);
    if (!is_dense(r.info->dtype))
        throw std::runtime_error(r.where + ": unsupported source dtype for download_host_fp16");
    const std::size_t n = static_cast<std::size_t>(rows) * cols;
    out.resize(n);
    if (r.info->dtype == bt::Dtype::FP16) {
        std::memcpy(out.data(), r.info->data, n * sizeof(std::uint16_t));
        return;
    }
    const std::vector<float> f = dense_as_fp32(*r.info);
    for (std::size_t i = 0; i < n; ++i) out[i] = bt::fp32_to_fp16_bits(f[i]);
}

}  // namespace brolm::detail::weights
