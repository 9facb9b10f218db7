#pragma once

// brotensor::Tensor — the subset of the (absent) brotensor sibling's tensor
// type that brolm's Qwen3 path uses (reconstructed from its call sites:
// include/brolm/detail/weights.h, src/detail/dense_decoder.cpp,
// src/detail/generate.cpp, tests/test_compute.h).
//
// A Tensor is a movable value type that owns its storage (host memory for
// Device::CPU, HBM for Device::ROCm); view() wraps foreign storage without
// owning it.  Quantized dtypes keep (rows, cols) as logical element counts;
// on the ROCm device their bytes are the carrier layout of libbrolm_hip
// (a byte permutation of the GGUF blocks), on the CPU the GGUF layout.

#include <cstddef>
#include <cstdint>
#include <string>
#include <vector>

namespace brotensor {

enum class Device { CPU, ROCm };
enum class Dtype { FP32, FP16, BF16, INT32, Q8_0, Q4_K, Q6_K };

const char* dtype_name(Dtype dt);
bool dtype_is_quant(Dtype dt);
// Elements per block: 32 (Q8_0), 256 (Q4_K, Q6_K), 1 for dense types.
int dtype_block_size(Dtype dt);
// Bytes per element of a dense dtype (0 for quant dtypes).
int dtype_size_bytes(Dtype dt);
// Bytes of one row of `cols` elements (cols must be a multiple of the block size).
std::int64_t dtype_storage_bytes(Dtype dt, std::int64_t cols);
// ggml type id <-> Dtype (GGUF tensor types F32, F16, BF16, Q8_0, Q4_K, Q6_K).
int dtype_to_ggml(Dtype dt);
Dtype dtype_from_ggml(int ggml_type);  // throws std::runtime_error if unsupported

float fp16_bits_to_fp32(std::uint16_t h);
std::uint16_t fp32_to_fp16_bits(float f);  // round to nearest even, subnormals kept
float bf16_bits_to_fp32(std::uint16_t h);
std::uint16_t fp32_to_bf16_bits(float f);

class Tensor {
public:
    Device device = Device::CPU;
    void* data = nullptr;
    int rows = 0;
    int cols = 0;
    Dtype dtype = Dtype::FP32;

    Tensor() = default;
    ~Tensor();
    Tensor(Tensor&& o) noexcept;
    Tensor& operator=(Tensor&& o) noexcept;
    Tensor(const Tensor&) = delete;
    Tensor& operator=(const Tensor&) = delete;

    static Tensor empty_on(Device dev, int rows, int cols, Dtype dt);
    static Tensor zeros_on(Device dev, int rows, int cols, Dtype dt);
    // FP32 values on the default device.
    static Tensor from_host(const float* src, int rows, int cols);
    static Tensor from_host_on(Device dev, const float* src, int rows, int cols);
    // FP16 bit patterns on the default device.
    static Tensor from_host_fp16(const std::uint16_t* src, int rows, int cols);
    // Non-owning view of existing storage.
    static Tensor view(Device dev, void* data, int rows, int cols, Dtype dt);

    std::int64_t size() const { return static_cast<std::int64_t>(rows) * cols; }
    std::size_t bytes() const;
    bool owns() const { return owns_; }

    Tensor clone() const;
    Tensor to(Device dev) const;
    // Reshape storage to (rows, cols, dt); reuses the allocation when it is
    // large enough (the same-shape fast path), otherwise reallocates on
    // `device`.  Contents are unspecified after a reallocation.
    void resize(int rows, int cols, Dtype dt);

    void copy_to_host_fp16(std::uint16_t* dst) const;   // FP16 tensors
    std::vector<float> to_host_vector() const;           // FP32 / FP16 / BF16 -> FP32
    std::vector<std::uint16_t> to_host_vector_fp16() const;
    void* host_raw_mut();
    const void* host_raw() const;

private:
    std::size_t capacity_ = 0;
    bool owns_ = false;
    void release_();
};

}  // namespace brotensor
