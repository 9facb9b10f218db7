// brotensor::Tensor on HBM (hipMalloc) or host memory.
#include "brotensor/tensor.h"

#include <hip/hip_runtime_api.h>

#include <cstdlib>
#include <cstring>
#include <stdexcept>
#include <string>

#include "brolm_hip.h"
#include "brotensor/runtime.h"
#include "hip_util.h"

namespace brotensor {

const char* dtype_name(Dtype dt) {
    switch (dt) {
        case Dtype::FP32: return "FP32";
        case Dtype::FP16: return "FP16";
        case Dtype::BF16: return "BF16";
        case Dtype::INT32: return "INT32";
        case Dtype::Q8_0: return "Q8_0";
        case Dtype::Q4_K: return "Q4_K";
        case Dtype::Q6_K: return "Q6_K";
    }
    return "?";
}

bool dtype_is_quant(Dtype dt) { return dt == Dtype::Q8_0 || dt == Dtype::Q4_K || dt == Dtype::Q6_K; }

int dtype_block_size(Dtype dt) {
    switch (dt) {
        case Dtype::Q8_0: return 32;
        case Dtype::Q4_K:
        case Dtype::Q6_K: return 256;
        default: return 1;
    }
}

int dtype_size_bytes(Dtype dt) {
    switch (dt) {
        case Dtype::FP32:
        case Dtype::INT32: return 4;
        case Dtype::FP16:
        case Dtype::BF16: return 2;
        default: return 0;
    }
}

std::int64_t dtype_storage_bytes(Dtype dt, std::int64_t cols) {
    switch (dt) {
        case Dtype::Q8_0: return cols / 32 * 34;
        case Dtype::Q4_K: return cols / 256 * 144;
        case Dtype::Q6_K: return cols / 256 * 210;
        default: return cols * dtype_size_bytes(dt);
    }
}

int dtype_to_ggml(Dtype dt) {
    switch (dt) {
        case Dtype::FP32: return 0;
        case Dtype::FP16: return 1;
        case Dtype::Q8_0: return 8;
        case Dtype::Q4_K: return 12;
        case Dtype::Q6_K: return 14;
        case Dtype::BF16: return 30;
        default: throw std::runtime_error(std::string("dtype_to_ggml: no ggml type for ") + dtype_name(dt));
    }
}

Dtype dtype_from_ggml(int t) {
    switch (t) {
        case 0: return Dtype::FP32;
        case 1: return Dtype::FP16;
        case 8: return Dtype::Q8_0;
        case 12: return Dtype::Q4_K;
        case 14: return Dtype::Q6_K;
        case 30: return Dtype::BF16;
        default: throw std::runtime_error("gguf: unsupported ggml tensor type " + std::to_string(t));
    }
}

float fp16_bits_to_fp32(std::uint16_t h) {
    const std::uint32_t sign = static_cast<std::uint32_t>(h & 0x8000u) << 16;
    const std::uint32_t e = (h >> 10) & 0x1fu, m = h & 0x3ffu;
    std::uint32_t bits;
    if (e == 0) {
        if (m == 0) {
            bits = sign;
        } else {
            const float v = static_cast<float>(m) * 0x1p-24f;
            std::memcpy(&bits, &v, 4);
            bits |= sign;
        }
    } else if (e == 31) {
        bits = sign | 0x7f800000u | (m << 13);
    } else {
        bits = sign | ((e + 112u) << 23) | (m << 13);
    }
    float f;
    std::memcpy(&f, &bits, 4);
    return f;
}

std::uint16_t fp32_to_fp16_bits(float f) {
    std::uint32_t x;
    std::memcpy(&x, &f, 4);
    const std::uint32_t sign = (x >> 16) & 0x8000u;
    const std::uint32_t a = x & 0x7fffffffu;
    if (a >= 0x7f800000u) return static_cast<std::uint16_t>(sign | 0x7c00u | (a > 0x7f800000u ? 0x200u : 0u));
    if (a >= 0x477ff000u) return static_cast<std::uint16_t>(sign | 0x7c00u);
    const std::uint32_t e = a >> 23;
    if (e < 113) {
        // result is a multiple of 2^-24: round a's value / 2^-24 to an integer
        if (e < 102) return static_cast<std::uint16_t>(sign);
        const std::uint32_t mant = (a & 0x7fffffu) | 0x800000u;
        const int sh = 126 - static_cast<int>(e);
        std::uint32_t q = mant >> sh;
        const std::uint32_t rest = mant & ((1u << sh) - 1u), half = 1u << (sh - 1);
        if (rest > half || (rest == half && (q & 1u))) ++q;
        return static_cast<std::uint16_t>(sign | q);
    }
    std::uint32_t h = ((e - 112u) << 10) | ((a & 0x7fffffu) >> 13);
    const std::uint32_t rest = a & 0x1fffu;
    if (rest > 0x1000u || (rest == 0x1000u && (h & 1u))) ++h;
    return static_cast<std::uint16_t>(sign | h);
}

float bf16_bits_to_fp32(std::uint16_t h) {
    const std::uint32_t bits = static_cast<std::uint32_t>(h) << 16;
    float f;
    std::memcpy(&f, &bits, 4);
    return f;
}

std::uint16_t fp32_to_bf16_bits(float f) {
    std::uint32_t x;
    std::memcpy(&x, &f, 4);
    if ((x & 0x7fffffffu) > 0x7f800000u) return static_cast<std::uint16_t>((x >> 16) | 0x40u);
    x += 0x7fffu + ((x >> 16) & 1u);
    return static_cast<std::uint16_t>(x >> 16);
}

// ---------------------------------------------------------------- Tensor

static std::size_t bytes_for(int rows, int cols, Dtype dt) {
    if (rows < 0 || cols < 0) throw std::runtime_error("Tensor: negative shape");
    if (dtype_is_quant(dt) && cols % dtype_block_size(dt) != 0)
        throw std::runtime_error(std::string("Tensor: ") + dtype_name(dt) + " cols " + std::to_string(cols) +
                                 " not a multiple of the block size");
    return static_cast<std::size_t>(rows) * static_cast<std::size_t>(dtype_storage_bytes(dt, cols));
}

static void* alloc_on(Device dev, std::size_t n) {
    if (n == 0) return nullptr;
    if (dev == Device::CPU) {
        void* p = std::aligned_alloc(64, (n + 63) / 64 * 64);
        if (!p) throw std::runtime_error("Tensor: host allocation failed");
        return p;
    }
    if (!initialized()) throw std::runtime_error("Tensor: ROCm allocation before brotensor::init()");
    void* p = nullptr;
    hipx::check(hipMalloc(&p, n), "hipMalloc");
    return p;
}

static void free_on(Device dev, void* p) {
    if (!p) return;
    if (dev == Device::CPU) std::free(p);
    else (void)hipFree(p);
}

Tensor::~Tensor() { release_(); }

void Tensor::release_() {
    if (owns_ && data) free_on(device, data);
    data = nullptr;
    owns_ = false;
    capacity_ = 0;
}

Tensor::Tensor(Tensor&& o) noexcept
    : device(o.device), data(o.data), rows(o.rows), cols(o.cols), dtype(o.dtype), capacity_(o.capacity_),
      owns_(o.owns_) {
    o.data = nullptr;
    o.owns_ = false;
    o.capacity_ = 0;
    o.rows = o.cols = 0;
}

Tensor& Tensor::operator=(Tensor&& o) noexcept {
    if (this != &o) {
        release_();
        device = o.device;
        data = o.data;
        rows = o.rows;
        cols = o.cols;
        dtype = o.dtype;
        capacity_ = o.capacity_;
        owns_ = o.owns_;
        o.data = nullptr;
        o.owns_ = false;
        o.capacity_ = 0;
        o.rows = o.cols = 0;
    }
    return *this;
}

std::size_t Tensor::bytes() const { return bytes_for(rows, cols, dtype); }

Tensor Tensor::empty_on(Device dev, int r, int c, Dtype dt) {
    Tensor t;
    t.device = dev;
    t.rows = r;
    t.cols = c;
    t.dtype = dt;
    t.capacity_ = bytes_for(r, c, dt);
    t.data = alloc_on(dev, t.capacity_);
    t.owns_ = true;
    return t;
}

Tensor Tensor::zeros_on(Device dev, int r, int c, Dtype dt) {
    Tensor t = empty_on(dev, r, c, dt);
    if (t.capacity_ == 0) return t;
    if (dev == Device::CPU) std::memset(t.data, 0, t.capacity_);
    else hipx::check(hipMemsetAsync(t.data, 0, t.capacity_, hipx::stream()), "hipMemsetAsync");
    return t;
}

Tensor Tensor::from_host_on(Device dev, const float* src, int r, int c) {
    Tensor t = empty_on(dev, r, c, Dtype::FP32);
    if (t.capacity_ == 0) return t;
    if (dev == Device::CPU) std::memcpy(t.data, src, t.capacity_);
    else hipx::h2d(t.data, src, t.capacity_);
    return t;
}

Tensor Tensor::from_host(const float* src, int r, int c) { return from_host_on(default_device(), src, r, c); }

Tensor Tensor::from_host_fp16(const std::uint16_t* src, int r, int c) {
    Tensor t = empty_on(default_device(), r, c, Dtype::FP16);
    if (t.capacity_ == 0) return t;
    if (t.device == Device::CPU) std::memcpy(t.data, src, t.capacity_);
    else hipx::h2d(t.data, src, t.capacity_);
    return t;
}

Tensor Tensor::view(Device dev, void* p, int r, int c, Dtype dt) {
    Tensor t;
    t.device = dev;
    t.data = p;
    t.rows = r;
    t.cols = c;
    t.dtype = dt;
    t.owns_ = false;
    t.capacity_ = bytes_for(r, c, dt);
    return t;
}

Tensor Tensor::clone() const {
    Tensor t = empty_on(device, rows, cols, dtype);
    const std::size_t n = bytes();
    if (n == 0) return t;
    if (device == Device::CPU) std::memcpy(t.data, data, n);
    else hipx::check(hipMemcpyAsync(t.data, data, n, hipMemcpyDeviceToDevice, hipx::stream()), "clone");
    return t;
}

Tensor Tensor::to(Device dev) const {
    if (dev == device) return clone();
    const std::size_t n = bytes();
    Tensor t = empty_on(dev, rows, cols, dtype);
    if (n == 0) return t;
    if (dev == Device::ROCm) {
        if (dtype_is_quant(dtype)) {
            // host GGUF blocks -> staging -> carrier layout
            void* stage = nullptr;
            hipx::check(hipMalloc(&stage, n), "hipMalloc staging");
            hipx::h2d(stage, data, n);
            const int rc = bx_repack_gguf_rows(dtype_to_ggml(dtype), stage, t.data, rows, cols, hipx::stream());
            hipx::sync();
            (void)hipFree(stage);
            hipx::bx(rc, "repack");
        } else {
            hipx::h2d(t.data, data, n);
        }
    } else {
        if (dtype_is_quant(dtype)) {
            void* stage = nullptr;
            hipx::check(hipMalloc(&stage, n), "hipMalloc staging");
            hipx::bx(bx_unpack_carrier_rows(dtype_to_ggml(dtype), data, stage, rows, cols, hipx::stream()),
                     "unpack");
            hipx::d2h(t.data, stage, n);
            (void)hipFree(stage);
        } else {
            hipx::d2h(t.data, data, n);
        }
    }
    return t;
}

void Tensor::resize(int r, int c, Dtype dt) {
    const std::size_t need = bytes_for(r, c, dt);
    if (data && need <= capacity_) {
        rows = r;
        cols = c;
        dtype = dt;
        return;
    }
    if (data && !owns_) throw std::runtime_error("Tensor::resize: cannot grow a view");
    release_();
    rows = r;
    cols = c;
    dtype = dt;
    capacity_ = need;
    data = alloc_on(device, need);
    owns_ = true;
}

void Tensor::copy_to_host_fp16(std::uint16_t* dst) const {
    if (dtype != Dtype::FP16) throw std::runtime_error("copy_to_host_fp16: tensor is not FP16");
    const std::size_t n = bytes();
    if (device == Device::CPU) std::memcpy(dst, data, n);
    else hipx::d2h(dst, data, n);
}

std::vector<std::uint16_t> Tensor::to_host_vector_fp16() const {
    std::vector<std::uint16_t> out(static_cast<std::size_t>(size()));
    copy_to_host_fp16(out.data());
    return out;
}

std::vector<float> Tensor::to_host_vector() const {
    const std::size_t n = static_cast<std::size_t>(size());
    std::vector<float> out(n);
    if (dtype == Dtype::FP32) {
        if (device == Device::CPU) std::memcpy(out.data(), data, n * 4);
        else hipx::d2h(out.data(), data, n * 4);
        return out;
    }
    if (dtype == Dtype::FP16 || dtype == Dtype::BF16) {
        std::vector<std::uint16_t> bits(n);
        if (device == Device::CPU) std::memcpy(bits.data(), data, n * 2);
        else hipx::d2h(bits.data(), data, n * 2);
        for (std::size_t i = 0; i < n; ++i)
            out[i] = dtype == Dtype::FP16 ? fp16_bits_to_fp32(bits[i]) : bf16_bits_to_fp32(bits[i]);
        return out;
    }
    throw std::runtime_error(std::string("to_host_vector: unsupported dtype ") + dtype_name(dtype));
}

void* Tensor::host_raw_mut() {
    if (device != Device::CPU) throw std::runtime_error("host_raw_mut: tensor is not on the CPU");
    return data;
}

const void* Tensor::host_raw() const {
    if (device != Device::CPU) throw std::runtime_error("host_raw: tensor is not on the CPU");
    return data;
}

}  // namespace brotensor
