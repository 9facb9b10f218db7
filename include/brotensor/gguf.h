#pragma once

// GGUF v3 container (the brotensor::gguf surface brolm reads:
// File::open / find_meta / find_tensor / tensors / metadata, TensorInfo
// {name, dtype, numel, nbytes, data}, upload_raw; call sites src/qwen.cpp:52-149,
// include/brolm/detail/weights.h:294-395) plus a writer used to build
// synthetic checkpoints.

#include <cstddef>
#include <cstdint>
#include <map>
#include <memory>
#include <string>
#include <utility>
#include <vector>

#include "brotensor/tensor.h"

namespace brotensor::gguf {

enum class ValueType : std::uint32_t {
    U8 = 0, I8 = 1, U16 = 2, I16 = 3, U32 = 4, I32 = 5, F32 = 6, Bool = 7,
    String = 8, Array = 9, U64 = 10, I64 = 11, F64 = 12
};

struct Value {
    ValueType type = ValueType::U8;
    union {
        std::uint8_t u8; std::int8_t i8; std::uint16_t u16; std::int16_t i16;
        std::uint32_t u32; std::int32_t i32; std::uint64_t u64; std::int64_t i64;
        float f32; double f64; bool b;
    } scalar{};
    std::string str;               // String
    ValueType array_type = ValueType::U8;
    std::vector<Value> array;      // Array
};

struct TensorInfo {
    std::string name;
    Dtype dtype = Dtype::FP32;
    std::vector<std::int64_t> dims;  // ggml order: dims[0] is the row length
    std::int64_t numel = 0;
    std::size_t nbytes = 0;
    std::uint64_t offset = 0;        // relative to the data section
    const std::uint8_t* data = nullptr;
};

class File {
public:
    File();
    ~File();
    File(File&&) noexcept;
    File& operator=(File&&) noexcept;
    File(const File&) = delete;
    File& operator=(const File&) = delete;

    static File open(const std::string& path);                // memory-maps the file
    static File from_memory(std::vector<std::uint8_t> bytes);  // takes ownership

    const Value* find_meta(const std::string& key) const;
    const TensorInfo* find_tensor(const std::string& name) const;
    const std::vector<TensorInfo>& tensors() const { return tensors_; }
    const std::vector<std::pair<std::string, Value>>& metadata() const { return meta_; }
    std::size_t tensor_count() const { return tensors_.size(); }
    std::uint32_t alignment() const { return alignment_; }

private:
    struct Storage;
    std::unique_ptr<Storage> storage_;
    std::vector<std::pair<std::string, Value>> meta_;
    std::vector<TensorInfo> tensors_;
    std::map<std::string, std::size_t> tensor_index_;
    std::uint32_t alignment_ = 32;
    void parse_();
};

// Upload a tensor's raw bytes as (rows, cols) to the default device, keeping a
// quant dtype as a device carrier.  Throws on a numel mismatch.
void upload_raw(const TensorInfo& info, int rows, int cols, Tensor& dst);
// Same from host bytes in GGUF layout (used after a host-side row permute).
void upload_raw_bytes(const std::uint8_t* bytes, std::size_t nbytes, Dtype dt, int rows, int cols, Tensor& dst);

class Writer {
public:
    void set_alignment(std::uint32_t a) { alignment_ = a; }
    void add_string(const std::string& key, const std::string& v);
    void add_u32(const std::string& key, std::uint32_t v);
    void add_i32(const std::string& key, std::int32_t v);
    void add_u64(const std::string& key, std::uint64_t v);
    void add_f32(const std::string& key, float v);
    void add_bool(const std::string& key, bool v);
    void add_string_array(const std::string& key, const std::vector<std::string>& v);
    void add_i32_array(const std::string& key, const std::vector<std::int32_t>& v);
    // dims in ggml order (dims[0] = row length); bytes must match the type.
    void add_tensor(const std::string& name, Dtype dt, const std::vector<std::int64_t>& dims,
                    std::vector<std::uint8_t> bytes);
    // Reserve a tensor whose bytes are filled in later (zeros until then).
    void add_tensor_placeholder(const std::string& name, Dtype dt, const std::vector<std::int64_t>& dims);
    // Serialized file; when data_offsets is non-null it receives each tensor's
    // absolute byte offset in the returned buffer (in add order).
    std::vector<std::uint8_t> to_bytes(std::vector<std::size_t>* data_offsets = nullptr) const;
    void write(const std::string& path) const;

private:
    struct KV { std::string key; ValueType type; std::vector<std::uint8_t> payload; };
    struct T { std::string name; Dtype dt; std::vector<std::int64_t> dims; std::size_t nbytes; std::vector<std::uint8_t> bytes; };
    std::vector<KV> kvs_;
    std::vector<T> tensors_;
    std::uint32_t alignment_ = 32;
};

}  // namespace brotensor::gguf
