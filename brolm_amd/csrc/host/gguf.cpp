// GGUF v3 reader (mmap) and writer.
//
// Layout: "GGUF", u32 version, u64 tensor_count, u64 kv_count, kv pairs
// (string key, u32 type, value), tensor infos (string name, u32 n_dims,
// u64 dims[n_dims], u32 ggml type, u64 offset), padding to `alignment`
// (general.alignment, default 32), tensor data.  Strings are u64 length +
// bytes; arrays are u32 element type + u64 count + elements.
#include "brotensor/gguf.h"

#include <fcntl.h>
#include <sys/mman.h>
#include <sys/stat.h>
#include <unistd.h>

#include <cstring>
#include <fstream>
#include <stdexcept>

#include "brolm_hip.h"
#include "brotensor/runtime.h"
#include "hip_util.h"

namespace brotensor::gguf {

struct File::Storage {
    std::vector<std::uint8_t> owned;
    void* map = nullptr;
    std::size_t map_len = 0;
    const std::uint8_t* base = nullptr;
    std::size_t size = 0;
    ~Storage() {
        if (map) munmap(map, map_len);
    }
};

File::File() = default;
File::~File() = default;
File::File(File&&) noexcept = default;
File& File::operator=(File&&) noexcept = default;

namespace {

[[noreturn]] void bad(const std::string& m) { throw std::runtime_error("gguf: " + m); }

struct Reader {
    const std::uint8_t* p;
    const std::uint8_t* end;
    void need(std::size_t n) const {
        if (static_cast<std::size_t>(end - p) < n) bad("truncated file");
    }
    template <typename T>
    T get() {
        need(sizeof(T));
        T v;
        std::memcpy(&v, p, sizeof(T));
        p += sizeof(T);
        return v;
    }
    std::string str() {
        const std::uint64_t n = get<std::uint64_t>();
        need(n);
        std::string s(reinterpret_cast<const char*>(p), n);
        p += n;
        return s;
    }
};

// Smallest encoding of one value of type t (strings: the u64 length; arrays:
// element type + count).
std::uint64_t min_encoded_bytes(ValueType t) {
    switch (t) {
        case ValueType::U8: case ValueType::I8: case ValueType::Bool: return 1;
        case ValueType::U16: case ValueType::I16: return 2;
        case ValueType::U32: case ValueType::I32: case ValueType::F32: return 4;
        case ValueType::U64: case ValueType::I64: case ValueType::F64: case ValueType::String: return 8;
        case ValueType::Array: return 12;
        default: bad("unknown metadata value type " + std::to_string(static_cast<unsigned>(t)));
    }
}

Value read_value(Reader& r, ValueType t, int depth) {
    Value v;
    v.type = t;
    switch (t) {
        case ValueType::U8: v.scalar.u8 = r.get<std::uint8_t>(); break;
        case ValueType::I8: v.scalar.i8 = r.get<std::int8_t>(); break;
        case ValueType::U16: v.scalar.u16 = r.get<std::uint16_t>(); break;
        case ValueType::I16: v.scalar.i16 = r.get<std::int16_t>(); break;
        case ValueType::U32: v.scalar.u32 = r.get<std::uint32_t>(); break;
        case ValueType::I32: v.scalar.i32 = r.get<std::int32_t>(); break;
        case ValueType::F32: v.scalar.f32 = r.get<float>(); break;
        case ValueType::Bool: v.scalar.b = r.get<std::uint8_t>() != 0; break;
        case ValueType::U64: v.scalar.u64 = r.get<std::uint64_t>(); break;
        case ValueType::I64: v.scalar.i64 = r.get<std::int64_t>(); break;
        case ValueType::F64: v.scalar.f64 = r.get<double>(); break;
        case ValueType::String: v.str = r.str(); break;
        case ValueType::Array: {
            if (depth > 4) bad("nested arrays too deep");
            v.array_type = static_cast<ValueType>(r.get<std::uint32_t>());
            const std::uint64_t n = r.get<std::uint64_t>();
            // every element takes at least min_encoded_bytes of the file: a
            // count the remaining bytes cannot hold is malformed (and is
            // refused before anything is reserved for it)
            const std::uint64_t room = static_cast<std::uint64_t>(r.end - r.p);
            if (n > room / min_encoded_bytes(v.array_type)) bad("array count exceeds the file");
            v.array.reserve(static_cast<std::size_t>(n));
            for (std::uint64_t i = 0; i < n; ++i) v.array.push_back(read_value(r, v.array_type, depth + 1));
            break;
        }
        default: bad("unknown metadata value type " + std::to_string(static_cast<unsigned>(t)));
    }
    return v;
}

}  // namespace

void File::parse_() {
    Reader r{storage_->base, storage_->base + storage_->size};
    r.need(4);
    if (std::memcmp(r.p, "GGUF", 4) != 0) bad("bad magic (not a GGUF file)");
    r.p += 4;
    const std::uint32_t version = r.get<std::uint32_t>();
    if (version != 3) bad("unsupported version " + std::to_string(version));
    const std::uint64_t n_t = r.get<std::uint64_t>();
    const std::uint64_t n_kv = r.get<std::uint64_t>();
    if (n_t > (1u << 24) || n_kv > (1u << 24)) bad("implausible header counts");
    for (std::uint64_t i = 0; i < n_kv; ++i) {
        std::string key = r.str();
        const auto t = static_cast<ValueType>(r.get<std::uint32_t>());
        Value v = read_value(r, t, 0);
        if (key == "general.alignment") {
            // a u32 in the spec, which asks for a multiple of 8; offsets are
            // rounded to it by division, so no power of two is needed
            std::uint64_t a = 0;
            if (t == ValueType::U32) a = v.scalar.u32;
            else if (t == ValueType::U64) a = v.scalar.u64;
            else bad("general.alignment is not an unsigned integer");
            if (a == 0 || a % 8 != 0 || a > (1u << 20))
                bad("general.alignment " + std::to_string(a) + " is not a nonzero multiple of 8 up to 1 MiB");
            alignment_ = static_cast<std::uint32_t>(a);
        }
        meta_.emplace_back(std::move(key), std::move(v));
    }
    tensors_.reserve(static_cast<std::size_t>(n_t));
    for (std::uint64_t i = 0; i < n_t; ++i) {
        TensorInfo ti;
        ti.name = r.str();
        const std::uint32_t nd = r.get<std::uint32_t>();
        if (nd < 1 || nd > 4) bad("tensor '" + ti.name + "' has " + std::to_string(nd) + " dims");
        ti.numel = 1;
        for (std::uint32_t d = 0; d < nd; ++d) {
            const std::uint64_t x = r.get<std::uint64_t>();
            if (x == 0 || x > static_cast<std::uint64_t>(INT64_MAX) ||
                __builtin_mul_overflow(ti.numel, static_cast<std::int64_t>(x), &ti.numel))
                bad("tensor '" + ti.name + "' has a zero or overflowing dim");
            ti.dims.push_back(static_cast<std::int64_t>(x));
        }
        ti.dtype = dtype_from_ggml(static_cast<int>(r.get<std::uint32_t>()));
        ti.offset = r.get<std::uint64_t>();
        if (ti.dims[0] % dtype_block_size(ti.dtype) != 0)
            bad("tensor '" + ti.name + "' row length is not a multiple of the block size");
        std::uint64_t nbytes = 0;
        if (__builtin_mul_overflow(static_cast<std::uint64_t>(dtype_storage_bytes(ti.dtype, ti.dims[0])),
                                   static_cast<std::uint64_t>(ti.numel / ti.dims[0]), &nbytes))
            bad("tensor '" + ti.name + "' byte size overflows");
        ti.nbytes = static_cast<std::size_t>(nbytes);
        tensors_.push_back(std::move(ti));
    }
    const std::size_t hdr = static_cast<std::size_t>(r.p - storage_->base);
    const std::size_t data0 = (hdr + alignment_ - 1) / alignment_ * alignment_;
    if (data0 > storage_->size && !tensors_.empty()) bad("data section starts past the end of the file");
    const std::uint64_t room = storage_->size > data0 ? storage_->size - data0 : 0;
    for (std::size_t i = 0; i < tensors_.size(); ++i) {
        TensorInfo& ti = tensors_[i];
        if (ti.offset % alignment_ != 0) bad("tensor '" + ti.name + "' offset is not a multiple of the alignment");
        // offset and size each checked against what is left, so no sum can wrap
        if (ti.offset > room || ti.nbytes > room - ti.offset) bad("tensor '" + ti.name + "' data out of range");
        ti.data = storage_->base + data0 + ti.offset;
        if (!tensor_index_.emplace(ti.name, i).second) bad("duplicate tensor '" + ti.name + "'");
    }
}

File File::open(const std::string& path) {
    File f;
    f.storage_ = std::make_unique<Storage>();
    const int fd = ::open(path.c_str(), O_RDONLY);
    if (fd < 0) bad("cannot open '" + path + "'");
    struct stat st;
    if (fstat(fd, &st) != 0) {
        ::close(fd);
        bad("cannot stat '" + path + "'");
    }
    const std::size_t len = static_cast<std::size_t>(st.st_size);
    void* m = mmap(nullptr, len, PROT_READ, MAP_PRIVATE, fd, 0);
    ::close(fd);
    if (m == MAP_FAILED) bad("cannot map '" + path + "'");
    f.storage_->map = m;
    f.storage_->map_len = len;
    f.storage_->base = static_cast<const std::uint8_t*>(m);
    f.storage_->size = len;
    f.parse_();
    return f;
}

File File::from_memory(std::vector<std::uint8_t> bytes) {
    File f;
    f.storage_ = std::make_unique<Storage>();
    f.storage_->owned = std::move(bytes);
    f.storage_->base = f.storage_->owned.data();
    f.storage_->size = f.storage_->owned.size();
    f.parse_();
    return f;
}

const Value* File::find_meta(const std::string& key) const {
    for (const auto& kv : meta_)
        if (kv.first == key) return &kv.second;
    return nullptr;
}

const TensorInfo* File::find_tensor(const std::string& name) const {
    const auto it = tensor_index_.find(name);
    return it == tensor_index_.end() ? nullptr : &tensors_[it->second];
}

void upload_raw_bytes(const std::uint8_t* bytes, std::size_t nbytes, Dtype dt, int rows, int cols, Tensor& dst) {
    if (!initialized()) throw std::runtime_error("gguf::upload_raw: brotensor::init() has not been called");
    const std::size_t need = static_cast<std::size_t>(rows) * static_cast<std::size_t>(dtype_storage_bytes(dt, cols));
    if (need != nbytes) bad("upload_raw: byte count mismatch");
    Tensor cpu = Tensor::view(Device::CPU, const_cast<std::uint8_t*>(bytes), rows, cols, dt);
    dst = cpu.to(Device::ROCm);
}

void upload_raw(const TensorInfo& info, int rows, int cols, Tensor& dst) {
    if (static_cast<std::int64_t>(rows) * cols != info.numel)
        bad("upload_raw: '" + info.name + "' numel mismatch");
    if (cols % dtype_block_size(info.dtype) != 0) bad("upload_raw: '" + info.name + "' ragged rows");
    upload_raw_bytes(info.data, info.nbytes, info.dtype, rows, cols, dst);
}

// ------------------------------------------------------------------ Writer

namespace {
template <typename T>
void put(std::vector<std::uint8_t>& b, T v) {
    const auto* p = reinterpret_cast<const std::uint8_t*>(&v);
    b.insert(b.end(), p, p + sizeof(T));
}
void put_str(std::vector<std::uint8_t>& b, const std::string& s) {
    put<std::uint64_t>(b, s.size());
    b.insert(b.end(), s.begin(), s.end());
}
}  // namespace

void Writer::add_string(const std::string& key, const std::string& v) {
    KV kv{key, ValueType::String, {}};
    put_str(kv.payload, v);
    kvs_.push_back(std::move(kv));
}
void Writer::add_u32(const std::string& key, std::uint32_t v) {
    KV kv{key, ValueType::U32, {}};
    put(kv.payload, v);
    kvs_.push_back(std::move(kv));
}
void Writer::add_i32(const std::string& key, std::int32_t v) {
    KV kv{key, ValueType::I32, {}};
    put(kv.payload, v);
    kvs_.push_back(std::move(kv));
}
void Writer::add_u64(const std::string& key, std::uint64_t v) {
    KV kv{key, ValueType::U64, {}};
    put(kv.payload, v);
    kvs_.push_back(std::move(kv));
}
void Writer::add_f32(const std::string& key, float v) {
    KV kv{key, ValueType::F32, {}};
    put(kv.payload, v);
    kvs_.push_back(std::move(kv));
}
void Writer::add_bool(const std::string& key, bool v) {
    KV kv{key, ValueType::Bool, {}};
    put<std::uint8_t>(kv.payload, v ? 1 : 0);
    kvs_.push_back(std::move(kv));
}
void Writer::add_string_array(const std::string& key, const std::vector<std::string>& v) {
    KV kv{key, ValueType::Array, {}};
    put<std::uint32_t>(kv.payload, static_cast<std::uint32_t>(ValueType::String));
    put<std::uint64_t>(kv.payload, v.size());
    for (const auto& s : v) put_str(kv.payload, s);
    kvs_.push_back(std::move(kv));
}

void Writer::add_i32_array(const std::string& key, const std::vector<std::int32_t>& v) {
    KV kv{key, ValueType::Array, {}};
    put<std::uint32_t>(kv.payload, static_cast<std::uint32_t>(ValueType::I32));
    put<std::uint64_t>(kv.payload, v.size());
    for (std::int32_t x : v) put<std::int32_t>(kv.payload, x);
    kvs_.push_back(std::move(kv));
}

void Writer::add_tensor(const std::string& name, Dtype dt, const std::vector<std::int64_t>& dims,
                        std::vector<std::uint8_t> bytes) {
    if (dims.empty() || dims.size() > 4) bad("writer: 1..4 dims required");
    std::int64_t n = 1;
    for (auto d : dims) n *= d;
    if (dims[0] % dtype_block_size(dt) != 0) bad("writer: ragged row for '" + name + "'");
    const std::size_t want = static_cast<std::size_t>(dtype_storage_bytes(dt, dims[0]) * (n / dims[0]));
    if (want != bytes.size()) bad("writer: byte count mismatch for '" + name + "'");
    tensors_.push_back(T{name, dt, dims, want, std::move(bytes)});
}

void Writer::add_tensor_placeholder(const std::string& name, Dtype dt, const std::vector<std::int64_t>& dims) {
    if (dims.empty() || dims.size() > 4) bad("writer: 1..4 dims required");
    std::int64_t n = 1;
    for (auto d : dims) n *= d;
    if (dims[0] % dtype_block_size(dt) != 0) bad("writer: ragged row for '" + name + "'");
    const std::size_t want = static_cast<std::size_t>(dtype_storage_bytes(dt, dims[0]) * (n / dims[0]));
    tensors_.push_back(T{name, dt, dims, want, {}});
}

std::vector<std::uint8_t> Writer::to_bytes(std::vector<std::size_t>* data_offsets) const {
    std::vector<std::uint8_t> b;
    b.insert(b.end(), {'G', 'G', 'U', 'F'});
    put<std::uint32_t>(b, 3);
    put<std::uint64_t>(b, tensors_.size());
    const bool write_align = alignment_ != 32;
    put<std::uint64_t>(b, kvs_.size() + (write_align ? 1 : 0));
    if (write_align) {
        put_str(b, "general.alignment");
        put<std::uint32_t>(b, static_cast<std::uint32_t>(ValueType::U32));
        put<std::uint32_t>(b, alignment_);
    }
    for (const auto& kv : kvs_) {
        put_str(b, kv.key);
        put<std::uint32_t>(b, static_cast<std::uint32_t>(kv.type));
        b.insert(b.end(), kv.payload.begin(), kv.payload.end());
    }
    std::uint64_t off = 0;
    std::vector<std::uint64_t> offs;
    for (const auto& t : tensors_) {
        put_str(b, t.name);
        put<std::uint32_t>(b, static_cast<std::uint32_t>(t.dims.size()));
        for (auto d : t.dims) put<std::uint64_t>(b, static_cast<std::uint64_t>(d));
        put<std::uint32_t>(b, static_cast<std::uint32_t>(dtype_to_ggml(t.dt)));
        put<std::uint64_t>(b, off);
        offs.push_back(off);
        off += (t.nbytes + alignment_ - 1) / alignment_ * alignment_;
    }
    b.resize((b.size() + alignment_ - 1) / alignment_ * alignment_, 0);
    const std::size_t data0 = b.size();
    b.resize(data0 + off, 0);
    for (std::size_t i = 0; i < tensors_.size(); ++i)
        if (!tensors_[i].bytes.empty())
            std::memcpy(b.data() + data0 + offs[i], tensors_[i].bytes.data(), tensors_[i].bytes.size());
    if (data_offsets) {
        data_offsets->clear();
        for (auto o : offs) data_offsets->push_back(data0 + o);
    }
    return b;
}

void Writer::write(const std::string& path) const {
    const std::vector<std::uint8_t> b = to_bytes();
    std::ofstream f(path, std::ios::binary | std::ios::trunc);
    if (!f) bad("cannot write '" + path + "'");
    f.write(reinterpret_cast<const char*>(b.data()), static_cast<std::streamsize>(b.size()));
    if (!f) bad("short write to '" + path + "'");
}

}  // namespace brotensor::gguf
