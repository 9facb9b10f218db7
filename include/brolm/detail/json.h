#pragma once

// Minimal JSON document reader for tokenizer containers (vocab.json,
// tokenizer.json).  The reference reads them with its own reader
// (reference include/brolm/detail/json.h, src/detail/byte_level_bpe.cpp:107-224);
// this one keeps objects as ordered (key, value) lists so that duplicate keys
// resolve the way a first-wins map insert would.

#include <cstdint>
#include <string>
#include <string_view>
#include <utility>
#include <vector>

namespace brolm::detail::json {

struct Value {
    enum class Kind { Null, Bool, Number, String, Array, Object };
    Kind kind = Kind::Null;
    bool b = false;
    double num = 0.0;
    std::string str;
    std::vector<Value> arr;
    std::vector<std::pair<std::string, Value>> obj;

    bool is_object() const { return kind == Kind::Object; }
    bool is_array() const { return kind == Kind::Array; }
    bool is_string() const { return kind == Kind::String; }
    bool is_number() const { return kind == Kind::Number; }
    bool is_bool() const { return kind == Kind::Bool; }
    // First member named `key`, or nullptr.
    const Value* find(std::string_view key) const;
};

// Parse a complete document; throws std::runtime_error("json: ...") on syntax
// errors.  Strings decode every JSON escape, \uXXXX surrogate pairs included,
// to UTF-8.
Value parse(std::string_view text);

}  // namespace brolm::detail::json
