// Recursive-descent JSON reader (see include/brolm/detail/json.h).
#include "brolm/detail/json.h"

#include <cstdlib>
#include <stdexcept>

namespace brolm::detail::json {

namespace {

[[noreturn]] void bad(const std::string& what, std::size_t at) {
    throw std::runtime_error("json: " + what + " at offset " + std::to_string(at));
}

void put_utf8(uint32_t cp, std::string& out) {
    if (cp < 0x80) {
        out += static_cast<char>(cp);
    } else if (cp < 0x800) {
        out += static_cast<char>(0xC0 | (cp >> 6));
        out += static_cast<char>(0x80 | (cp & 0x3F));
    } else if (cp < 0x10000) {
        out += static_cast<char>(0xE0 | (cp >> 12));
        out += static_cast<char>(0x80 | ((cp >> 6) & 0x3F));
        out += static_cast<char>(0x80 | (cp & 0x3F));
    } else {
        out += static_cast<char>(0xF0 | (cp >> 18));
        out += static_cast<char>(0x80 | ((cp >> 12) & 0x3F));
        out += static_cast<char>(0x80 | ((cp >> 6) & 0x3F));
        out += static_cast<char>(0x80 | (cp & 0x3F));
    }
}

struct Reader {
    std::string_view s;
    std::size_t i = 0;
    int depth = 0;

    void ws() {
        while (i < s.size() && (s[i] == ' ' || s[i] == '\t' || s[i] == '\n' || s[i] == '\r')) ++i;
    }
    char peek() {
        ws();
        if (i >= s.size()) bad("unexpected end", i);
        return s[i];
    }
    void expect(char c) {
        if (peek() != c) bad(std::string("expected '") + c + "'", i);
        ++i;
    }
    uint32_t hex4() {
        if (i + 4 > s.size()) bad("short \\u escape", i);
        uint32_t v = 0;
        for (int k = 0; k < 4; ++k) {
            const char c = s[i++];
            v <<= 4;
            if (c >= '0' && c <= '9') v |= c - '0';
            else if (c >= 'a' && c <= 'f') v |= c - 'a' + 10;
            else if (c >= 'A' && c <= 'F') v |= c - 'A' + 10;
            else bad("bad hex digit", i - 1);
        }
        return v;
    }
    std::string string() {
        expect('"');
        std::string out;
        while (true) {
            if (i >= s.size()) bad("unterminated string", i);
            const char c = s[i++];
            if (c == '"') break;
            if (c != '\\') {
                out += c;
                continue;
            }
            if (i >= s.size()) bad("unterminated escape", i);
            const char e = s[i++];
            switch (e) {
                case '"': out += '"'; break;
                case '\\': out += '\\'; break;
                case '/': out += '/'; break;
                case 'b': out += '\b'; break;
                case 'f': out += '\f'; break;
                case 'n': out += '\n'; break;
                case 'r': out += '\r'; break;
                case 't': out += '\t'; break;
                case 'u': {
                    uint32_t cp = hex4();
                    if (cp >= 0xD800 && cp < 0xDC00 && i + 6 <= s.size() && s[i] == '\\' && s[i + 1] == 'u') {
                        const std::size_t save = i;
                        i += 2;
                        const uint32_t lo = hex4();
                        if (lo >= 0xDC00 && lo < 0xE000) cp = 0x10000 + ((cp - 0xD800) << 10) + (lo - 0xDC00);
                        else i = save;
                    }
                    put_utf8(cp, out);
                    break;
                }
                default: bad("bad escape", i - 1);
            }
        }
        return out;
    }
    Value value() {
        if (++depth > 256) bad("nesting too deep", i);
        Value v;
        const char c = peek();
        if (c == '{') {
            ++i;
            v.kind = Value::Kind::Object;
            if (peek() == '}') {
                ++i;
            } else {
                while (true) {
                    std::string k = string();
                    expect(':');
                    v.obj.emplace_back(std::move(k), value());
                    const char d = peek();
                    ++i;
                    if (d == '}') break;
                    if (d != ',') bad("expected ',' or '}'", i - 1);
                }
            }
        } else if (c == '[') {
            ++i;
            v.kind = Value::Kind::Array;
            if (peek() == ']') {
                ++i;
            } else {
                while (true) {
                    v.arr.push_back(value());
                    const char d = peek();
                    ++i;
                    if (d == ']') break;
                    if (d != ',') bad("expected ',' or ']'", i - 1);
                }
            }
        } else if (c == '"') {
            v.kind = Value::Kind::String;
            v.str = string();
        } else if (s.compare(i, 4, "true") == 0) {
            v.kind = Value::Kind::Bool;
            v.b = true;
            i += 4;
        } else if (s.compare(i, 5, "false") == 0) {
            v.kind = Value::Kind::Bool;
            i += 5;
        } else if (s.compare(i, 4, "null") == 0) {
            i += 4;
        } else {
            const std::size_t b = i;
            while (i < s.size() && (s[i] == '-' || s[i] == '+' || s[i] == '.' || s[i] == 'e' || s[i] == 'E' ||
                                    (s[i] >= '0' && s[i] <= '9')))
                ++i;
            if (i == b) bad("unexpected character", i);
            const std::string num(s.substr(b, i - b));
            char* end = nullptr;
            v.kind = Value::Kind::Number;
            v.num = std::strtod(num.c_str(), &end);
            if (!end || *end) bad("bad number", b);
        }
        --depth;
        return v;
    }
};

}  // namespace

const Value* Value::find(std::string_view key) const {
    for (const auto& kv : obj)
        if (kv.first == key) return &kv.second;
    return nullptr;
}

Value parse(std::string_view text) {
    Reader r{text};
    Value v = r.value();
    r.ws();
    if (r.i != text.size()) bad("trailing characters", r.i);
    return v;
}

}  // namespace brolm::detail::json
