// Qwen3 byte-level BPE tokenizer (see include/brolm/qwen_tokenizer.h).
// Behaviour follows the reference src/qwen_tokenizer.cpp (pre-tokenization
// :29-111, loaders :122-390, encode / decode / chat template :392-471) and
// src/detail/byte_level_bpe.cpp (byte alphabet :60-105, merges.txt :225-251,
// merge loop :255-304, special matching :451-468).
#include "brolm/qwen_tokenizer.h"

#include <algorithm>
#include <fstream>
#include <sstream>
#include <stdexcept>

#include "brolm/detail/json.h"
#include "brotensor/gguf.h"

namespace brolm::qwen {

namespace {

namespace gg = brotensor::gguf;
namespace js = brolm::detail::json;

[[noreturn]] void fail(const std::string& where, const std::string& what) {
    throw std::runtime_error("qwen::Tokenizer::" + where + ": " + what);
}

std::string read_file(const std::string& path, const char* where) {
    std::ifstream f(path, std::ios::binary);
    if (!f) fail(where, "cannot open '" + path + "'");
    std::ostringstream ss;
    ss << f.rdbuf();
    return ss.str();
}

void utf8(uint32_t cp, std::string& out) {
    if (cp < 0x80) {
        out += static_cast<char>(cp);
    } else if (cp < 0x800) {
        out += static_cast<char>(0xC0 | (cp >> 6));
        out += static_cast<char>(0x80 | (cp & 0x3F));
    } else {
        out += static_cast<char>(0xE0 | (cp >> 12));
        out += static_cast<char>(0x80 | ((cp >> 6) & 0x3F));
        out += static_cast<char>(0x80 | (cp & 0x3F));
    }
}

// Length of the UTF-8 sequence starting with lead byte c (1 for stray bytes).
std::size_t seq_len(unsigned char c) {
    if (c >= 0xF0) return 4;
    if (c >= 0xE0) return 3;
    if (c >= 0xC0) return 2;
    return 1;
}

uint32_t decode_cp(const std::string& s, std::size_t& i) {
    const unsigned char c = static_cast<unsigned char>(s[i]);
    const std::size_t n = std::min(seq_len(c), s.size() - i);
    uint32_t cp = n == 1 ? c : (n == 2 ? c & 0x1F : (n == 3 ? c & 0x0F : c & 0x07));
    for (std::size_t k = 1; k < n; ++k) cp = (cp << 6) | (static_cast<unsigned char>(s[i + k]) & 0x3F);
    i += n;
    return cp;
}

bool letter(unsigned char c) { return (c >= 'a' && c <= 'z') || (c >= 'A' && c <= 'Z'); }
bool digit(unsigned char c) { return c >= '0' && c <= '9'; }
bool space(unsigned char c) { return c == ' ' || c == '\t' || c == '\n' || c == '\r' || c == '\f' || c == '\v'; }

// Contraction at text[i] (which is an apostrophe): its length or 0.
std::size_t contraction(std::string_view t, std::size_t i) {
    static const char* const k3[] = {"'re", "'ve", "'ll"};
    static const char* const k2[] = {"'s", "'t", "'m", "'d"};
    for (const char* c : k3)
        if (t.compare(i, 3, c) == 0) return 3;
    for (const char* c : k2)
        if (t.compare(i, 2, c) == 0) return 2;
    return 0;
}

// GPT-2 style ASCII pre-tokenization (reference src/qwen_tokenizer.cpp:38-111).
template <class Emit>
void pre_tokenize(std::string_view t, Emit&& emit) {
    std::size_t i = 0;
    const std::size_t n = t.size();
    while (i < n) {
        unsigned char c = static_cast<unsigned char>(t[i]);
        if (c == '\'') {
            if (const std::size_t k = contraction(t, i)) {
                emit(t.substr(i, k));
                i += k;
                continue;
            }
        }
        const std::size_t start = i;
        if (c == ' ') {
            // one space folds into the run after it unless whitespace follows
            if (i + 1 < n && !space(static_cast<unsigned char>(t[i + 1]))) {
                ++i;
                c = static_cast<unsigned char>(t[i]);
            } else {
                emit(t.substr(i, 1));
                ++i;
                continue;
            }
        } else if (space(c)) {
            std::size_t j = i;
            while (j < n && space(static_cast<unsigned char>(t[j])) && t[j] != ' ') ++j;
            emit(t.substr(i, j - i));
            i = j;
            continue;
        }
        std::size_t j = i;
        if (letter(c)) {
            while (j < n && letter(static_cast<unsigned char>(t[j]))) ++j;
        } else if (digit(c)) {
            while (j < n && digit(static_cast<unsigned char>(t[j]))) ++j;
        } else {
            // any other bytes; an apostrophe that starts a contraction ends
            // the run unless it is the run's first byte
            while (j < n) {
                const unsigned char u = static_cast<unsigned char>(t[j]);
                if (space(u) || letter(u) || digit(u)) break;
                if (u == '\'' && j != i && contraction(t, j)) break;
                ++j;
            }
        }
        emit(t.substr(start, j - start));
        i = j;
    }
}

}  // namespace

// ---------------------------------------------------------------- specials

void Tokenizer::Special::add(const std::string& tok, int32_t id) {
    if (tok.empty()) return;
    auto it = by_str.find(tok);
    if (it != by_str.end()) {
        auto old = by_id.find(it->second);
        if (old != by_id.end() && old->second == tok) by_id.erase(old);
        it->second = id;
    } else {
        by_str.emplace(tok, id);
        by_first[static_cast<unsigned char>(tok[0])].push_back(tok);
    }
    by_id[id] = tok;
}

std::pair<std::size_t, int32_t> Tokenizer::Special::match(std::string_view text, std::size_t pos) const {
    std::size_t best = 0;
    int32_t id = -1;
    for (const std::string& tok : by_first[static_cast<unsigned char>(text[pos])]) {
        if (tok.size() > best && text.compare(pos, tok.size(), tok) == 0) {
            best = tok.size();
            id = by_str.at(tok);
        }
    }
    return {best, id};
}

// ---------------------------------------------------------------- set-up

Tokenizer::Tokenizer() {
    // GPT-2 byte alphabet: printable bytes keep their codepoint, the rest take
    // U+0100, U+0101, ... in byte order
    int next = 256;
    for (int b = 0; b < 256; ++b) {
        const bool self = (b >= 33 && b <= 126) || (b >= 161 && b <= 172) || (b >= 174 && b <= 255);
        const uint32_t cp = self ? static_cast<uint32_t>(b) : static_cast<uint32_t>(next++);
        utf8(cp, byte_cp_[b]);
        cp_byte_[cp] = static_cast<unsigned char>(b);
    }
}

int32_t Tokenizer::intern_(const std::string& s) {
    auto it = sym_.find(s);
    if (it != sym_.end()) return it->second;
    const int32_t id = static_cast<int32_t>(sym_str_.size());
    sym_.emplace(s, id);
    sym_str_.push_back(s);
    return id;
}

void Tokenizer::add_merge_(const std::string& a, const std::string& b, int32_t rank) {
    const int32_t ia = intern_(a), ib = intern_(b);
    const int32_t iab = intern_(a + b);
    const uint64_t key = (static_cast<uint64_t>(static_cast<uint32_t>(ia)) << 32) | static_cast<uint32_t>(ib);
    if (merges_.emplace(key, std::make_pair(rank, iab)).second) ++merge_count_;
}

void Tokenizer::finish_(const std::vector<std::string>& extra_special_tokens) {
    std::vector<std::string> names = {"<|endoftext|>", "<|im_start|>", "<|im_end|>"};
    names.insert(names.end(), extra_special_tokens.begin(), extra_special_tokens.end());
    for (const auto& s : names) {
        auto it = vocab_.find(s);
        if (it != vocab_.end()) specials_.add(s, it->second);
    }
    auto id_of = [&](const char* s) {
        auto it = vocab_.find(s);
        return it != vocab_.end() ? static_cast<int>(it->second) : -1;
    };
    endoftext_id_ = id_of("<|endoftext|>");
    im_start_id_ = id_of("<|im_start|>");
    im_end_id_ = id_of("<|im_end|>");
}

Tokenizer Tokenizer::load(const std::string& vocab_json_path, const std::string& merges_txt_path,
                          const std::vector<std::string>& extra_special_tokens) {
    Tokenizer t;
    js::Value root;
    try {
        root = js::parse(read_file(vocab_json_path, "load"));
    } catch (const std::runtime_error& e) {
        fail("load", std::string("vocab.json: ") + e.what());
    }
    if (!root.is_object()) fail("load", "vocab.json is not an object");
    for (const auto& [tok, v] : root.obj) {
        if (!v.is_number()) fail("load", "vocab.json value for '" + tok + "' is not a number");
        t.vocab_.emplace(tok, static_cast<int32_t>(v.num));
    }
    for (const auto& [tok, id] : t.vocab_) t.id_to_token_.emplace(id, tok);

    std::istringstream mf(read_file(merges_txt_path, "load"));
    std::string line;
    int32_t rank = 0;
    bool first = true;
    while (std::getline(mf, line)) {
        if (!line.empty() && line.back() == '\r') line.pop_back();
        if (line.empty()) continue;
        if (first) {
            first = false;
            if (line[0] == '#') continue;
        }
        const auto sp = line.find(' ');
        if (sp == std::string::npos) fail("load", "merges.txt: malformed line '" + line + "'");
        t.add_merge_(line.substr(0, sp), line.substr(sp + 1), rank++);
    }
    t.finish_(extra_special_tokens);
    return t;
}

Tokenizer Tokenizer::from_gguf(const gg::File& f, const std::vector<std::string>& extra_special_tokens) {
    auto array_of = [&](const char* key, gg::ValueType et) -> const std::vector<gg::Value>& {
        const gg::Value* v = f.find_meta(key);
        if (!v) fail("from_gguf", std::string("missing metadata '") + key + "'");
        if (v->type != gg::ValueType::Array || v->array_type != et)
            fail("from_gguf", std::string("metadata '") + key + "' is not an array of the expected element type");
        return v->array;
    };
    Tokenizer t;
    const auto& tokens = array_of("tokenizer.ggml.tokens", gg::ValueType::String);
    for (std::size_t i = 0; i < tokens.size(); ++i) {
        t.vocab_.emplace(tokens[i].str, static_cast<int32_t>(i));
        t.id_to_token_.emplace(static_cast<int32_t>(i), tokens[i].str);
    }
    const auto& merges = array_of("tokenizer.ggml.merges", gg::ValueType::String);
    for (std::size_t i = 0; i < merges.size(); ++i) {
        const std::string& m = merges[i].str;
        const auto sp = m.find(' ');
        if (sp == std::string::npos) fail("from_gguf", "malformed merges entry '" + m + "'");
        t.add_merge_(m.substr(0, sp), m.substr(sp + 1), static_cast<int32_t>(i));
    }
    if (const gg::Value* tt = f.find_meta("tokenizer.ggml.token_type");
        tt && tt->type == gg::ValueType::Array && tt->array_type == gg::ValueType::I32) {
        for (std::size_t i = 0; i < tt->array.size() && i < tokens.size(); ++i)
            if (tt->array[i].scalar.i32 == 3) t.specials_.add(tokens[i].str, static_cast<int32_t>(i));
    }
    t.finish_(extra_special_tokens);
    return t;
}

Tokenizer Tokenizer::from_tokenizer_json(const std::string& tokenizer_json_path,
                                         const std::vector<std::string>& extra_special_tokens) {
    Tokenizer t;
    js::Value root;
    try {
        root = js::parse(read_file(tokenizer_json_path, "from_tokenizer_json"));
    } catch (const std::runtime_error& e) {
        fail("from_tokenizer_json", std::string("json parse: ") + e.what());
    }
    if (!root.is_object()) fail("from_tokenizer_json", "root is not a JSON object");
    const js::Value* model = root.find("model");
    if (!model || !model->is_object()) fail("from_tokenizer_json", "missing 'model' object");
    const js::Value* vocab = model->find("vocab");
    if (!vocab || !vocab->is_object())
        fail("from_tokenizer_json", "model.vocab is not an object (not a byte-level BPE tokenizer.json)");
    for (const auto& [tok, v] : vocab->obj)
        if (v.is_number()) t.vocab_.emplace(tok, static_cast<int32_t>(v.num));
    if (const js::Value* merges = model->find("merges"); merges && merges->is_array()) {
        for (std::size_t i = 0; i < merges->arr.size(); ++i) {
            const js::Value& m = merges->arr[i];
            if (m.is_array()) {
                if (m.arr.size() != 2 || !m.arr[0].is_string() || !m.arr[1].is_string())
                    fail("from_tokenizer_json", "malformed model.merges pair entry");
                t.add_merge_(m.arr[0].str, m.arr[1].str, static_cast<int32_t>(i));
            } else if (m.is_string()) {
                const auto sp = m.str.find(' ');
                if (sp == std::string::npos) fail("from_tokenizer_json", "malformed model.merges entry '" + m.str + "'");
                t.add_merge_(m.str.substr(0, sp), m.str.substr(sp + 1), static_cast<int32_t>(i));
            }
        }
    }
    if (const js::Value* added = root.find("added_tokens"); added && added->is_array()) {
        for (const js::Value& a : added->arr) {
            if (!a.is_object()) continue;
            const js::Value* content = a.find("content");
            const js::Value* idv = a.find("id");
            if (!content || !content->is_string() || !idv || !idv->is_number()) continue;
            const int32_t id = static_cast<int32_t>(idv->num);
            t.vocab_[content->str] = id;
            const js::Value* sp = a.find("special");
            if (!(sp && sp->is_bool() && !sp->b)) t.specials_.add(content->str, id);
        }
    }
    for (const auto& [tok, id] : t.vocab_) t.id_to_token_.emplace(id, tok);
    t.finish_(extra_special_tokens);
    return t;
}

void Tokenizer::register_special_token(const std::string& token, int32_t id) {
    specials_.add(token, id);
    if (token == "<|endoftext|>") endoftext_id_ = id;
    else if (token == "<|im_start|>") im_start_id_ = id;
    else if (token == "<|im_end|>") im_end_id_ = id;
}

// ---------------------------------------------------------------- encode / decode

void Tokenizer::encode_piece_(std::string_view piece, std::vector<int32_t>& out) const {
    if (piece.empty()) return;
    // symbols of the byte-mapped piece; a codepoint never interned gets a
    // negative placeholder (it takes part in no merge)
    std::vector<int32_t> w;
    std::vector<std::string> extra;
    w.reserve(piece.size());
    for (char ch : piece) {
        const std::string& cp = byte_cp_[static_cast<unsigned char>(ch)];
        auto it = sym_.find(cp);
        if (it != sym_.end()) {
            w.push_back(it->second);
        } else {
            extra.push_back(cp);
            w.push_back(-static_cast<int32_t>(extra.size()));
        }
    }
    auto key = [](int32_t a, int32_t b) {
        return (static_cast<uint64_t>(static_cast<uint32_t>(a)) << 32) | static_cast<uint32_t>(b);
    };
    while (w.size() > 1) {
        int32_t best_rank = -1, best_a = 0, best_b = 0, merged = 0;
        for (std::size_t i = 0; i + 1 < w.size(); ++i) {
            if (w[i] < 0 || w[i + 1] < 0) continue;
            auto it = merges_.find(key(w[i], w[i + 1]));
            if (it != merges_.end() && (best_rank < 0 || it->second.first < best_rank)) {
                best_rank = it->second.first;
                best_a = w[i];
                best_b = w[i + 1];
                merged = it->second.second;
            }
        }
        if (best_rank < 0) break;
        std::size_t o = 0;
        for (std::size_t i = 0; i < w.size();) {
            if (i + 1 < w.size() && w[i] == best_a && w[i + 1] == best_b) {
                w[o++] = merged;
                i += 2;
            } else {
                w[o++] = w[i++];
            }
        }
        w.resize(o);
    }
    for (int32_t s : w) {
        const std::string& str = s >= 0 ? sym_str_[static_cast<std::size_t>(s)] : extra[static_cast<std::size_t>(-s - 1)];
        auto it = vocab_.find(str);
        if (it != vocab_.end()) out.push_back(it->second);   // a unit outside the vocab is dropped
    }
}

void Tokenizer::encode_span_(std::string_view span, std::vector<int32_t>& out) const {
    pre_tokenize(span, [&](std::string_view piece) { encode_piece_(piece, out); });
}

std::vector<int32_t> Tokenizer::encode(std::string_view text, bool add_special) const {
    std::vector<int32_t> ids;
    ids.reserve(text.size());
    std::size_t span = 0;
    for (std::size_t i = 0; i < text.size();) {
        const auto m = specials_.match(text, i);
        if (m.first == 0) {
            ++i;
            continue;
        }
        if (i > span) encode_span_(text.substr(span, i - span), ids);
        ids.push_back(m.second);
        i += m.first;
        span = i;
    }
    if (span < text.size()) encode_span_(text.substr(span), ids);
    if (add_special && endoftext_id_ >= 0) ids.push_back(endoftext_id_);
    return ids;
}

std::string Tokenizer::decode(const std::vector<int32_t>& ids) const {
    std::string out, pending;
    auto flush = [&]() {
        for (std::size_t i = 0; i < pending.size();) {
            auto it = cp_byte_.find(decode_cp(pending, i));
            if (it != cp_byte_.end()) out += static_cast<char>(it->second);
        }
        pending.clear();
    };
    for (int32_t id : ids) {
        if (auto sp = specials_.by_id.find(id); sp != specials_.by_id.end()) {
            flush();
            out += sp->second;
            continue;
        }
        if (auto it = id_to_token_.find(id); it != id_to_token_.end()) pending += it->second;
    }
    flush();
    return out;
}

std::string Tokenizer::apply_chat_template(const std::vector<std::pair<std::string, std::string>>& messages,
                                           bool add_generation_prompt) const {
    std::string out;
    for (const auto& [role, content] : messages) out += "<|im_start|>" + role + "\n" + content + "<|im_end|>\n";
    if (add_generation_prompt) out += "<|im_start|>assistant\n";
    return out;
}

}  // namespace brolm::qwen
