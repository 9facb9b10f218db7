#pragma once

// Qwen3 byte-level BPE tokenizer (reference include/brolm/qwen_tokenizer.h:41-151,
// src/qwen_tokenizer.cpp, src/detail/byte_level_bpe.cpp).  Same interface and
// token ids as the reference:
//   - pre-tokenization: GPT-2 style and ASCII-only - contractions 's 't 're
//     've 'm 'll 'd; runs of letters, of digits, of other bytes ("punct", every
//     non-ASCII byte included), each optionally led by one folded space;
//     whitespace other than ' ' in runs; a space before whitespace stands alone;
//   - each piece is mapped byte by byte into the GPT-2 byte-level unicode
//     alphabet, then merged: repeatedly the lowest-ranked adjacent pair, every
//     non-overlapping occurrence of it in one left-to-right pass;
//   - registered special tokens are matched verbatim (longest first) before
//     pre-tokenization and decode to their literal text.
// Symbols are interned to integers, so the merge loop compares pair keys, not
// strings.

#include <cstddef>
#include <cstdint>
#include <string>
#include <string_view>
#include <unordered_map>
#include <utility>
#include <vector>

namespace brotensor::gguf {
class File;
}

namespace brolm::qwen {

class Tokenizer {
public:
    // HF GPT-2 format vocab.json + merges.txt (merges.txt: an optional first
    // "#..." line, blank lines skipped, "a b" per line in priority order).
    static Tokenizer load(const std::string& vocab_json_path, const std::string& merges_txt_path,
                          const std::vector<std::string>& extra_special_tokens = {});
    // GGUF metadata: tokenizer.ggml.tokens (strings, id = index),
    // tokenizer.ggml.merges ("a b" strings), optional tokenizer.ggml.token_type
    // (i32; type 3 = control -> special).
    static Tokenizer from_gguf(const brotensor::gguf::File& f,
                               const std::vector<std::string>& extra_special_tokens = {});
    // HF tokenizer.json: model.vocab, model.merges ("a b" or ["a", "b"]),
    // added_tokens (special unless "special": false).
    static Tokenizer from_tokenizer_json(const std::string& tokenizer_json_path,
                                         const std::vector<std::string>& extra_special_tokens = {});

    // add_special appends <|endoftext|> (Qwen3 has no BOS).
    std::vector<int32_t> encode(std::string_view text, bool add_special = false) const;
    // Special ids render literally, others through the byte-level alphabet;
    // unknown ids are skipped.
    std::string decode(const std::vector<int32_t>& ids) const;
    // ChatML: "<|im_start|>role\ncontent<|im_end|>\n" per message, then
    // "<|im_start|>assistant\n" when add_generation_prompt.
    std::string apply_chat_template(const std::vector<std::pair<std::string, std::string>>& messages,
                                    bool add_generation_prompt = true) const;

    std::size_t vocab_count() const { return vocab_.size(); }
    std::size_t merge_count() const { return merge_count_; }

    // Register (or re-bind) an atomic special token; the three ChatML names
    // also update the cached ids below.
    void register_special_token(const std::string& token, int32_t id);

    int eos_id() const { return im_end_id_; }  // <|im_end|>, the ChatML turn end
    int im_start_id() const { return im_start_id_; }
    int im_end_id() const { return im_end_id_; }
    int endoftext_id() const { return endoftext_id_; }

private:
    Tokenizer();

    struct Special {
        std::unordered_map<std::string, int32_t> by_str;
        std::unordered_map<int32_t, std::string> by_id;
        std::vector<std::string> by_first[256];   // candidates by first byte
        void add(const std::string& tok, int32_t id);
        // longest registered token at text[pos..]: (length, id) or (0, -1)
        std::pair<std::size_t, int32_t> match(std::string_view text, std::size_t pos) const;
    };

    int32_t intern_(const std::string& s);
    void add_merge_(const std::string& a, const std::string& b, int32_t rank);
    void finish_(const std::vector<std::string>& extra_special_tokens);
    void encode_span_(std::string_view span, std::vector<int32_t>& out) const;
    void encode_piece_(std::string_view piece, std::vector<int32_t>& out) const;

    std::unordered_map<std::string, int32_t> vocab_;
    std::unordered_map<int32_t, std::string> id_to_token_;
    // interned symbols (every vocab string and merge part / result)
    std::unordered_map<std::string, int32_t> sym_;
    std::vector<std::string> sym_str_;
    // (left symbol << 32 | right symbol) -> (rank, merged symbol); first rank wins
    std::unordered_map<uint64_t, std::pair<int32_t, int32_t>> merges_;
    std::size_t merge_count_ = 0;
    Special specials_;
    std::string byte_cp_[256];                   // byte -> UTF-8 of its codepoint
    std::unordered_map<uint32_t, unsigned char> cp_byte_;
    int endoftext_id_ = -1, im_start_id_ = -1, im_end_id_ = -1;
};

}  // namespace brolm::qwen
