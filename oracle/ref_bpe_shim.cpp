// Test harness (oracle/_ref only): a C entry point over the reference's own
// byte-level BPE core, compiled from reference src/detail/byte_level_bpe.cpp
// (load_vocab_json, load_merges_txt, build_byte_to_unicode, encode_piece,
// SpecialTokens).  Used by tests/ to check the tokenizer oracle's merge loop
// against the reference's compiled code; never linked into the product.
#include <cstring>
#include <map>
#include <memory>
#include <string>
#include <unordered_map>
#include <vector>

#include "brolm/detail/byte_level_bpe.h"

namespace bpe = brolm::detail::bpe;

namespace {
struct Tables {
    std::unordered_map<std::string, int32_t> vocab, ranks;
    std::string b2u[256];
};
std::map<std::string, std::unique_ptr<Tables>> g_tables;
std::string g_err;
}  // namespace

extern "C" {

const char* ref_bpe_error(void) { return g_err.c_str(); }

// ids of encode_piece(piece) under the vocab.json / merges.txt pair (loaded
// once per pair); returns the id count (may exceed cap) or -1.
int ref_bpe_encode_piece(const char* vocab_json, const char* merges_txt, const char* piece, long len, int* out,
                         int cap) {
    try {
        const std::string key = std::string(vocab_json) + '\n' + merges_txt;
        auto& t = g_tables[key];
        if (!t) {
            t = std::make_unique<Tables>();
            t->vocab = bpe::load_vocab_json(vocab_json);
            t->ranks = bpe::load_merges_txt(merges_txt);
            bpe::build_byte_to_unicode(t->b2u);
        }
        std::vector<int32_t> ids;
        bpe::encode_piece(std::string_view(piece, static_cast<std::size_t>(len)), t->b2u, t->vocab, t->ranks, false,
                          ids);
        for (std::size_t i = 0; i < ids.size() && static_cast<int>(i) < cap; ++i) out[i] = ids[i];
        return static_cast<int>(ids.size());
    } catch (const std::exception& e) {
        g_err = e.what();
        return -1;
    }
}

// SpecialTokens::match over a '\n'-separated list of tokens (ids = their
// position): writes (length, id) of the longest special at text[pos].
int ref_bpe_special_match(const char* tokens, const char* text, long len, long pos, long* match_len, int* id) {
    try {
        bpe::SpecialTokens sp;
        int k = 0;
        std::string cur;
        for (const char* p = tokens;; ++p) {
            if (*p == '\n' || *p == 0) {
                if (!cur.empty()) sp.add(cur, k++);
                cur.clear();
                if (*p == 0) break;
            } else {
                cur += *p;
            }
        }
        const auto m = sp.match(std::string_view(text, static_cast<std::size_t>(len)), static_cast<std::size_t>(pos));
        *match_len = static_cast<long>(m.first);
        *id = m.second;
        return 0;
    } catch (const std::exception& e) {
        g_err = e.what();
        return -1;
    }
}

}  // extern "C"
