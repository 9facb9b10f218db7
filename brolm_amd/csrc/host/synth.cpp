// Synthetic Qwen3 GGUF generator (see include/brolm/synth.h).
#include "brolm/synth.h"

#include <algorithm>
#include <cctype>
#include <cmath>
#include <cstring>
#include <fstream>
#include <map>
#include <stdexcept>
#include <thread>

#include "brotensor/gguf.h"

namespace brolm::synth {

namespace bt = ::brotensor;

namespace {

constexpr std::uint64_t kGolden = 0x9E3779B97F4A7C15ull;

// i-th output of the splitmix64 generator seeded with `key`.
inline std::uint64_t splitmix_at(std::uint64_t key, std::uint64_t i) {
    std::uint64_t z = key + (i + 1) * kGolden;
    z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
    z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
    return z ^ (z >> 31);
}

template <typename F>
void parallel_for(std::int64_t n, F&& f) {
    unsigned nt = std::thread::hardware_concurrency();
    if (nt == 0) nt = 4;
    if (nt > 64) nt = 64;
    if (n < 4096 || nt == 1) {
        f(0, n);
        return;
    }
    std::vector<std::thread> th;
    const std::int64_t chunk = (n + nt - 1) / nt;
    for (unsigned t = 0; t < nt; ++t) {
        const std::int64_t b = t * chunk, e = std::min<std::int64_t>(n, b + chunk);
        if (b >= e) break;
        th.emplace_back([&f, b, e] { f(b, e); });
    }
    for (auto& x : th) x.join();
}

inline int nearest(float x) { return static_cast<int>(std::lrintf(x)); }

void quant_q8_0(const float* x, std::uint8_t* out) {
    float amax = 0.f;
    for (int i = 0; i < 32; ++i) amax = std::max(amax, std::fabs(x[i]));
    const float d = amax / 127.f;
    const std::uint16_t dh = bt::fp32_to_fp16_bits(d);
    const float d16 = bt::fp16_bits_to_fp32(dh);
    std::memcpy(out, &dh, 2);
    for (int i = 0; i < 32; ++i) {
        const int q = d16 > 0.f ? std::clamp(nearest(x[i] / d16), -127, 127) : 0;
        out[2 + i] = static_cast<std::uint8_t>(static_cast<std::int8_t>(q));
    }
}

// Q4_K: 8 sub-blocks of 32, y = (d*sc)*q - (dmin*m), q in [0,15], sc, m 6-bit.
void quant_q4_k(const float* x, std::uint8_t* out) {
    float scale[8], mn[8];
    for (int j = 0; j < 8; ++j) {
        float lo = x[32 * j], hi = x[32 * j];
        for (int i = 1; i < 32; ++i) {
            lo = std::min(lo, x[32 * j + i]);
            hi = std::max(hi, x[32 * j + i]);
        }
        if (lo > 0.f) lo = 0.f;
        scale[j] = (hi - lo) / 15.f;
        mn[j] = -lo;
    }
    const float max_scale = *std::max_element(scale, scale + 8);
    const float max_min = *std::max_element(mn, mn + 8);
    const std::uint16_t dh = bt::fp32_to_fp16_bits(max_scale / 63.f);
    const std::uint16_t mh = bt::fp32_to_fp16_bits(max_min / 63.f);
    const float d = bt::fp16_bits_to_fp32(dh), dmin = bt::fp16_bits_to_fp32(mh);
    int sc[8], m[8];
    for (int j = 0; j < 8; ++j) {
        sc[j] = d > 0.f ? std::clamp(nearest(scale[j] / d), 0, 63) : 0;
        m[j] = dmin > 0.f ? std::clamp(nearest(mn[j] / dmin), 0, 63) : 0;
    }
    std::memcpy(out, &dh, 2);
    std::memcpy(out + 2, &mh, 2);
    std::uint8_t* s = out + 4;
    for (int j = 0; j < 4; ++j) {
        s[j] = static_cast<std::uint8_t>((sc[j] & 63) | ((sc[j + 4] >> 4) << 6));
        s[j + 4] = static_cast<std::uint8_t>((m[j] & 63) | ((m[j + 4] >> 4) << 6));
        s[j + 8] = static_cast<std::uint8_t>((sc[j + 4] & 15) | ((m[j + 4] & 15) << 4));
    }
    std::uint8_t q[256];
    for (int j = 0; j < 8; ++j) {
        const float ds = d * static_cast<float>(sc[j]), dm = dmin * static_cast<float>(m[j]);
        for (int i = 0; i < 32; ++i)
            q[32 * j + i] = static_cast<std::uint8_t>(ds > 0.f ? std::clamp(nearest((x[32 * j + i] + dm) / ds), 0, 15) : 0);
    }
    std::uint8_t* qs = out + 16;
    for (int c = 0; c < 4; ++c)
        for (int l = 0; l < 32; ++l) qs[32 * c + l] = static_cast<std::uint8_t>(q[64 * c + l] | (q[64 * c + 32 + l] << 4));
}

// Q6_K: 16 sub-blocks of 16, y = d*sc*(q-32), q in [0,63], sc int8.
void quant_q6_k(const float* x, std::uint8_t* out) {
    float scale[16];
    float max_scale = 0.f, max_abs = 0.f;
    for (int j = 0; j < 16; ++j) {
        float best = 0.f, bv = 0.f;
        for (int i = 0; i < 16; ++i) {
            const float v = x[16 * j + i];
            if (std::fabs(v) > best) {
                best = std::fabs(v);
                bv = v;
            }
        }
        scale[j] = bv / -32.f;  // the largest magnitude maps to q = -32 exactly
        if (std::fabs(scale[j]) > max_abs) {
            max_abs = std::fabs(scale[j]);
            max_scale = scale[j];
        }
    }
    const std::uint16_t dh = bt::fp32_to_fp16_bits(max_scale != 0.f ? max_scale / -128.f : 0.f);
    const float d = bt::fp16_bits_to_fp32(dh);
    std::int8_t sc[16];
    for (int j = 0; j < 16; ++j) sc[j] = static_cast<std::int8_t>(d != 0.f ? std::clamp(nearest(scale[j] / d), -128, 127) : 0);
    std::uint8_t Q[256];
    for (int j = 0; j < 16; ++j) {
        const float ds = d * static_cast<float>(sc[j]);
        for (int i = 0; i < 16; ++i)
            Q[16 * j + i] = static_cast<std::uint8_t>((ds != 0.f ? std::clamp(nearest(x[16 * j + i] / ds), -32, 31) : 0) + 32);
    }
    std::uint8_t* ql = out;
    std::uint8_t* qh = out + 128;
    for (int h = 0; h < 2; ++h) {
        const std::uint8_t* q = Q + 128 * h;
        for (int l = 0; l < 32; ++l) {
            ql[64 * h + l] = static_cast<std::uint8_t>((q[l] & 15) | ((q[l + 64] & 15) << 4));
            ql[64 * h + 32 + l] = static_cast<std::uint8_t>((q[l + 32] & 15) | ((q[l + 96] & 15) << 4));
            qh[32 * h + l] = static_cast<std::uint8_t>((q[l] >> 4) | ((q[l + 32] >> 4) << 2) | ((q[l + 64] >> 4) << 4) |
                                                       ((q[l + 96] >> 4) << 6));
        }
    }
    std::memcpy(out + 192, sc, 16);
    std::memcpy(out + 208, &dh, 2);
}

}  // namespace

std::uint64_t tensor_key(std::uint64_t seed, const std::string& name) {
    std::uint64_t h = 0xcbf29ce484222325ull;
    for (unsigned char c : name) {
        h ^= c;
        h *= 0x100000001b3ull;
    }
    return h ^ (seed * kGolden);
}

void normal_bf16(std::uint64_t key, std::int64_t n, float stddev, float* out) {
    parallel_for((n + 1) / 2, [&](std::int64_t b, std::int64_t e) {
        for (std::int64_t j = b; j < e; ++j) {
            const double u1 = (static_cast<double>(splitmix_at(key, 2 * j) >> 11) + 1.0) * 0x1p-53;
            const double u2 = static_cast<double>(splitmix_at(key, 2 * j + 1) >> 11) * 0x1p-53;
            const double r = std::sqrt(-2.0 * std::log(u1));
            const double a = 6.283185307179586476925286766559 * u2;
            const float z0 = static_cast<float>(stddev * r * std::cos(a));
            const float z1 = static_cast<float>(stddev * r * std::sin(a));
            out[2 * j] = bt::bf16_bits_to_fp32(bt::fp32_to_bf16_bits(z0));
            if (2 * j + 1 < n) out[2 * j + 1] = bt::bf16_bits_to_fp32(bt::fp32_to_bf16_bits(z1));
        }
    });
}

void quantize(bt::Dtype dt, const float* src, std::int64_t n, std::uint8_t* dst) {
    const std::int64_t be = bt::dtype_block_size(dt);
    if (n % be) throw std::runtime_error("synth::quantize: n not a multiple of the block size");
    const std::int64_t bb = bt::dtype_storage_bytes(dt, be);
    switch (dt) {
        case bt::Dtype::Q8_0:
            parallel_for(n / 32, [&](std::int64_t b, std::int64_t e) {
                for (std::int64_t i = b; i < e; ++i) quant_q8_0(src + 32 * i, dst + bb * i);
            });
            return;
        case bt::Dtype::Q4_K:
            parallel_for(n / 256, [&](std::int64_t b, std::int64_t e) {
                for (std::int64_t i = b; i < e; ++i) quant_q4_k(src + 256 * i, dst + bb * i);
            });
            return;
        case bt::Dtype::Q6_K:
            parallel_for(n / 256, [&](std::int64_t b, std::int64_t e) {
                for (std::int64_t i = b; i < e; ++i) quant_q6_k(src + 256 * i, dst + bb * i);
            });
            return;
        case bt::Dtype::FP16: {
            auto* d = reinterpret_cast<std::uint16_t*>(dst);
            for (std::int64_t i = 0; i < n; ++i) d[i] = bt::fp32_to_fp16_bits(src[i]);
            return;
        }
        case bt::Dtype::BF16: {
            auto* d = reinterpret_cast<std::uint16_t*>(dst);
            for (std::int64_t i = 0; i < n; ++i) d[i] = bt::fp32_to_bf16_bits(src[i]);
            return;
        }
        case bt::Dtype::FP32: std::memcpy(dst, src, static_cast<std::size_t>(n) * 4); return;
        default: throw std::runtime_error("synth::quantize: unsupported dtype");
    }
}

namespace {

// A byte-level BPE vocabulary for synthetic checkpoints: the 256 byte tokens
// (GPT-2 byte alphabet, id = byte), up to 256 merges learned greedily from a
// fixed English paragraph (most frequent adjacent pair first, ties to the
// smaller pair), the three ChatML specials (token type 3), then reserved
// fillers up to the model's vocab size.
const char kCorpus[] =
    "The quick brown fox jumps over the lazy dog while the model reads the tokens of the prompt. "
    "A decoder turns the hidden state into logits, and the sampler picks the next token from them. "
    "In the beginning there was the word, and the word was split into pieces, and the pieces were merged "
    "again by the rules that were learned from the text. Numbers such as 2024, 128 and 4096 appear too. "
    "She said that they're going to the station, but we'll see whether it's true. "
    "Weights are stored in blocks; each block keeps its scale and its small integers. "
    "The cache holds the keys and the values of every position, so that attention can look back.";

struct SynthVocab {
    std::vector<std::string> tokens, merges;
    std::vector<std::int32_t> types;
};

std::string byte_symbol(unsigned char b) {
    int next = 256;
    auto self = [](int x) { return (x >= 33 && x <= 126) || (x >= 161 && x <= 172) || (x >= 174 && x <= 255); };
    for (int i = 0; i < b; ++i)
        if (!self(i)) ++next;
    const unsigned cp = self(b) ? b : static_cast<unsigned>(next);
    std::string out;
    if (cp < 0x80) {
        out += static_cast<char>(cp);
    } else {
        out += static_cast<char>(0xC0 | (cp >> 6));
        out += static_cast<char>(0x80 | (cp & 0x3F));
    }
    return out;
}

SynthVocab synth_vocab(int vocab) {
    SynthVocab v;
    for (int b = 0; b < 256; ++b) {
        v.tokens.push_back(byte_symbol(static_cast<unsigned char>(b)));
        v.types.push_back(1);
    }
    // words: letter runs with one folded leading space, other bytes alone
    std::vector<std::vector<std::string>> words;
    const std::string text(kCorpus);
    for (std::size_t i = 0; i < text.size();) {
        std::size_t j = i;
        if (text[j] == ' ' && j + 1 < text.size()) ++j;
        const bool alpha = std::isalpha(static_cast<unsigned char>(text[j])) != 0;
        if (alpha)
            while (j < text.size() && std::isalpha(static_cast<unsigned char>(text[j]))) ++j;
        else
            ++j;
        std::vector<std::string> w;
        for (std::size_t k = i; k < j; ++k) w.push_back(byte_symbol(static_cast<unsigned char>(text[k])));
        words.push_back(std::move(w));
        i = j;
    }
    const int max_merges = std::min(256, vocab - 256 - 3);
    for (int m = 0; m < max_merges; ++m) {
        std::map<std::pair<std::string, std::string>, int> counts;
        for (const auto& w : words)
            for (std::size_t k = 0; k + 1 < w.size(); ++k) ++counts[{w[k], w[k + 1]}];
        const std::pair<std::string, std::string>* best = nullptr;
        int best_n = 1;
        for (const auto& [pair, n] : counts)
            if (n > best_n) {   // map order: ties keep the smaller pair
                best_n = n;
                best = &pair;
            }
        if (!best) break;
        const std::string a = best->first, b = best->second;
        v.merges.push_back(a + " " + b);
        v.tokens.push_back(a + b);
        v.types.push_back(1);
        for (auto& w : words) {
            std::vector<std::string> nw;
            for (std::size_t k = 0; k < w.size();) {
                if (k + 1 < w.size() && w[k] == a && w[k + 1] == b) {
                    nw.push_back(a + b);
                    k += 2;
                } else {
                    nw.push_back(w[k++]);
                }
            }
            w = std::move(nw);
        }
    }
    for (const char* sp : {"<|endoftext|>", "<|im_start|>", "<|im_end|>"}) {
        v.tokens.push_back(sp);
        v.types.push_back(3);
    }
    for (int i = 0; static_cast<int>(v.tokens.size()) < vocab; ++i) {
        v.tokens.push_back("<|reserved_" + std::to_string(i) + "|>");
        v.types.push_back(1);
    }
    return v;
}

}  // namespace

bool use_more_bits(int i_layer, int n_layers) {
    const int e = n_layers / 8;
    return i_layer < e || i_layer >= 7 * n_layers / 8 || (i_layer - e) % 3 == 2;
}

std::vector<std::uint8_t> make_qwen3_gguf(const Qwen3Spec& s) {
    if (s.hidden <= 0 || s.intermediate <= 0 || s.layers <= 0 || s.vocab <= 0 || s.n_q <= 0 || s.n_kv <= 0 ||
        s.head_dim <= 0)
        throw std::runtime_error("synth: non-positive dimension");
    if (s.arch.empty()) throw std::runtime_error("synth: empty architecture name");
    const bool qk_norm = s.arch == "qwen3";
    const std::string a = s.arch + ".";
    bt::gguf::Writer w;
    w.add_string("general.architecture", s.arch);
    w.add_string("general.name", "brolm-synthetic-" + s.arch);
    w.add_u32(a + "embedding_length", static_cast<std::uint32_t>(s.hidden));
    w.add_u32(a + "feed_forward_length", static_cast<std::uint32_t>(s.intermediate));
    w.add_u32(a + "block_count", static_cast<std::uint32_t>(s.layers));
    w.add_u32(a + "attention.head_count", static_cast<std::uint32_t>(s.n_q));
    w.add_u32(a + "attention.head_count_kv", static_cast<std::uint32_t>(s.n_kv));
    w.add_u32(a + "attention.key_length", static_cast<std::uint32_t>(s.head_dim));
    w.add_u32(a + "attention.value_length", static_cast<std::uint32_t>(s.head_dim));
    w.add_f32(a + "attention.layer_norm_rms_epsilon", s.eps);
    w.add_f32(a + "rope.freq_base", s.theta);
    w.add_u32(a + "context_length", static_cast<std::uint32_t>(s.context));
    w.add_u32(a + "vocab_size", static_cast<std::uint32_t>(s.vocab));
    if (s.vocab >= 256 + 3) {
        const SynthVocab tv = synth_vocab(s.vocab);
        w.add_string("tokenizer.ggml.model", "gpt2");
        w.add_string("tokenizer.ggml.pre", "qwen2");
        w.add_string_array("tokenizer.ggml.tokens", tv.tokens);
        w.add_i32_array("tokenizer.ggml.token_type", tv.types);
        w.add_string_array("tokenizer.ggml.merges", tv.merges);
        const auto id_of = [&](const char* t) {
            return static_cast<std::uint32_t>(std::find(tv.tokens.begin(), tv.tokens.end(), t) - tv.tokens.begin());
        };
        w.add_u32("tokenizer.ggml.eos_token_id", id_of("<|im_end|>"));
        w.add_u32("tokenizer.ggml.padding_token_id", id_of("<|endoftext|>"));
    }

    struct Item {
        std::string name;
        bt::Dtype dt;
        std::int64_t rows, cols;
        bool gamma;
    };
    std::vector<Item> items;
    const std::int64_t H = s.hidden, F = s.intermediate, qd = s.n_q * s.head_dim, kvd = s.n_kv * s.head_dim;
    items.push_back({"token_embd.weight", s.embed, s.vocab, H, false});
    for (int l = 0; l < s.layers; ++l) {
        const std::string p = "blk." + std::to_string(l) + ".";
        items.push_back({p + "attn_norm.weight", bt::Dtype::FP32, 1, H, true});
        items.push_back({p + "attn_q.weight", s.q, qd, H, false});
        items.push_back({p + "attn_k.weight", s.k, kvd, H, false});
        const bool more = s.more_bits_type >= 0 && use_more_bits(l, s.layers);
        const bt::Dtype vt = more ? bt::dtype_from_ggml(s.more_bits_type) : s.v;
        const bt::Dtype dt = more ? bt::dtype_from_ggml(s.more_bits_type) : s.down;
        items.push_back({p + "attn_v.weight", vt, kvd, H, false});
        items.push_back({p + "attn_output.weight", s.o, H, qd, false});
        if (qk_norm) {
            items.push_back({p + "attn_q_norm.weight", bt::Dtype::FP32, 1, s.head_dim, true});
            items.push_back({p + "attn_k_norm.weight", bt::Dtype::FP32, 1, s.head_dim, true});
        }
        items.push_back({p + "ffn_norm.weight", bt::Dtype::FP32, 1, H, true});
        items.push_back({p + "ffn_gate.weight", s.gate, F, H, false});
        items.push_back({p + "ffn_up.weight", s.up, F, H, false});
        items.push_back({p + "ffn_down.weight", dt, H, F, false});
    }
    items.push_back({"output_norm.weight", bt::Dtype::FP32, 1, H, true});
    if (!s.tied) items.push_back({"output.weight", s.output, s.vocab, H, false});

    for (const Item& it : items) {
        if (it.gamma) w.add_tensor_placeholder(it.name, it.dt, {it.cols});
        else w.add_tensor_placeholder(it.name, it.dt, {it.cols, it.rows});
    }
    std::vector<std::size_t> offs;
    std::vector<std::uint8_t> bytes = w.to_bytes(&offs);
    std::vector<float> buf;
    for (std::size_t i = 0; i < items.size(); ++i) {
        const Item& it = items[i];
        const std::int64_t n = it.rows * it.cols;
        buf.resize(static_cast<std::size_t>(n));
        if (it.gamma) std::fill(buf.begin(), buf.end(), 1.0f);
        else normal_bf16(tensor_key(s.seed, it.name), n, s.stddev, buf.data());
        quantize(it.dt, buf.data(), n, bytes.data() + offs[i]);
    }
    return bytes;
}

void write_qwen3_gguf(const Qwen3Spec& spec, const std::string& path) {
    const std::vector<std::uint8_t> b = make_qwen3_gguf(spec);
    std::ofstream f(path, std::ios::binary | std::ios::trunc);
    if (!f) throw std::runtime_error("synth: cannot write '" + path + "'");
    f.write(reinterpret_cast<const char*>(b.data()), static_cast<std::streamsize>(b.size()));
    if (!f) throw std::runtime_error("synth: short write to '" + path + "'");
}

void write_mistral3_gguf(Qwen3Spec spec, const std::string& path) {
    spec.arch = "llama";
    write_qwen3_gguf(spec, path);
}

}  // namespace brolm::synth
