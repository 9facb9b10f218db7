#pragma once

// Synthetic Qwen3 GGUF checkpoints for benchmarks and parity tests (no network,
// no real weights).  Every linear weight is drawn N(0, stddev) from a
// counter-based splitmix64 stream keyed by (seed, tensor name), Box-Muller in
// double, rounded to BF16 (RNE), then stored as the requested GGUF type.
// Norm gammas are 1 (F32).
//
// The quantizers here are this project's own (round-to-nearest per block with
// the ggml block layouts); they are not ggml's iterative quantizers.  They
// only produce inputs: parity is checked on the dequantized values of the
// blocks they write.

#include <cstdint>
#include <string>
#include <vector>

#include "brotensor/tensor.h"

namespace brolm::synth {

struct Qwen3Spec {
    int vocab = 151936;
    int hidden = 1024;
    int intermediate = 3072;
    int layers = 28;
    int n_q = 16;
    int n_kv = 8;
    int head_dim = 128;
    float eps = 1e-6f;
    float theta = 1000000.0f;
    int context = 40960;
    bool tied = true;  // no output.weight
    brotensor::Dtype embed = brotensor::Dtype::Q8_0;
    brotensor::Dtype q = brotensor::Dtype::Q8_0, k = brotensor::Dtype::Q8_0, v = brotensor::Dtype::Q8_0,
                     o = brotensor::Dtype::Q8_0;
    brotensor::Dtype gate = brotensor::Dtype::Q8_0, up = brotensor::Dtype::Q8_0, down = brotensor::Dtype::Q8_0;
    brotensor::Dtype output = brotensor::Dtype::Q6_K;
    float stddev = 0.02f;
    std::uint64_t seed = 0;
    // general.architecture and metadata-key prefix.  "qwen3" writes per-head
    // attn_q_norm / attn_k_norm gammas; any other name ("llama", the arch
    // llama.cpp gives Mistral text models) writes none (no QK-norm).
    std::string arch = "qwen3";
    // ggml type id written for attn_v and ffn_down on the layers llama.cpp's
    // Q4_K_M recipe gives more bits (use_more_bits: the first and last eighth
    // of the layers and every third layer between), or -1 for none: the
    // per-layer format mix of a real Q4_K_M file (base type from v / down).
    int more_bits_type = -1;
};

// llama.cpp's layer rule for the larger attn_v / ffn_down type of its _M
// mixes: i < n/8, i >= 7n/8, or (i - n/8) % 3 == 2.
bool use_more_bits(int i_layer, int n_layers);

// Key of a tensor's random stream: seed mixed with the FNV-1a hash of its name.
std::uint64_t tensor_key(std::uint64_t seed, const std::string& name);
// out[i] = bf16(stddev * z_i), z the i-th standard normal of stream `key`.
void normal_bf16(std::uint64_t key, std::int64_t n, float stddev, float* out);
// Quantize n values (multiple of the block size) into GGUF blocks of `dt`
// (Q8_0, Q4_K, Q6_K, or dense FP16 / BF16 / FP32).
void quantize(brotensor::Dtype dt, const float* src, std::int64_t n, std::uint8_t* dst);

std::vector<std::uint8_t> make_qwen3_gguf(const Qwen3Spec& spec);
void write_qwen3_gguf(const Qwen3Spec& spec, const std::string& path);
// Mistral 3.1 text checkpoint: the same tensors under arch "llama", no
// QK-norm gammas; untied when spec.tied is false (output.weight present).
void write_mistral3_gguf(Qwen3Spec spec, const std::string& path);

}  // namespace brolm::synth
