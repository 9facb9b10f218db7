#pragma once

// Qwen3 generation binding (reference include/brolm/qwen_generate.h:45-53).

#include <cstdint>
#include <string>
#include <string_view>
#include <vector>

#include "brolm/detail/generate.h"
#include "brolm/qwen.h"
#include "brolm/qwen_tokenizer.h"

namespace brolm::qwen {

using SamplingParams = brolm::detail::SamplingParams;
using GenerateOptions = brolm::detail::GenerateOptions;
using brolm::detail::sample_token;

std::vector<int32_t> generate(Qwen3Model& model, const std::vector<int32_t>& prompt_ids, int eos_id,
                              const GenerateOptions& opts);

// Text in, text out: encode(prompt) -> generate (stop token tok.eos_id()) ->
// decode of the new ids only (reference src/qwen_generate.cpp:19-25).
std::string generate_text(Qwen3Model& model, const Tokenizer& tok, std::string_view prompt,
                          const GenerateOptions& opts);

}  // namespace brolm::qwen
