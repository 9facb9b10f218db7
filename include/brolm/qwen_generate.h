#pragma once

// Qwen3 generation binding (reference include/brolm/qwen_generate.h:45-53).
// generate_text needs the Qwen tokenizer, which is outside this build's scope.

#include <cstdint>
#include <vector>

#include "brolm/detail/generate.h"
#include "brolm/qwen.h"

namespace brolm::qwen {

using SamplingParams = brolm::detail::SamplingParams;
using GenerateOptions = brolm::detail::GenerateOptions;
using brolm::detail::sample_token;

std::vector<int32_t> generate(Qwen3Model& model, const std::vector<int32_t>& prompt_ids, int eos_id,
                              const GenerateOptions& opts);

}  // namespace brolm::qwen
