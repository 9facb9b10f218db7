#pragma once

// Mistral 3.1 generation binding (reference include/brolm/mistral3_generate.h:40-43):
// sizes and resets the KV cache for prompt + max_new_tokens, prefills the
// prompt in one forward, then decodes; returns only the new ids, without the
// stop token.  generate_text (:52-54) needs the Tekken tokenizer, which this
// build does not carry.

#include <cstdint>
#include <vector>

#include "brolm/detail/generate.h"
#include "brolm/mistral3_text.h"

namespace brolm::mistral3 {

using GenerateOptions = brolm::detail::GenerateOptions;

std::vector<int32_t> generate(TextModel& model, const std::vector<int32_t>& prompt_ids, int eos_id,
                              const GenerateOptions& opts);

}  // namespace brolm::mistral3
