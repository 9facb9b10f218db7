// Arguments of the split-K attention kernels (attention.hip) and the MFMA
// flash-attention entry (attention_mfma.hip).
#pragma once

#include "common.h"

namespace bx {

constexpr int kAttnMaxGroup = 8;   // query heads per KV head

struct AttnArgs {
    const uint16_t* q;
    const uint16_t* Kc;
    const uint16_t* Vc;
    const float* mask;  // optional: keys with mask[j] == 0 are skipped
    int L, valid_len, n_q, n_kv, hd;
    float softcap;
    int window;
    int kps, S;
    float* ws;  // partials [L][n_q][S][hd + 2]
    int bidir;  // 1: every row attends all valid_len keys (no causal limit)
    // per-row key ranges (batched decode of independent sequences): row r
    // attends cache rows rbase[r] .. rbase[r] + rlen[r] - 1; null otherwise
    const int32_t* rlen;
    const int64_t* rbase;
};

// Flash attention on MFMA for L >= 16 query rows (attention_mfma.hip): head
// dims 64 and 128, no softcap / window / key mask.
bool attn_mfma_supported(int L, int hd, float softcap, int window, const float* mask);
int attn_mfma(const uint16_t* q, const uint16_t* Kc, const uint16_t* Vc, int L, int valid_len, int n_q, int n_kv,
              int hd, int bidir, uint16_t* out, hipStream_t st);

}  // namespace bx
