// spec.cpp -- host side of lossless speculative decoding: the n-gram (prompt
// lookup) drafter and the draft-length rule (reference: mega.cu:557-589 ngram_draft /
// best_draft_len, the acceptance EWMA :613, 877-880; cuda_infer.cu:1212-1225 is the
// fixed-n host variant). Plain C++; the engine calls these between verify steps.
#include "minfer.h"

#include <algorithm>
#include <cstdint>

extern "C" {

// Draft up to kmax tokens for the history h[0..len): for n = ngmax down to 1, find
// the latest earlier start j (j + n < len) where h[j..j+n) equals the last n tokens,
// and propose the tokens that followed it, h[j+n .. j+n+K), K = min(kmax, len-j-n).
// Returns K (0: no match of any length, or kmax <= 0).
int32_t mi_ngram_draft(const int32_t* h, int32_t len, int32_t ngmax, int32_t kmax, int32_t* out) {
    if (!h || !out || kmax <= 0) return 0;
    for (int n = ngmax; n >= 1; n--) {
        if (len < n + 1) continue;
        const int32_t* suf = h + len - n;
        for (int j = len - n - 1; j >= 0; j--) {
            if (!std::equal(suf, suf + n, h + j)) continue;
            const int K = std::min<int>(kmax, len - (j + n));
            for (int k = 0; k < K; k++) out[k] = h[j + n + k];
            return K;
        }
    }
    return 0;
}

// Draft length for the next verify step. A step that carries k drafts costs 1 + slope*k
// single-token steps and, when each draft survives with probability alpha independently,
// yields (1 - alpha^(k+1)) / (1 - alpha) tokens on average (the accepted prefix plus the
// correction). Returns the k in 0..tmax-1 with the highest yield per unit of cost; k = 0
// (a plain step) yields exactly one token per unit, and a larger k must beat the best so
// far strictly. alpha^(k+1) is built by repeated multiplication, so the choice matches
// the reference's rule (mega.cu:581-589) float for float.
int32_t mi_best_draft_len(float alpha, float slope, int32_t tmax) {
    int32_t best_k = 0;
    float best_rate = 1.f;
    float all_accepted = alpha;                    // alpha^(k+1) once updated for k
    for (int32_t k = 1; k < tmax; ++k) {
        all_accepted *= alpha;
        const float expected_tokens = (1.f - all_accepted) / (1.f - alpha);
        const float rate = expected_tokens / (1.f + slope * k);
        if (rate > best_rate) {
            best_rate = rate;
            best_k = k;
        }
    }
    return best_k;
}

}  // extern "C"
