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

// Draft length K in 0..tmax-1 that maximises the expected tokens per unit of step
// cost when each draft is accepted with probability alpha: E(K) = (1-alpha^(K+1)) /
// (1-alpha) tokens for a step costing 1 + slope*K single-token steps. K = 0 scores 1.
int32_t mi_best_draft_len(float alpha, float slope, int32_t tmax) {
    int kb = 0;
    float vb = 1.f, pw = alpha;
    for (int K = 1; K < tmax; K++) {
        pw *= alpha;   // alpha^(K+1)
        const float v = (1.f - pw) / (1.f - alpha) / (1.f + slope * K);
        if (v > vb) { vb = v; kb = K; }
    }
    return kb;
}

}  // extern "C"
