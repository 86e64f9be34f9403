// teacher.cpp -- the exactness hash of teacher-forced runs (mega.cu:1197-1201). Host code.
#include "minfer.h"

#include <cstring>

extern "C" uint64_t mi_fnv1a64(const void* data, size_t n, uint64_t basis) {
    const unsigned char* p = static_cast<const unsigned char*>(data);
    uint64_t h = basis;
    for (size_t i = 0; i < n; i++) {
        h ^= p[i];
        h *= 1099511628211ull;
    }
    return h;
}

// FNV-1a over (token, margin bits) per position, each 32-bit value byte by byte from the
// low byte up, from the offset basis mega.cu:1197 uses
extern "C" uint64_t mi_pred_hash(const int32_t* pred, const float* margin, int32_t n) {
    uint64_t h = 1469598103934665603ull;
    if (!pred || !margin) return h;
    for (int32_t i = 0; i < n; i++) {
        uint32_t v[2];
        v[0] = (uint32_t)pred[i];
        std::memcpy(&v[1], &margin[i], 4);
        for (uint32_t w : v) {
            unsigned char b[4] = {(unsigned char)w, (unsigned char)(w >> 8), (unsigned char)(w >> 16),
                                  (unsigned char)(w >> 24)};
            h = mi_fnv1a64(b, 4, h);
        }
    }
    return h;
}
