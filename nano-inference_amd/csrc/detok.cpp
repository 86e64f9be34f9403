// detok.cpp -- byte-level BPE detokenizer for Qwen2/GPT-2 vocabularies (reference:
// src/detok.h:13-41). A vocab piece is the UTF-8 of code points that stand for bytes:
// the printable bytes '!'..'~', 0xA1..0xAC and 0xAE..0xFF stand for themselves, the
// other 68 bytes (0x00..0x20, 0x7F..0xA0, 0xAD) for 256, 257, ... in increasing byte
// order. Decoding maps each code point back to its byte; code points outside that map
// and malformed lead bytes are dropped, as the reference does.
#include "minfer.h"

#include <cstdint>

namespace {

// byte for code point cp, or -1
int cp_byte(uint32_t cp) {
    auto printable = [](uint32_t b) { return (b >= 0x21 && b <= 0x7E) || (b >= 0xA1 && b <= 0xAC) || (b >= 0xAE && b <= 0xFF); };
    if (cp < 256) return printable(cp) ? (int)cp : -1;
    // the k-th non-printable byte (k = cp - 256) in increasing order
    uint32_t k = cp - 256;
    for (uint32_t b = 0; b < 256; b++) {
        if (printable(b)) continue;
        if (k == 0) return (int)b;
        k--;
    }
    return -1;
}

}  // namespace

extern "C" {

// Decode `len` bytes of a vocab piece into out[0..cap). Returns the number of decoded
// bytes (which may exceed cap: only the first cap are written), or -1 on bad arguments.
int32_t mi_detok_piece(const char* piece, int32_t len, char* out, int32_t cap) {
    if (!piece || len < 0 || cap < 0 || (cap > 0 && !out)) return -1;
    const unsigned char* s = reinterpret_cast<const unsigned char*>(piece);
    int32_t n = 0;
    for (int32_t i = 0; i < len;) {
        const unsigned c = s[i];
        uint32_t cp;
        int l;
        if (c < 0x80) { cp = c; l = 1; }
        else if ((c >> 5) == 0x6) { cp = c & 0x1F; l = 2; }
        else if ((c >> 4) == 0xE) { cp = c & 0x0F; l = 3; }
        else if ((c >> 3) == 0x1E) { cp = c & 0x07; l = 4; }
        else { i++; continue; }
        for (int k = 1; k < l && i + k < len; k++) cp = (cp << 6) | (s[i + k] & 0x3F);
        i += l;
        const int b = cp_byte(cp);
        if (b < 0) continue;
        if (n < cap) out[n] = (char)b;
        n++;
    }
    return n;
}

}  // extern "C"
