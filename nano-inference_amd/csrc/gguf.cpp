// gguf.cpp -- see gguf.hpp. Reference: src/gguf.h:19-222.
#include "gguf.hpp"

#include <cstring>
#include <fcntl.h>
#include <sys/mman.h>
#include <sys/stat.h>
#include <unistd.h>

namespace mi {

size_t GTensor::nbytes() const {
    const int64_t c = cols(), r = rows();
    switch (type) {
        case GT_F32: return (size_t)(c * r) * 4;
        case GT_F16: return (size_t)(c * r) * 2;
        case GT_Q4_0: return (size_t)(c / 32 * r) * 18;
        case GT_Q4_1: return (size_t)(c / 32 * r) * 20;
        case GT_Q8_0: return (size_t)(c / 32 * r) * 34;
        case GT_Q6_K: return (size_t)(c / 256 * r) * 210;
        default: return 0;
    }
}

GGUFFile::~GGUFFile() {
    if (base_) munmap(const_cast<uint8_t*>(base_), size_);
    if (fd_ >= 0) close(fd_);
}

bool GGUFFile::open(const std::string& path) {
    fd_ = ::open(path.c_str(), O_RDONLY);
    if (fd_ < 0) { err_ = "cannot open " + path; return false; }
    struct stat st;
    if (fstat(fd_, &st) != 0) { err_ = "cannot stat " + path; return false; }
    size_ = (size_t)st.st_size;
    void* p = mmap(nullptr, size_, PROT_READ, MAP_PRIVATE, fd_, 0);
    if (p == MAP_FAILED) { err_ = "mmap failed for " + path; return false; }
    base_ = (const uint8_t*)p; cur_ = base_; end_ = base_ + size_;
    return parse();
}

#define NEED(n) do { if ((size_t)(end_ - cur_) < (size_t)(n)) { err_ = "truncated GGUF"; return false; } } while (0)
#define RD(T, out) do { NEED(sizeof(T)); memcpy(&(out), cur_, sizeof(T)); cur_ += sizeof(T); } while (0)

bool GGUFFile::read_value(uint32_t vt, const std::string& key, bool store) {
    double v = 0;
    switch (vt) {
        case 0: { uint8_t x; RD(uint8_t, x); v = x; break; }
        case 1: { int8_t x; RD(int8_t, x); v = x; break; }
        case 2: { uint16_t x; RD(uint16_t, x); v = x; break; }
        case 3: { int16_t x; RD(int16_t, x); v = x; break; }
        case 4: { uint32_t x; RD(uint32_t, x); v = x; break; }
        case 5: { int32_t x; RD(int32_t, x); v = x; break; }
        case 6: { float x; RD(float, x); v = x; break; }
        case 7: { uint8_t x; RD(uint8_t, x); v = x; break; }
        case 10: { uint64_t x; RD(uint64_t, x); v = (double)x; break; }
        case 11: { int64_t x; RD(int64_t, x); v = (double)x; break; }
        case 12: { double x; RD(double, x); v = x; break; }
        case 8: {
            uint64_t n; RD(uint64_t, n); NEED(n);
            if (store) str_[key] = std::string((const char*)cur_, n);
            cur_ += n;
            return true;
        }
        case 9: {
            uint32_t et; uint64_t n;
            RD(uint32_t, et); RD(uint64_t, n);
            const bool keep = store && key == "tokenizer.ggml.tokens" && et == 8;
            if (keep) tokens_.reserve(n);
            for (uint64_t i = 0; i < n; i++) {
                if (et == 8) {
                    uint64_t sl; RD(uint64_t, sl); NEED(sl);
                    if (keep) tokens_.emplace_back((const char*)cur_, sl);
                    cur_ += sl;
                } else if (!read_value(et, std::string(), false)) return false;
            }
            return true;
        }
        default: err_ = "bad GGUF metadata type " + std::to_string(vt); return false;
    }
    if (store) num_[key] = v;
    return true;
}

bool GGUFFile::parse() {
    uint32_t magic, version; uint64_t n_t, n_kv;
    RD(uint32_t, magic);
    if (magic != 0x46554747u) { err_ = "not a GGUF file"; return false; }
    RD(uint32_t, version);
    if (version < 2 || version > 3) { err_ = "unsupported GGUF version " + std::to_string(version); return false; }
    RD(uint64_t, n_t); RD(uint64_t, n_kv);
    for (uint64_t i = 0; i < n_kv; i++) {
        uint64_t kl; RD(uint64_t, kl); NEED(kl);
        std::string key((const char*)cur_, kl); cur_ += kl;
        uint32_t vt; RD(uint32_t, vt);
        if (!read_value(vt, key, true)) return false;
    }
    std::vector<std::pair<std::string, GTensor>> infos;
    for (uint64_t i = 0; i < n_t; i++) {
        uint64_t nl; RD(uint64_t, nl); NEED(nl);
        std::string name((const char*)cur_, nl); cur_ += nl;
        uint32_t nd; RD(uint32_t, nd);
        if (nd < 1 || nd > 4) { err_ = "bad tensor rank for " + name; return false; }
        GTensor t; t.ne.resize(nd);
        for (uint32_t d = 0; d < nd; d++) { uint64_t e; RD(uint64_t, e); t.ne[d] = (int64_t)e; }
        RD(uint32_t, t.type);
        RD(uint64_t, t.offset);
        infos.emplace_back(std::move(name), std::move(t));
    }
    const uint64_t align = (uint64_t)num("general.alignment", 32);
    if (align == 0) { err_ = "bad alignment"; return false; }
    const size_t pos = (size_t)(cur_ - base_), start = (pos + align - 1) / align * align;
    for (auto& kv : infos) {
        GTensor& t = kv.second;
        t.data = base_ + start + t.offset;
        const size_t nb = t.nbytes();
        if (!gtype_known(t.type)) {
            // kept (a model may carry tensors the engine never reads); size unknown
        } else if (start + t.offset + nb > size_) {
            err_ = "tensor " + kv.first + " runs past the end of the file"; return false;
        }
        tensors_.emplace(kv.first, t);
    }
    return true;
}

double GGUFFile::num(const std::string& key, double def) const {
    auto it = num_.find(key); return it == num_.end() ? def : it->second;
}
const std::string& GGUFFile::str(const std::string& key) const {
    static const std::string empty;
    auto it = str_.find(key); return it == str_.end() ? empty : it->second;
}
const GTensor* GGUFFile::tensor(const std::string& name) const {
    auto it = tensors_.find(name); return it == tensors_.end() ? nullptr : &it->second;
}
void GGUFFile::release(const GTensor& t) const {
    if (!t.data) return;
    const long ps = sysconf(_SC_PAGESIZE);
    const uintptr_t a = (uintptr_t)t.data, s = a & ~(uintptr_t)(ps - 1);
    madvise((void*)s, (a - s) + t.nbytes(), MADV_DONTNEED);
}

float f16_to_f32(uint16_t h) {
    uint32_t sign = (uint32_t)(h & 0x8000) << 16, ex = (h >> 10) & 0x1F, mant = h & 0x3FF, f;
    if (ex == 0) {
        if (mant == 0) f = sign;
        else {
            int e = -14;
            while ((mant & 0x400) == 0) { mant <<= 1; e--; }
            f = sign | ((uint32_t)(e + 127) << 23) | ((mant & 0x3FF) << 13);
        }
    } else if (ex == 0x1F) f = sign | 0x7F800000u | (mant << 13);
    else f = sign | ((ex + 112) << 23) | (mant << 13);
    float out; memcpy(&out, &f, 4); return out;
}

uint16_t f32_to_f16(float v) {
    uint32_t x; memcpy(&x, &v, 4);
    const uint32_t sign = (x >> 16) & 0x8000u, ex = (x >> 23) & 0xFF, mant = x & 0x7FFFFFu;
    if (ex == 0xFF) return (uint16_t)(sign | 0x7C00u | (mant ? 0x200u : 0));
    const int e = (int)ex - 112;
    if (e >= 31) return (uint16_t)(sign | 0x7C00u);
    if (e <= 0) {
        if (e < -10) return (uint16_t)sign;
        const uint32_t m = mant | 0x800000u;
        const int sh = 14 - e;
        uint32_t q = m >> sh;
        const uint32_t rem = m & ((1u << sh) - 1), half = 1u << (sh - 1);
        if (rem > half || (rem == half && (q & 1))) q++;
        return (uint16_t)(sign | q);
    }
    uint32_t q = ((uint32_t)e << 10) | (mant >> 13);
    const uint32_t rem = mant & 0x1FFFu;
    if (rem > 0x1000u || (rem == 0x1000u && (q & 1))) q++;
    return (uint16_t)(sign | q);
}

}  // namespace mi
