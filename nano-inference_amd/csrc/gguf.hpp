// gguf.hpp -- GGUF v3 model-file reader for the engine host.
//
// Same file semantics as the reference loader src/gguf.h:19-222: little-endian
// header, metadata key/values (numbers kept as double, the token list kept),
// tensor infos, tensor data starting at the first multiple of
// general.alignment (default 32) after the infos (:215-217), ne[0] = row length
// (:56), q4_0 block = fp16 d + 16 bytes (:29, 94-101). Differences that a
// library needs: the file is mmapped read-only and every failure is reported as
// a status + message instead of exit(1) (gguf.h:33, 79, 185-192).
#pragma once
#include <cstdint>
#include <string>
#include <unordered_map>
#include <vector>

namespace mi {

enum GType : uint32_t { GT_F32 = 0, GT_F16 = 1, GT_Q4_0 = 2, GT_Q4_1 = 3, GT_Q8_0 = 8, GT_Q6_K = 14 };
// the tensor types the loader reads (gguf.h:22-35 lists the same set)
inline bool gtype_known(uint32_t t) {
    return t == GT_F32 || t == GT_F16 || t == GT_Q4_0 || t == GT_Q4_1 || t == GT_Q8_0 || t == GT_Q6_K;
}

struct GTensor {
    uint32_t type = 0;
    std::vector<int64_t> ne;
    const uint8_t* data = nullptr;
    uint64_t offset = 0;
    int64_t rows() const { int64_t r = 1; for (size_t i = 1; i < ne.size(); i++) r *= ne[i]; return r; }
    int64_t cols() const { return ne.empty() ? 0 : ne[0]; }
    size_t nbytes() const;
};

class GGUFFile {
public:
    GGUFFile() = default;
    ~GGUFFile();
    GGUFFile(const GGUFFile&) = delete;
    GGUFFile& operator=(const GGUFFile&) = delete;

    // returns false and sets error() on any failure
    bool open(const std::string& path);
    const std::string& error() const { return err_; }

    double num(const std::string& key, double def) const;
    bool has_num(const std::string& key) const { return num_.count(key) > 0; }
    const std::string& str(const std::string& key) const;
    const std::vector<std::string>& tokens() const { return tokens_; }
    const GTensor* tensor(const std::string& name) const;
    // drop the mmapped pages of a tensor once it has been uploaded
    void release(const GTensor& t) const;

private:
    bool parse();
    bool read_value(uint32_t vt, const std::string& key, bool store);
    int fd_ = -1;
    size_t size_ = 0;
    const uint8_t* base_ = nullptr;
    const uint8_t* cur_ = nullptr;
    const uint8_t* end_ = nullptr;
    std::string err_;
    std::unordered_map<std::string, double> num_;
    std::unordered_map<std::string, std::string> str_;
    std::vector<std::string> tokens_;
    std::unordered_map<std::string, GTensor> tensors_;
};

float f16_to_f32(uint16_t h);
uint16_t f32_to_f16(float f);

}  // namespace mi
