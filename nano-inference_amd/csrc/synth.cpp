// synth.cpp -- seeded random-init Qwen2-architecture GGUF writer.
//
// Writes exactly what the reference loaders read (cpu_infer.cpp:70-98,
// mega.cu:1010-1014, 1068-1112): the qwen2.* shape keys, a GPT-2 style token
// list whose length is n_vocab (cpu_infer.cpp:79), tokenizer.ggml.eos_token_id,
// token_embd.weight, output_norm.weight, output.weight and the per-layer
// attention/FFN tensors with q/k/v biases. Distributions:
// q4_0 matrices with uniform nibbles 0..15 and fp16 |N(0, 0.002)| scales; norms,
// biases and the embedding fp32 N(0, 0.02). Two optional knobs (off in every BASELINE
// config) make attention matter: q/k biases N(0, qk_bias_std) and norm weights
// norm_offset + N(0, 0.02), which give O(1) attention scores that depend on the
// relative position, so a RoPE or head-mapping mistake changes the output.
//
// Determinism: every tensor is cut into fixed segments, each filled from its own
// splitmix64 stream keyed by (seed, tensor index, segment index), and normals come
// from Box-Muller with log/sin/cos evaluated by series in plain double arithmetic
// (no libm), so the same binary writes the same bytes on any x86-64 host and for
// any thread count.
#include "gguf.hpp"
#include "minfer.h"

#include <algorithm>
#include <cmath>
#include <cstdio>
#include <cstring>
#include <string>
#include <thread>
#include <vector>

namespace {

inline uint64_t mix64(uint64_t z) {
    z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
    z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
    return z ^ (z >> 31);
}
struct Rng {
    uint64_t s;
    explicit Rng(uint64_t seed) : s(seed) {}
    uint64_t next() { s += 0x9E3779B97F4A7C15ull; return mix64(s); }
    double unit() { return (double)(next() >> 11) * (1.0 / 9007199254740992.0); }   // [0, 1)
};

// ln(x) for x in (0, 1]: x = m 2^e, m in [sqrt(.5), sqrt(2)), ln m = 2 atanh((m-1)/(m+1))
double det_log(double x) {
    int e = 0;
    double m = std::frexp(x, &e);
    if (m < 0.70710678118654752) { m *= 2.0; e -= 1; }
    const double s = (m - 1.0) / (m + 1.0), s2 = s * s;
    double term = s, sum = 0.0;
    for (int k = 1; k <= 25; k += 2) { sum += term / k; term *= s2; }
    return 2.0 * sum + e * 0.69314718055994530942;
}
// cos(2 pi u), u in [0, 1): quadrant reduction, then Taylor series on |r| <= pi/4
double det_cos2pi(double u) {
    const double x = 4.0 * u;
    const int k = (int)(x + 0.5);
    const double r = (x - k) * 1.57079632679489661923, r2 = r * r;
    double c = 1.0, s = r, tc = 1.0, ts = r;
    for (int n = 1; n <= 11; n++) {
        tc *= -r2 / ((2.0 * n - 1) * (2.0 * n));
        ts *= -r2 / ((2.0 * n) * (2.0 * n + 1));
        c += tc; s += ts;
    }
    switch (k & 3) { case 0: return c; case 1: return -s; case 2: return -c; default: return s; }
}
double normal(Rng& r) {
    const double u1 = 1.0 - r.unit(), u2 = r.unit();   // u1 in (0, 1]
    return std::sqrt(-2.0 * det_log(u1)) * det_cos2pi(u2);
}

struct Out {
    std::string name;
    uint32_t type;
    std::vector<int64_t> ne;
    std::vector<uint8_t> bytes;
};

constexpr size_t kSegF32 = 65536, kSegQ4 = 4096;

// segments are independent streams, so the split over threads never changes the bytes
template<class F> void parallel_segments(int64_t nseg, F f) {
    const int64_t nt = std::max<int64_t>(1, std::min<int64_t>(nseg, (int64_t)std::thread::hardware_concurrency()));
    std::vector<std::thread> th;
    for (int64_t t = 0; t < nt; t++)
        th.emplace_back([=] { for (int64_t s = t; s < nseg; s += nt) f(s); });
    for (auto& x : th) x.join();
}

void fill_f32(Out& t, uint64_t seed, uint64_t tid, int64_t n, float sigma) {
    t.bytes.resize((size_t)n * 4);
    float* p = reinterpret_cast<float*>(t.bytes.data());
    const int64_t nseg = (n + kSegF32 - 1) / kSegF32;
    parallel_segments(nseg, [=](int64_t sgi) {
        Rng r(mix64(seed ^ mix64(tid * 0x100000001B3ull + (uint64_t)sgi)));
        const int64_t a = sgi * kSegF32, b = std::min<int64_t>(n, a + kSegF32);
        for (int64_t i = a; i < b; i++) p[i] = (float)(sigma * normal(r));
    });
}

void fill_q4(Out& t, uint64_t seed, uint64_t tid, int64_t nblocks, float sigma) {
    t.bytes.resize((size_t)nblocks * 18);
    uint8_t* p = t.bytes.data();
    const int64_t nseg = (nblocks + kSegQ4 - 1) / kSegQ4;
    parallel_segments(nseg, [=](int64_t sgi) {
        Rng r(mix64(seed ^ mix64(tid * 0x100000001B3ull + (uint64_t)sgi)));
        const int64_t a = sgi * kSegQ4, b = std::min<int64_t>(nblocks, a + kSegQ4);
        for (int64_t i = a; i < b; i++) {
            uint8_t* blk = p + i * 18;
            const uint16_t d = mi::f32_to_f16((float)std::fabs(sigma * normal(r)));
            memcpy(blk, &d, 2);
            const uint64_t w0 = r.next(), w1 = r.next();
            memcpy(blk + 2, &w0, 8);
            memcpy(blk + 10, &w1, 8);
        }
    });
}

// q8_0 (int8 codes uniform in [-127, 127], fp16 d = |N(0, sigma)| / 16), q4_1 (nibbles
// uniform, d = |N(0, sigma)|, m = -8 d rounded to fp16) and q6_K (random 6-bit codes,
// int8 group scales uniform in [1, 63], fp16 d = |N(0, sigma)| / 256) blocks
void fill_blocks(Out& t, uint64_t seed, uint64_t tid, int64_t nblocks, float sigma) {
    const size_t bs = t.type == mi::GT_Q8_0 ? 34 : t.type == mi::GT_Q4_1 ? 20 : 210;
    t.bytes.resize((size_t)nblocks * bs);
    uint8_t* p = t.bytes.data();
    const int64_t nseg = (nblocks + kSegQ4 - 1) / kSegQ4;
    const uint32_t type = t.type;
    parallel_segments(nseg, [=](int64_t sgi) {
        Rng r(mix64(seed ^ mix64(tid * 0x100000001B3ull + (uint64_t)sgi)));
        const int64_t a = sgi * kSegQ4, b = std::min<int64_t>(nblocks, a + kSegQ4);
        for (int64_t i = a; i < b; i++) {
            uint8_t* blk = p + i * bs;
            const double g = std::fabs(sigma * normal(r));
            if (type == mi::GT_Q8_0) {
                const uint16_t d = mi::f32_to_f16((float)(g / 16.0));
                memcpy(blk, &d, 2);
                for (int j = 0; j < 32; j++) blk[2 + j] = (uint8_t)(int8_t)((int)(r.next() % 255) - 127);
            } else if (type == mi::GT_Q4_1) {
                const uint16_t d = mi::f32_to_f16((float)g), m = mi::f32_to_f16((float)(-8.0 * g));
                memcpy(blk, &d, 2);
                memcpy(blk + 2, &m, 2);
                const uint64_t w0 = r.next(), w1 = r.next();
                memcpy(blk + 4, &w0, 8);
                memcpy(blk + 12, &w1, 8);
            } else {
                for (int j = 0; j < 192; j += 8) { const uint64_t w = r.next(); memcpy(blk + j, &w, 8); }
                for (int j = 0; j < 16; j++) blk[192 + j] = (uint8_t)(int8_t)(1 + (int)(r.next() % 63));
                const uint16_t d = mi::f32_to_f16((float)(g / 256.0));
                memcpy(blk + 208, &d, 2);
            }
        }
    });
}

// GPT-2 byte-level alphabet (the inverse of detok.h's byte decoder): printable
// bytes map to themselves, the rest to U+0100 + k
std::string byte_token(int b) {
    auto printable = [](int c) { return (c >= 33 && c <= 126) || (c >= 161 && c <= 172) || (c >= 174 && c <= 255); };
    int cp;
    if (printable(b)) cp = b;
    else {
        int k = 0;
        for (int c = 0; c < b; c++) if (!printable(c)) k++;
        cp = 256 + k;
    }
    std::string s;
    if (cp < 0x80) s += (char)cp;
    else if (cp < 0x800) { s += (char)(0xC0 | (cp >> 6)); s += (char)(0x80 | (cp & 0x3F)); }
    return s;
}

struct W {
    FILE* f;
    bool ok = true;
    void raw(const void* p, size_t n) { if (ok && fwrite(p, 1, n, f) != n) ok = false; }
    template<class T> void put(T v) { raw(&v, sizeof v); }
    void str(const std::string& s) { put<uint64_t>(s.size()); raw(s.data(), s.size()); }
    void kv_u32(const char* k, uint32_t v) { str(k); put<uint32_t>(4); put<uint32_t>(v); }
    void kv_f32(const char* k, float v) { str(k); put<uint32_t>(6); put<float>(v); }
    void kv_str(const char* k, const std::string& v) { str(k); put<uint32_t>(8); str(v); }
};

}  // namespace

extern "C" int mi_synth_gguf(const char* path, const mi_synth_shape* sh, uint64_t seed) {
    if (!path || !sh) return MI_ERR_ARG;
    const int L = sh->n_layer, E = sh->n_embd, FF = sh->n_ff, NH = sh->n_head, NKV = sh->n_head_kv, V = sh->n_vocab;
    if (L < 1 || E < 32 || FF < 32 || NH < 1 || NKV < 1 || V < 256 || E % NH || NH % NKV || E % 32 || FF % 32)
        return MI_ERR_SHAPE;
    const int HD = E / NH, KVD = NKV * HD;
    std::vector<Out> ts;
    auto add = [&](const std::string& name, uint32_t type, std::vector<int64_t> ne) {
        ts.push_back(Out{name, type, std::move(ne), {}});
        return ts.size() - 1;
    };
    // tensor list and shapes: ne[0] is the input (row) length
    auto mtype = [](int32_t t, uint32_t def) -> uint32_t { return t == 0 ? def : (uint32_t)t; };
    const uint32_t emb_t = sh->emb_type == 2 ? mi::GT_Q4_0 : sh->emb_type == 8 ? mi::GT_Q8_0 : mi::GT_F32;
    const uint32_t head_t = mtype(sh->head_type, mi::GT_Q4_0), down_t = mtype(sh->down_type, mi::GT_Q4_0);
    if ((head_t != mi::GT_Q4_0 && head_t != mi::GT_Q8_0 && head_t != mi::GT_Q6_K) ||
        (down_t != mi::GT_Q4_0 && down_t != mi::GT_Q4_1) || (head_t == mi::GT_Q6_K && E % 256))
        return MI_ERR_ARG;
    add("token_embd.weight", emb_t, {E, V});
    for (int l = 0; l < L; l++) {
        const std::string p = "blk." + std::to_string(l) + ".";
        add(p + "attn_norm.weight", mi::GT_F32, {E});
        add(p + "attn_q.weight", mi::GT_Q4_0, {E, E});
        add(p + "attn_q.bias", mi::GT_F32, {E});
        add(p + "attn_k.weight", mi::GT_Q4_0, {E, KVD});
        add(p + "attn_k.bias", mi::GT_F32, {KVD});
        add(p + "attn_v.weight", mi::GT_Q4_0, {E, KVD});
        add(p + "attn_v.bias", mi::GT_F32, {KVD});
        add(p + "attn_output.weight", mi::GT_Q4_0, {E, E});
        add(p + "ffn_norm.weight", mi::GT_F32, {E});
        add(p + "ffn_gate.weight", mi::GT_Q4_0, {E, FF});
        add(p + "ffn_up.weight", mi::GT_Q4_0, {E, FF});
        add(p + "ffn_down.weight", down_t, {FF, E});
    }
    add("output_norm.weight", mi::GT_F32, {E});
    if (!sh->tied) add("output.weight", head_t, {E, V});

    FILE* f = fopen(path, "wb");
    if (!f) return MI_ERR_IO;
    W w{f};
    const uint32_t eos = (uint32_t)(V > 151645 ? 151645 : V - 1);
    w.put<uint32_t>(0x46554747u);
    w.put<uint32_t>(3);
    w.put<uint64_t>(ts.size());
    w.put<uint64_t>(15);
    w.kv_str("general.architecture", "qwen2");
    w.kv_str("general.name", "minfer-synthetic-" + std::to_string(seed));
    w.kv_u32("general.alignment", 32);
    w.kv_u32("qwen2.block_count", (uint32_t)L);
    w.kv_u32("qwen2.context_length", 32768);
    w.kv_u32("qwen2.embedding_length", (uint32_t)E);
    w.kv_u32("qwen2.feed_forward_length", (uint32_t)FF);
    w.kv_u32("qwen2.attention.head_count", (uint32_t)NH);
    w.kv_u32("qwen2.attention.head_count_kv", (uint32_t)NKV);
    w.kv_f32("qwen2.rope.freq_base", sh->rope_base);
    w.kv_f32("qwen2.attention.layer_norm_rms_epsilon", sh->rms_eps);
    w.kv_str("tokenizer.ggml.model", "gpt2");
    w.kv_u32("tokenizer.ggml.eos_token_id", eos);
    w.kv_u32("tokenizer.ggml.bos_token_id", eos);
    w.str("tokenizer.ggml.tokens"); w.put<uint32_t>(9); w.put<uint32_t>(8); w.put<uint64_t>((uint64_t)V);
    for (int i = 0; i < V; i++) {
        if (i < 256) w.str(byte_token(i));
        else if (i == (int)eos) w.str("<|im_end|>");
        else w.str((i % 3 == 0 ? "\xC4\xA0" : "") + std::string("t") + std::to_string(i));
    }
    // tensor infos with 32-byte aligned offsets
    auto nbytes = [](const Out& t) {
        int64_t n = 1; for (auto e : t.ne) n *= e;
        switch (t.type) {
            case mi::GT_F32: return (uint64_t)n * 4;
            case mi::GT_Q4_1: return (uint64_t)(n / 32) * 20;
            case mi::GT_Q8_0: return (uint64_t)(n / 32) * 34;
            case mi::GT_Q6_K: return (uint64_t)(n / 256) * 210;
            default: return (uint64_t)(n / 32) * 18;
        }
    };
    uint64_t off = 0;
    std::vector<uint64_t> offs;
    for (auto& t : ts) {
        w.str(t.name); w.put<uint32_t>((uint32_t)t.ne.size());
        for (auto e : t.ne) w.put<uint64_t>((uint64_t)e);
        w.put<uint32_t>(t.type); w.put<uint64_t>(off);
        offs.push_back(off);
        off = (off + nbytes(t) + 31) / 32 * 32;
    }
    long pos = ftell(f);
    const long start = (pos + 31) / 32 * 32;
    static const uint8_t zeros[32] = {0};
    w.raw(zeros, (size_t)(start - pos));
    for (size_t i = 0; i < ts.size() && w.ok; i++) {
        Out& t = ts[i];
        int64_t n = 1; for (auto e : t.ne) n *= e;
        if (t.type == mi::GT_F32) {
            const bool qk_bias = t.name.find("attn_q.bias") != std::string::npos ||
                                 t.name.find("attn_k.bias") != std::string::npos;
            const bool norm = t.name.find("norm.weight") != std::string::npos;
            fill_f32(t, seed, i, n, qk_bias && sh->qk_bias_std > 0.f ? sh->qk_bias_std : 0.02f);
            if (norm && sh->norm_offset != 0.f) {
                float* p = reinterpret_cast<float*>(t.bytes.data());
                for (int64_t k = 0; k < n; k++) p[k] += sh->norm_offset;
            }
        }
        else if (t.type == mi::GT_Q4_0) fill_q4(t, seed, i, n / 32, 0.002f);
        else fill_blocks(t, seed, i, t.type == mi::GT_Q6_K ? n / 256 : n / 32, 0.002f);
        pos = ftell(f);
        const long want = start + (long)offs[i];
        if (want > pos) w.raw(zeros, (size_t)(want - pos));
        w.raw(t.bytes.data(), t.bytes.size());
        std::vector<uint8_t>().swap(t.bytes);
    }
    const bool ok = w.ok && fclose(f) == 0;
    return ok ? MI_OK : MI_ERR_IO;
}
