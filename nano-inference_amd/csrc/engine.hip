// engine.hip -- host side of the engine and the C ABI (include/minfer.h).
//
// Load path (reference: cuda_infer.cu:844-901, mega.cu:1005-1139): parse the GGUF,
// repack every q4_0 matrix into the tile layout (common.hpp), fuse q|k|v rows and
// interleave gate/up row groups, upload everything into one device arena, build
// the RoPE table with cpu_infer's own float expressions (cpu_infer.cpp:54-55), and
// allocate the fp16 KV cache and the step's work buffers. Steps then run on one HIP
// stream without host round trips: the token of each position lives in device
// memory (tokbuf), and each step's argmax writes the next token there.
#include "common.hpp"
#include "gguf.hpp"
#include "kernels.hpp"
#include "layout.hpp"
#include "minfer.h"

#include <algorithm>
#include <chrono>
#include <cmath>
#include <cstdarg>
#include <cstdio>
#include <cstring>
#include <memory>
#include <string>
#include <thread>
#include <vector>

using namespace mi;

namespace {

thread_local std::string g_load_error;

}  // namespace

struct mi_engine {
    mi_opts opts{};
    GGUFFile gguf;
    std::string err;
    int n_cu = 0;
    int E = 0, FF = 0, NH = 0, NKV = 0, HD = 0, G = 0, KVD = 0, QKV = 0, V = 0, NL = 0, maxseq = 0, maxch = 0, eos = 0;
    float rope_base = 0, eps = 0;
    int cb[5] = {0}, ks[5] = {0};
    uint64_t weight_bytes = 0;
    std::vector<void*> allocs;
    DModel M{};
    DModel M_logits{};            // same as M with the logits buffer attached
    DModel* dM = nullptr;         // device copies the kernels read: [0] M, [1] M_logits, [2] profiling
    DLayer* d_layers = nullptr;
    hipStream_t stream = nullptr;
    hipEvent_t ev0 = nullptr, ev1 = nullptr;
    int nwg_persistent = 0;       // workgroups of the persistent step kernel (0: per-phase launches)
    bool coop = false;            // launch it cooperatively (after a plain launch's barrier failed)
    bool multi_persistent = false;   // multi-token steps as one persistent launch too (kT_step)
    int32_t* h_iota = nullptr;    // pinned host memory, h_iota[p] = p: the source of posT
    uint64_t* h_ring = nullptr;   // pinned, device-mapped host memory [maxseq]: streamed tokens (DModel::ring)
    hipGraphExec_t gexec[2][kMaxT + 1] = {};   // multi-token step per (logits, T), captured on first use
    int cur_len = 0;              // positions holding valid K/V
    bool next_ready = false;      // tokbuf[cur_len] holds the prediction of the last step
    mi_stats stats{};
    ~mi_engine() {
        if (stream) (void)hipStreamSynchronize(stream);
        for (auto& row : gexec)
            for (hipGraphExec_t g : row)
                if (g) (void)hipGraphExecDestroy(g);
        if (h_iota) (void)hipHostFree(h_iota);
        if (h_ring) (void)hipHostFree(h_ring);
        for (void* p : allocs) (void)hipFree(p);
        if (ev0) (void)hipEventDestroy(ev0);
        if (ev1) (void)hipEventDestroy(ev1);
        if (stream) (void)hipStreamDestroy(stream);
    }
};

namespace {

int set_err(mi_engine* e, int code, const char* fmt, ...) {
    char buf[512];
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(buf, sizeof buf, fmt, ap);
    va_end(ap);
    if (e) e->err = buf; else g_load_error = buf;
    return code;
}

#define HIPCHK(e, x)                                                                                   \
    do {                                                                                               \
        hipError_t st_ = (x);                                                                          \
        if (st_ != hipSuccess) return set_err(e, MI_ERR_DEVICE, "%s: %s", #x, hipGetErrorString(st_)); \
    } while (0)

int dev_alloc(mi_engine* e, void** p, size_t bytes) {
    if (hipMalloc(p, bytes) != hipSuccess) {
        (void)hipGetLastError();
        return set_err(e, MI_ERR_OOM, "hipMalloc(%zu MB) failed", bytes >> 20);
    }
    e->allocs.push_back(*p);
    if (hipMemset(*p, 0, bytes) != hipSuccess) return set_err(e, MI_ERR_DEVICE, "hipMemset failed");
    return MI_OK;
}

// Weights stored in another type are re-encoded as q4_0, the only format the kernels
// read (mega.cu:924-936 is the recipe; the oracle restates the same steps, so the two
// must agree bit for bit). For one block of 32 values:
//   step  = (largest |value|) / 7, stored as fp16
//   code  = lrintf(value * (1 / step)) + 8 (0 when step is 0), limited to 0..15
//   byte j of the 16 holds the code of value j in its low nibble, value j + 16 in its high
struct Q4Codec {
    static uint8_t code(float v, float recip) { return (uint8_t)std::clamp((int)lrintf(v * recip) + 8, 0, 15); }
    static void encode(const float* v, uint8_t* blk) {
        float peak = 0.f;
        for (int i = 0; i < 32; ++i) peak = std::max(peak, std::fabs(v[i]));
        const float step = peak / 7.f;
        const float recip = step > 0.f ? 1.f / step : 0.f;
        const uint16_t h = f32_to_f16(step);
        memcpy(blk, &h, sizeof h);
        uint8_t* q = blk + 2;
        for (int j = 0; j < 16; ++j) q[j] = (uint8_t)(code(v[j], recip) | (code(v[j + 16], recip) << 4));
    }
};

void dequant_row(const GTensor& t, int64_t r, float* out) {
    const int64_t c = t.cols();
    switch (t.type) {
        case GT_F32: memcpy(out, t.data + (size_t)r * c * 4, (size_t)c * 4); break;
        case GT_F16: {
            const uint16_t* h = reinterpret_cast<const uint16_t*>(t.data + (size_t)r * c * 2);
            for (int64_t i = 0; i < c; i++) out[i] = f16_to_f32(h[i]);
            break;
        }
        case GT_Q4_0: {
            const uint8_t* p = t.data + (size_t)r * (c / 32) * 18;
            for (int64_t b = 0; b < c / 32; b++, p += 18) {
                uint16_t hd; memcpy(&hd, p, 2);
                const float d = f16_to_f32(hd);
                for (int j = 0; j < 16; j++) {
                    out[b * 32 + j] = ((p[2 + j] & 0x0F) - 8) * d;
                    out[b * 32 + j + 16] = ((p[2 + j] >> 4) - 8) * d;
                }
            }
            break;
        }
        case GT_Q4_1: {     // 20-byte blocks: fp16 d, fp16 m, 16 B of nibbles (element j low, j+16 high)
            const uint8_t* p = t.data + (size_t)r * (c / 32) * 20;
            for (int64_t b = 0; b < c / 32; b++, p += 20) {
                uint16_t hd, hm; memcpy(&hd, p, 2); memcpy(&hm, p + 2, 2);
                const float d = f16_to_f32(hd), m = f16_to_f32(hm);
                for (int j = 0; j < 16; j++) {
                    out[b * 32 + j] = (p[4 + j] & 0x0F) * d + m;
                    out[b * 32 + j + 16] = (p[4 + j] >> 4) * d + m;
                }
            }
            break;
        }
        case GT_Q8_0: {
            const uint8_t* p = t.data + (size_t)r * (c / 32) * 34;
            for (int64_t b = 0; b < c / 32; b++, p += 34) {
                uint16_t hd; memcpy(&hd, p, 2);
                const float d = f16_to_f32(hd);
                for (int j = 0; j < 32; j++) out[b * 32 + j] = (int8_t)p[2 + j] * d;
            }
            break;
        }
        case GT_Q6_K: {
            // 210-byte superblocks of 256: ql[128] low nibbles, qh[64] 2-bit highs, int8
            // scales[16] (one per 16 values), fp16 d. Each 128-value half: value l (l < 32)
            // of quarter k takes its low nibble from ql[l + 32 (k & 1)] (low nibble for
            // k < 2, high for k >= 2) and its two high bits from qh[l] bits 2k..2k+1;
            // q - 32 times d times the scale of its 16-value group.
            const uint8_t* p = t.data + (size_t)r * (c / 256) * 210;
            for (int64_t b = 0; b < c / 256; b++, p += 210) {
                uint16_t hd; memcpy(&hd, p + 208, 2);
                const float d = f16_to_f32(hd);
                for (int half = 0; half < 2; half++) {
                    const uint8_t* ql = p + 64 * half;
                    const uint8_t* qh = p + 128 + 32 * half;
                    const int8_t* sc = reinterpret_cast<const int8_t*>(p + 192 + 8 * half);
                    float* y = out + b * 256 + 128 * half;
                    for (int l = 0; l < 32; l++)
                        for (int k = 0; k < 4; k++) {
                            const int lo = k < 2 ? (ql[l + 32 * (k & 1)] & 0x0F) : (ql[l + 32 * (k & 1)] >> 4);
                            const int q = (lo | (((qh[l] >> (2 * k)) & 3) << 4)) - 32;
                            y[32 * k + l] = d * sc[l / 16 + 2 * k] * q;
                        }
                }
            }
            break;
        }
        default: memset(out, 0, (size_t)c * 4);
    }
}

// The rows of a weight matrix as GGUF q4_0 bytes: a view of the mapped file when the
// tensor is stored as q4_0, otherwise an owned copy with every row dequantized and
// re-encoded block by block (Q4Codec).
class Q4View {
  public:
    explicit Q4View(const GTensor& t) {
        if (t.type == GT_Q4_0) {
            bytes_ = t.data;
            return;
        }
        const int64_t cols = t.cols(), nblk = cols / 32;
        owned_.resize((size_t)t.rows() * nblk * 18);
        std::vector<float> vals((size_t)cols);
        uint8_t* dst = owned_.data();
        for (int64_t r = 0; r < t.rows(); ++r) {
            dequant_row(t, r, vals.data());
            for (int64_t b = 0; b < nblk; ++b, dst += 18) Q4Codec::encode(vals.data() + 32 * b, dst);
        }
        bytes_ = owned_.data();
    }
    const uint8_t* data() const { return bytes_; }

  private:
    const uint8_t* bytes_ = nullptr;
    std::vector<uint8_t> owned_;
};

}  // namespace

extern "C" {

void mi_default_opts(mi_opts* o) {
    if (!o) return;
    o->max_ctx = 4096;
    o->tchunk = 8;
    o->spec = 0;
    o->ngmax = 3;
    o->spec_slope = 0.074f;
    o->persistent = 2;
    o->stop_eos = 0;
    o->device = 0;
    o->graphs = 0;
}

size_t mi_q4_packed_bytes(int32_t rows, int32_t nb, int32_t cb) {
    if (rows <= 0 || rows % 64 || nb <= 0 || (cb != 4 && cb != 8) || nb % cb) return 0;
    return (size_t)(rows / 64) * (nb / cb) * tile_bytes(cb);
}

int mi_q4_pack(const uint8_t* src, int32_t rows, int32_t nb, int32_t cb, uint8_t* dst) {
    if (!src || !dst || !mi_q4_packed_bytes(rows, nb, cb)) return MI_ERR_ARG;
    const int ng = rows / 64, nc = nb / cb;
    const size_t TB = tile_bytes(cb);
    for (int g = 0; g < ng; g++)
        for (int c = 0; c < nc; c++) {
            uint8_t* t = dst + ((size_t)g * nc + c) * TB;
            for (int r = 0; r < 64; r++) {
                const uint8_t* row = src + (size_t)(g * 64 + r) * nb * 18;
                for (int k = 0; k < cb; k++) {
                    const uint8_t* blk = row + (size_t)(c * cb + k) * 18;
                    memcpy(t + k * 1024 + r * 16, blk + 2, 16);
                    memcpy(t + (size_t)cb * 1024 + r * cb * 2 + k * 2, blk, 2);
                }
            }
        }
    return MI_OK;
}

const char* mi_last_error(const mi_engine* e) { return e ? e->err.c_str() : g_load_error.c_str(); }

}  // extern "C"

static int upload_mat(mi_engine* e, const uint8_t* rows_q4, int rows, int nb, int kind, PMat* out) {
    const int cb = e->cb[kind];
    const size_t bytes = mi_q4_packed_bytes(rows, nb, cb);
    if (!bytes) return set_err(e, MI_ERR_SHAPE, "matrix %dx%d blocks cannot be tiled (cb %d)", rows, nb, cb);
    std::vector<uint8_t> host(bytes);
    mi_q4_pack(rows_q4, rows, nb, cb, host.data());
    void* d = nullptr;
    int rc = dev_alloc(e, &d, bytes);
    if (rc) return rc;
    HIPCHK(e, hipMemcpy(d, host.data(), bytes, hipMemcpyHostToDevice));
    // placement of the work split (results do not depend on it): the QKV and O segments
    // go to the last workgroups, which hold no down segment (the phase before QKV) and
    // are not the gate/up phase's doubly loaded first ones (the phase after O); a
    // workgroup busy in one phase prefetches the next one's tiles late
    int rot = 0;
    const int nseg = (rows / 64) * e->ks[kind];
    if ((kind == 0 || kind == 1) && nseg < e->n_cu) rot = e->n_cu - nseg;
    *out = PMat{reinterpret_cast<const uint8_t*>(d), rows, nb, cb, nb / cb, e->ks[kind], rot};
    e->weight_bytes += (uint64_t)rows * nb * 18;
    return MI_OK;
}

static int upload_f32(mi_engine* e, const GTensor* t, int64_t n, const float** out) {
    std::vector<float> host((size_t)n);
    if (t->type == GT_F32) memcpy(host.data(), t->data, (size_t)n * 4);
    else {
        const int64_t c = t->cols();
        for (int64_t r = 0; r < n / c; r++) dequant_row(*t, r, host.data() + r * c);
    }
    void* d = nullptr;
    int rc = dev_alloc(e, &d, (size_t)n * 4);
    if (rc) return rc;
    HIPCHK(e, hipMemcpy(d, host.data(), (size_t)n * 4, hipMemcpyHostToDevice));
    *out = reinterpret_cast<const float*>(d);
    return MI_OK;
}

template <class T>
static int alloc_buf(mi_engine* e, T** p, size_t count) {
    void* d = nullptr;
    int rc = dev_alloc(e, &d, std::max<size_t>(count, 1) * sizeof(T));
    *p = reinterpret_cast<T*>(d);
    return rc;
}

// the buffer-layout facts of a model shape (layout.hpp)
static Dims step_dims(int NL, int E, int FF, int NH, int NKV, int V, int maxseq, const int cb[5], const int ks[5],
                      int nwg) {
    Dims d{};
    d.NL = NL; d.E = E; d.FF = FF; d.NH = NH; d.NKV = NKV; d.HD = E / NH; d.V = V;
    d.QKV = NH * d.HD + 2 * NKV * d.HD;
    d.maxseq = maxseq;
    d.maxch = (maxseq + kAttnChunk - 1) / kAttnChunk;
    d.arec = attn_record_floats(d.HD);
    d.ks_qkv = ks[0]; d.ks_o = ks[1]; d.ks_d = ks[3];
    d.ks_oT = (E / 32) / cb[1];
    d.nwg = nwg;
    return d;
}

static int load_impl(mi_engine* e, const char* path) {
    int ndev = 0;
    if (hipGetDeviceCount(&ndev) != hipSuccess || ndev <= e->opts.device)
        return set_err(e, MI_ERR_DEVICE, "no HIP device %d", e->opts.device);
    HIPCHK(e, hipSetDevice(e->opts.device));
    hipDeviceProp_t prop;
    HIPCHK(e, hipGetDeviceProperties(&prop, e->opts.device));
    if (strncmp(prop.gcnArchName, "gfx950", 6) != 0)
        return set_err(e, MI_ERR_DEVICE, "device %d is %s; the kernels are built for gfx950", e->opts.device, prop.gcnArchName);
    e->n_cu = prop.multiProcessorCount;

    GGUFFile& g = e->gguf;
    if (!g.open(path)) return set_err(e, MI_ERR_FORMAT, "%s", g.error().c_str());
    e->NL = (int)g.num("qwen2.block_count", 0);
    e->E = (int)g.num("qwen2.embedding_length", 0);
    e->FF = (int)g.num("qwen2.feed_forward_length", 0);
    e->NH = (int)g.num("qwen2.attention.head_count", 0);
    e->NKV = (int)g.num("qwen2.attention.head_count_kv", 0);
    e->rope_base = (float)g.num("qwen2.rope.freq_base", 1e6);
    e->eps = (float)g.num("qwen2.attention.layer_norm_rms_epsilon", 1e-6);
    e->V = (int)g.tokens().size();
    e->eos = (int)g.num("tokenizer.ggml.eos_token_id", 151645);
    if (e->NL < 1 || e->E < 32 || e->NH < 1 || e->NKV < 1 || e->E % e->NH || e->NH % e->NKV)
        return set_err(e, MI_ERR_FORMAT, "missing or inconsistent qwen2.* shape metadata");
    e->HD = e->E / e->NH;
    e->G = e->NH / e->NKV;
    e->KVD = e->NKV * e->HD;
    e->QKV = e->NH * e->HD + 2 * e->KVD;
    if (!kernels_support(e->G, e->HD) || e->E % 64 || e->E > kMaxE || e->FF % 32 || e->FF > kMaxFF ||
        e->QKV % 64 || e->V % 64 || e->V < 64 || (e->E / 32) % 4 || (e->FF / 32) % 4)
        return set_err(e, MI_ERR_SHAPE, "unsupported shape E=%d FF=%d heads=%d/%d hd=%d vocab=%d", e->E, e->FF, e->NH,
                       e->NKV, e->HD, e->V);
    e->maxseq = e->opts.max_ctx > 0 ? e->opts.max_ctx : 4096;
    e->maxch = (e->maxseq + kAttnChunk - 1) / kAttnChunk;
    if (e->maxch > kernels_max_ctx_chunks(e->HD))
        return set_err(e, MI_ERR_SHAPE, "max_ctx %d exceeds the %d positions the attention merge holds", e->maxseq,
                       kernels_max_ctx_chunks(e->HD) * kAttnChunk);

    // reduction plan (the float summation order; depends on the shape only)
    const int nbE = e->E / 32, nbF = e->FF / 32;
    if (!kernels_plan(e->E, e->FF, e->cb, e->ks))
        return set_err(e, MI_ERR_SHAPE, "E=%d FF=%d do not fit the kernels' staging", e->E, e->FF);
    {
        const int rows[5] = {e->QKV, e->E, 2 * e->FF, e->E, e->V}, nbs[5] = {nbE, nbE, nbE, nbF, nbE};
        for (int i = 0; i < 5; i++)
            if (kernels_tiles_per_wg(rows[i], nbs[i], e->cb[i], e->ks[i], e->n_cu) > kernels_max_tiles_per_wg() ||
                (nbs[i] / e->cb[i] + e->ks[i] - 1) / e->ks[i] > kernels_max_chunks_multi())
                return set_err(e, MI_ERR_SHAPE, "matrix %d needs %d tiles per workgroup on %d CUs (limit %d)", i,
                               kernels_tiles_per_wg(rows[i], nbs[i], e->cb[i], e->ks[i], e->n_cu), e->n_cu,
                               kernels_max_tiles_per_wg());
    }

    auto need = [&](const std::string& n) -> const GTensor* { return g.tensor(n); };
    const GTensor* te = need("token_embd.weight");
    const GTensor* tout = need("output.weight");
    const GTensor* tnorm = need("output_norm.weight");
    if (!te || !tnorm) return set_err(e, MI_ERR_FORMAT, "missing token_embd.weight or output_norm.weight");
    if (!tout) tout = te;   // tied embeddings (mega.cu:1071)
    if (te->cols() != e->E || te->rows() < e->V || tout->cols() != e->E || tout->rows() != e->V)
        return set_err(e, MI_ERR_FORMAT, "embedding/output shapes do not match the metadata");

    std::vector<DLayer> layers(e->NL);
    std::vector<uint8_t> cat;
    const size_t rbE = (size_t)nbE * 18, rbF = (size_t)nbF * 18;
    for (int l = 0; l < e->NL; l++) {
        const std::string p = "blk." + std::to_string(l) + ".";
        const char* names[] = {"attn_norm.weight", "attn_q.weight", "attn_q.bias", "attn_k.weight", "attn_k.bias",
                               "attn_v.weight", "attn_v.bias", "attn_output.weight", "ffn_norm.weight",
                               "ffn_gate.weight", "ffn_up.weight", "ffn_down.weight"};
        const GTensor* t[12];
        for (int i = 0; i < 12; i++) {
            t[i] = need(p + names[i]);
            if (!t[i]) return set_err(e, MI_ERR_FORMAT, "missing tensor %s%s", p.c_str(), names[i]);
        }
        const int NQ = e->NH * e->HD;
        if (t[1]->cols() != e->E || t[1]->rows() != NQ || t[3]->rows() != e->KVD || t[5]->rows() != e->KVD ||
            t[7]->cols() != NQ || t[7]->rows() != e->E || t[9]->rows() != e->FF || t[10]->rows() != e->FF ||
            t[11]->cols() != e->FF || t[11]->rows() != e->E)
            return set_err(e, MI_ERR_FORMAT, "layer %d tensor shapes do not match the metadata", l);
        // fused QKV rows [q; k; v]
        cat.resize((size_t)e->QKV * rbE);
        memcpy(cat.data(), Q4View(*t[1]).data(), (size_t)NQ * rbE);
        memcpy(cat.data() + (size_t)NQ * rbE, Q4View(*t[3]).data(), (size_t)e->KVD * rbE);
        memcpy(cat.data() + (size_t)(NQ + e->KVD) * rbE, Q4View(*t[5]).data(), (size_t)e->KVD * rbE);
        int rc = upload_mat(e, cat.data(), e->QKV, nbE, 0, &layers[l].qkv);
        if (rc) return rc;
        rc = upload_mat(e, Q4View(*t[7]).data(), e->E, nbE, 1, &layers[l].o);
        if (rc) return rc;
        // gate/up interleaved by 32-row groups
        {
            const Q4View gv(*t[9]), uv(*t[10]);
            const uint8_t* gr = gv.data();
            const uint8_t* ur = uv.data();
            cat.resize((size_t)2 * e->FF * rbE);
            for (int G32 = 0; G32 < e->FF / 32; G32++) {
                memcpy(cat.data() + (size_t)(64 * G32) * rbE, gr + (size_t)(32 * G32) * rbE, 32 * rbE);
                memcpy(cat.data() + (size_t)(64 * G32 + 32) * rbE, ur + (size_t)(32 * G32) * rbE, 32 * rbE);
            }
            rc = upload_mat(e, cat.data(), 2 * e->FF, nbE, 2, &layers[l].gu);
            if (rc) return rc;
        }
        rc = upload_mat(e, Q4View(*t[11]).data(), e->E, nbF, 3, &layers[l].d);
        if (rc) return rc;
        (void)rbF;
        rc = upload_f32(e, t[0], e->E, &layers[l].an);
        if (rc) return rc;
        rc = upload_f32(e, t[8], e->E, &layers[l].fn);
        if (rc) return rc;
        {
            std::vector<float> b((size_t)e->QKV);
            for (int i = 0; i < 3; i++) {
                const GTensor* bt = t[2 + 2 * i];
                const int n = i == 0 ? NQ : e->KVD, off = i == 0 ? 0 : (i == 1 ? NQ : NQ + e->KVD);
                if (bt->cols() != n) return set_err(e, MI_ERR_FORMAT, "layer %d bias shape", l);
                dequant_row(*bt, 0, b.data() + off);
            }
            void* d = nullptr;
            rc = dev_alloc(e, &d, b.size() * 4);
            if (rc) return rc;
            HIPCHK(e, hipMemcpy(d, b.data(), b.size() * 4, hipMemcpyHostToDevice));
            layers[l].bqkv = reinterpret_cast<const float*>(d);
        }
        for (int i : {1, 3, 5, 7, 9, 10, 11}) g.release(*t[i]);
    }
    DModel& M = e->M;
    M.E = e->E; M.FF = e->FF; M.NH = e->NH; M.NKV = e->NKV; M.HD = e->HD; M.G = e->G; M.KVD = e->KVD;
    M.QKV = e->QKV; M.V = e->V; M.NL = e->NL; M.maxseq = e->maxseq; M.maxch = e->maxch;
    M.eps = e->eps;
    M.scale = 1.f / sqrtf((float)e->HD);
    int rc = upload_mat(e, Q4View(*tout).data(), e->V, nbE, 4, &M.lm);
    if (rc) return rc;
    rc = upload_f32(e, te, (int64_t)e->V * e->E, &M.emb);
    if (rc) return rc;
    rc = upload_f32(e, tnorm, e->E, &M.out_norm);
    if (rc) return rc;
    g.release(*tout);
    g.release(*te);
    // RoPE table: cpu_infer.cpp:54-55 evaluated with the same float expressions
    {
        const int half = e->HD / 2;
        std::vector<float2> rope((size_t)e->maxseq * half);
        for (int pos = 0; pos < e->maxseq; pos++)
            for (int i = 0; i < half; i++) {
                const float theta = pos * powf(e->rope_base, -2.f * i / e->HD);
                rope[(size_t)pos * half + i] = make_float2(cosf(theta), sinf(theta));
            }
        float2* d = nullptr;
        rc = alloc_buf(e, &d, rope.size());
        if (rc) return rc;
        HIPCHK(e, hipMemcpy(d, rope.data(), rope.size() * sizeof(float2), hipMemcpyHostToDevice));
        M.rope = d;
    }
    rc = alloc_buf(e, &e->d_layers, e->NL);
    if (rc) return rc;
    HIPCHK(e, hipMemcpy(e->d_layers, layers.data(), layers.size() * sizeof(DLayer), hipMemcpyHostToDevice));
    M.layers = e->d_layers;
    if (e->opts.persistent) {
        int coop = 0;
        HIPCHK(e, hipDeviceGetAttribute(&coop, hipDeviceAttributeCooperativeLaunch, e->opts.device));
        const int per_cu = persistent_max_grid(e->G, e->HD);
        if (!coop || per_cu < 1)
            return set_err(e, MI_ERR_DEVICE, "persistent step kernel cannot be co-resident (cooperative %d, %d per CU)",
                           coop, per_cu);
        e->nwg_persistent = e->n_cu;      // one workgroup per CU
        e->multi_persistent = e->opts.persistent >= 2 && multi_persistent_max_grid(e->HD) >= 1;
    }
    M.arec = attn_record_floats(e->HD);
    const size_t NL = (size_t)e->NL;
    const Dims D = step_dims(e->NL, e->E, e->FF, e->NH, e->NKV, e->V, e->maxseq, e->cb, e->ks, e->n_cu);
    if ((rc = alloc_buf(e, &M.kc, lay::kv_size(D))) || (rc = alloc_buf(e, &M.vc, lay::kv_size(D))) ||
        (rc = alloc_buf(e, &M.tokbuf, (size_t)e->maxseq + 1)) ||
        (rc = alloc_buf(e, &M.hbuf, lay::hbuf_size(D))) ||
        (rc = alloc_buf(e, &M.qkv_part, lay::qkv_part_size(D))) ||
        (rc = alloc_buf(e, &M.att, lay::att_size(D))) ||
        (rc = alloc_buf(e, &M.att_out, NL * e->E)) ||
        (rc = alloc_buf(e, &M.o_part, lay::o_part_size(D))) ||
        (rc = alloc_buf(e, &M.act, lay::act_size(D))) ||
        (rc = alloc_buf(e, &M.d_part, lay::d_part_size(D))) ||
        (rc = alloc_buf(e, &M.cand, (size_t)e->n_cu * 32)) ||
        (rc = alloc_buf(e, &M.bar, (size_t)barrier_words())) || (rc = alloc_buf(e, &M.err, 64)) ||
        (rc = alloc_buf(e, &M.out_tok, (size_t)e->maxseq)) ||
        (rc = alloc_buf(e, &M.out_margin, (size_t)e->maxseq)))
        return rc;
    // multi-token step buffers (mi_step with T > 1)
    if ((rc = alloc_buf(e, &M.posT, 1)) || (rc = alloc_buf(e, &M.hT, lay::hT_size(D))) ||
        (rc = alloc_buf(e, &M.qkvT, lay::qkvT_size(D))) ||
        (rc = alloc_buf(e, &M.attT, lay::attT_size(D))) ||
        (rc = alloc_buf(e, &M.xT, lay::xT_size(D))) ||
        (rc = alloc_buf(e, &M.oT, lay::oT_size(D))) ||
        (rc = alloc_buf(e, &M.actT, lay::actT_size(D))) ||
        (rc = alloc_buf(e, &M.dT, lay::dT_size(D))) ||
        (rc = alloc_buf(e, &M.candT, lay::candT_size(D))) || (rc = alloc_buf(e, &M.spec, 1)))
        return rc;
    M.logits = nullptr;
    M.logitsT = nullptr;
    M.prof = nullptr;
    // the token ring of streaming generation: fine-grained (coherent) pinned host memory,
    // so the host sees each launch's system-scope store as soon as it lands
    HIPCHK(e, hipHostMalloc((void**)&e->h_ring, sizeof(uint64_t) * (size_t)e->maxseq,
                            hipHostMallocMapped | hipHostMallocCoherent));
    HIPCHK(e, hipHostGetDevicePointer((void**)&M.ring, e->h_ring, 0));
    // a kGenRing launch whose input token is M.eos does nothing: only when generation
    // stops at eos; with stop_eos off an eos is an ordinary token and the steps go on
    // (the reference's RAWIDS mode keeps generating past it, cuda_infer.cu:1192)
    M.eos = e->opts.stop_eos ? e->eos : -1;
    e->M_logits = M;
    if ((rc = alloc_buf(e, &e->M_logits.logits, (size_t)e->V))) return rc;
    if ((rc = alloc_buf(e, &e->M_logits.logitsT, lay::logitsT_size(D)))) return rc;
    if ((rc = alloc_buf(e, &e->dM, 3))) return rc;
    HIPCHK(e, hipMemcpy(e->dM, &e->M, sizeof(DModel), hipMemcpyHostToDevice));
    HIPCHK(e, hipMemcpy(e->dM + 1, &e->M_logits, sizeof(DModel), hipMemcpyHostToDevice));
    HIPCHK(e, hipStreamCreateWithFlags(&e->stream, hipStreamNonBlocking));
    HIPCHK(e, hipHostMalloc((void**)&e->h_iota, sizeof(int32_t) * ((size_t)e->maxseq + 1), hipHostMallocDefault));
    for (int p = 0; p <= e->maxseq; p++) e->h_iota[p] = p;
    HIPCHK(e, hipEventCreate(&e->ev0));
    HIPCHK(e, hipEventCreate(&e->ev1));
    HIPCHK(e, hipDeviceSynchronize());
    return MI_OK;
}

extern "C" {

int mi_load(const char* gguf_path, const mi_opts* opts, mi_engine** out) {
    if (!gguf_path || !out) return set_err(nullptr, MI_ERR_ARG, "null argument");
    *out = nullptr;
    std::unique_ptr<mi_engine> e(new mi_engine());
    if (opts) e->opts = *opts; else mi_default_opts(&e->opts);
    if (e->opts.tchunk < 1 || e->opts.tchunk > 8 || e->opts.max_ctx < 0 || e->opts.persistent < 0 || e->opts.persistent > 2 ||
        e->opts.spec < 0 || e->opts.spec > 2)
        return set_err(nullptr, MI_ERR_ARG, "bad options");
    const int rc = load_impl(e.get(), gguf_path);
    if (rc) { g_load_error = e->err; return rc; }
    *out = e.release();
    return MI_OK;
}

void mi_free(mi_engine* e) { delete e; }

int mi_info(const mi_engine* e, mi_model_info* o) {
    if (!e || !o) return MI_ERR_ARG;
    memset(o, 0, sizeof *o);
    o->n_layer = e->NL; o->n_embd = e->E; o->n_ff = e->FF; o->n_head = e->NH; o->n_head_kv = e->NKV;
    o->head_dim = e->HD; o->n_vocab = e->V; o->eos = e->eos; o->rope_base = e->rope_base; o->rms_eps = e->eps;
    o->max_ctx = e->maxseq;
    for (int i = 0; i < 5; i++) { o->plan_cb[i] = e->cb[i]; o->plan_ks[i] = e->ks[i]; }
    o->attn_chunk = kAttnChunk;
    o->kv_f16 = 1;
    o->n_cu = e->n_cu;
    o->persistent = e->nwg_persistent > 0;
    o->weight_bytes = e->weight_bytes;
    o->coop = e->coop ? 1 : 0;
    return MI_OK;
}

// Host-side walk over every buffer index the step kernels form for one step of T
// tokens at pos (T = 1: the single-token step; T > 1: the multi-token phase bodies),
// with the loop bounds of each body, checked against the allocation sizes (layout.hpp).
int mi_check_layout(const mi_synth_shape* sh, int32_t max_ctx, int32_t n_cu, int32_t T, int32_t pos, char* err,
                    int32_t errlen) {
    auto fail = [&](const char* fmt, ...) {
        if (err && errlen > 0) {
            va_list ap;
            va_start(ap, fmt);
            vsnprintf(err, (size_t)errlen, fmt, ap);
            va_end(ap);
        }
        return MI_ERR_SHAPE;
    };
    if (!sh || max_ctx < 1 || n_cu < 1 || T < 1 || T > kMaxT || pos < 0) return MI_ERR_ARG;
    const int NL = sh->n_layer, E = sh->n_embd, FF = sh->n_ff, NH = sh->n_head, NKV = sh->n_head_kv, V = sh->n_vocab;
    if (NL < 1 || NH < 1 || NKV < 1 || E % NH || NH % NKV || E % 64 || FF % 64 || V % 64) return MI_ERR_ARG;
    int cb[5], ks[5];
    if (!kernels_plan(E, FF, cb, ks)) return fail("no plan for E=%d FF=%d", E, FF);
    const Dims D = step_dims(NL, E, FF, NH, NKV, V, max_ctx, cb, ks, n_cu);
    const int HD = D.HD, G = NH / NKV, QKV = D.QKV, KVD = NKV * HD, nbE = E / 32, nbF = FF / 32;
    if (pos + T > D.maxseq) return fail("positions %d..%d past the context %d (the engine rejects the step)", pos,
                                        pos + T - 1, D.maxseq);
    // every (buffer, element) formed below must lie inside the buffer
    auto in = [&](const char* buf, size_t idx, size_t size) { return idx < size ? 0 : 1; };
    int bad = 0;
    const char* what = "";
    size_t at = 0, lim = 0;
    auto chk = [&](const char* buf, size_t idx, size_t size) {
        if (!bad && in(buf, idx, size)) { bad = 1; what = buf; at = idx; lim = size; }
    };
    // GEMM outputs: segment t = g * ks + s (tseg), rows g * 64 + lane, tokens < T
    auto gemm_out = [&](const char* buf, size_t base, int rows, int kseg, size_t size) {
        for (int t = 0; t < (rows / 64) * kseg; t++) {
            const int g = t / kseg, sg = t % kseg;
            for (int tok = 0; tok < T; tok++)
                chk(buf, base + ((size_t)sg * (T > 1 ? kMaxT : 1) + (T > 1 ? tok : 0)) * rows + g * 64 + 63, size);
        }
    };
    const int nch = (pos + T - 1 + kAttnChunk) / kAttnChunk;      // chunks of the last token's context
    if (nch > D.maxch) return fail("%d attention chunks > maxch %d", nch, D.maxch);
    for (int l = 0; l < NL; l++) {
        // K/V rows appended and read: positions 0 .. pos + T - 1 of every kv head
        for (int kvh = 0; kvh < NKV; kvh++) chk("kc/vc", lay::kv(NKV, D.maxseq, HD, l, kvh, pos + T - 1) + HD - 1, lay::kv_size(D));
        if (T == 1) {
            gemm_out("qkv_part", lay::qkv_part(ks[0], QKV, l), QKV, ks[0], lay::qkv_part_size(D));
            for (int h = 0; h < NH; h++)
                for (int c = 0; c < nch; c++) chk("att", lay::att(NH, D.maxch, D.arec, l) + (size_t)(h * D.maxch + c) * D.arec + HD + 1, lay::att_size(D));
            gemm_out("o_part", lay::o_part(ks[1], E, l), E, ks[1], lay::o_part_size(D));
            for (int g = 0; g < FF / 32; g++) chk("act", lay::act(FF, l) + (size_t)g * kActRec + 39, lay::act_size(D));
            gemm_out("d_part", lay::d_part(ks[3], E, l), E, ks[3], lay::d_part_size(D));
            continue;
        }
        // kT_in (qkv and gate/up inputs): residual rows of hT, the int8 records in xT
        for (int t = 0; t < T; t++) {
            chk("hT", lay::hT(E, 2 * l, t) + E - 1, lay::hT_size(D));
            chk("hT", lay::hT(E, 2 * l + 1, t) + E - 1, lay::hT_size(D));
            for (int w : {lay::kXtQkv, lay::kXtO, lay::kXtGu}) {
                // the writers' last byte, and the last byte of the GEMMs' copy of T tokens
                chk("xT", lay::xT(E, lay::xt_slot(NL, l, w)) + t * lay::xT_tok(E) + (size_t)(nbE - 1) * kTRec + kTRec - 1,
                    lay::xT_size(D));
                chk("xT", lay::xT(E, lay::xt_slot(NL, l, w)) + (size_t)(t + 1) * lay::xT_tok(E) - 1, lay::xT_size(D));
            }
            for (int sg = 0; sg < ks[3]; sg++)
                chk("dT", lay::dT(ks[3], E, l) + ((size_t)sg * kMaxT + t) * E + E - 1, lay::dT_size(D));
            for (int sg = 0; sg < D.ks_oT; sg++)
                chk("oT", lay::oT(D.ks_oT, E, l) + ((size_t)sg * kMaxT + t) * E + E - 1, lay::oT_size(D));
        }
        gemm_out("qkvT", lay::qkvT(ks[0], QKV, l), QKV, ks[0], lay::qkvT_size(D));
        // kT_attn items (kv head, chunk, token group) and the q/k/v rows they read
        int tg = 1;
        while (tg < T && NKV * nch * ((T + tg - 1) / tg) > n_cu) tg *= 2;
        const int ngrp = (T + tg - 1) / tg;
        for (int it = 0; it < NKV * nch * ngrp; it++) {
            const int grp = it % ngrp, rest = it / ngrp, c = rest % nch, kvh = rest / nch;
            const int ta = grp * tg, tb = std::min(T, ta + tg) - 1, t0 = c * kAttnChunk;
            if (t0 > pos + tb) continue;
            for (int t = ta; t <= tb; t++)
                for (int hh = 0; hh < G; hh++) {
                    const int h = kvh * G + hh;
                    for (int sg = 0; sg < ks[0]; sg++)
                        chk("qkvT", lay::qkvT(ks[0], QKV, l) + ((size_t)sg * kMaxT + t) * QKV + NH * HD + KVD + kvh * HD + HD - 1, lay::qkvT_size(D));
                    if (t0 <= pos + t)
                        chk("attT", lay::attT(NH, D.maxch, D.arec, l, t) + (size_t)(h * D.maxch + c) * D.arec + HD + 1, lay::attT_size(D));
                }
        }
        // kT_comb: token t merges its chunks 0 .. (pos + t) / 64
        for (int t = 0; t < T; t++)
            for (int h = 0; h < NH; h++) {
                const int nct = (pos + t + kAttnChunk) / kAttnChunk;
                chk("attT", lay::attT(NH, D.maxch, D.arec, l, t) + (size_t)(h * D.maxch + nct - 1) * D.arec + HD + 1, lay::attT_size(D));
            }
        gemm_out("oT", lay::oT(D.ks_oT, E, l), E, D.ks_oT, lay::oT_size(D));
        for (int t = 0; t < T; t++)
            for (int g = 0; g < FF / 32; g++) chk("actT", lay::actT(FF, l, t) + (size_t)g * kActRec + 39, lay::actT_size(D));
        for (int t = 0; t < T; t++) chk("actT", lay::actT(FF, l, t) + (size_t)(nbF - 1) * kActRec + kTRec - 1, lay::actT_size(D));
        gemm_out("dT", lay::dT(ks[3], E, l), E, ks[3], lay::dT_size(D));
    }
    if (T > 1) {
        for (int t = 0; t < T; t++) {
            chk("hT", lay::hT(E, 2 * (NL - 1) + 1, t) + E - 1, lay::hT_size(D));
            chk("xT", lay::xT(E, lay::xt_slot(NL, NL, 0)) + t * lay::xT_tok(E) + (size_t)(nbE - 1) * kTRec + kTRec - 1,
                lay::xT_size(D));
            chk("xT", lay::xT(E, lay::xt_slot(NL, NL, 0)) + (size_t)(t + 1) * lay::xT_tok(E) - 1, lay::xT_size(D));
            chk("logitsT", (size_t)t * V + V - 1, lay::logitsT_size(D));
            for (int w = 0; w < n_cu; w++) chk("candT", lay::candT(w, t) + 3, lay::candT_size(D));
        }
    }
    if (bad) return fail("%s index %zu outside its %zu elements (T=%d pos=%d)", what, at, lim, T, pos);
    return MI_OK;
}

int mi_debug_flag_barrier(mi_engine* e) {
    if (!e) return MI_ERR_ARG;
    if (!e->nwg_persistent) return set_err(e, MI_ERR_STATE, "no persistent step kernel");
    const int32_t one = 1;
    HIPCHK(e, hipMemcpy(e->M.err, &one, 4, hipMemcpyHostToDevice));
    return MI_OK;
}

}  // extern "C"

// One multi-token step (T > 1) at positions pos..pos+T-1: with the persistent step, one
// persistent launch (kT_step), otherwise one launch per phase. The kernels read the
// position from posT, so the launch sequence of each (logits, T) can be captured once
// into a HIP graph and replayed at any position.
static int run_multi(mi_engine* e, int pos, int T, bool want_logits) {
    const DModel& M = want_logits ? e->M_logits : e->M;
    const DModel* dM = e->dM + (want_logits ? 1 : 0);
    HIPCHK(e, hipMemcpyAsync(e->M.posT, e->h_iota + pos, sizeof(int32_t), hipMemcpyHostToDevice, e->stream));
    auto launch = [&]() -> hipError_t {
        if (e->nwg_persistent && e->multi_persistent) {
            const hipError_t err = launch_step_multi_persistent(M, dM, e->nwg_persistent, T, e->coop, e->stream);
            if (err != hipErrorIllegalState && err != hipErrorCooperativeLaunchTooLarge) return err;
            // the runtime refused the cooperative launch itself (nothing ran): the per-phase
            // launches compute the same values
            (void)hipGetLastError();
            e->multi_persistent = false;
        }
        launch_step_multi(M, dM, e->n_cu, T, e->stream);
        return hipGetLastError();
    };
    // A cooperative launch is never captured: the fallback must reach the runtime as a
    // cooperative dispatch every time (check_barrier drops the graphs when it switches).
    if (!e->opts.graphs || (e->coop && e->nwg_persistent && e->multi_persistent)) {
        HIPCHK(e, launch());
        return MI_OK;
    }
    hipGraphExec_t& g = e->gexec[want_logits ? 1 : 0][T];
    if (!g) {
        hipGraph_t graph = nullptr;
        HIPCHK(e, hipStreamBeginCapture(e->stream, hipStreamCaptureModeThreadLocal));
        const hipError_t launched = launch();
        const hipError_t ended = hipStreamEndCapture(e->stream, &graph);
        HIPCHK(e, launched);
        HIPCHK(e, ended);
        const hipError_t inst = hipGraphInstantiate(&g, graph, nullptr, nullptr, 0);
        (void)hipGraphDestroy(graph);
        if (inst != hipSuccess) g = nullptr;
        HIPCHK(e, inst);
    }
    HIPCHK(e, hipGraphLaunch(g, e->stream));
    return MI_OK;
}

static int run_step(mi_engine* e, int pos, int gen, bool want_logits) {
    const DModel& M = want_logits ? e->M_logits : e->M;
    const DModel* dM = e->dM + (want_logits ? 1 : 0);
    if (e->nwg_persistent) {
        const hipError_t err = launch_step_persistent(M, dM, e->nwg_persistent, pos, gen, e->coop, e->stream);
        if (err == hipErrorIllegalState || err == hipErrorCooperativeLaunchTooLarge) {
            // The runtime refused the cooperative launch itself (seen while another process
            // holds the device's cooperative dispatch); nothing ran. The per-phase launches
            // compute the same values, so the engine continues in that mode (mi_info reports it).
            (void)hipGetLastError();
            e->nwg_persistent = 0;
            launch_step_phases(M, dM, e->n_cu, pos, gen, e->stream);
        } else {
            HIPCHK(e, err);
        }
    } else {
        launch_step_phases(M, dM, e->n_cu, pos, gen, e->stream);
    }
    HIPCHK(e, hipGetLastError());
    return MI_OK;
}

// after a synchronization: a grid barrier that timed out leaves a flag. The persistent
// kernel goes out as a plain launch, which needs every workgroup resident at once (true
// on an otherwise idle device). If a barrier gave up (another process held CUs), the
// barrier state is cleared, the engine switches to cooperative launches (the runtime
// then waits until all workgroups fit) and the caller recomputes: kRetry.
constexpr int kRetry = 1 << 20;
static int check_barrier(mi_engine* e) {
    if (!e->nwg_persistent) return MI_OK;
    int32_t flag = 0;
    HIPCHK(e, hipMemcpy(&flag, e->M.err, 4, hipMemcpyDeviceToHost));
    if (flag) {
        // a failed launch may leave its counters set: clear them for the next launch
        HIPCHK(e, hipMemset(e->M.bar, 0, sizeof(uint32_t) * barrier_words()));
        HIPCHK(e, hipMemset(e->M.err, 0, 4));
        if (!e->coop) {
            e->coop = true;
            // graphs captured so far hold plain launches of the persistent kernel
            for (auto& row : e->gexec)
                for (hipGraphExec_t& g : row)
                    if (g) {
                        (void)hipGraphExecDestroy(g);
                        g = nullptr;
                    }
            return kRetry;
        }
        return set_err(e, MI_ERR_DEVICE, "grid barrier timed out under a cooperative launch");
    }
    return MI_OK;
}

// Generation that hands each token over as it is made (a callback, or a stop at eos),
// from token t0 on: one step, then its token fetched and delivered. Token t is the
// prediction at position p0 + t - 1 (t = 0: the prefill's). `steps0` steps already ran.
static int generate_sync(mi_engine* e, int p0, int t0, int steps0, int n_gen, int32_t* out, float* margins,
                         int32_t* n_out, mi_token_cb cb, void* user) {
    auto fetch = [&](int pos, int32_t* t, float* m) -> int {
        HIPCHK(e, hipMemcpyAsync(t, e->M.out_tok + pos, 4, hipMemcpyDeviceToHost, e->stream));
        HIPCHK(e, hipMemcpyAsync(m, e->M.out_margin + pos, 4, hipMemcpyDeviceToHost, e->stream));
        HIPCHK(e, hipStreamSynchronize(e->stream));
        return MI_OK;
    };
    if (t0 == 0) HIPCHK(e, hipEventRecord(e->ev0, e->stream));
    int emitted = t0, steps = steps0;
    for (int t = t0; t < n_gen; t++) {
        if (t > 0) {
            const int rc = run_step(e, p0 + t - 1, 1, false);
            if (rc) return rc;
            steps++;
        }
        int32_t tok; float m;
        int rc = fetch(p0 + t - 1, &tok, &m);
        if (rc) return rc;
        if (t > 0 && (rc = check_barrier(e))) {
            if (rc != kRetry) return rc;
            if ((rc = run_step(e, p0 + t - 1, 1, false)) || (rc = fetch(p0 + t - 1, &tok, &m))) return rc;
            if ((rc = check_barrier(e))) return rc == kRetry ? MI_ERR_DEVICE : rc;
        }
        if (out) out[t] = tok;
        if (margins) margins[t] = m;
        emitted++;
        if ((cb && cb(tok, user)) || (e->opts.stop_eos && tok == e->eos)) break;
    }
    HIPCHK(e, hipEventRecord(e->ev1, e->stream));
    HIPCHK(e, hipStreamSynchronize(e->stream));
    float ms = 0.f;
    HIPCHK(e, hipEventElapsedTime(&ms, e->ev0, e->ev1));
    e->stats.decode_ms = ms;
    e->stats.steps = e->stats.tokens = steps;
    e->cur_len = p0 + steps;
    if (n_out) *n_out = emitted;
    return MI_OK;
}

// Streaming generation with the persistent step (mega.cu:847-856, 1165-1178): the steps
// go out up to kRingAhead launches ahead of the tokens the host has delivered; each
// writes its token and margin to the mapped host ring (one 64-bit word at ring[pos]),
// which the host polls, so no step waits for the host. A stop (the callback, or eos)
// leaves at most kRingAhead - 1 queued steps to run past it; after an eos they return
// at once (k_step passes the eos on). Their K/V rows lie past the context length the
// call leaves, so nothing reads them. A ring entry kRingFail (a grid barrier of that
// launch gave up) is never delivered: the launches drain, the barrier state is reset,
// and the rest runs through generate_sync with cooperative launches.
constexpr int kRingAhead = 8;
static int generate_ring(mi_engine* e, int n_gen, int32_t* out, float* margins, int32_t* n_out, mi_token_cb cb,
                         void* user) {
    const int p0 = e->cur_len;
    if (n_gen == 0) {
        if (n_out) *n_out = 0;
        e->stats.steps = e->stats.tokens = 0;
        e->stats.decode_ms = 0;
        return MI_OK;
    }
    int32_t tok = 0;
    float m = 0.f;
    HIPCHK(e, hipMemcpyAsync(&tok, e->M.out_tok + p0 - 1, 4, hipMemcpyDeviceToHost, e->stream));
    HIPCHK(e, hipMemcpyAsync(&m, e->M.out_margin + p0 - 1, 4, hipMemcpyDeviceToHost, e->stream));
    HIPCHK(e, hipStreamSynchronize(e->stream));
    for (int p = p0; p < p0 + n_gen - 1; p++) __atomic_store_n(e->h_ring + p, kRingEmpty, __ATOMIC_RELAXED);
    HIPCHK(e, hipEventRecord(e->ev0, e->stream));
    int emitted = 0, got = 0, enq = 0;
    bool stop = false, failed = false;
    auto deliver = [&](int32_t t, float mg) {
        if (out) out[emitted] = t;
        if (margins) margins[emitted] = mg;
        emitted++;
        if ((cb && cb(t, user)) || (e->opts.stop_eos && t == e->eos)) stop = true;
    };
    deliver(tok, m);
    auto last = std::chrono::steady_clock::now();
    while (!stop && got < n_gen - 1) {
        for (; enq < n_gen - 1 && enq < got + kRingAhead; enq++)
            if (int rc = run_step(e, p0 + enq, kGenRing, false)) return rc;
        const uint64_t w = __atomic_load_n(e->h_ring + p0 + got, __ATOMIC_ACQUIRE);
        if (w == kRingEmpty) {
            const hipError_t q = hipStreamQuery(e->stream);
            if (q == hipSuccess) {
                // the stream is idle: the entry is there now, or no launch will write it
                if (__atomic_load_n(e->h_ring + p0 + got, __ATOMIC_ACQUIRE) != kRingEmpty) continue;
                return set_err(e, MI_ERR_DEVICE, "streaming generate: no token for position %d", p0 + got);
            }
            if (q != hipErrorNotReady) return set_err(e, MI_ERR_DEVICE, "hipStreamQuery: %s", hipGetErrorString(q));
            if (std::chrono::steady_clock::now() - last > std::chrono::seconds(30))
                return set_err(e, MI_ERR_DEVICE, "streaming generate: no token for 30 s");
            std::this_thread::sleep_for(std::chrono::microseconds(20));
            continue;
        }
        if (w == kRingFail) {
            failed = true;
            break;
        }
        last = std::chrono::steady_clock::now();
        got++;
        const uint32_t mb = (uint32_t)(w >> 32);
        float mg;
        std::memcpy(&mg, &mb, 4);
        deliver((int32_t)(uint32_t)w, mg);
    }
    HIPCHK(e, hipEventRecord(e->ev1, e->stream));
    HIPCHK(e, hipStreamSynchronize(e->stream));
    if (failed) {
        const int rc = check_barrier(e);
        if (rc != kRetry) return rc ? rc : set_err(e, MI_ERR_DEVICE, "streaming generate: failed step at %d", p0 + got);
        // positions before p0 + got are good and tokbuf[p0 + got] holds their last token
        return generate_sync(e, p0, got + 1, got, n_gen, out, margins, n_out, cb, user);
    }
    // a barrier that gave up only at a launch's last barrier (after its results were
    // complete) still leaves the flag: reset it (the delivered tokens are right)
    if (int rc = check_barrier(e); rc && rc != kRetry) return rc;
    float ms = 0.f;
    HIPCHK(e, hipEventElapsedTime(&ms, e->ev0, e->ev1));
    e->stats.decode_ms = ms;
    e->stats.steps = e->stats.tokens = got;
    e->cur_len = p0 + got;
    if (n_out) *n_out = emitted;
    return MI_OK;
}

extern "C" {

int mi_step(mi_engine* e, const int32_t* toks, int32_t T, int32_t pos, int32_t* argmax, float* margin, float* logits) {
    if (!e || !toks) return MI_ERR_ARG;
    if (T < 1 || T > kernels_max_tokens())
        return set_err(e, MI_ERR_ARG, "mi_step: T=%d outside 1..%d", T, kernels_max_tokens());
    if (pos < 0 || pos > e->cur_len || pos + T > e->maxseq) return set_err(e, MI_ERR_ARG, "mi_step: position %d out of range (length %d, capacity %d)", pos, e->cur_len, e->maxseq);
    for (int t = 0; t < T; t++)
        if (toks[t] < 0 || toks[t] >= e->V) return set_err(e, MI_ERR_ARG, "mi_step: token %d out of range", toks[t]);
    HIPCHK(e, hipMemcpyAsync(e->M.tokbuf + pos, toks, sizeof(int32_t) * T, hipMemcpyHostToDevice, e->stream));
    int rc;
    if (T == 1) {
        rc = run_step(e, pos, 1, logits != nullptr);
    } else {
        rc = run_multi(e, pos, T, logits != nullptr);
    }
    if (rc) return rc;
    std::vector<int32_t> tok(T);
    std::vector<float> mg(T);
    HIPCHK(e, hipMemcpyAsync(tok.data(), e->M.out_tok + pos, 4 * T, hipMemcpyDeviceToHost, e->stream));
    HIPCHK(e, hipMemcpyAsync(mg.data(), e->M.out_margin + pos, 4 * T, hipMemcpyDeviceToHost, e->stream));
    if (logits)
        HIPCHK(e, hipMemcpyAsync(logits, T == 1 ? e->M_logits.logits : e->M_logits.logitsT, sizeof(float) * e->V * T,
                                 hipMemcpyDeviceToHost, e->stream));
    HIPCHK(e, hipStreamSynchronize(e->stream));
    if ((rc = check_barrier(e))) return rc == kRetry ? mi_step(e, toks, T, pos, argmax, margin, logits) : rc;
    for (int t = 0; t < T; t++) {
        if (argmax) argmax[t] = tok[t];
        if (margin) margin[t] = mg[t];
    }
    // the next position's token is the last prediction (mi_generate continues from it)
    HIPCHK(e, hipMemcpyAsync(e->M.tokbuf + pos + T, &tok[T - 1], 4, hipMemcpyHostToDevice, e->stream));
    HIPCHK(e, hipStreamSynchronize(e->stream));
    e->cur_len = pos + T;
    e->next_ready = true;
    return MI_OK;
}

int mi_prefill(mi_engine* e, const int32_t* ids, int32_t n, int32_t* first, float* margin) {
    if (!e || !ids || n < 1) return MI_ERR_ARG;
    if (n >= e->maxseq) return set_err(e, MI_ERR_ARG, "prompt of %d tokens exceeds the context capacity %d", n, e->maxseq);
    for (int i = 0; i < n; i++)
        if (ids[i] < 0 || ids[i] >= e->V) return set_err(e, MI_ERR_ARG, "prompt token %d out of range", ids[i]);
    HIPCHK(e, hipMemcpyAsync(e->M.tokbuf, ids, sizeof(int32_t) * n, hipMemcpyHostToDevice, e->stream));
    HIPCHK(e, hipEventRecord(e->ev0, e->stream));
    // chunks of tchunk tokens through the multi-token step (cuda_infer.cu:1133-1144,
    // mega.cu:622, 819-820); its results equal one step per token bit for bit
    for (int p = 0; p < n;) {
        const int T = std::min(e->opts.tchunk, n - p);
        if (T == 1) {
            if (int rc = run_step(e, p, p == n - 1, false)) return rc;
        } else {
            if (int rc = run_multi(e, p, T, false)) return rc;
            if (p + T == n)   // the next position's token is the last prediction
                HIPCHK(e, hipMemcpyAsync(e->M.tokbuf + n, e->M.out_tok + n - 1, 4, hipMemcpyDeviceToDevice, e->stream));
        }
        p += T;
    }
    HIPCHK(e, hipEventRecord(e->ev1, e->stream));
    int32_t tok = 0;
    float mg = 0.f;
    HIPCHK(e, hipMemcpyAsync(&tok, e->M.out_tok + n - 1, 4, hipMemcpyDeviceToHost, e->stream));
    HIPCHK(e, hipMemcpyAsync(&mg, e->M.out_margin + n - 1, 4, hipMemcpyDeviceToHost, e->stream));
    HIPCHK(e, hipStreamSynchronize(e->stream));
    if (int rc = check_barrier(e)) return rc == kRetry ? mi_prefill(e, ids, n, first, margin) : rc;
    float ms = 0.f;
    HIPCHK(e, hipEventElapsedTime(&ms, e->ev0, e->ev1));
    e->stats.prefill_ms = ms;
    if (first) *first = tok;
    if (margin) *margin = mg;
    e->cur_len = n;
    e->next_ready = true;
    return MI_OK;
}

// Teacher forcing (mega.cu:857-862): the prefill's chunks over the whole sequence; every
// step writes its positions' argmax and margin to out_tok / out_margin, which are read
// back at the end. No step feeds its prediction forward (ids are the context).
int mi_teacher(mi_engine* e, const int32_t* ids, int32_t n, int32_t* pred, float* margin) {
    if (!e || !ids || !pred || !margin || n < 1) return MI_ERR_ARG;
    if (n > e->maxseq) return set_err(e, MI_ERR_ARG, "teacher sequence of %d tokens exceeds the context capacity %d", n, e->maxseq);
    for (int i = 0; i < n; i++)
        if (ids[i] < 0 || ids[i] >= e->V) return set_err(e, MI_ERR_ARG, "teacher token %d out of range", ids[i]);
    HIPCHK(e, hipMemcpyAsync(e->M.tokbuf, ids, sizeof(int32_t) * n, hipMemcpyHostToDevice, e->stream));
    for (int p = 0; p < n;) {
        const int T = std::min(e->opts.tchunk, n - p);
        if (T == 1) {
            if (int rc = run_step(e, p, 0, false)) return rc;
        } else {
            if (int rc = run_multi(e, p, T, false)) return rc;
        }
        p += T;
    }
    HIPCHK(e, hipMemcpyAsync(pred, e->M.out_tok, sizeof(int32_t) * n, hipMemcpyDeviceToHost, e->stream));
    HIPCHK(e, hipMemcpyAsync(margin, e->M.out_margin, sizeof(float) * n, hipMemcpyDeviceToHost, e->stream));
    HIPCHK(e, hipStreamSynchronize(e->stream));
    if (int rc = check_barrier(e)) return rc == kRetry ? mi_teacher(e, ids, n, pred, margin) : rc;
    e->cur_len = n;
    e->next_ready = false;
    return MI_OK;
}

}  // extern "C"

// T tokens already in tokbuf[pos..pos+T-1]: one step, predictions back to the host
static int run_tokens(mi_engine* e, int pos, int T, int32_t* tok, float* mg) {
    if (T == 1) {
        if (int rc = run_step(e, pos, 1, false)) return rc;
    } else {
        if (int rc = run_multi(e, pos, T, false)) return rc;
    }
    HIPCHK(e, hipMemcpyAsync(tok, e->M.out_tok + pos, 4 * T, hipMemcpyDeviceToHost, e->stream));
    HIPCHK(e, hipMemcpyAsync(mg, e->M.out_margin + pos, 4 * T, hipMemcpyDeviceToHost, e->stream));
    HIPCHK(e, hipStreamSynchronize(e->stream));
    const int rc = check_barrier(e);
    return rc == kRetry ? run_tokens(e, pos, T, tok, mg) : rc;
}

// Speculative generation driven on the device (mega.cu:863-895: the reference drafts,
// commits and adapts K inside its persistent loop): the same steps as generate_spec below,
// in the same float arithmetic, but each verify launch reads its T and position from
// M.spec / posT and commits on the device (spec_commit), so the host only drafts the first
// step, queues launches and reads the result once. A launch after the generation finished
// returns at once; at most n_gen - 1 steps are needed (each emits at least one token).
// (sp below is the host copy; it is read back from the device after each batch.)
static int generate_spec_device(mi_engine* e, int n_gen, int32_t* out, float* margins, int32_t* n_out) {
    const int p0 = e->cur_len;
    const int TM = kernels_max_tokens();
    std::vector<int32_t> hist((size_t)p0 + TM + 1);
    HIPCHK(e, hipMemcpy(hist.data(), e->M.tokbuf, sizeof(int32_t) * (p0 + 1), hipMemcpyDeviceToHost));
    const int eos = e->opts.stop_eos ? e->eos : -1;
    SpecDev sp{};
    sp.emitted = n_gen > 0 ? 1 : 0;                  // the prefill's prediction, tokbuf[p0]
    sp.n_gen = n_gen;
    sp.eos = eos;
    sp.last_pos = p0;
    sp.ngmax = e->opts.ngmax;
    sp.maxseq = e->maxseq;
    sp.tmax = TM;
    sp.acc_num = 0.6f;
    sp.acc_den = 1.f;
    sp.slope = e->opts.spec_slope;
    sp.done = n_gen <= 1 || (eos >= 0 && hist[p0] == eos);
    if (!sp.done) {
        const float alpha = std::min(std::max(sp.acc_num / sp.acc_den, 0.01f), 0.99f);
        const int kmax = std::min(mi_best_draft_len(alpha, sp.slope, TM), std::min(n_gen - 2, e->maxseq - 1 - p0));
        const int K = kmax > 0 ? mi_ngram_draft(hist.data(), p0 + 1, sp.ngmax, kmax, hist.data() + p0 + 1) : 0;
        sp.T = K + 1;                                // tokbuf[p0] already holds the current token
        if (K > 0)
            HIPCHK(e, hipMemcpyAsync(e->M.tokbuf + p0 + 1, hist.data() + p0 + 1, sizeof(int32_t) * K, hipMemcpyHostToDevice, e->stream));
    }
    HIPCHK(e, hipMemcpyAsync(e->M.spec, &sp, sizeof(SpecDev), hipMemcpyHostToDevice, e->stream));
    HIPCHK(e, hipMemcpyAsync(e->M.posT, e->h_iota + p0, sizeof(int32_t), hipMemcpyHostToDevice, e->stream));
    const auto t_start = std::chrono::steady_clock::now();
    // launches in batches of kSpecBatch, the state read back after each: a generation
    // that finished early leaves at most kSpecBatch - 1 launches that return at once
    constexpr int kSpecBatch = 16;
    for (int queued = 0; !sp.done && queued < n_gen - 1;) {
        const int nb = std::min(kSpecBatch, n_gen - 1 - queued);
        for (int i = 0; i < nb; i++) HIPCHK(e, launch_spec_step(e->M, e->dM, e->nwg_persistent, e->coop, e->stream));
        queued += nb;
        HIPCHK(e, hipMemcpyAsync(&sp, e->M.spec, sizeof(SpecDev), hipMemcpyDeviceToHost, e->stream));
        HIPCHK(e, hipStreamSynchronize(e->stream));
    }
    if (int rc = check_barrier(e)) return rc == kRetry ? generate_spec_device(e, n_gen, out, margins, n_out) : rc;
    const double ms = std::chrono::duration<double, std::milli>(std::chrono::steady_clock::now() - t_start).count();
    const int emitted = sp.emitted;
    if (emitted > 0) {
        // emitted token k is the prediction after position p0 - 1 + k
        if (out) HIPCHK(e, hipMemcpy(out, e->M.out_tok + p0 - 1, sizeof(int32_t) * emitted, hipMemcpyDeviceToHost));
        if (margins) HIPCHK(e, hipMemcpy(margins, e->M.out_margin + p0 - 1, sizeof(float) * emitted, hipMemcpyDeviceToHost));
    }
    e->stats.decode_ms = ms;
    e->stats.steps = sp.steps;
    e->stats.tokens = emitted;
    e->stats.drafted = sp.drafted;
    e->stats.accepted = sp.accepted;
    e->cur_len = sp.last_pos;                        // the last emitted token sits there (tokbuf), K/V not computed
    e->next_ready = true;
    if (n_out) *n_out = emitted;
    return MI_OK;
}

// Lossless speculative generation (mega.cu:863-895): each step runs [cur, draft]
// at positions pos..pos+K and commits the predictions up to and including the first
// one that disagrees with its draft. A token's logits do not depend on how many
// tokens share the step, so the output is the plain greedy decode token for token.
static int generate_spec(mi_engine* e, int n_gen, int32_t* out, float* margins, int32_t* n_out, mi_token_cb cb,
                         void* user) {
    const int p0 = e->cur_len;                   // position of the current (first) token
    const int TM = kernels_max_tokens();
    std::vector<int32_t> hist((size_t)p0 + n_gen + TM + 1);
    HIPCHK(e, hipMemcpy(hist.data(), e->M.tokbuf, sizeof(int32_t) * (p0 + 1), hipMemcpyDeviceToHost));
    float mg0 = 0.f;
    HIPCHK(e, hipMemcpy(&mg0, e->M.out_margin + p0 - 1, 4, hipMemcpyDeviceToHost));
    int pos = p0, emitted = 0, last_pos = p0, steps = 0, drafted = 0, accepted = 0;
    bool done = n_gen == 0;
    auto emit = [&](int32_t t, float m, int at) {
        if (out) out[emitted] = t;
        if (margins) margins[emitted] = m;
        emitted++;
        last_pos = at;
        const bool stop = cb && cb(t, user);     // every emitted token reaches the callback
        done = stop || emitted >= n_gen || (e->opts.stop_eos && t == e->eos);
    };
    int32_t cur = hist[p0];
    if (!done) emit(cur, mg0, p0);
    float acc_num = 0.6f, acc_den = 1.f;         // EWMA of accepted drafts / (accepted + rejections), mega.cu:613
    const auto t_start = std::chrono::steady_clock::now();
    while (!done) {
        const float alpha = std::min(std::max(acc_num / acc_den, 0.01f), 0.99f);
        const int kmax = std::min(mi_best_draft_len(alpha, e->opts.spec_slope, TM),
                                  std::min(n_gen - emitted - 1, e->maxseq - 1 - pos));
        int32_t toks[16], y[16];
        float ym[16];
        toks[0] = cur;
        const int K = kmax > 0 ? mi_ngram_draft(hist.data(), pos + 1, e->opts.ngmax, kmax, toks + 1) : 0;
        HIPCHK(e, hipMemcpyAsync(e->M.tokbuf + pos, toks, sizeof(int32_t) * (K + 1), hipMemcpyHostToDevice, e->stream));
        if (int rc = run_tokens(e, pos, K + 1, y, ym)) return rc;
        int a = 0;
        while (a < K && toks[1 + a] == y[a]) a++;
        for (int i = 0; i <= a && !done; i++) {
            hist[pos + 1 + i] = y[i];
            emit(y[i], ym[i], pos + 1 + i);
        }
        cur = y[a];
        pos += a + 1;
        if (K > 0) {
            acc_num = 0.85f * acc_num + 0.15f * a;
            acc_den = 0.85f * acc_den + 0.15f * (a + (a < K ? 1 : 0));
        }
        steps++;
        drafted += K;
        accepted += a;
    }
    const double ms = std::chrono::duration<double, std::milli>(std::chrono::steady_clock::now() - t_start).count();
    // the last emitted token sits at last_pos with its K/V not yet computed (as after a plain generate)
    HIPCHK(e, hipMemcpy(e->M.tokbuf + last_pos, &hist[last_pos], 4, hipMemcpyHostToDevice));
    e->stats.decode_ms = ms;
    e->stats.steps = steps;
    e->stats.tokens = emitted;
    e->stats.drafted = drafted;
    e->stats.accepted = accepted;
    e->cur_len = last_pos;
    e->next_ready = true;
    if (n_out) *n_out = emitted;
    return MI_OK;
}

extern "C" {

int mi_generate(mi_engine* e, int32_t n_gen, int32_t* out, float* margins, int32_t* n_out, mi_token_cb cb, void* user) {
    if (!e || n_gen < 0) return MI_ERR_ARG;
    if (!e->next_ready || e->cur_len < 1) return set_err(e, MI_ERR_STATE, "mi_generate needs mi_prefill first");
    if (e->cur_len + n_gen > e->maxseq) return set_err(e, MI_ERR_ARG, "n_gen %d exceeds the context capacity", n_gen);
    if (e->opts.spec) {
        if (e->opts.spec == 2 && e->nwg_persistent && e->multi_persistent && !cb)
            return generate_spec_device(e, n_gen, out, margins, n_out);
        return generate_spec(e, n_gen, out, margins, n_out, cb, user);
    }
    e->stats.drafted = e->stats.accepted = 0;
    const int p0 = e->cur_len;                   // position of the first generated token
    const bool sync_each = cb != nullptr || e->opts.stop_eos;
    if (sync_each && e->nwg_persistent) return generate_ring(e, n_gen, out, margins, n_out, cb, user);
    if (sync_each) return generate_sync(e, p0, 0, 0, n_gen, out, margins, n_out, cb, user);
    HIPCHK(e, hipEventRecord(e->ev0, e->stream));
    int steps = 0;
    for (int t = 1; t < n_gen; t++, steps++) {
        const int rc = run_step(e, p0 + t - 1, 1, false);
        if (rc) return rc;
    }
    HIPCHK(e, hipEventRecord(e->ev1, e->stream));
    std::vector<int32_t> tk(n_gen > 0 ? n_gen : 1);
    std::vector<float> mg(n_gen > 0 ? n_gen : 1);
    if (n_gen > 0) {
        HIPCHK(e, hipMemcpyAsync(tk.data(), e->M.out_tok + p0 - 1, sizeof(int32_t) * n_gen, hipMemcpyDeviceToHost, e->stream));
        HIPCHK(e, hipMemcpyAsync(mg.data(), e->M.out_margin + p0 - 1, sizeof(float) * n_gen, hipMemcpyDeviceToHost, e->stream));
    }
    HIPCHK(e, hipStreamSynchronize(e->stream));
    if (int rc = check_barrier(e))   // the launches only wrote positions p0.. and tokbuf[p0+1..]
        return rc == kRetry ? mi_generate(e, n_gen, out, margins, n_out, cb, user) : rc;
    for (int t = 0; t < n_gen; t++) {
        if (out) out[t] = tk[t];
        if (margins) margins[t] = mg[t];
    }
    float ms = 0.f;
    HIPCHK(e, hipEventElapsedTime(&ms, e->ev0, e->ev1));
    e->stats.decode_ms = ms;
    e->stats.steps = e->stats.tokens = steps;
    e->cur_len = p0 + steps;
    if (n_out) *n_out = n_gen;
    return MI_OK;
}

int mi_time_phase(mi_engine* e, int32_t phase, int32_t layer, int32_t reps, double* avg_ms) {
    if (!e || !avg_ms || phase < 0 || phase > 8 || layer < 0 || layer >= e->NL || reps < 1) return MI_ERR_ARG;
    if (e->cur_len < 1) return set_err(e, MI_ERR_STATE, "mi_time_phase needs a completed step");
    if (phase == 8 && !e->nwg_persistent) return set_err(e, MI_ERR_STATE, "phase 8 is the persistent step kernel");
    const int pos = e->cur_len - 1;
    HIPCHK(e, hipEventRecord(e->ev0, e->stream));
    for (int r = 0; r < reps; r++) {
        if (phase == 8) HIPCHK(e, launch_step_persistent(e->M, e->dM, e->nwg_persistent, pos, 1, e->coop, e->stream));
        else launch_phase(e->M, e->dM, e->n_cu, phase, layer, pos, 1, e->stream);
    }
    HIPCHK(e, hipGetLastError());
    HIPCHK(e, hipEventRecord(e->ev1, e->stream));
    HIPCHK(e, hipEventSynchronize(e->ev1));
    if (phase == 8) {
        const int rc = check_barrier(e);
        if (rc) return rc == kRetry ? mi_time_phase(e, phase, layer, reps, avg_ms) : rc;
    }
    float ms = 0.f;
    HIPCHK(e, hipEventElapsedTime(&ms, e->ev0, e->ev1));
    *avg_ms = ms / reps;
    return MI_OK;
}

int mi_profile_step(mi_engine* e, double* us, int32_t n) {
    if (!e || !us) return MI_ERR_ARG;
    if (!e->nwg_persistent) return set_err(e, MI_ERR_STATE, "profiling needs the persistent step kernel");
    if (e->cur_len < 1) return set_err(e, MI_ERR_STATE, "mi_profile_step needs a completed step");
    const int nslot = prof_slots(e->NL), nwg = e->nwg_persistent;
    const size_t total = (size_t)nslot * nwg;
    if ((size_t)n < total) return set_err(e, MI_ERR_ARG, "mi_profile_step needs %zu entries", total);
    uint64_t* prof = nullptr;
    HIPCHK(e, hipMalloc(&prof, sizeof(uint64_t) * total));
    DModel M = e->M;
    M.prof = prof;
    hipError_t st = hipMemcpy(e->dM + 2, &M, sizeof(DModel), hipMemcpyHostToDevice);
    if (st == hipSuccess) st = launch_step_persistent(M, e->dM + 2, nwg, e->cur_len - 1, 1, e->coop, e->stream);
    std::vector<uint64_t> t(total);
    if (st == hipSuccess) st = hipStreamSynchronize(e->stream);
    if (st == hipSuccess) st = hipMemcpy(t.data(), prof, sizeof(uint64_t) * total, hipMemcpyDeviceToHost);
    (void)hipFree(prof);
    if (st != hipSuccess) return set_err(e, MI_ERR_DEVICE, "profile step: %s", hipGetErrorString(st));
    uint64_t t0 = t[0];
    for (int w = 1; w < nwg; w++) t0 = std::min(t0, t[(size_t)w * nslot]);
    for (size_t i = 0; i < total; i++) us[i] = (double)(int64_t)(t[i] - t0) * 0.01;   // 100 MHz ticks
    const int rc = check_barrier(e);
    return rc == kRetry ? mi_profile_step(e, us, n) : rc;
}

int mi_barrier_cost(int32_t nwg, int32_t n, double* us_per_barrier) {
    if (nwg < 1 || n < 1 || !us_per_barrier) return MI_ERR_ARG;
    uint32_t* bar = nullptr;
    int32_t* err = nullptr;
    hipEvent_t a, b;
    if (hipMalloc(&bar, sizeof(uint32_t) * barrier_words()) != hipSuccess || hipMalloc(&err, 64) != hipSuccess) return MI_ERR_OOM;
    (void)hipMemset(err, 0, 64);
    (void)hipEventCreate(&a);
    (void)hipEventCreate(&b);
    hipError_t st = launch_barriers(bar, err, nwg, 8, nullptr);   // warm up
    (void)hipEventRecord(a, nullptr);
    if (st == hipSuccess) st = launch_barriers(bar, err, nwg, n, nullptr);
    (void)hipEventRecord(b, nullptr);
    if (st == hipSuccess) st = hipEventSynchronize(b);
    float ms = 0.f;
    int32_t flag = 0;
    if (st == hipSuccess) st = hipEventElapsedTime(&ms, a, b);
    if (st == hipSuccess) st = hipMemcpy(&flag, err, 4, hipMemcpyDeviceToHost);
    (void)hipEventDestroy(a);
    (void)hipEventDestroy(b);
    (void)hipFree(bar);
    (void)hipFree(err);
    if (st != hipSuccess || flag) return MI_ERR_DEVICE;
    *us_per_barrier = ms * 1000.0 / n;
    return MI_OK;
}

int mi_get_stats(const mi_engine* e, mi_stats* out) {
    if (!e || !out) return MI_ERR_ARG;
    *out = e->stats;
    return MI_OK;
}

int32_t mi_token_text(const mi_engine* e, int32_t id, char* out, int32_t cap) {
    if (!e || cap < 0 || (cap > 0 && !out)) return MI_ERR_ARG;
    const auto& v = e->gguf.tokens();
    if (id < 0 || id >= (int32_t)v.size()) return MI_ERR_ARG;
    return mi_detok_piece(v[id].data(), (int32_t)v[id].size(), out, cap);
}

// ---------------------------------------------------------------- kernel-level entry points
static int g_ncu = 0;
static int ncu() {
    if (!g_ncu) {
        int dev = 0;
        if (hipGetDevice(&dev) != hipSuccess || hipDeviceGetAttribute(&g_ncu, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess)
            g_ncu = 256;
    }
    return g_ncu;
}

int mi_quant_q8(const float* x, int32_t n, int8_t* xq, float* xd, int32_t* xs8, void* stream) {
    if (!x || !xq || !xd || !xs8 || n <= 0 || n % 32) return MI_ERR_ARG;
    launch_quant(x, n, xq, xd, xs8, (hipStream_t)stream);
    return hipGetLastError() == hipSuccess ? MI_OK : MI_ERR_DEVICE;
}

int mi_gemv_q4(const uint8_t* packed, int32_t rows, int32_t nb, int32_t cb, int32_t ks, const int8_t* xq,
               const float* xd, const int32_t* xs8, float* part, float* y, void* stream) {
    if (!packed || !xq || !xd || !xs8 || !part || !mi_q4_packed_bytes(rows, nb, cb) || ks < 1 || ks > nb / cb ||
        nb * 32 > kMaxFF)
        return MI_ERR_ARG;
    const PMat W{packed, rows, nb, cb, nb / cb, ks};
    launch_gemv(W, xq, xd, xs8, part, y, ncu(), (hipStream_t)stream);
    return hipGetLastError() == hipSuccess ? MI_OK : MI_ERR_DEVICE;
}

int mi_q4_block_isums(const uint8_t* packed, int32_t rows, int32_t nb, int32_t cb, const int8_t* xq, int32_t* isum,
                      void* stream) {
    if (!packed || !xq || !isum || !mi_q4_packed_bytes(rows, nb, cb)) return MI_ERR_ARG;
    const PMat W{packed, rows, nb, cb, nb / cb, 1};
    launch_isums(W, xq, isum, (hipStream_t)stream);
    return hipGetLastError() == hipSuccess ? MI_OK : MI_ERR_DEVICE;
}

int mi_attn_decode(const float* q, const uint16_t* kc, const uint16_t* vc, int32_t n_head, int32_t n_head_kv, int32_t hd,
                   int32_t L, int32_t ctx, float scale, float* scratch, float* out, void* stream) {
    if (!q || !kc || !vc || !scratch || !out || n_head < 1 || n_head_kv < 1 || L < 1 || L > ctx) return MI_ERR_ARG;
    if (!launch_attn_decode(q, reinterpret_cast<const __half*>(kc), reinterpret_cast<const __half*>(vc), n_head,
                            n_head_kv, hd, L, ctx, scale, scratch, out, (hipStream_t)stream))
        return MI_ERR_SHAPE;
    return hipGetLastError() == hipSuccess ? MI_OK : MI_ERR_DEVICE;
}

int mi_attn_decode_mfma(const float* q, const uint16_t* kc, const uint16_t* vc, int32_t n_head, int32_t n_head_kv,
                        int32_t hd, int32_t L, int32_t ctx, float scale, float* scratch, float* out, void* stream) {
    if (!q || !kc || !vc || !scratch || !out || n_head < 1 || n_head_kv < 1 || L < 1 || L > ctx) return MI_ERR_ARG;
    if (!launch_attn_decode_mfma(q, reinterpret_cast<const __half*>(kc), reinterpret_cast<const __half*>(vc), n_head,
                                 n_head_kv, hd, L, ctx, scale, scratch, out, (hipStream_t)stream))
        return MI_ERR_SHAPE;
    return hipGetLastError() == hipSuccess ? MI_OK : MI_ERR_DEVICE;
}

static_assert(kNoAllocScratchFloats == MI_ATTN_NOALLOC_SCRATCH_FLOATS, "scratch size in minfer.h and kernels.hpp");

int mi_attn_decode_noalloc(const float* q, const uint16_t* kc, const uint16_t* vc, int32_t n_head, int32_t n_head_kv,
                           int32_t hd, int32_t L, int32_t ctx, float scale, float* out, void* stream) {
    if (!q || !kc || !vc || !out || n_head < 1 || n_head_kv < 1 || hd < 1 || L < 1 || L > ctx)
        return set_err(nullptr, MI_ERR_ARG, "mi_attn_decode_noalloc: bad argument");
    const size_t need = attn_scratch_floats(n_head, hd, L);
    if (need > MI_ATTN_NOALLOC_SCRATCH_FLOATS)
        return set_err(nullptr, MI_ERR_SHAPE,
                       "mi_attn_decode_noalloc: %d heads of %d over %d positions need %zu scratch floats, more than "
                       "the %u the library holds (use mi_attn_decode with a workspace)",
                       n_head, hd, L, need, (unsigned)MI_ATTN_NOALLOC_SCRATCH_FLOATS);
    float* scr = nullptr;
    const hipError_t e = noalloc_scratch((hipStream_t)stream, &scr);
    if (e != hipSuccess) return set_err(nullptr, MI_ERR_DEVICE, "mi_attn_decode_noalloc: %s", hipGetErrorString(e));
    if (!launch_attn_decode(q, reinterpret_cast<const __half*>(kc), reinterpret_cast<const __half*>(vc), n_head,
                            n_head_kv, hd, L, ctx, scale, scr, out, (hipStream_t)stream))
        return set_err(nullptr, MI_ERR_SHAPE, "mi_attn_decode_noalloc: unsupported shape");
    return hipGetLastError() == hipSuccess ? MI_OK : MI_ERR_DEVICE;
}

size_t mi_attn_scratch_floats(int32_t n_head, int32_t hd, int32_t L) {
    return n_head < 1 || hd < 1 || L < 1 ? 0 : attn_scratch_floats(n_head, hd, L);
}

int mi_stream_read(const void* buf, size_t bytes, uint32_t* sink, void* stream) {
    if (!buf || !sink || bytes % 16) return MI_ERR_ARG;
    launch_stream(buf, bytes, sink, ncu(), (hipStream_t)stream);
    return hipGetLastError() == hipSuccess ? MI_OK : MI_ERR_DEVICE;
}

int mi_stream_sync(void* stream) { return hipStreamSynchronize((hipStream_t)stream) == hipSuccess ? MI_OK : MI_ERR_DEVICE; }

int mi_device_count(int32_t* n) {
    int c = 0;
    if (!n) return MI_ERR_ARG;
    if (hipGetDeviceCount(&c) != hipSuccess) c = 0;
    *n = c;
    return MI_OK;
}

}  // extern "C"
