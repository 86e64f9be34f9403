/* gguf_reader.c -- GGUF v3 reader and row dequantization for the oracle.
 * TEST INFRASTRUCTURE ONLY (see oracle.h).
 *
 * Restates src/gguf.h: header + metadata (:183-200, rd_value :156-181), tensor
 * infos (:202-212), data start aligned to general.alignment (default 32,
 * :215-217), ne[0] is the contiguous row length (:56), q4_0 block = fp16 d then
 * 16 bytes whose low nibble is element j and high nibble element j+16, value
 * (n-8)*d (:94-101). Unlike gguf.h it reports errors instead of exiting.
 */
#define _GNU_SOURCE
#include "oracle.h"
#include <fcntl.h>
#include <stdio.h>
#include <stdlib.h>
#include <math.h>
#include <string.h>
#include <sys/mman.h>
#include <sys/stat.h>
#include <unistd.h>

#define MAXKV 256
#define MAXT 2048

typedef struct { char* key; double val; } num_kv;
typedef struct { char* name; orc_tensor t; uint64_t off; } tinfo;

struct orc_gguf {
    int fd;
    size_t size;
    const uint8_t* base;
    const uint8_t* cur;
    const uint8_t* end;
    num_kv num[MAXKV];
    int n_num;
    int64_t n_tokens;
    tinfo* tens;
    int n_tens;
};

static __thread char g_err[256];
const char* orc_gguf_error(void) { return g_err; }

static int need(orc_gguf* g, size_t n) {
    if ((size_t)(g->end - g->cur) < n) { snprintf(g_err, sizeof g_err, "truncated GGUF"); return 0; }
    return 1;
}
#define RD(T, out) do { if (!need(g, sizeof(T))) return 0; memcpy(&(out), g->cur, sizeof(T)); g->cur += sizeof(T); } while (0)

static int rd_str(orc_gguf* g, const uint8_t** s, uint64_t* n) {
    RD(uint64_t, *n);
    if (!need(g, *n)) return 0;
    *s = g->cur; g->cur += *n;
    return 1;
}

static void put_num(orc_gguf* g, const uint8_t* k, uint64_t kn, double v) {
    if (g->n_num >= MAXKV) return;
    char* key = (char*)malloc(kn + 1);
    memcpy(key, k, kn); key[kn] = 0;
    g->num[g->n_num].key = key; g->num[g->n_num].val = v; g->n_num++;
}

/* gguf.h:156-181: numeric metadata kept as double, strings skipped except the
 * token list, whose length gives n_vocab (cpu_infer.cpp:79) */
static int rd_value(orc_gguf* g, uint32_t vt, const uint8_t* k, uint64_t kn, int store) {
    union { uint8_t u8; int8_t i8; uint16_t u16; int16_t i16; uint32_t u32; int32_t i32; float f; uint64_t u64; int64_t i64; double d; } v;
    double val;
    switch (vt) {
        case 0: RD(uint8_t, v.u8); val = v.u8; break;
        case 1: RD(int8_t, v.i8); val = v.i8; break;
        case 2: RD(uint16_t, v.u16); val = v.u16; break;
        case 3: RD(int16_t, v.i16); val = v.i16; break;
        case 4: RD(uint32_t, v.u32); val = v.u32; break;
        case 5: RD(int32_t, v.i32); val = v.i32; break;
        case 6: RD(float, v.f); val = v.f; break;
        case 7: RD(uint8_t, v.u8); val = v.u8; break;
        case 10: RD(uint64_t, v.u64); val = (double)v.u64; break;
        case 11: RD(int64_t, v.i64); val = (double)v.i64; break;
        case 12: RD(double, v.d); val = v.d; break;
        case 8: { const uint8_t* s; uint64_t n; if (!rd_str(g, &s, &n)) return 0; return 1; }
        case 9: {
            uint32_t et; uint64_t n;
            RD(uint32_t, et); RD(uint64_t, n);
            int is_tokens = store && kn == strlen("tokenizer.ggml.tokens") && memcmp(k, "tokenizer.ggml.tokens", kn) == 0 && et == 8;
            for (uint64_t i = 0; i < n; i++)
                if (!rd_value(g, et, NULL, 0, 0)) return 0;
            if (is_tokens) g->n_tokens = (int64_t)n;
            return 1;
        }
        default: snprintf(g_err, sizeof g_err, "bad meta type %u", vt); return 0;
    }
    if (store) put_num(g, k, kn, val);
    return 1;
}

static int parse(orc_gguf* g) {
    uint32_t magic, version; uint64_t n_t, n_kv;
    RD(uint32_t, magic);
    if (magic != 0x46554747u) { snprintf(g_err, sizeof g_err, "not a GGUF file"); return 0; }
    RD(uint32_t, version);
    RD(uint64_t, n_t); RD(uint64_t, n_kv);
    if (n_t > MAXT) { snprintf(g_err, sizeof g_err, "too many tensors"); return 0; }
    for (uint64_t i = 0; i < n_kv; i++) {
        const uint8_t* k; uint64_t kn; uint32_t vt;
        if (!rd_str(g, &k, &kn)) return 0;
        RD(uint32_t, vt);
        if (!rd_value(g, vt, k, kn, 1)) return 0;
    }
    g->tens = (tinfo*)calloc(n_t ? n_t : 1, sizeof(tinfo));
    for (uint64_t i = 0; i < n_t; i++) {
        const uint8_t* s; uint64_t n; uint32_t nd;
        if (!rd_str(g, &s, &n)) return 0;
        tinfo* ti = &g->tens[g->n_tens++];
        ti->name = (char*)malloc(n + 1); memcpy(ti->name, s, n); ti->name[n] = 0;
        RD(uint32_t, nd);
        if (nd < 1 || nd > 4) { snprintf(g_err, sizeof g_err, "bad tensor rank"); return 0; }
        ti->t.nd = (int32_t)nd;
        for (int d = 0; d < 4; d++) ti->t.ne[d] = 1;
        for (uint32_t d = 0; d < nd; d++) { uint64_t e; RD(uint64_t, e); ti->t.ne[d] = (int64_t)e; }
        RD(uint32_t, ti->t.type);
        RD(uint64_t, ti->off);
    }
    uint64_t align = (uint64_t)orc_gguf_num(g, "general.alignment", 32);
    size_t pos = (size_t)(g->cur - g->base);
    size_t start = (pos + align - 1) / align * align;
    for (int i = 0; i < g->n_tens; i++) {
        g->tens[i].t.data = g->base + start + g->tens[i].off;
        if (g->tens[i].t.data > g->end) { snprintf(g_err, sizeof g_err, "tensor data out of file"); return 0; }
    }
    return 1;
}

orc_gguf* orc_gguf_open(const char* path) {
    orc_gguf* g = (orc_gguf*)calloc(1, sizeof *g);
    g->fd = open(path, O_RDONLY);
    if (g->fd < 0) { snprintf(g_err, sizeof g_err, "cannot open %s", path); free(g); return NULL; }
    struct stat st; fstat(g->fd, &st); g->size = (size_t)st.st_size;
    void* p = mmap(NULL, g->size, PROT_READ, MAP_PRIVATE, g->fd, 0);
    if (p == MAP_FAILED) { snprintf(g_err, sizeof g_err, "mmap failed"); close(g->fd); free(g); return NULL; }
    g->base = (const uint8_t*)p; g->cur = g->base; g->end = g->base + g->size;
    if (!parse(g)) { orc_gguf_close(g); return NULL; }
    return g;
}

void orc_gguf_close(orc_gguf* g) {
    if (!g) return;
    for (int i = 0; i < g->n_num; i++) free(g->num[i].key);
    for (int i = 0; i < g->n_tens; i++) free(g->tens[i].name);
    free(g->tens);
    if (g->base) munmap((void*)g->base, g->size);
    if (g->fd >= 0) close(g->fd);
    free(g);
}

double orc_gguf_num(const orc_gguf* g, const char* key, double def) {
    for (int i = 0; i < g->n_num; i++) if (strcmp(g->num[i].key, key) == 0) return g->num[i].val;
    return def;
}
int64_t orc_gguf_n_tokens(const orc_gguf* g) { return g->n_tokens; }
const orc_tensor* orc_gguf_tensor(const orc_gguf* g, const char* name) {
    for (int i = 0; i < g->n_tens; i++) if (strcmp(g->tens[i].name, name) == 0) return &g->tens[i].t;
    return NULL;
}

/* gguf.h:37-52, bit manipulation (exact) */
float orc_f16_to_f32(uint16_t h) {
    uint32_t sign = (uint32_t)(h & 0x8000) << 16, ex = (h >> 10) & 0x1F, mant = h & 0x3FF, f;
    if (ex == 0) {
        if (mant == 0) f = sign;
        else {
            ex = 127 - 15 + 1;
            while ((mant & 0x400) == 0) { mant <<= 1; ex--; }
            mant &= 0x3FF; f = sign | (ex << 23) | (mant << 13);
        }
    } else if (ex == 0x1F) f = sign | 0x7F800000u | (mant << 13);
    else f = sign | ((ex - 15 + 127) << 23) | (mant << 13);
    float out; memcpy(&out, &f, 4); return out;
}

/* binary32 -> binary16, round to nearest even, subnormals and overflow to inf:
 * the conversion the reference's __float2half performs (cuda_infer.cu:88) */
uint16_t orc_f32_to_f16(float f) {
    uint32_t x; memcpy(&x, &f, 4);
    uint32_t sign = (x >> 16) & 0x8000u, ex = (x >> 23) & 0xFF, mant = x & 0x7FFFFFu;
    if (ex == 0xFF) return (uint16_t)(sign | 0x7C00u | (mant ? 0x200u : 0));
    int e = (int)ex - 127 + 15;
    if (e >= 31) return (uint16_t)(sign | 0x7C00u);
    if (e <= 0) {                       /* subnormal half (or zero) */
        if (e < -10) return (uint16_t)sign;
        uint32_t m = mant | 0x800000u;
        int shift = 14 - e;             /* 24-bit significand -> 10-bit at exponent 1-15 */
        uint32_t q = m >> shift, rem = m & ((1u << shift) - 1), half = 1u << (shift - 1);
        if (rem > half || (rem == half && (q & 1))) q++;
        return (uint16_t)(sign | q);
    }
    uint32_t q = ((uint32_t)e << 10) | (mant >> 13), rem = mant & 0x1FFFu;
    if (rem > 0x1000u || (rem == 0x1000u && (q & 1))) q++;   /* carry may round up to inf: correct */
    return (uint16_t)(sign | q);
}

/* gguf.h:85-142 (F32, F16, Q4_0, Q4_1, Q8_0, Q6_K) */
static void dequant(const orc_tensor* t, int64_t r, float* out, int fma_q41) {
    const int64_t cols = t->ne[0];
    switch (t->type) {
        case ORC_F32: memcpy(out, t->data + (size_t)r * cols * 4, (size_t)cols * 4); return;
        case ORC_F16: {
            const uint16_t* h = (const uint16_t*)(t->data + (size_t)r * cols * 2);
            for (int64_t i = 0; i < cols; i++) out[i] = orc_f16_to_f32(h[i]);
            return;
        }
        case ORC_Q4_0: {
            const int64_t bpr = cols / 32;
            const uint8_t* p = t->data + (size_t)(r * bpr) * 18;
            for (int64_t b = 0; b < bpr; b++, p += 18) {
                uint16_t hd; memcpy(&hd, p, 2);
                const float d = orc_f16_to_f32(hd);
                const uint8_t* qs = p + 2; float* y = out + b * 32;
                for (int j = 0; j < 16; j++) {
                    y[j] = ((qs[j] & 0x0F) - 8) * d;
                    y[j + 16] = ((qs[j] >> 4) - 8) * d;
                }
            }
            return;
        }
        case ORC_Q4_1: {   /* gguf.h:103-113: fp16 d, fp16 m, 16 B of nibbles */
            const int64_t bpr = cols / 32;
            const uint8_t* p = t->data + (size_t)(r * bpr) * 20;
            for (int64_t b = 0; b < bpr; b++, p += 20) {
                uint16_t hd, hm; memcpy(&hd, p, 2); memcpy(&hm, p + 2, 2);
                const float d = orc_f16_to_f32(hd), m = orc_f16_to_f32(hm);
                const uint8_t* qs = p + 4; float* y = out + b * 32;
                for (int j = 0; j < 16; j++) {
                    const float q0 = (float)(qs[j] & 0x0F), q1 = (float)(qs[j] >> 4);
                    y[j] = fma_q41 ? fmaf(q0, d, m) : q0 * d + m;
                    y[j + 16] = fma_q41 ? fmaf(q1, d, m) : q1 * d + m;
                }
            }
            return;
        }
        case ORC_Q8_0: {
            const int64_t bpr = cols / 32;
            const uint8_t* p = t->data + (size_t)(r * bpr) * 34;
            for (int64_t b = 0; b < bpr; b++, p += 34) {
                uint16_t hd; memcpy(&hd, p, 2);
                const float d = orc_f16_to_f32(hd);
                const int8_t* qs = (const int8_t*)(p + 2); float* y = out + b * 32;
                for (int j = 0; j < 32; j++) y[j] = qs[j] * d;
            }
            return;
        }
        case ORC_Q6_K: {   /* gguf.h:120-139: ql[128], qh[64], int8 scales[16], fp16 d per 256 */
            const int64_t bpr = cols / 256;
            const uint8_t* p = t->data + (size_t)(r * bpr) * 210;
            for (int64_t b = 0; b < bpr; b++, p += 210) {
                uint16_t hd; memcpy(&hd, p + 208, 2);
                const float d = orc_f16_to_f32(hd);
                const uint8_t* ql = p; const uint8_t* qh = p + 128; const int8_t* sc = (const int8_t*)(p + 192);
                float* y = out + b * 256;
                for (int n = 0; n < 256; n += 128) {
                    for (int l = 0; l < 32; l++) {
                        const int is = l / 16;
                        const int q1 = ((ql[l] & 0xF) | (((qh[l] >> 0) & 3) << 4)) - 32;
                        const int q2 = ((ql[l + 32] & 0xF) | (((qh[l] >> 2) & 3) << 4)) - 32;
                        const int q3 = ((ql[l] >> 4) | (((qh[l] >> 4) & 3) << 4)) - 32;
                        const int q4 = ((ql[l + 32] >> 4) | (((qh[l] >> 6) & 3) << 4)) - 32;
                        y[l] = d * sc[is + 0] * q1;
                        y[l + 32] = d * sc[is + 2] * q2;
                        y[l + 64] = d * sc[is + 4] * q3;
                        y[l + 96] = d * sc[is + 6] * q4;
                    }
                    ql += 64; qh += 32; sc += 8; y += 128;
                }
            }
            return;
        }
        default: for (int64_t i = 0; i < cols; i++) out[i] = 0.f; return;
    }
}
void orc_dequant_row(const orc_tensor* t, int64_t r, float* out) { dequant(t, r, out, 0); }
void orc_dequant_row_fma(const orc_tensor* t, int64_t r, float* out) { dequant(t, r, out, 1); }

void orc_requant_q4_0_row(const float* y, int n, uint8_t* out) {
    for (int b = 0; b < n / 32; b++, y += 32, out += 18) {
        float amax = 0.f;
        for (int j = 0; j < 32; j++) amax = fmaxf(amax, fabsf(y[j]));
        const float d = amax / 7.f, inv = d > 0.f ? 1.f / d : 0.f;
        const uint16_t hd = orc_f32_to_f16(d);
        memcpy(out, &hd, 2);
        for (int j = 0; j < 16; j++) {
            int q0 = (int)lrintf(y[j] * inv) + 8, q1 = (int)lrintf(y[j + 16] * inv) + 8;
            q0 = q0 < 0 ? 0 : (q0 > 15 ? 15 : q0);
            q1 = q1 < 0 ? 0 : (q1 > 15 ? 15 : q1);
            out[2 + j] = (uint8_t)(q0 | (q1 << 4));
        }
    }
}
