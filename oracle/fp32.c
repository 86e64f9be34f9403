/* fp32.c -- cpu_infer.cpp restated in C (ORC_MODE_FP32).
 * TEST INFRASTRUCTURE ONLY (see oracle.h). Built with the reference's float
 * semantics: gnu dialect, -O3, -ffp-contract=fast (CMakeLists.txt:4,10 build
 * cpu_infer as gnu++17 -O3 -march=native), so GCC contracts the same
 * multiply-adds it contracts in cpu_infer. Each function keeps the expression
 * shape of the line it restates. Parity: the greedy token streams of the
 * reference cpu_infer compiled from /root/reference (tests/golden/cpu_infer_*.json fixtures,
 * tests/test_oracle_golden.py).
 */
#include "internal.h"
#include <math.h>
#include <stdlib.h>
#include <string.h>

/* cpu_infer.cpp:22-32 */
static void matvec(const orc_tensor* W, const float* x, float* y, int nthr) {
    const int64_t in = W->ne[0], out = W->ne[1] * W->ne[2];
    #pragma omp parallel for schedule(static) num_threads(nthr)
    for (int64_t j = 0; j < out; j++) {
        float row[16384];
        orc_dequant_row_fma(W, j, row);
        float acc = 0.f;
        for (int64_t k = 0; k < in; k++) acc += row[k] * x[k];
        y[j] = acc;
    }
}

/* cpu_infer.cpp:34-38 */
static void add_bias(float* y, const orc_tensor* b, int n) {
    const float* bb = (const float*)b->data;
    for (int i = 0; i < n; i++) y[i] += bb[i];
}

/* cpu_infer.cpp:40-46 */
static void rmsnorm(const float* x, const orc_tensor* w, int n, float eps, float* out) {
    const float* wb = (const float*)w->data;
    double ss = 0;
    for (int i = 0; i < n; i++) ss += (double)x[i] * x[i];
    float scale = 1.f / sqrtf((float)(ss / n) + eps);
    for (int i = 0; i < n; i++) out[i] = x[i] * scale * wb[i];
}

/* cpu_infer.cpp:54-55 */
void orc_rope_cs(int pos, int i, int hd, float base, float* c, float* s) {
    float theta = pos * powf(base, -2.f * i / hd);
    *c = cosf(theta);
    *s = sinf(theta);
}

/* cpu_infer.cpp:49-61 (exported as orc_rope_fp32) */
static void rope(float* v, int n_head, int hd, int pos, float base) {
    int half = hd / 2;
    for (int h = 0; h < n_head; h++) {
        float* p = v + (size_t)h * hd;
        for (int i = 0; i < half; i++) {
            float theta = pos * powf(base, -2.f * i / hd);
            float c = cosf(theta), s = sinf(theta);
            float x0 = p[i], x1 = p[i + half];
            p[i] = x0 * c - x1 * s;
            p[i + half] = x0 * s + x1 * c;
        }
    }
}

void orc_rope_fp32(float* v, int n_head, int hd, int pos, float base) { rope(v, n_head, hd, pos, base); }

/* cpu_infer.cpp:121-140 for one head */
void orc_attention_fp32(const float* qh, const float* k, const float* v, int L, int hd,
                        int stride, float inv, float* oh) {
    float* sc = (float*)malloc(sizeof(float) * (size_t)L);
    float mx = -1e30f;
    for (int t = 0; t < L; t++) {
        const float* kt = k + (size_t)t * stride;
        float d = 0; for (int i = 0; i < hd; i++) d += qh[i] * kt[i];
        sc[t] = d * inv; if (sc[t] > mx) mx = sc[t];
    }
    float sum = 0; for (int t = 0; t < L; t++) { sc[t] = expf(sc[t] - mx); sum += sc[t]; }
    for (int i = 0; i < hd; i++) oh[i] = 0;
    for (int t = 0; t < L; t++) {
        const float* vt = v + (size_t)t * stride;
        float p = sc[t] / sum;
        for (int i = 0; i < hd; i++) oh[i] += p * vt[i];
    }
    free(sc);
}

/* cpu_infer.cpp:109-155 (the lambda `forward`), logits left in m->logits */
int32_t orc_forward_fp32(struct orc_model* m, int32_t token, int32_t pos) {
    const orc_config* c = &m->c;
    const int kv_dim = c->n_head_kv * c->head_dim, gqa = c->n_head / c->n_head_kv;
    orc_dequant_row_fma(m->tok_emb, token, m->h);
    for (int l = 0; l < c->n_layer; l++) {
        const orc_layer* ly = &m->L[l];
        rmsnorm(m->h, ly->an, c->n_embd, c->rms_eps, m->xb);
        matvec(ly->wq, m->xb, m->q, m->n_threads); add_bias(m->q, ly->bq, c->n_head * c->head_dim);
        matvec(ly->wk, m->xb, m->k, m->n_threads); add_bias(m->k, ly->bk, kv_dim);
        matvec(ly->wv, m->xb, m->v, m->n_threads); add_bias(m->v, ly->bv, kv_dim);
        rope(m->q, c->n_head, c->head_dim, pos, c->rope_base);
        rope(m->k, c->n_head_kv, c->head_dim, pos, c->rope_base);
        memcpy(m->kc + ((size_t)l * m->max_seq + pos) * kv_dim, m->k, (size_t)kv_dim * 4);
        memcpy(m->vc + ((size_t)l * m->max_seq + pos) * kv_dim, m->v, (size_t)kv_dim * 4);
        float inv = 1.f / sqrtf((float)c->head_dim);
        for (int hh = 0; hh < c->n_head; hh++) {
            int kvh = hh / gqa;
            orc_attention_fp32(m->q + (size_t)hh * c->head_dim,
                               m->kc + (size_t)l * m->max_seq * kv_dim + kvh * c->head_dim,
                               m->vc + (size_t)l * m->max_seq * kv_dim + kvh * c->head_dim,
                               pos + 1, c->head_dim, kv_dim, inv, m->att + (size_t)hh * c->head_dim);
        }
        matvec(ly->wo, m->att, m->proj, m->n_threads);
        for (int i = 0; i < c->n_embd; i++) m->h[i] += m->proj[i];
        rmsnorm(m->h, ly->fn, c->n_embd, c->rms_eps, m->xb);
        matvec(ly->wg, m->xb, m->gbuf, m->n_threads);
        matvec(ly->wu, m->xb, m->ubuf, m->n_threads);
        for (int i = 0; i < c->n_ff; i++) { float x = m->gbuf[i]; m->gbuf[i] = (x / (1.f + expf(-x))) * m->ubuf[i]; }
        matvec(ly->wd, m->gbuf, m->proj, m->n_threads);
        for (int i = 0; i < c->n_embd; i++) m->h[i] += m->proj[i];
    }
    rmsnorm(m->h, m->out_norm, c->n_embd, c->rms_eps, m->xb);
    matvec(m->out_w, m->xb, m->logits, m->n_threads);
    return 0;
}
