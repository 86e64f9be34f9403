/* model.c -- oracle model setup, the greedy argmax and the generate loop.
 * TEST INFRASTRUCTURE ONLY (see oracle.h).
 * Config and tensor names follow cpu_infer.cpp:70-98; the generate loop follows
 * cpu_infer.cpp:161-167 (sequential prefill, then print `next` and step).
 */
#define _GNU_SOURCE
#include "internal.h"
#include <math.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>
#include <time.h>
#ifdef _OPENMP
#include <omp.h>
#endif

/* first maximum wins (cpu_infer.cpp:153-154); second = best of all the others */
void orc_argmax(const float* x, int n, int32_t* idx, float* margin) {
    int best = 0; float bv = x[0], sv = -INFINITY;
    for (int i = 1; i < n; i++) {
        if (x[i] > bv) { sv = bv; bv = x[i]; best = i; }
        else if (x[i] > sv) sv = x[i];
    }
    *idx = best;
    if (margin) *margin = bv - sv;
}

static const orc_tensor* need_t(const orc_gguf* g, const char* name, int* ok) {
    const orc_tensor* t = orc_gguf_tensor(g, name);
    if (!t) *ok = 0;
    return t;
}

orc_model* orc_model_new(const orc_gguf* g, int mode, const orc_plan* plan, int max_seq, int n_threads) {
    orc_model* m = (orc_model*)calloc(1, sizeof *m);
    m->mode = mode;
    if (plan) m->plan = *plan;
    if (mode == ORC_MODE_Q8ACT && !plan) { free(m); return NULL; }
    orc_config* c = &m->c;
    c->n_layer = (int)orc_gguf_num(g, "qwen2.block_count", 0);
    c->n_embd = (int)orc_gguf_num(g, "qwen2.embedding_length", 0);
    c->n_ff = (int)orc_gguf_num(g, "qwen2.feed_forward_length", 0);
    c->n_head = (int)orc_gguf_num(g, "qwen2.attention.head_count", 0);
    c->n_head_kv = (int)orc_gguf_num(g, "qwen2.attention.head_count_kv", 0);
    if (c->n_head <= 0 || c->n_head_kv <= 0 || c->n_layer <= 0) { free(m); return NULL; }
    c->head_dim = c->n_embd / c->n_head;
    c->rope_base = (float)orc_gguf_num(g, "qwen2.rope.freq_base", 1e6);
    c->rms_eps = (float)orc_gguf_num(g, "qwen2.attention.layer_norm_rms_epsilon", 1e-6);
    c->n_vocab = (int)orc_gguf_n_tokens(g);
    m->max_seq = max_seq;
#ifdef _OPENMP
    m->n_threads = n_threads > 0 ? n_threads : omp_get_max_threads();
#else
    m->n_threads = 1;
#endif
    int ok = 1;
    m->tok_emb = need_t(g, "token_embd.weight", &ok);
    m->out_w = orc_gguf_tensor(g, "output.weight");
    if (!m->out_w) m->out_w = m->tok_emb;          /* tied embeddings (mega.cu:1071) */
    m->out_norm = need_t(g, "output_norm.weight", &ok);
    m->L = (orc_layer*)calloc((size_t)c->n_layer, sizeof(orc_layer));
    char name[128];
#define T(field, suffix) do { snprintf(name, sizeof name, "blk.%d.%s", i, suffix); m->L[i].field = need_t(g, name, &ok); } while (0)
    for (int i = 0; i < c->n_layer; i++) {
        T(an, "attn_norm.weight"); T(wq, "attn_q.weight"); T(bq, "attn_q.bias");
        T(wk, "attn_k.weight"); T(bk, "attn_k.bias"); T(wv, "attn_v.weight"); T(bv, "attn_v.bias");
        T(wo, "attn_output.weight"); T(fn, "ffn_norm.weight");
        T(wg, "ffn_gate.weight"); T(wu, "ffn_up.weight"); T(wd, "ffn_down.weight");
    }
#undef T
    if (!ok || c->n_vocab <= 0) { orc_model_free(m); return NULL; }
    if (mode == ORC_MODE_Q8ACT) {
        const int nmat = 7 * c->n_layer + 1;
        m->own_t = (orc_tensor*)calloc((size_t)nmat, sizeof(orc_tensor));
        m->own_buf = (uint8_t**)calloc((size_t)nmat, sizeof(uint8_t*));
        for (int i = 0; i <= c->n_layer; i++) {
            const orc_tensor** mats[7];
            int k = 0;
            if (i < c->n_layer) {
                orc_layer* Ly = &m->L[i];
                mats[k++] = &Ly->wq; mats[k++] = &Ly->wk; mats[k++] = &Ly->wv; mats[k++] = &Ly->wo;
                mats[k++] = &Ly->wg; mats[k++] = &Ly->wu; mats[k++] = &Ly->wd;
            } else {
                mats[k++] = &m->out_w;
            }
            for (int j = 0; j < k; j++) {
                const orc_tensor* t = *mats[j];
                if (t->type == ORC_Q4_0) continue;
                const int64_t n = t->ne[0], rows = t->ne[1] * t->ne[2] * t->ne[3];
                uint8_t* buf = (uint8_t*)malloc((size_t)rows * (n / 32) * 18);
                float* row = (float*)malloc(sizeof(float) * (size_t)n);
                for (int64_t r = 0; r < rows; r++) {
                    orc_dequant_row(t, r, row);
                    orc_requant_q4_0_row(row, (int)n, buf + (size_t)r * (n / 32) * 18);
                }
                free(row);
                orc_tensor* o = &m->own_t[m->n_own];
                *o = *t;
                o->type = ORC_Q4_0;
                o->data = buf;
                m->own_buf[m->n_own++] = buf;
                *mats[j] = o;
            }
        }
    }
    const int kvd = c->n_head_kv * c->head_dim, E = c->n_embd;
    m->kc = (float*)calloc((size_t)c->n_layer * max_seq * kvd, 4);
    m->vc = (float*)calloc((size_t)c->n_layer * max_seq * kvd, 4);
    m->h = (float*)calloc(E, 4); m->xb = (float*)calloc(E, 4);
    m->q = (float*)calloc(c->n_head * c->head_dim, 4);
    m->k = (float*)calloc(kvd, 4); m->v = (float*)calloc(kvd, 4);
    m->att = (float*)calloc(c->n_head * c->head_dim, 4); m->proj = (float*)calloc(E, 4);
    m->gbuf = (float*)calloc(c->n_ff, 4); m->ubuf = (float*)calloc(c->n_ff, 4);
    m->logits = (float*)calloc(c->n_vocab, 4);
    const int nmax = c->n_ff > E ? c->n_ff : E;
    m->xq = (int8_t*)calloc(nmax, 1); m->xd = (float*)calloc(nmax / 32 + 1, 4); m->xs8 = (int32_t*)calloc(nmax / 32 + 1, 4);
    const int half = c->head_dim / 2;
    m->rope_c = (float*)calloc((size_t)max_seq * half, 4);
    m->rope_s = (float*)calloc((size_t)max_seq * half, 4);
    for (int p = 0; p < max_seq; p++)
        for (int i = 0; i < half; i++)
            orc_rope_cs(p, i, c->head_dim, c->rope_base, &m->rope_c[(size_t)p * half + i], &m->rope_s[(size_t)p * half + i]);
    return m;
}

void orc_model_free(orc_model* m) {
    if (!m) return;
    free(m->L); free(m->kc); free(m->vc); free(m->h); free(m->xb); free(m->q); free(m->k); free(m->v);
    free(m->att); free(m->proj); free(m->gbuf); free(m->ubuf); free(m->logits);
    free(m->xq); free(m->xd); free(m->xs8); free(m->rope_c); free(m->rope_s); free(m->scores);
    for (int i = 0; i < m->n_own; i++) free(m->own_buf[i]);
    free(m->own_buf); free(m->own_t);
    free(m);
}

void orc_model_config(const orc_model* m, orc_config* out) { *out = m->c; }

int32_t orc_forward(orc_model* m, int32_t token, int32_t pos, float* logits, float* margin) {
    if (pos < 0 || pos >= m->max_seq || token < 0 || token >= m->c.n_vocab) return -1;
    const int32_t rc = m->mode == ORC_MODE_FP32 ? orc_forward_fp32(m, token, pos) : orc_forward_q8act(m, token, pos);
    if (rc < 0) return -1;
    if (logits) memcpy(logits, m->logits, sizeof(float) * (size_t)m->c.n_vocab);
    int32_t best; float mg;
    orc_argmax(m->logits, m->c.n_vocab, &best, &mg);
    if (margin) *margin = mg;
    return best;
}

static double now_s(void) {
    struct timespec ts; clock_gettime(CLOCK_MONOTONIC, &ts);
    return ts.tv_sec + ts.tv_nsec * 1e-9;
}

int orc_generate(orc_model* m, const int32_t* prompt, int32_t n_prompt, int32_t n_gen,
                 int32_t* out, float* margins, double* t_prefill, double* t_decode) {
    if (n_prompt < 1 || n_prompt + n_gen > m->max_seq) return -1;
    int pos = 0; int32_t next = -1; float mg = 0.f;
    const double t0 = now_s();
    for (int i = 0; i < n_prompt; i++) { next = orc_forward(m, prompt[i], pos++, NULL, &mg); if (next < 0) return -1; }
    const double t1 = now_s();
    for (int t = 0; t < n_gen; t++) {
        out[t] = next;
        if (margins) margins[t] = mg;
        if (t + 1 < n_gen) { next = orc_forward(m, next, pos++, NULL, &mg); if (next < 0) return -1; }
    }
    const double t2 = now_s();
    if (t_prefill) *t_prefill = t1 - t0;
    if (t_decode) *t_decode = t2 - t1;
    return 0;
}
