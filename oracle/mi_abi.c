/* The engine's C ABI (include/minfer.h) over the CPU oracle: a second backend that the
 * parity harness loads in place of the HIP library and drives with the same calls.
 * TEST INFRASTRUCTURE, like the rest of oracle/: only tests/ load it, never the product.
 *
 * It implements the engine entry points -- mi_default_opts, mi_load, mi_free,
 * mi_last_error, mi_info, mi_prefill, mi_step, mi_generate, mi_teacher, mi_get_stats --
 * with the argument meaning, state rules and status codes minfer.h gives them (the
 * reference has no such API: its seams are cuda_infer.cu:990-1026 forward_batch,
 * :1031-1083 record, :1133-1200 prefill and generate, mega.cu:857-895 teacher and
 * speculative modes). Every position is one orc_forward, in the mode and reduction plan
 * set before mi_load with orc_mi_set_mode / orc_mi_set_plan: ORC_MODE_FP32 gives
 * cpu_infer.cpp's numbers, ORC_MODE_Q8ACT (the default) the GPU engine's bits when given
 * the plan the GPU engine reports (mi_info). A multi-token step or a chunked prefill is
 * its tokens one at a time (the GPU's multi-token results equal that bit for bit), and
 * opts.spec changes nothing in the output (speculation is lossless), so it is ignored. */
#include <math.h>
#include <stdarg.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>
#include <time.h>

#include "../include/minfer.h"
#include "oracle.h"

struct mi_engine {
    orc_gguf* g;
    orc_model* m;
    mi_opts opts;
    mi_model_info info;
    mi_stats stats;
    int32_t cur_len;        /* positions holding K/V */
    int32_t next_tok;       /* the prediction after position cur_len - 1 */
    float next_margin;
    int next_ready;
    char err[256];
};

static int g_mode = ORC_MODE_Q8ACT;
static int g_plan_set = 0;
static orc_plan g_plan;
static char g_load_err[256];

/* the forward mode of engines loaded after this call */
void orc_mi_set_mode(int mode) { g_mode = mode; }
/* the q8act reduction plan of engines loaded after this call (cb, ks per matrix:
 * qkv, o, gate/up, down, lm_head); without it every matrix is cb 8, ks 1 */
void orc_mi_set_plan(const int32_t* cb, const int32_t* ks) {
    for (int i = 0; i < ORC_NMAT; i++) {
        g_plan.cb[i] = cb[i];
        g_plan.ks[i] = ks[i];
    }
    g_plan.attn_chunk = 64;
    g_plan.kv_f16 = 1;
    g_plan_set = 1;
}

static int fail(mi_engine* e, int rc, const char* fmt, ...) {
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(e ? e->err : g_load_err, sizeof(g_load_err), fmt, ap);
    va_end(ap);
    return rc;
}

static double now_s(void) {
    struct timespec ts;
    clock_gettime(CLOCK_MONOTONIC, &ts);
    return ts.tv_sec + 1e-9 * ts.tv_nsec;
}

void mi_default_opts(mi_opts* o) {
    memset(o, 0, sizeof(*o));
    o->max_ctx = 4096;
    o->tchunk = 8;
    o->spec = 0;
    o->ngmax = 3;
    o->spec_slope = 0.074f;
    o->persistent = 1;
    o->stop_eos = 0;
}

int mi_load(const char* gguf_path, const mi_opts* opts, mi_engine** out) {
    if (!gguf_path || !out) return fail(NULL, MI_ERR_ARG, "null argument");
    *out = NULL;
    mi_engine* e = (mi_engine*)calloc(1, sizeof(mi_engine));
    if (!e) return fail(NULL, MI_ERR_OOM, "out of host memory");
    if (opts) e->opts = *opts;
    else mi_default_opts(&e->opts);
    if (e->opts.max_ctx == 0) e->opts.max_ctx = 4096;
    if (e->opts.tchunk < 1 || e->opts.tchunk > 8 || e->opts.max_ctx < 0 || e->opts.persistent < 0 ||
        e->opts.persistent > 2) {
        free(e);
        return fail(NULL, MI_ERR_ARG, "bad options");
    }
    FILE* f = fopen(gguf_path, "rb");
    if (!f) {
        free(e);
        return fail(NULL, MI_ERR_IO, "cannot open %s", gguf_path);
    }
    fclose(f);
    e->g = orc_gguf_open(gguf_path);
    if (!e->g) {
        free(e);
        return fail(NULL, MI_ERR_FORMAT, "%s: %s", gguf_path, orc_gguf_error());
    }
    orc_plan plan = g_plan;
    if (!g_plan_set) {
        for (int i = 0; i < ORC_NMAT; i++) { plan.cb[i] = 8; plan.ks[i] = 1; }
        plan.attn_chunk = 64;
        plan.kv_f16 = 1;
    }
    e->m = orc_model_new(e->g, g_mode, g_mode == ORC_MODE_Q8ACT ? &plan : NULL, e->opts.max_ctx, 0);
    if (!e->m) {
        orc_gguf_close(e->g);
        free(e);
        return fail(NULL, MI_ERR_FORMAT, "%s: model tensors missing or unsupported", gguf_path);
    }
    orc_config c;
    orc_model_config(e->m, &c);
    mi_model_info* i = &e->info;
    i->n_layer = c.n_layer; i->n_embd = c.n_embd; i->n_ff = c.n_ff; i->n_head = c.n_head;
    i->n_head_kv = c.n_head_kv; i->head_dim = c.head_dim; i->n_vocab = c.n_vocab;
    i->eos = (int32_t)orc_gguf_num(e->g, "tokenizer.ggml.eos_token_id", 151645);
    i->rope_base = c.rope_base;
    i->rms_eps = c.rms_eps;
    i->max_ctx = e->opts.max_ctx;
    for (int k = 0; k < 5; k++) { i->plan_cb[k] = plan.cb[k]; i->plan_ks[k] = plan.ks[k]; }
    i->attn_chunk = plan.attn_chunk;
    i->kv_f16 = g_mode == ORC_MODE_Q8ACT;
    *out = e;
    return MI_OK;
}

void mi_free(mi_engine* e) {
    if (!e) return;
    orc_model_free(e->m);
    orc_gguf_close(e->g);
    free(e);
}

const char* mi_last_error(const mi_engine* e) { return e ? e->err : g_load_err; }

int mi_info(const mi_engine* e, mi_model_info* out) {
    if (!e || !out) return MI_ERR_ARG;
    *out = e->info;
    return MI_OK;
}

int mi_get_stats(const mi_engine* e, mi_stats* out) {
    if (!e || !out) return MI_ERR_ARG;
    *out = e->stats;
    return MI_OK;
}

static int check_ids(mi_engine* e, const int32_t* ids, int32_t n, const char* what) {
    for (int32_t k = 0; k < n; k++)
        if (ids[k] < 0 || ids[k] >= e->info.n_vocab) return fail(e, MI_ERR_ARG, "%s token %d out of range", what, ids[k]);
    return MI_OK;
}

int mi_prefill(mi_engine* e, const int32_t* ids, int32_t n, int32_t* first, float* margin) {
    if (!e || !ids || n < 1) return MI_ERR_ARG;
    if (n >= e->opts.max_ctx)
        return fail(e, MI_ERR_ARG, "prompt of %d tokens exceeds the context capacity %d", n, e->opts.max_ctx);
    int rc = check_ids(e, ids, n, "prompt");
    if (rc) return rc;
    const double t0 = now_s();
    int32_t tok = 0;
    float mg = 0.f;
    for (int32_t p = 0; p < n; p++) {
        tok = orc_forward(e->m, ids[p], p, NULL, &mg);
        if (tok < 0) return fail(e, MI_ERR_STATE, "forward failed at position %d", p);
    }
    e->stats.prefill_ms = 1e3 * (now_s() - t0);
    e->cur_len = n;
    e->next_tok = tok;
    e->next_margin = mg;
    e->next_ready = 1;
    if (first) *first = tok;
    if (margin) *margin = mg;
    return MI_OK;
}

int mi_step(mi_engine* e, const int32_t* toks, int32_t T, int32_t pos, int32_t* argmax, float* margin, float* logits) {
    if (!e || !toks) return MI_ERR_ARG;
    if (T < 1 || T > 8) return fail(e, MI_ERR_ARG, "mi_step: T=%d outside 1..8", T);
    if (pos < 0 || pos > e->cur_len || pos + T > e->opts.max_ctx)
        return fail(e, MI_ERR_ARG, "mi_step: position %d out of range (length %d, capacity %d)", pos, e->cur_len,
                    e->opts.max_ctx);
    int rc = check_ids(e, toks, T, "mi_step:");
    if (rc) return rc;
    int32_t tok = 0;
    float mg = 0.f;
    for (int32_t t = 0; t < T; t++) {
        tok = orc_forward(e->m, toks[t], pos + t, logits ? logits + (size_t)t * e->info.n_vocab : NULL, &mg);
        if (tok < 0) return fail(e, MI_ERR_STATE, "forward failed at position %d", pos + t);
        if (argmax) argmax[t] = tok;
        if (margin) margin[t] = mg;
    }
    e->cur_len = pos + T;
    e->next_tok = tok;
    e->next_margin = mg;
    e->next_ready = 1;
    return MI_OK;
}

int mi_generate(mi_engine* e, int32_t n_gen, int32_t* out, float* margins, int32_t* n_out, mi_token_cb cb,
                void* user) {
    if (!e || n_gen < 0) return MI_ERR_ARG;
    if (!e->next_ready || e->cur_len < 1) return fail(e, MI_ERR_STATE, "mi_generate needs mi_prefill first");
    if (e->cur_len + n_gen > e->opts.max_ctx) return fail(e, MI_ERR_ARG, "n_gen %d exceeds the context capacity", n_gen);
    const double t0 = now_s();
    const int32_t p0 = e->cur_len;
    int32_t tok = e->next_tok, emitted = 0;
    float mg = e->next_margin;
    for (int32_t t = 0; t < n_gen; t++) {
        if (t > 0) {
            tok = orc_forward(e->m, tok, p0 + t - 1, NULL, &mg);
            if (tok < 0) return fail(e, MI_ERR_STATE, "forward failed at position %d", p0 + t - 1);
        }
        if (out) out[t] = tok;
        if (margins) margins[t] = mg;
        emitted = t + 1;
        if ((cb && cb(tok, user)) || (e->opts.stop_eos && tok == e->info.eos)) break;
    }
    e->stats.steps = e->stats.tokens = emitted > 0 ? emitted - 1 : 0;   /* decode steps run, as the engine counts */
    e->stats.decode_ms = 1e3 * (now_s() - t0);
    e->stats.drafted = e->stats.accepted = 0;
    if (emitted > 1) e->cur_len = p0 + emitted - 1;
    e->next_tok = tok;
    e->next_margin = mg;
    if (n_out) *n_out = emitted;
    return MI_OK;
}

int mi_teacher(mi_engine* e, const int32_t* ids, int32_t n, int32_t* pred, float* margin) {
    if (!e || !ids || !pred || !margin || n < 1) return MI_ERR_ARG;
    if (n > e->opts.max_ctx)
        return fail(e, MI_ERR_ARG, "teacher sequence of %d tokens exceeds the context capacity %d", n, e->opts.max_ctx);
    int rc = check_ids(e, ids, n, "teacher");
    if (rc) return rc;
    for (int32_t p = 0; p < n; p++) {
        pred[p] = orc_forward(e->m, ids[p], p, NULL, &margin[p]);
        if (pred[p] < 0) return fail(e, MI_ERR_STATE, "forward failed at position %d", p);
    }
    e->cur_len = n;
    e->next_ready = 0;
    return MI_OK;
}
