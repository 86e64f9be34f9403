/* internal.h -- shared state of the oracle's two forward modes (test infrastructure). */
#ifndef MINFER_ORACLE_INTERNAL_H
#define MINFER_ORACLE_INTERNAL_H
#include "oracle.h"

typedef struct {
    const orc_tensor *an, *wq, *bq, *wk, *bk, *wv, *bv, *wo, *fn, *wg, *wu, *wd;
} orc_layer;

struct orc_model {
    int mode;
    orc_plan plan;
    orc_config c;
    int max_seq, n_threads;
    const orc_tensor *tok_emb, *out_w, *out_norm;
    orc_layer* L;
    /* KV cache [layer][pos][kv_dim] (cpu_infer.cpp:101-103), fp32 storage */
    float *kc, *vc;
    /* activations (cpu_infer.cpp:105-107) */
    float *h, *xb, *q, *k, *v, *att, *proj, *gbuf, *ubuf, *logits;
    /* q8act scratch */
    int8_t* xq; float* xd; int32_t* xs8;
    float* rope_c; float* rope_s;   /* [max_seq][head_dim/2], cpu_infer.cpp:54-55 values */
    float* scores;                   /* [max_seq] */
    /* q8act: q4_0 copies of the matrices stored in other types (the engine requantizes
     * them at load, mega.cu:1091-1111) */
    orc_tensor* own_t; uint8_t** own_buf; int n_own;
};

int32_t orc_forward_fp32(struct orc_model* m, int32_t token, int32_t pos);
int32_t orc_forward_q8act(struct orc_model* m, int32_t token, int32_t pos);
void orc_argmax(const float* x, int n, int32_t* idx, float* margin);

#endif
