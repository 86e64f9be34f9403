/* cli.c -- oracle_infer: cpu_infer's command line (cpu_infer.cpp:5, 63-68, 158-167)
 * over the oracle, with wall-clock timers around prefill and decode that the
 * reference does not print. TEST INFRASTRUCTURE / CPU BASELINE ONLY.
 *
 *   oracle_infer <model.gguf> <n_gen> <id0> <id1> ...
 *   env ORACLE_MODE=fp32 (default, cpu_infer semantics) | q8act (needs ORACLE_PLAN)
 *       ORACLE_PLAN="cb0,..,cb4:ks0,..,ks4:chunk:kvf16"
 * stdout: the n_gen greedy token IDs separated by spaces, then a newline.
 * stderr: the cpu_infer banner line and a timing line.
 */
#include "oracle.h"
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

static int parse_plan(const char* s, orc_plan* p) {
    return sscanf(s, "%d,%d,%d,%d,%d:%d,%d,%d,%d,%d:%d:%d", &p->cb[0], &p->cb[1], &p->cb[2], &p->cb[3], &p->cb[4],
                  &p->ks[0], &p->ks[1], &p->ks[2], &p->ks[3], &p->ks[4], &p->attn_chunk, &p->kv_f16) == 12;
}

int main(int argc, char** argv) {
    if (argc < 4) { fprintf(stderr, "usage: %s <model.gguf> <n_gen> <id...>\n", argv[0]); return 1; }
    orc_gguf* g = orc_gguf_open(argv[1]);
    if (!g) { fprintf(stderr, "oracle: %s\n", orc_gguf_error()); return 1; }
    const int n_gen = atoi(argv[2]);
    const int np = argc - 3;
    int32_t* ids = (int32_t*)malloc(sizeof(int32_t) * np);
    for (int i = 0; i < np; i++) ids[i] = atoi(argv[3 + i]);
    const char* mode_s = getenv("ORACLE_MODE");
    const int mode = mode_s && strcmp(mode_s, "q8act") == 0 ? ORC_MODE_Q8ACT : ORC_MODE_FP32;
    orc_plan plan; memset(&plan, 0, sizeof plan);
    if (mode == ORC_MODE_Q8ACT && (!getenv("ORACLE_PLAN") || !parse_plan(getenv("ORACLE_PLAN"), &plan))) {
        fprintf(stderr, "oracle: q8act mode needs ORACLE_PLAN\n"); return 1;
    }
    orc_model* m = orc_model_new(g, mode, mode == ORC_MODE_Q8ACT ? &plan : NULL, np + n_gen, 0);
    if (!m) { fprintf(stderr, "oracle: model setup failed (missing tensor or metadata)\n"); return 1; }
    orc_config c; orc_model_config(m, &c);
    fprintf(stderr, "minfer-cpu: qwen2 L=%d d=%d ff=%d H=%d/%d hd=%d vocab=%d\n",
            c.n_layer, c.n_embd, c.n_ff, c.n_head, c.n_head_kv, c.head_dim, c.n_vocab);
    int32_t* out = (int32_t*)malloc(sizeof(int32_t) * (n_gen > 0 ? n_gen : 1));
    double tp = 0, td = 0;
    if (orc_generate(m, ids, np, n_gen, out, NULL, &tp, &td)) { fprintf(stderr, "oracle: generate failed\n"); return 1; }
    for (int i = 0; i < n_gen; i++) printf("%d ", out[i]);
    printf("\n");
    fprintf(stderr, "oracle-%s: prefill %d tok in %.3f s (%.3f tok/s) | decode %d tok in %.3f s (%.3f tok/s)\n",
            mode == ORC_MODE_FP32 ? "fp32" : "q8act", np, tp, np / (tp > 0 ? tp : 1e-9),
            n_gen > 1 ? n_gen - 1 : 0, td, n_gen > 1 ? (n_gen - 1) / (td > 0 ? td : 1e-9) : 0.0);
    orc_model_free(m); orc_gguf_close(g); free(ids); free(out);
    return 0;
}
