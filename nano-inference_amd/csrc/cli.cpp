// cli.cpp -- the reference's command-line contract over the C ABI (cpu_infer.cpp:64-68,
// 161-167; cuda_infer.cu:845-868, 1146-1200, 1288-1291; mega.cu:1233-1249):
//
//   minfer <model.gguf> <n_gen> <id...>
//
// stdout: the generated tokens' text, streamed and flushed per token, stopping at the
// GGUF's eos token; with RAWIDS=1 the generated IDs separated by spaces instead (the
// format the reference's correctness gates parse). A newline ends the output either way.
// stderr: the stat lines the reference's tools parse ("... = X tok/s", and with SPEC=1
// "N generation steps, X tokens/step | drafted D, accepted A (P%)").
// Environment: RAWIDS, SPEC (n-gram speculative decode, output identical to greedy; 2: the
// loop on the device), NG (longest n-gram drafted, default 3), PERSISTENT (0: one launch per
// phase; 1: multi-token steps per phase, single tokens persistent; default 2), GRAPHS (1:
// multi-token steps replay a HIP graph instead of launching kernel by kernel), TCHUNK
// (prompt tokens per step, 1..8), DEVICE, and TEACHER=<k> (mega.cu:28-29, 1192-1205): the
// ids are a reference sequence whose first k are the prompt; every position is predicted
// under teacher forcing, and stderr gets the mismatches past the prompt and the line
// "teacher-forced top-1 agreement: A/T | P positions in X ms (Y ms per C-token step) |
// logit hash H" (H: the FNV-1a hash of all predictions and margins, equal across TCHUNK
// exactly when the runs are bit-identical); MARGINS=1 adds every "i:token:margin".
#include "minfer.h"

#include <chrono>
#include <cstdio>
#include <cstdlib>
#include <vector>

namespace {

int env_int(const char* name, int def) {
    const char* v = std::getenv(name);
    return v && *v ? std::atoi(v) : def;
}

struct Sink {
    mi_engine* e;
    bool raw;
    int eos;
    int printed;
};

int on_token(int32_t id, void* user) {
    Sink* s = static_cast<Sink*>(user);
    if (s->raw) {
        std::printf("%d ", id);
    } else {
        if (id == s->eos) return 0;            // the engine stops after it; not printed
        char buf[512];
        const int32_t n = mi_token_text(s->e, id, buf, (int32_t)sizeof buf);
        if (n > 0) std::fwrite(buf, 1, n < (int32_t)sizeof buf ? (size_t)n : sizeof buf, stdout);
        std::fflush(stdout);
    }
    s->printed++;
    return 0;
}

int fail(mi_engine* e, const char* what, int rc) {
    std::fprintf(stderr, "minfer: %s failed (%d): %s\n", what, rc, mi_last_error(e));
    if (e) mi_free(e);
    return 1;
}

}  // namespace

int main(int argc, char** argv) {
    if (argc < 4) {
        std::fprintf(stderr, "usage: %s <model.gguf> <n_gen> <id...>\n", argv[0]);
        return 1;
    }
    const int n_gen = std::atoi(argv[2]);
    std::vector<int32_t> ids;
    for (int i = 3; i < argc; i++) ids.push_back((int32_t)std::atoi(argv[i]));
    if (n_gen < 0) {
        std::fprintf(stderr, "minfer: n_gen must be >= 0\n");
        return 1;
    }
    const bool raw = env_int("RAWIDS", 0) != 0;

    mi_opts o;
    mi_default_opts(&o);
    o.max_ctx = (int32_t)ids.size() + n_gen + 16;     // verify steps write ahead of the committed tokens
    o.spec = std::min(std::max(env_int("SPEC", 0), 0), 2);
    o.ngmax = env_int("NG", o.ngmax);
    o.persistent = env_int("PERSISTENT", o.persistent);
    o.device = env_int("DEVICE", o.device);
    o.graphs = env_int("GRAPHS", o.graphs);
    o.tchunk = env_int("TCHUNK", o.tchunk);
    o.stop_eos = raw ? 0 : 1;
    const int teacher = env_int("TEACHER", 0);

    mi_engine* e = nullptr;
    if (int rc = mi_load(argv[1], &o, &e)) return fail(e, "load", rc);
    mi_model_info info;
    mi_info(e, &info);

    if (teacher > 0) {
        const int P = (int)ids.size();
        std::vector<int32_t> pred(P);
        std::vector<float> mg(P);
        const auto t0 = std::chrono::steady_clock::now();
        if (int rc = mi_teacher(e, ids.data(), P, pred.data(), mg.data())) return fail(e, "teacher", rc);
        const double ms = std::chrono::duration<double, std::milli>(std::chrono::steady_clock::now() - t0).count();
        int agree = 0, total = 0;
        for (int i = teacher - 1; i + 1 < P; i++, total++) {
            if (pred[i] == ids[i + 1]) {
                agree++;
                continue;
            }
            std::fprintf(stderr, "  pos %d: ref %d, minfer-hip %d (margin %.4f)\n", i + 1, ids[i + 1], pred[i], mg[i]);
        }
        std::printf("\n");
        std::fflush(stdout);
        std::fprintf(stderr,
                     "teacher-forced top-1 agreement: %d/%d | %d positions in %.1f ms (%.2f ms per %d-token step) | "
                     "logit hash %016llx\n",
                     agree, total, P, ms, ms * o.tchunk / P, o.tchunk,
                     (unsigned long long)mi_pred_hash(pred.data(), mg.data(), P));
        if (env_int("MARGINS", 0))
            for (int i = 0; i < P; i++) std::fprintf(stderr, "%d:%d:%.4f%c", i, pred[i], mg[i], i + 1 < P ? ' ' : '\n');
        mi_free(e);
        return 0;
    }

    int32_t first = 0;
    if (int rc = mi_prefill(e, ids.data(), (int32_t)ids.size(), &first, nullptr)) return fail(e, "prefill", rc);
    mi_stats st;
    mi_get_stats(e, &st);
    std::fprintf(stderr, "minfer-hip prefill: %zu tok in %.1f ms (sequential)\n", ids.size(), st.prefill_ms);

    Sink sink{e, raw, info.eos, 0};
    std::vector<int32_t> out((size_t)n_gen + 1);
    int32_t n_out = 0;
    if (n_gen > 0) {
        if (int rc = mi_generate(e, n_gen, out.data(), nullptr, &n_out, on_token, &sink)) return fail(e, "generate", rc);
    }
    std::printf("\n");
    std::fflush(stdout);
    mi_get_stats(e, &st);
    mi_model_info after;
    mi_info(e, &after);
    if (o.persistent && !after.persistent)
        std::fprintf(stderr, "minfer-hip: the persistent step was refused by the device (cooperative dispatch "
                             "busy); ran one launch per phase\n");
    // the tokens the timed decode steps made (the first printed token is the prefill's),
    // over their device time, as the reference's "n - 1 tok in ... ms" (mega.cu:1186-1190)
    const double ms = st.decode_ms;
    std::fprintf(stderr, "minfer-hip decode: %d tok in %.1f ms = %.2f tok/s\n", st.tokens, ms,
                 ms > 0 ? st.tokens * 1000.0 / ms : 0.0);
    if (o.spec)
        std::fprintf(stderr, "minfer-hip: %d generation steps, %.2f tokens/step | drafted %d, accepted %d (%.0f%%)\n",
                     st.steps, st.steps ? (double)st.tokens / st.steps : 0.0, st.drafted, st.accepted,
                     st.drafted ? 100.0 * st.accepted / st.drafted : 0.0);
    mi_free(e);
    return 0;
}
