/* minfer.h -- C ABI of the MI355X (gfx950) batch-1 decode engine.
 *
 * The reference has no library interface: its engines are executables whose
 * seams are internal (src/cuda_infer.cu record() :1031-1083 = one token at a
 * device-held position, forward_batch() :990-1026 = T <= 8 tokens at pos0,
 * src/mega.cu run<Shape>() :1005-1243 + kernel mega<M>(n_gen) :597-903 = load +
 * whole generate). This header turns those seams into plain C entry points
 * (int32 token IDs, plain pointers and sizes, int status codes, no exits), so
 * the reference's host (GGUF loader, CLI, drafter) can drive this engine in place
 * of the CUDA path. Every function is single-threaded per engine, as the
 * reference is (one host thread, cuda_infer.cu:1170-1200).
 *
 * Errors: every entry point returns MI_OK (0) or a negative MI_ERR_* code and
 * records a message readable with mi_last_error(); the reference instead prints
 * and exits (cuda_infer.cu:20, mega.cu:46-47, gguf.h:33/79/185-192).
 */
#ifndef MINFER_H
#define MINFER_H
#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define MI_OK 0
#define MI_ERR_ARG (-1)      /* bad argument / out-of-range position or token */
#define MI_ERR_IO (-2)       /* file cannot be opened or written */
#define MI_ERR_FORMAT (-3)   /* not a GGUF / missing tensor / unsupported tensor type */
#define MI_ERR_SHAPE (-4)    /* model shape the kernels do not support (mega.cu:47 REQUIRE) */
#define MI_ERR_DEVICE (-5)   /* HIP runtime error or no gfx950 device */
#define MI_ERR_OOM (-6)      /* device allocation failed */
#define MI_ERR_STATE (-7)    /* call out of order (e.g. generate before prefill) */

typedef struct mi_engine mi_engine;

/* Engine options. Environment knobs of the reference map onto fields:
 * TCHUNK (mega.cu:1019) -> tchunk, SPEC (mega.cu:1020) -> spec, NGMAX (:1021) -> ngmax,
 * SPEC_SLOPE (:1022) -> spec_slope; maxseq = P + n_gen + TMAX (:1023) -> max_ctx. */
typedef struct mi_opts {
    int32_t max_ctx;       /* KV cache capacity in positions (0: 4096) */
    int32_t tchunk;        /* prompt tokens per step, 1..8 */
    int32_t spec;          /* n-gram speculative decoding inside mi_generate: 0 off; 1 the host drafts,
                              launches each verify step and commits its result; 2 the whole loop runs
                              on the device (mega.cu:863-895: each persistent verify launch commits
                              and drafts the next step itself; needs persistent 2 and no token
                              callback, else as 1). Same tokens either way; 1 measured faster on
                              MI355X (3117 vs 2942 tok/s on config 2). */
    int32_t ngmax;         /* longest n-gram the drafter matches (mega.cu:561-578) */
    float spec_slope;      /* cost of each extra token in a step, relative to a 1-token step */
    int32_t persistent;    /* 1: one persistent kernel per step (a plain launch of one workgroup per CU;
                              if a grid barrier ever gives up because the workgroups were not all
                              resident, the engine recomputes with cooperative launches from then
                              on); 0: one launch per phase; 2 (default): as 1, and each multi-token
                              step (prompt chunks, verify steps) also one persistent launch, the same
                              bits as its per-phase launches (1), and faster on MI355X: T = 8 verify
                              2.20 vs 2.25 ms, 512-token prefill 90.2 vs 91.4 ms */
    int32_t stop_eos;      /* mi_generate stops after tokenizer.ggml.eos_token_id */
    int32_t device;        /* HIP device ordinal */
    int32_t graphs;        /* 1: each multi-token step replays a HIP graph captured once per (T, logits)
                              instead of ~300 kernel launches (same results; saves host launch work).
                              Default 0: rocprofv3 --kernel-trace crashed in the HIP runtime while
                              capturing on this ROCm image, and the GPU time differs by <1%. */
} mi_opts;

/* reference defaults: TCHUNK 8, SPEC 1 (mega) / 0 (cuda_infer), NGMAX 3, SPEC_SLOPE 0.074 */
void mi_default_opts(mi_opts* o);

/* cuda_infer.cu:844-901 / mega.cu:1005-1113: parse the GGUF, repack every q4_0
 * matrix into the device tile layout, upload, allocate the KV cache and state. */
int mi_load(const char* gguf_path, const mi_opts* opts, mi_engine** out);
void mi_free(mi_engine* e);
/* message of the last failure on e (or of the last failed mi_load when e is NULL) */
const char* mi_last_error(const mi_engine* e);

/* Model shape and the engine's reduction plan (the fixed float summation order
 * the kernels follow; the CPU oracle takes the same plan to match them bit for bit). */
typedef struct mi_model_info {
    int32_t n_layer, n_embd, n_ff, n_head, n_head_kv, head_dim, n_vocab, eos;
    float rope_base, rms_eps;
    int32_t max_ctx;
    int32_t plan_cb[5];    /* blocks per chunk: qkv, o, gate/up, down, lm_head */
    int32_t plan_ks[5];    /* K segments per row, same order */
    int32_t attn_chunk;    /* positions per attention partial */
    int32_t kv_f16;        /* 1: the KV cache holds fp16 */
    int32_t n_cu;          /* compute units of the device */
    int32_t persistent;    /* step mode in use */
    uint64_t weight_bytes; /* q4_0 bytes streamed per token (all layers + lm_head) */
    int32_t coop;          /* 1: the persistent kernel goes out as a cooperative launch */
} mi_model_info;
int mi_info(const mi_engine* e, mi_model_info* out);

/* Prefill: cuda_infer.cu:1133-1159 / mega.cu:622, 819-820 prompt steps. Runs ids[0..n)
 * at positions 0..n-1 (from an empty cache) in chunks of opts.tchunk tokens (each chunk
 * one multi-token step; results bit-identical to one step per token) and returns the
 * greedy prediction after the last one (= the first generated token) and its margin. */
int mi_prefill(mi_engine* e, const int32_t* ids, int32_t n, int32_t* first, float* margin);

/* One step: forward_batch(toks, T, pos0) (cuda_infer.cu:990-1026). Runs toks[0..T)
 * at positions pos..pos+T-1 (pos <= current length: a smaller pos rewinds, which is
 * how rejected drafts are dropped), writes their K/V, returns per token the argmax
 * (lowest index on ties), the margin best - second, and optionally the logits
 * [T][n_vocab] (nullable; the reference never exposes logits). 1 <= T <= 8 (TMAX,
 * mega.cu:50). T > 1 is the verify step of speculative decoding: one pass over the
 * weights with int8 MFMA tiles; every token's logits are bit-identical to running
 * the tokens one at a time with T = 1. */
int mi_step(mi_engine* e, const int32_t* toks, int32_t T, int32_t pos,
            int32_t* argmax, float* margin, float* logits);

/* Host side of speculative decoding (mega.cu:557-589), exported so callers and tests
 * can use them directly. mi_ngram_draft: for n = ngmax..1, the latest earlier
 * occurrence of the last n tokens of h[0..len) proposes the up to kmax tokens that
 * followed it; returns the draft length. mi_best_draft_len: the K in 0..tmax-1 that
 * maximises (1-alpha^(K+1))/(1-alpha) / (1+slope*K). */
int32_t mi_ngram_draft(const int32_t* h, int32_t len, int32_t ngmax, int32_t kmax, int32_t* out);
int32_t mi_best_draft_len(float alpha, float slope, int32_t tmax);

/* Token callback for mi_generate; returning nonzero stops generation. */
typedef int (*mi_token_cb)(int32_t id, void* user);

/* Greedy generation after mi_prefill (cuda_infer.cu:1170-1200, mega.cu:819-895):
 * emits n_gen tokens, the first being mi_prefill's prediction. out[n_gen] and
 * margins[n_gen] (nullable) receive them; *n_out the count actually emitted
 * (fewer when stop_eos hits eos or the callback stops). With opts.spec = 1 each step
 * verifies [current token, n-gram draft] in one multi-token step and commits the
 * predictions up to the first one that disagrees with its draft (mega.cu:863-895):
 * the output is token for token the plain greedy decode. */
int mi_generate(mi_engine* e, int32_t n_gen, int32_t* out, float* margins, int32_t* n_out,
                mi_token_cb cb, void* user);

/* Teacher forcing: the TEACHER=<k> mode of mega.cu:28-29, 596, 857-862, 1192-1205. Runs
 * ids[0..n) as the context at positions 0..n-1 (from an empty cache) in chunks of
 * opts.tchunk tokens, as mi_prefill does, and returns every position's greedy
 * prediction: pred[i], margin[i] = the argmax (lowest index on ties) and best - second
 * after position i, i.e. the prediction for position i+1. The caller compares
 * pred[i] with ids[i+1] for the positions past its prompt (the reference's "top-1
 * agreement"). Leaves the context at length n. */
int mi_teacher(mi_engine* e, const int32_t* ids, int32_t n, int32_t* pred, float* margin);

/* The reference's exactness hash of a teacher-forced run (mega.cu:1197-1201): FNV-1a 64
 * over, for i = 0..n-1, the 4 little-endian bytes of pred[i] then the 4 of margin[i]'s
 * bit pattern, from the reference's offset basis 1469598103934665603 (mega.cu:1197;
 * the published FNV basis is 14695981039346656037). Runs with different chunk sizes
 * give the same hash exactly when every prediction and margin is bit-identical. */
uint64_t mi_pred_hash(const int32_t* pred, const float* margin, int32_t n);
/* FNV-1a 64 of n bytes from offset basis `basis` (prime 1099511628211): the building
 * block of mi_pred_hash, exported so the published FNV vectors can pin it. No reference
 * counterpart. */
uint64_t mi_fnv1a64(const void* data, size_t n, uint64_t basis);

/* Timing of the last mi_generate: device time of its decode steps measured with
 * HIP events on the engine stream (the reference prints the same figure,
 * mega.cu:1186-1190, cuda_infer.cu:1196-1199). */
typedef struct mi_stats {
    int32_t steps;          /* decode steps run (with speculation: verify steps) */
    int32_t tokens;         /* tokens emitted by those steps */
    double decode_ms;       /* device time of those steps (with speculation: wall time) */
    double prefill_ms;      /* device time of the last mi_prefill */
    int32_t drafted;        /* draft tokens proposed (speculation; mega.cu stats[1]) */
    int32_t accepted;       /* draft tokens accepted (speculation; mega.cu stats[2]) */
} mi_stats;
int mi_get_stats(const mi_engine* e, mi_stats* out);

/* Text of one token (src/detok.h:28-41 detok_piece over the GGUF's
 * tokenizer.ggml.tokens): the vocab piece decoded from byte-level BPE code points to
 * raw bytes into out[0..cap). Returns the byte count (only the first cap are written;
 * it may exceed cap) or a negative status (MI_ERR_ARG for an id outside the vocab). */
int32_t mi_token_text(const mi_engine* e, int32_t id, char* out, int32_t cap);
/* The same decoding for any piece of `len` bytes (src/detok.h:13-41); -1 on bad
 * arguments. Needs no engine and no device. */
int32_t mi_detok_piece(const char* piece, int32_t len, char* out, int32_t cap);

/* Measurement hook, no counterpart in the reference (which profiles with nsys/ncu and
 * in-kernel clock64 marks, mega.cu:111-119): re-launches one phase kernel of the
 * last step `reps` times on the engine stream and returns its mean duration from
 * HIP events. phase: 0 qkv, 1 attention, 2 chunk merge (launched only past 16 chunks),
 * 3 o, 4 gate/up + SiLU + quant, 5 down, 6 lm_head, 7 argmax, 8 the whole persistent
 * step kernel (persistent mode). Needs a completed step; re-running a phase rewrites
 * the same values, so the engine state is unchanged. */
int mi_time_phase(mi_engine* e, int32_t phase, int32_t layer, int32_t reps, double* avg_ms);

/* In-kernel phase profile of one persistent step (the reference's PROFILE=1,
 * mega.cu:111-119, 1206-1224): reruns the last step once with every workgroup
 * stamping the device wall clock (100 MHz). With S = 1 + 8*(5*n_layer + 1) slots and
 * W = the persistent grid (mi_model_info.n_cu workgroups), us[w*S + s] receives slot s
 * of workgroup w in microseconds since the earliest start, n >= W*S. Slots: 0 start;
 * then eight per phase, for qkv, attention, o, gate/up and down of every layer and
 * finally lm_head: prologue end (inputs loaded, normalised and quantised), the
 * first worker wave's tiles done, its stores drained (lm_head: the workgroup's
 * argmax candidate written), phase end, barrier exit, the control wave's input
 * staging landed, the first worker's staging landed (with its prefetched tiles), the
 * residual add done (norm phases). Slots never stamped read as 0 - earliest start. */
int mi_profile_step(mi_engine* e, double* us, int32_t n);

/* Cost of a grid barrier of the persistent kernel: one cooperative launch of nwg
 * workgroups doing n barriers and nothing else; returns microseconds per barrier. */
int mi_barrier_cost(int32_t nwg, int32_t n, double* us_per_barrier);

/* Test hook of the launch-mode fallback: raise the persistent kernel's barrier error
 * flag from the host, as a grid barrier that gave up would. The next completed
 * single-token step then takes the recovery path (clear, switch to cooperative
 * launches, recompute); the kernels themselves run normally. */
int mi_debug_flag_barrier(mi_engine* e);

/* ---------------- synthetic model files ---------------- */
typedef struct mi_synth_shape {
    int32_t n_layer, n_embd, n_ff, n_head, n_head_kv, n_vocab;
    float rope_base, rms_eps;
    int32_t emb_type;      /* token embedding: 0 F32 (the configs), 2 q4_0, 8 q8_0 */
    int32_t head_type;     /* output.weight: 0 or 2 q4_0, 8 q8_0, 14 q6_K (real Qwen files carry q6_K) */
    int32_t down_type;     /* ffn_down.weight: 0 or 2 q4_0, 3 q4_1 (llama.cpp's q4_0 recipe) */
    int32_t tied;          /* 1: no output.weight, the embedding serves as lm_head */
    float qk_bias_std;     /* > 0: attn_q/attn_k biases N(0, qk_bias_std) instead of N(0, 0.02) */
    float norm_offset;     /* != 0: norm weights norm_offset + N(0, 0.02) (real models carry ~1) */
} mi_synth_shape;
/* Writes a seeded random-init qwen2 GGUF: q4_0 matrices (uniform nibbles, fp16
 * |N(0,0.002)| scales), fp32 N(0,0.02) norms/biases/embedding, a token list of
 * n_vocab entries. Same seed -> same bytes. Other matrix types, when asked for, have
 * random codes with scales of a similar weight range. qk_bias_std and norm_offset
 * (0: off) give attention scores of order 1 (parity tests of RoPE and the GQA head
 * mapping need them; at the defaults the scores are ~1e-2 and attention is near
 * uniform). No reference counterpart (the reference runs downloaded Qwen files,
 * README.md:58). */
int mi_synth_gguf(const char* path, const mi_synth_shape* shape, uint64_t seed);

/* Host-side bounds check of the step kernels' buffer indexing (no GPU needed). No
 * counterpart in the reference: for a model shape, a context of max_ctx positions and a
 * grid of n_cu workgroups, walks every index the single-token step (T = 1) or the
 * multi-token phase bodies (T = 2..8) form for a step at pos, with each body's loop
 * bounds, against the allocation sizes the engine uses. Returns MI_OK, MI_ERR_SHAPE with
 * the buffer and index in err, or MI_ERR_ARG. */
int mi_check_layout(const mi_synth_shape* shape, int32_t max_ctx, int32_t n_cu, int32_t T, int32_t pos, char* err,
                    int32_t errlen);

/* ---------------- kernel-level entry points (device pointers) ----------------
 * For the microbenchmarks and bit-exact parity tests. `stream` is a hipStream_t
 * (NULL = the null stream). All pointers are device pointers unless noted. */

/* bytes of a rows x (nb*32) q4_0 matrix in the device tile layout: 64-row groups,
 * chunks of cb blocks; tile (group g, chunk c) holds cb slabs of 64 x 16 quant
 * bytes then 64 x cb fp16 scales. Replaces mega.cu pack_q4 (:966-984). */
size_t mi_q4_packed_bytes(int32_t rows, int32_t nb, int32_t cb);
/* host: GGUF row-major q4_0 blocks (18 B each) -> tile layout (host buffers) */
int mi_q4_pack(const uint8_t* src, int32_t rows, int32_t nb, int32_t cb, uint8_t* dst);

/* per-32 symmetric int8 quantization of x[n] (cuda_infer.cu:80-89 quant_x_q8,
 * mega.cu:303-325 quant32): xq[n], xd[n/32] (fp16-rounded scale), xs8[n/32] = 8*sum(q) */
int mi_quant_q8(const float* x, int32_t n, int8_t* xq, float* xd, int32_t* xs8, void* stream);

/* q4_0 x int8 GEMV on a packed matrix (cuda_infer.cu:94-127 gemv_dp4a, mega.cu:178-196
 * row_dot): part[ks][rows] = per-segment row sums, y[rows] = segments added in order
 * (y may be NULL). */
int mi_gemv_q4(const uint8_t* packed, int32_t rows, int32_t nb, int32_t cb, int32_t ks,
               const int8_t* xq, const float* xd, const int32_t* xs8,
               float* part, float* y, void* stream);

/* integer block sums isum[rows][nb] = sum_j n_j * x_j of the packed matrix against xq
 * (the exact integer part of dot_q4, mega.cu:157-165) */
int mi_q4_block_isums(const uint8_t* packed, int32_t rows, int32_t nb, int32_t cb,
                      const int8_t* xq, int32_t* isum, void* stream);

/* single-query GQA attention over an fp16 cache (cuda_infer.cu:650-702 attn_partial +
 * attn_combine, mega.cu:414-521), two kernel launches on `stream` (chunk records, then
 * their merge): q[n_head][hd] fp32, kc/vc [n_head_kv][ctx][hd] fp16, positions 0..L-1,
 * out[n_head][hd]; n_head / n_head_kv <= 8, at most 512 splits of 16 64-position chunks
 * (L <= 524288). scratch holds mi_attn_scratch_floats(n_head, hd, L) floats: a record
 * per head and 64-position chunk, written and read within the call (no initial
 * contents needed). Calls that share a scratch buffer must not overlap. */
size_t mi_attn_scratch_floats(int32_t n_head, int32_t hd, int32_t L);
int mi_attn_decode(const float* q, const uint16_t* kc, const uint16_t* vc, int32_t n_head,
                   int32_t n_head_kv, int32_t hd, int32_t L, int32_t ctx, float scale,
                   float* scratch, float* out, void* stream);

/* The same attention (same arguments, scratch and record layout, same merge) with each
 * chunk's scores and p.v as fp16 matrix-core contractions: q and the probabilities are
 * split into two fp16 parts each (~22 significant bits), K and V are used as stored, the
 * products are exact and accumulate in fp32. Within ~1e-6 relative of mi_attn_decode,
 * not bit-identical to it (the order of the sums inside a matrix instruction is the
 * hardware's). Replaces the same reference kernels (cuda_infer.cu:650-702
 * attn_partial + attn_combine); config-3 tolerance 1e-3 relative. */
int mi_attn_decode_mfma(const float* q, const uint16_t* kc, const uint16_t* vc, int32_t n_head,
                        int32_t n_head_kv, int32_t hd, int32_t L, int32_t ctx, float scale,
                        float* scratch, float* out, void* stream);

/* The same attention as mi_attn_decode without a workspace argument and without any
 * allocation. No counterpart in the reference: it is for callers that cannot allocate
 * (code under HIP graph capture, serving loops, harnesses that forbid hipMalloc). The
 * scratch is a library-held device array of MI_ATTN_NOALLOC_SCRATCH_FLOATS floats (16 MiB,
 * one per GPU, held until the process ends); a shape that needs more than
 * mi_attn_scratch_floats() allows returns MI_ERR_SHAPE (message via mi_last_error(NULL)).
 * The first call on a device looks the array's address up on the host (no stream work):
 * code that captures the call into a HIP graph makes one call on that device before the
 * capture. All calls on one GPU share the array: calls that overlap on one GPU race. */
#define MI_ATTN_NOALLOC_SCRATCH_FLOATS (4u << 20)
int mi_attn_decode_noalloc(const float* q, const uint16_t* kc, const uint16_t* vc, int32_t n_head,
                           int32_t n_head_kv, int32_t hd, int32_t L, int32_t ctx, float scale,
                           float* out, void* stream);

/* stream-read roofline (bench/roofline.cu:39-71 k_gridstride): one launch reading
 * `bytes` (multiple of 16) with several 16-byte loads in flight per thread */
int mi_stream_read(const void* buf, size_t bytes, uint32_t* sink, void* stream);

/* device-side timing helpers for callers without a HIP binding */
int mi_stream_sync(void* stream);
int mi_device_count(int32_t* n);

#ifdef __cplusplus
}
#endif
#endif
