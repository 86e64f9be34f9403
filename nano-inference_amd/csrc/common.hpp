// common.hpp -- device-side model description shared by the host engine and the
// gfx950 kernels.
//
// HBM layout (one GPU, everything resident):
//   q4_0 matrices   "tile layout": rows in groups of 64 (one wave64 lane per row),
//                   blocks in chunks of cb (4 or 8); tile (g, c) = cb slabs of
//                   64 x 16 quant bytes (slab k, lane r at k*1024 + r*16) followed
//                   by 64 x cb fp16 scales (lane r at cb*1024 + r*cb*2). Tiles of a
//                   group are consecutive. A wave's load of one slab is 1 KB
//                   contiguous; its scale load is 64 x (2*cb) B contiguous.
//                   (Reference: mega.cu:55-59 PM / pack_q4 :966-984 use 32-row
//                   groups for 32-wide warps.)
//   fused QKV       rows [q (NH*HD); k (KVD); v (KVD)] in GGUF order
//   fused gate/up   row group G = 32 gate rows 32G.. then the 32 matching up rows,
//                   so one group's outputs are one 32-element SiLU*up quant block
//   KV cache        fp16 [layer][kv_head][position][head_dim]
//   residual stream fp32 h_in(l) / h_mid(l) per layer, never overwritten in a step
#pragma once
#include <hip/hip_fp16.h>
#include <hip/hip_runtime.h>
#include <cstdint>

namespace mi {

constexpr int kGroupRows = 64;     // rows per tile group = lanes per wave
constexpr int kWaves = 4;          // waves per workgroup of the per-phase kernels
constexpr int kThreads = kGroupRows * kWaves;
constexpr int kPWaves = 8;         // waves per workgroup of the persistent step kernel
constexpr int kPThreads = kGroupRows * kPWaves;
constexpr int kMaxWaves = 8;
constexpr int kAttnChunk = 64;     // positions per attention partial
constexpr int kInlineComb = 4;     // up to this many chunks the O phase merges them itself
constexpr int kAttnSplit = 16;     // past this many chunks the records merge as a two-level tree
constexpr int kActRec = 128;       // bytes per act block record (32 int8, scale, 8*sum, padding)
constexpr int kTRec = 40;          // block record stride of the multi-token steps: 32 codes, scale, 8*sum
constexpr int kMaxE = 2048;        // largest hidden size the LDS staging holds
constexpr int kMaxFF = 11264;      // largest FFN width the LDS staging holds
constexpr int kMaxT = 8;           // tokens of one multi-token step (mega.cu:50 TMAX)

struct PMat {                      // one q4_0 matrix in the tile layout
    const uint8_t* base;
    int32_t rows, nb, cb, nc, ks;
    int32_t rot;                   // segment t of the work split runs on workgroup (t + rot) % grid
};

struct DLayer {
    PMat qkv, o, gu, d;
    const float* an;               // attn_norm [E]
    const float* fn;               // ffn_norm  [E]
    const float* bqkv;             // q|k|v bias [QKV]
};

struct DModel {
    int32_t E, FF, NH, NKV, HD, G, KVD, QKV, V, NL, maxseq, maxch;
    float eps, scale;              // rms eps, 1/sqrt(head_dim)
    const DLayer* layers;          // [NL], device memory
    PMat lm;
    const float* emb;              // [V][E] fp32
    const float* out_norm;         // [E]
    const float2* rope;            // [maxseq][HD/2] (cos, sin)
    __half* kc;                    // [NL][NKV][maxseq][HD]
    __half* vc;
    int32_t* tokbuf;               // [maxseq+1] token at each position (prompt, then generated)
    float* hbuf;                   // [2*NL+1][E]: h_in(l) at 2l, h_mid(l) at 2l+1, lm input at 2NL
    // Values exchanged between workgroups inside one step live in per-layer buffers:
    // every 128-byte line has a single writer and is written once per launch (with
    // agent-coherent stores) before any workgroup reads it, so readers may use
    // ordinary, L2-shared loads.
    float* qkv_part;               // [NL][ks_qkv][QKV]
    float* att;                    // [NL][NH][maxch][arec] chunk output o[HD], max, sum
    float* att_out;                // [NL][E] merged attention (long contexts)
    float* o_part;                 // [NL][ks_o][E]
    uint8_t* act;                  // [NL][FF/32][kActRec] int8 block, scale, 8*sum(q)
    float* d_part;                 // [NL][ks_d][E]
    int32_t arec;                  // floats per attention record (HD + 32)
    float* logits;                 // [V] (written when non-null)
    float* cand;                   // [lm workgroups][32] (best, idx bits, second) per 128-byte line
    uint32_t* bar;                 // grid-barrier arrival counter (persistent kernel)
    uint64_t* prof;                // when non-null: [workgroup][prof_slots] s_memrealtime stamps
    int32_t* err;                  // set when a grid barrier times out
    int32_t* out_tok;              // [maxseq] prediction made at each position
    float* out_margin;             // [maxseq]
    // streaming generation (k_step launched with gen = kGenRing): each launch also writes
    // its (token, margin bits) as one 64-bit word to ring[pos], pinned host memory the
    // host polls while later launches run (mega.cu:847-856, 1165-1178)
    uint64_t* ring;                // [maxseq] device address of the mapped host ring
    int32_t eos;                   // the GGUF's eos token when generation stops there, else -1: a kGenRing
                                   // launch whose input is eos does nothing
    // multi-token steps (T <= kMaxT tokens at positions pos..pos+T-1, one launch per
    // phase): per-token copies of the exchange buffers, token index after the segment
    int32_t* posT;                 // [1] position of the step's first token (set before each launch sequence)
    float* hT;                     // [2*NL+1][kMaxT][E]
    float* qkvT;                   // [NL][ks_qkv][kMaxT][QKV]
    float* attT;                   // [NL][kMaxT][NH][maxch][arec]
    float* oT;                     // [NL][ks_oT = O's chunks per row][kMaxT][E]
    uint8_t* actT;                 // [NL][kMaxT][FF/32][kActRec]
    uint8_t* xT;                   // [3*NL+1][kMaxT][E/32][kTRec] int8 records of the GEMM inputs: per
                                   // layer the qkv, o and gate/up inputs, then lm_head's (xT_slots)
    float* dT;                     // [NL][ks_d][kMaxT][E]
    float* candT;                  // [workgroups][kMaxT][4]
    float* logitsT;                // [kMaxT][V] (written when non-null)
    struct SpecDev* spec;          // [1] state of speculative generation driven on the device
};

// Speculative generation on the device (mega.cu:863-895): each persistent multi-token
// launch verifies tokbuf[pos..pos+T-1] = [current token, drafts] at pos = *posT, then its
// workgroup 0 commits the accepted prefix plus the correction, updates the acceptance
// average, drafts the next step into tokbuf and sets T and *posT for the next launch.
// The emitted tokens are out_tok[p0-1 ..] (p0: the first generated position).
struct SpecDev {
    int32_t T;                     // tokens of the next verify step (1 + drafts)
    int32_t done;                  // 1: generation finished; later launches return at once
    int32_t emitted;               // tokens emitted so far (the first is the prefill's prediction)
    int32_t n_gen;                 // tokens to emit
    int32_t eos;                   // stop after emitting this token (-1: no stop)
    int32_t last_pos;              // position of the last emitted token (its K/V not computed)
    int32_t steps, drafted, accepted;
    int32_t ngmax, maxseq, tmax;
    float acc_num, acc_den;        // EWMA of accepted / (accepted + rejections) (mega.cu:613)
    float slope;                   // opts.spec_slope
    int32_t pad;
};

inline __host__ __device__ size_t tile_bytes(int cb) { return (size_t)cb * 1152; }

// k_step's gen argument: 0 = the prediction is only recorded (prefill, teacher, mi_step);
// 1 = it is also the next position's input token; kGenRing = as 1, plus the ring entry,
// and the step does nothing when its input token is eos (generation stopped there)
constexpr int kGenRing = 2;
// ring words: low 32 bits the token, high 32 the margin's bit pattern
constexpr uint64_t kRingEmpty = ~0ull;                    // not written yet (token -1)
constexpr uint64_t kRingFail = 0x00000000FFFFFFFEull;     // token -2: a grid barrier of that launch failed

}  // namespace mi
