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
constexpr int kWaves = 4;          // waves per workgroup of every phase kernel
constexpr int kThreads = kGroupRows * kWaves;
constexpr int kAttnChunk = 64;     // positions per attention partial
constexpr int kMaxE = 2048;        // largest hidden size the LDS staging holds
constexpr int kMaxFF = 11264;      // largest FFN width the LDS staging holds

struct PMat {                      // one q4_0 matrix in the tile layout
    const uint8_t* base;
    int32_t rows, nb, cb, nc, ks;
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
    float* qkv_part;               // [ks_qkv][QKV]
    float* qf;                     // [NH*HD] rotated q
    float* att_ml;                 // [NH][maxch][2] chunk max and sum
    float* att_o;                  // [NH][maxch][HD] chunk outputs
    float* att_out;                // [E]
    float* o_part;                 // [ks_o][E]
    float* gu_part;                // [ks_gu][2*FF]
    int8_t* act_q;                 // [FF]
    float2* act_ds;                // [FF/32] (scale, 8*sum(q) as int bits)
    float* d_part;                 // [ks_d][E]
    float* logits;                 // [V] (written when non-null)
    float4* cand;                  // [lm workgroups] (best, idx bits, second, 0)
    int32_t* out_tok;              // [maxseq] prediction made at each position
    float* out_margin;             // [maxseq]
};

inline __host__ __device__ size_t tile_bytes(int cb) { return (size_t)cb * 1152; }

}  // namespace mi
