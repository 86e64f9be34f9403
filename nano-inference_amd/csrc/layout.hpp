// layout.hpp -- sizes and offsets of the buffers the step kernels exchange through
// (DModel), in one place: the engine allocates with the *_size functions, the kernels
// index with the offset functions, and mi_check_layout (engine.hip) walks every index
// the phase bodies form against the sizes on the host, without a GPU.
//
// Offsets are in elements of the buffer's type (bytes for the int8 record buffers).
#pragma once
#include "common.hpp"

namespace mi {


// the shape facts the layouts depend on (filled from the model and the options)
struct Dims {
    int NL, E, FF, NH, NKV, HD, QKV, V, maxseq, maxch, arec;
    int ks_qkv, ks_o, ks_d;        // split-K segments of qkv, o and down (the plan)
    int ks_oT;                     // O's split in the multi-token steps: one segment per chunk
    int nwg;                       // workgroups of the persistent kernels (argmax candidates)
};

namespace lay {
#define LAYFN __host__ __device__ __forceinline__
// ---- single-token step
LAYFN size_t hbuf_size(const Dims& d) { return (size_t)(2 * d.NL + 1) * d.E; }
LAYFN size_t qkv_part(int ks, int QKV, int l) { return (size_t)l * ks * QKV; }        // + s * QKV + row
LAYFN size_t qkv_part_size(const Dims& d) { return (size_t)d.NL * d.ks_qkv * d.QKV; }
LAYFN size_t att(int NH, int maxch, int arec, int l) { return (size_t)l * NH * maxch * arec; }   // + (h * maxch + c) * arec + i
LAYFN size_t att_size(const Dims& d) { return (size_t)d.NL * d.NH * d.maxch * d.arec; }
LAYFN size_t o_part(int ks, int E, int l) { return (size_t)l * ks * E; }                  // + s * E + row
LAYFN size_t o_part_size(const Dims& d) { return (size_t)d.NL * d.ks_o * d.E; }
LAYFN size_t act(int FF, int l) { return (size_t)l * (FF / 32) * kActRec; }            // bytes; + g * kActRec + byte
LAYFN size_t act_size(const Dims& d) { return (size_t)d.NL * (d.FF / 32) * kActRec; }
LAYFN size_t d_part(int ks, int E, int l) { return (size_t)l * ks * E; }                  // + s * E + row
LAYFN size_t d_part_size(const Dims& d) { return (size_t)d.NL * d.ks_d * d.E; }
LAYFN size_t kv(int NKV, int maxseq, int HD, int l, int kvh, int p) {                    // + dim
    return (((size_t)l * NKV + kvh) * maxseq + p) * HD;
}
LAYFN size_t kv_size(const Dims& d) { return (size_t)d.NL * d.NKV * d.maxseq * d.HD; }
// ---- multi-token steps (T <= kMaxT tokens)
LAYFN size_t hT(int E, int slot, int t) { return ((size_t)slot * kMaxT + t) * E; }        // + e
LAYFN size_t hT_size(const Dims& d) { return (size_t)(2 * d.NL + 1) * kMaxT * d.E; }
LAYFN size_t qkvT(int ks, int QKV, int l) { return (size_t)l * ks * kMaxT * QKV; }        // + (s * kMaxT + t) * QKV + row
LAYFN size_t qkvT_size(const Dims& d) { return (size_t)d.NL * d.ks_qkv * kMaxT * d.QKV; }
LAYFN size_t attT(int NH, int maxch, int arec, int l, int t) {                           // + (h * maxch + c) * arec + i
    return ((size_t)l * kMaxT + t) * NH * maxch * arec;
}
LAYFN size_t attT_size(const Dims& d) { return (size_t)d.NL * kMaxT * d.NH * d.maxch * d.arec; }
// the GEMM inputs' int8 records, one slot per (layer, input) so that every line is
// written once per step: slot 3l = layer l's qkv input, 3l + 1 its o input, 3l + 2 its
// gate/up input, 3 NL the lm_head input
constexpr int kXtQkv = 0, kXtO = 1, kXtGu = 2;
LAYFN int xt_slot(int NL, int l, int which) { return l < NL ? 3 * l + which : 3 * NL; }
// bytes per token in an xT slot: E/32 records of kTRec bytes, rounded up to 16 mod 128.
// The GEMMs copy a slot's tokens into LDS as they lie, and at a stride that is a multiple
// of 128 bytes the eight tokens' records of one block would share LDS banks.
LAYFN size_t xT_tok(int E) {
    const size_t s = (size_t)(E / 32) * kTRec;
    return s + ((16 - s) & 127);
}
LAYFN size_t xT(int E, int slot) { return (size_t)slot * kMaxT * xT_tok(E); }   // bytes; + t * xT_tok(E) + b * kTRec + byte
LAYFN size_t xT_size(const Dims& d) { return (size_t)(3 * d.NL + 1) * kMaxT * xT_tok(d.E); }
LAYFN size_t oT(int ks, int E, int l) { return (size_t)l * ks * kMaxT * E; }              // + (s * kMaxT + t) * E + row
LAYFN size_t oT_size(const Dims& d) { return (size_t)d.NL * d.ks_oT * kMaxT * d.E; }
LAYFN size_t actT(int FF, int l, int t) { return ((size_t)l * kMaxT + t) * (FF / 32) * kActRec; }  // bytes
LAYFN size_t actT_size(const Dims& d) { return (size_t)d.NL * kMaxT * (d.FF / 32) * kActRec; }
LAYFN size_t dT(int ks, int E, int l) { return (size_t)l * ks * kMaxT * E; }              // + (s * kMaxT + t) * E + row
LAYFN size_t dT_size(const Dims& d) { return (size_t)d.NL * d.ks_d * kMaxT * d.E; }
LAYFN size_t candT(int wg, int t) { return ((size_t)wg * kMaxT + t) * 4; }                // + 0..3
LAYFN size_t candT_size(const Dims& d) { return (size_t)d.nwg * kMaxT * 4; }
LAYFN size_t logitsT_size(const Dims& d) { return (size_t)kMaxT * d.V; }                  // t * V + row
#undef LAYFN
}  // namespace lay

}  // namespace mi
