// kernels.hip -- gfx950 kernels of the batch-1 decode step.
//
// Every floating-point operation below is an explicitly rounded IEEE-754 binary32
// operation (__fadd_rn, __fmul_rn, __fmaf_rn, __fdiv_rn, __builtin_sqrtf) issued in a
// fixed order, so the results do not depend on how work is split across waves
// and workgroups, and equal the CPU restatement of the same order bit for bit.
// The orders (the reduction plan) are:
//   q4_0 x int8 row   per block isum = sum(nibble * x) via v_dot4_i32_i8, minus
//                     8*sum(x); acc = fma(dw*dx, float(isum - 8 sum x), acc) over the
//                     cb blocks of a chunk, from 0 (mega.cu:153-155); the chunk sums
//                     of a K segment are added left to right, then the ks segments
//                     of the row left to right (mega.cu:665-673)
//   RMSNorm           64 lane partials (lane l: elements 256j + 4l + i, i < 4, in
//                     order) by fma, then xor butterfly 32..1; x * (1/sqrt(mean+eps))
//                     * w (cpu_infer.cpp:40-46, mega.cu:336-347)
//   int8 quant        per 32 elements: amax, 127/amax, round half even, fp16(amax/127),
//                     8*sum(q) (cuda_infer.cu:80-89, mega.cu:303-325)
//   attention         64-position chunks: lane = position for q.k (4 fma chains over
//                     d mod 4), lane max, exp, butterfly sum; lane = dim for p.v
//                     (fma chain over positions); chunks merged by max rescaling in
//                     chunk order (cuda_infer.cu:650-702)
//   exp               mi_expf: Cody-Waite by ln2 + Taylor-7 Horner (no libm)
// Compile with -ffp-contract=off (nothing else gets fused) and without packed fp32.
//
// Work split of a step workgroup (512 threads = 8 waves, one workgroup per CU):
//   wave 0, "control"      the grid barrier, then the phase prologue: it gathers the
//                          phase input (split-K partials, attention records, act
//                          records) into LDS by DMA, adds the residual, normalises
//                          and quantises it into int8 block records in LDS
//   waves 1..7, "workers"  the phase's q4_0 weight tiles. A worker loads its tiles
//                          of the NEXT phase into registers as soon as its part of
//                          the current phase is stored, so the weight stream runs
//                          during the grid barrier and the control wave's prologue.
// A wave's vector memory reads complete in issue order, so a prefetch issued by a
// wave delays every later load of that same wave; keeping the barrier polls and the
// prologue loads in a wave that never prefetches is what lets them overlap.
#include "common.hpp"
#include "kernels.hpp"
#include "layout.hpp"

#include <algorithm>
#include <climits>
#include <mutex>
#include <type_traits>

namespace mi {

// The model description is read through constant-address-space pointers: a read of
// a generic pointer compiles to a vector load (the compiler cannot prove that the
// kernel's own stores leave it unchanged), which would queue behind a wave's weight
// prefetch; constant-space reads are scalar loads on their own counter, and the
// compiler reloads them instead of keeping every field live in registers.
#define AS4 __attribute__((address_space(4)))
typedef const AS4 DModel* MPtr;
typedef const AS4 DLayer* LPtr;
__device__ __forceinline__ LPtr LY(MPtr M, int l) { return (LPtr)M->layers + l; }
__device__ __forceinline__ PMat ldmat(const AS4 PMat* m) {
    PMat r;
    r.base = m->base; r.rows = m->rows; r.nb = m->nb; r.cb = m->cb; r.nc = m->nc; r.ks = m->ks; r.rot = m->rot;
    return r;
}

// ------------------------------------------------------------------ scalar helpers
__device__ __forceinline__ float mi_expf(float x) {
    if (x != x) return x;
    if (x > 88.72283f) return __builtin_inff();
    if (x < -87.0f) return 0.0f;
    const float n = __builtin_rintf(__fmul_rn(x, 0x1.715476p+0f));
    float r = __fmaf_rn(n, -0x1.62e4p-1f, x);
    r = __fmaf_rn(n, -0x1.7f7d1cp-20f, r);
    float p = 0x1.a01a02p-13f;
    p = __fmaf_rn(p, r, 0x1.6c16c2p-10f);
    p = __fmaf_rn(p, r, 0x1.111112p-7f);
    p = __fmaf_rn(p, r, 0x1.555556p-5f);
    p = __fmaf_rn(p, r, 0x1.555556p-3f);
    p = __fmaf_rn(p, r, 0x1p-1f);
    p = __fmaf_rn(p, r, 1.0f);
    p = __fmaf_rn(p, r, 1.0f);
    return __builtin_ldexpf(p, (int)n);
}

// LDS hand-off between lanes of one wave (waves run independently, so a workgroup
// barrier cannot be used): DS operations of one wave complete in order
// (the s_waitcnt builtin, unlike inline asm, is seen by the compiler's own wait
// insertion, which then knows nothing is outstanding afterwards; gfx9 encoding:
// vmcnt in bits 3:0 + 15:14, expcnt 6:4, lgkmcnt 11:8)
__device__ __forceinline__ void wave_lds_sync() { __builtin_amdgcn_s_waitcnt(0xC07F); }   // lgkmcnt(0)
__device__ __forceinline__ float h2f_lo(uint32_t u) { return __half2float(__ushort_as_half((unsigned short)(u & 0xFFFFu))); }
__device__ __forceinline__ float h2f_hi(uint32_t u) { return __half2float(__ushort_as_half((unsigned short)(u >> 16))); }
__device__ __forceinline__ float fp16_round(float v) { return __half2float(__float2half(v)); }

// Cross-lane partners without the LDS pipe. The xor butterfly pairs lane l with
// l ^ off for off = 32, 16, ..., 1; every step leaves a pair holding the same value
// (IEEE add and max are commutative), which the cheaper permutations rely on:
//   off 32, 16: v_permlane32_swap / v_permlane16_swap of v with itself leave the two
//               values of each pair (l, l ^ off) in the two results on lane l;
//   off 8:      DPP row_ror:8 is l ^ 8 inside each 16-lane row;
//   off 4:      DPP row_ror:4 reads lane (l + 4) mod 16, which holds the value of
//               l ^ 4 once the values are symmetric under xor 8;
//   off 2, 1:   DPP quad_perm [2,3,0,1] and [1,0,3,2] are l ^ 2 and l ^ 1.
// So each step adds exactly the same two values as the xor butterfly.
template <int CTRL>
__device__ __forceinline__ float dppf(float v) {
    return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), CTRL, 0xF, 0xF, false));
}
template <int CTRL>
__device__ __forceinline__ int dppi(int v) {
    return __builtin_amdgcn_update_dpp(0, v, CTRL, 0xF, 0xF, false);
}
constexpr int kDppXor1 = 0xB1, kDppXor2 = 0x4E, kDppRor4 = 0x124, kDppRor8 = 0x128, kDppHalfMirror = 0x141;
__device__ __forceinline__ void pair32(float v, float& a, float& b) {
    const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
    a = __uint_as_float(r[0]);
    b = __uint_as_float(r[1]);
}
__device__ __forceinline__ void pair16(float v, float& a, float& b) {
    const auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
    a = __uint_as_float(r[0]);
    b = __uint_as_float(r[1]);
}
__device__ __forceinline__ float bfly_sum64(float v) {
    float a, b;
    pair32(v, a, b);
    v = __fadd_rn(a, b);
    pair16(v, a, b);
    v = __fadd_rn(a, b);
    v = __fadd_rn(v, dppf<kDppRor8>(v));
    v = __fadd_rn(v, dppf<kDppRor4>(v));
    v = __fadd_rn(v, dppf<kDppXor2>(v));
    return __fadd_rn(v, dppf<kDppXor1>(v));
}
__device__ __forceinline__ float wave_max(float v) {
    float a, b;
    pair32(v, a, b);
    v = fmaxf(a, b);
    pair16(v, a, b);
    v = fmaxf(a, b);
    v = fmaxf(v, dppf<kDppRor8>(v));
    v = fmaxf(v, dppf<kDppRor4>(v));
    v = fmaxf(v, dppf<kDppXor2>(v));
    return fmaxf(v, dppf<kDppXor1>(v));
}
// max / integer sum over aligned groups of 8 lanes (exact in any order): quad steps,
// then the half-row mirror pairs lane i of a quad with the other quad of its 8
__device__ __forceinline__ float max8(float v) {
    v = fmaxf(v, dppf<kDppXor1>(v));
    v = fmaxf(v, dppf<kDppXor2>(v));
    return fmaxf(v, dppf<kDppHalfMirror>(v));
}
__device__ __forceinline__ int sum8(int v) {
    v += dppi<kDppXor1>(v);
    v += dppi<kDppXor2>(v);
    return v + dppi<kDppHalfMirror>(v);
}

// max / integer sum over each 32-lane half (exact in any order; pairings as in
// bfly_sum64: permlane16 swap, then DPP inside 16-lane rows)
__device__ __forceinline__ float max32(float v) {
    float a, b;
    pair16(v, a, b);
    v = fmaxf(a, b);
    v = fmaxf(v, dppf<kDppRor8>(v));
    v = fmaxf(v, dppf<kDppRor4>(v));
    v = fmaxf(v, dppf<kDppXor2>(v));
    return fmaxf(v, dppf<kDppXor1>(v));
}
__device__ __forceinline__ int sum32(int v) {
    const auto r = __builtin_amdgcn_permlane16_swap((unsigned)v, (unsigned)v, false, false);
    v = (int)(r[0] + r[1]);
    v += dppi<kDppRor8>(v);
    v += dppi<kDppRor4>(v);
    v += dppi<kDppXor2>(v);
    return v + dppi<kDppXor1>(v);
}

// quantize one 32-element block per half-wave: the lane's code, the block scale and
// 8*sum(q) on every lane (cuda_infer.cu:80-89, mega.cu:303-325)
__device__ __forceinline__ void quant32_vals(float v, int& q, float& d, int& s8) {
    const float a = max32(fabsf(v));
    const float inv = a > 0.f ? __fdiv_rn(127.f, a) : 0.f;
    q = __float2int_rn(__fmul_rn(v, inv));
    d = fp16_round(__fdiv_rn(a, 127.f));
    s8 = 8 * sum32(q);
}

// ------------------------------------------------------------------ memory helpers
// Inside one step, values that one workgroup writes and others read (GEMV partials,
// attention records, the int8 act, argmax candidates) are written once per launch
// into per-layer buffers whose 128-byte lines each have a single writer, with
// agent-coherent stores (global_store sc1: written through past the per-XCD L2).
// After the grid barrier every reader sees them with ordinary loads: no reader can
// hold an older copy of a line that is written once per launch, and the 32
// workgroups of an XCD share one L2 fill. That keeps the barrier free of agent-scope
// fences (an L2 write-back/invalidate per workgroup costs ~1.7 us at 256 workgroups).
__device__ __forceinline__ uint32_t ldc(const uint32_t* p) {
    return __hip_atomic_load(const_cast<uint32_t*>(p), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ void stc(float* p, float v) { __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT); }
__device__ __forceinline__ void stc(uint32_t* p, uint32_t v) { __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT); }
__device__ __forceinline__ void drain_vm() { __builtin_amdgcn_s_waitcnt(0x0F70); }      // vmcnt(0)
// a store to memory that other workgroups of the same launch read (P: agent-coherent)
// or that only later launches read (plain)
template <bool P>
__device__ __forceinline__ void st_x(float* p, float v) {
    if constexpr (P) stc(p, v);
    else *p = v;
}
template <bool P>
__device__ __forceinline__ void st_x(uint32_t* p, uint32_t v) {
    if constexpr (P) stc(p, v);
    else *p = v;
}

typedef __attribute__((address_space(3))) void* lds_ptr;
// one wave copies `bytes` (multiple of 16, both ends 16-byte aligned) from global
// memory straight into LDS, 1 KB per instruction (lane l moves bytes 16l..16l+15)
__device__ __forceinline__ void dma_wave(const void* g, void* lds, int bytes, int lane) {
    for (int off = 0; off < bytes; off += 1024)
        if (off + lane * 16 < bytes)
            __builtin_amdgcn_global_load_lds(static_cast<const uint8_t*>(g) + off + lane * 16,
                                             (lds_ptr)(static_cast<uint8_t*>(lds) + off), 16, 0, 0);
}

typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));
// weights are read once per token (868 MB > the 256 MB MALL): streaming loads
__device__ __forceinline__ uint4 ntload16(const uint8_t* p) {
    const u32x4 v = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(p));
    return make_uint4(v.x, v.y, v.z, v.w);
}

// ------------------------------------------------------------------ q4_0 x int8
// q4_0 block (16 bytes: byte j = element j low nibble, element j+16 high nibble)
// against 32 int8: the nibbles stay 0..15 (the -8 is folded into 8*sum(x))
__device__ __forceinline__ int dot_q4(uint4 w, int4 x0, int4 x1) {
    const unsigned M = 0x0F0F0F0Fu;
    int s = __builtin_amdgcn_sdot4((int)(w.x & M), x0.x, 0, false);
    s = __builtin_amdgcn_sdot4((int)(w.y & M), x0.y, s, false);
    s = __builtin_amdgcn_sdot4((int)(w.z & M), x0.z, s, false);
    s = __builtin_amdgcn_sdot4((int)(w.w & M), x0.w, s, false);
    s = __builtin_amdgcn_sdot4((int)((w.x >> 4) & M), x1.x, s, false);
    s = __builtin_amdgcn_sdot4((int)((w.y >> 4) & M), x1.y, s, false);
    s = __builtin_amdgcn_sdot4((int)((w.z >> 4) & M), x1.z, s, false);
    s = __builtin_amdgcn_sdot4((int)((w.w >> 4) & M), x1.w, s, false);
    return s;
}

// One lane's row of one tile (64-row group x cb blocks): cb x 16 quant bytes and cb
// fp16 scales. Int8 activations are "block records" in LDS: block b at x + b*rs holds
// 32 int8 codes, then the fp32 scale and 8*sum(q) as int32.
struct Tile { uint4 q[8]; uint4 s; };
constexpr int kXRec = 48;          // record stride of a quantised E vector (act records use kActRec)

__device__ __forceinline__ void tile_load(Tile& t, const uint8_t* p, int cb, int lane) {
    if (cb == 8) {
#pragma unroll
        for (int k = 0; k < 8; k++) t.q[k] = ntload16(p + k * 1024 + lane * 16);
        t.s = ntload16(p + 8192 + lane * 16);
    } else {
#pragma unroll
        for (int k = 0; k < 4; k++) t.q[k] = ntload16(p + k * 1024 + lane * 16);
        const uint2 v = *reinterpret_cast<const uint2*>(p + 4096 + lane * 8);
        t.s = make_uint4(v.x, v.y, 0u, 0u);
    }
}
// the same loads for a chunk size known at compile time (one straight-line sequence)
template <int CB>
__device__ __forceinline__ void tile_load_cb(Tile& t, const uint8_t* p, int lane) {
#pragma unroll
    for (int k = 0; k < CB; k++) t.q[k] = ntload16(p + k * 1024 + lane * 16);
    if constexpr (CB == 8) {
        t.s = ntload16(p + 8192 + lane * 16);
    } else {
        const uint2 v = *reinterpret_cast<const uint2*>(p + 4096 + lane * 8);
        t.s = make_uint4(v.x, v.y, 0u, 0u);
    }
}
__device__ __forceinline__ uint32_t u4_at(const uint4& v, int i) { return i == 0 ? v.x : i == 1 ? v.y : i == 2 ? v.z : v.w; }

// sum of one chunk: an fma chain over its CB blocks, from 0
template <int CB>
__device__ __forceinline__ float chunk_dot(const Tile& t, const uint8_t* x, int rs, int b0) {
    float acc = 0.f;
#pragma unroll
    for (int k = 0; k < CB; k++) {
        const uint8_t* xb = x + (b0 + k) * rs;
        const int4 x0 = *reinterpret_cast<const int4*>(xb);
        const int4 x1 = *reinterpret_cast<const int4*>(xb + 16);
        const float2 ds = *reinterpret_cast<const float2*>(xb + 32);
        const int isum = dot_q4(t.q[k], x0, x1);
        const uint32_t sw = u4_at(t.s, k >> 1);
        const float dw = (k & 1) ? h2f_hi(sw) : h2f_lo(sw);
        acc = __fmaf_rn(__fmul_rn(dw, ds.x), __int2float_rn(isum - __float_as_int(ds.y)), acc);
    }
    return acc;
}
__device__ __forceinline__ float chunk_dot(const Tile& t, int cb, const uint8_t* x, int rs, int b0) {
    return cb == 8 ? chunk_dot<8>(t, x, rs, b0) : chunk_dot<4>(t, x, rs, b0);
}
__device__ __forceinline__ const uint8_t* tile_ptr(const PMat W, int g, int c) {
    return W.base + ((size_t)g * W.nc + c) * tile_bytes(W.cb);
}
// floor(k / d) for 0 <= k < 2^22, d >= 1, without the ~30-instruction integer divide:
// the float estimate is at most one off, then corrected
__device__ __forceinline__ int div_small(int k, int d) {
    int q = (int)((float)k * __builtin_amdgcn_rcpf((float)d));
    if (q * d > k) q--;
    else if ((q + 1) * d <= k) q++;
    return q;
}
// first chunk of K segment s: s * nc / ks (integer division, the oracle's boundaries)
__device__ __forceinline__ int seg_c0(const PMat W, int s) { return W.ks == 1 ? s * W.nc : div_small(s * W.nc, W.ks); }

// ------------------------------------------------------------------ workgroup work split
constexpr int kWorkers = kPWaves - 1;      // waves 1..7
constexpr int kPartTiles = 96;             // chunk sums a workgroup stages per phase
constexpr int kCtlBytes = 72 * 1024;       // phase-input DMA staging (hd 128's attention union is larger)
constexpr int kMaxKsQkv = 2;               // q/k/v partials an attention item stages
constexpr int kMaxKsRes = 12;              // split-K partials a residual add takes

// Segments (64-row group g, K segment s; t = g*ks + s) go round-robin to
// workgroups, t -> workgroup (t + W.rot) % nwg. A workgroup's tiles are its segments'
// chunks in order; tile k belongs to worker k % kWorkers, which holds it in
// register slot (k / kWorkers) % 2.
struct TileRef { const uint8_t* p; int b0; };
// the workgroup's place in W's round-robin (W.rot < nwg); wg_tile and wg_segments take
// the place, which their callers compute once
__device__ __forceinline__ int wg_place(const PMat W, int wg, int nwg) {
    const int v = wg - W.rot;
    return v < 0 ? v + nwg : v;
}
__device__ __forceinline__ bool wg_tile(const PMat W, int wg, int nwg, int k, TileRef& r) {
    const int nseg = (W.rows >> 6) * W.ks;
    int t, c;
    if (W.ks == 1) {
        const int round = div_small(k, W.nc);
        t = wg + round * nwg;
        c = k - round * W.nc;
        if (t >= nseg) return false;
        r.p = tile_ptr(W, t, c);
    } else {
        t = wg;
        for (;;) {
            if (t >= nseg) return false;
            const int g = div_small(t, W.ks), s = t - g * W.ks, c0 = seg_c0(W, s), len = seg_c0(W, s + 1) - c0;
            if (k < len) { c = c0 + k; r.p = tile_ptr(W, g, c); break; }
            k -= len;
            t += nwg;
        }
    }
    r.b0 = c * W.cb;
    return true;
}

// calls f(g, s, k0, k1) for the workgroup's segments that worker kw finishes
// (segment r of the workgroup -> worker r % kWorkers); tiles k0..k1-1 are its chunks
template <class F>
__device__ __forceinline__ void wg_segments(const PMat W, int wg, int nwg, int kw, F f) {
    const int nseg = (W.rows >> 6) * W.ks;
    if (W.ks == 1) {          // every segment is a whole row group of nc chunks
        for (int t = wg + kw * nwg, r = kw; t < nseg; t += kWorkers * nwg, r += kWorkers) f(t, 0, r * W.nc, (r + 1) * W.nc);
        return;
    }
    int k0 = 0, r = 0;
    for (int t = wg; t < nseg; t += nwg, r++) {
        const int g = div_small(t, W.ks), s = t - g * W.ks, len = seg_c0(W, s + 1) - seg_c0(W, s);
        if (r % kWorkers == kw) f(g, s, k0, k0 + len);
        k0 += len;
    }
}
__device__ __forceinline__ float seg_sum(const float* P, int k0, int k1, int lane) {
    float v = P[k0 * 64 + lane];
    for (int k = k0 + 1; k < k1; k++) v = __fadd_rn(v, P[k * 64 + lane]);
    return v;
}

// the worker's first two tiles of W into registers. Both slots are written either
// way, so no older tile stays live (in registers) across the phases in between.
__device__ __forceinline__ void prefetch(const PMat W, int wg, int nwg, int kw, Tile (&tl)[2], int lane) {
    TileRef r;
    tl[0] = Tile{};
    tl[1] = Tile{};
    wg = wg_place(W, wg, nwg);
    if (wg_tile(W, wg, nwg, kw, r)) tile_load(tl[0], r.p, W.cb, lane);
    if (wg_tile(W, wg, nwg, kw + kWorkers, r)) tile_load(tl[1], r.p, W.cb, lane);
}

// chunk sums of the worker's tiles into P[k][64]: the two prefetched tiles, then any
// further ones loaded one at a time (only lm_head has more than two per worker; its
// 1792 workers keep ~16 MB in flight, enough to stay bandwidth-bound)
template <int CB>
__device__ __forceinline__ void gemv_tiles_cb(const PMat W, int wg, int nwg, int kw, Tile (&tl)[2], const uint8_t* x,
                                              int rs, float* P, int lane) {
    TileRef r;
    wg = wg_place(W, wg, nwg);
    if (!wg_tile(W, wg, nwg, kw, r)) return;
    P[kw * 64 + lane] = chunk_dot<CB>(tl[0], x, rs, r.b0);
    if (!wg_tile(W, wg, nwg, kw + kWorkers, r)) return;
    P[(kw + kWorkers) * 64 + lane] = chunk_dot<CB>(tl[1], x, rs, r.b0);
    for (int k = kw + 2 * kWorkers; wg_tile(W, wg, nwg, k, r); k += kWorkers) {
        tile_load(tl[0], r.p, CB, lane);
        P[k * 64 + lane] = chunk_dot<CB>(tl[0], x, rs, r.b0);
    }
}
__device__ __forceinline__ void gemv_tiles(const PMat W, int wg, int nwg, int kw, Tile (&tl)[2], const uint8_t* x, int rs,
                                           float* P, int lane) {
    if (W.cb == 8) gemv_tiles_cb<8>(W, wg, nwg, kw, tl, x, rs, P, lane);
    else gemv_tiles_cb<4>(W, wg, nwg, kw, tl, x, rs, P, lane);
}

// worker epilogue: segment sums stored as split-K partials part[s][row]
__device__ __forceinline__ void seg_store(const PMat W, int wg, int nwg, int kw, const float* P, float* part, int lane) {
    wg_segments(W, wg_place(W, wg, nwg), nwg, kw, [&](int g, int s, int k0, int k1) {
        stc(part + (size_t)s * W.rows + g * 64 + lane, seg_sum(P, k0, k1, lane));
    });
}

// ------------------------------------------------------------------ LDS layout
// attention unit (kv head, chunk): the K and V tiles, shared by the unit's head waves,
// then one area per wave: q / k / v split-K partials, q, and the wave's probability row
template <int HD>
constexpr int attn_head_lds() { return 3 * kMaxKsQkv * HD * 4 + 2 * HD * 4 + 64 * 4; }
template <int HD>
constexpr int attn_unit_lds() { return 2 * 64 * HD * 2 + kPWaves * attn_head_lds<HD>(); }
template <int HD>
constexpr int union_bytes() { return attn_unit_lds<HD>() > kCtlBytes ? attn_unit_lds<HD>() : kCtlBytes; }
constexpr int kFixedLds = 8 * kMaxE + (kMaxE / 32) * kXRec + kPartTiles * 256 + 1024;
template <int HD>
constexpr int step_lds() { return kFixedLds + union_bytes<HD>(); }

// R     the residual stream h [kMaxE] (the persistent kernel keeps it resident)
// T     the vector the control wave normalises / quantises [kMaxE]
// X     int8 block records of the phase input [kMaxE/32][kXRec]
// P     chunk sums [kPartTiles][64]
// misc  256 floats: per-wave argmax candidates, per-head merge weights
// U     control-wave DMA staging, or the attention waves' K/V (never both at once)
struct Lds {
    float* R; float* T; uint8_t* X; float* P; float* misc; uint8_t* U;
    __device__ explicit Lds(uint8_t* s)
        : R(reinterpret_cast<float*>(s)), T(reinterpret_cast<float*>(s + 4 * kMaxE)), X(s + 8 * kMaxE),
          P(reinterpret_cast<float*>(s + 8 * kMaxE + (kMaxE / 32) * kXRec)),
          misc(reinterpret_cast<float*>(s + 8 * kMaxE + (kMaxE / 32) * kXRec + kPartTiles * 256)),
          U(s + kFixedLds) {}
};

// ------------------------------------------------------------------ argmax candidates
struct Top2 { float best; int idx; float second; };
__device__ __forceinline__ void top2_push(Top2& t, float v, int row) {   // rows arrive increasing
    if (v > t.best) { t.second = t.best; t.best = v; t.idx = row; }
    else if (v > t.second) t.second = v;
}
__device__ __forceinline__ void top2_merge(Top2& a, float ob, int oi, float os) {
    const bool take = ob > a.best || (ob == a.best && oi < a.idx);
    a.second = fmaxf(fmaxf(a.second, os), take ? a.best : ob);
    if (take) { a.best = ob; a.idx = oi; }
}
// the xor butterfly over 64 lanes with the pairings of bfly_sum64; the pair merge is
// symmetric (max, lowest index on ties), so each step gives the xor result
__device__ __forceinline__ void top2_wave(Top2& t) {
    auto swap_merge = [&](bool p32) {
        const unsigned b = __float_as_uint(t.best), i = (unsigned)t.idx, s2 = __float_as_uint(t.second);
        const auto rb = p32 ? __builtin_amdgcn_permlane32_swap(b, b, false, false) : __builtin_amdgcn_permlane16_swap(b, b, false, false);
        const auto ri = p32 ? __builtin_amdgcn_permlane32_swap(i, i, false, false) : __builtin_amdgcn_permlane16_swap(i, i, false, false);
        const auto rs = p32 ? __builtin_amdgcn_permlane32_swap(s2, s2, false, false) : __builtin_amdgcn_permlane16_swap(s2, s2, false, false);
        Top2 x{__uint_as_float(rb[0]), (int)ri[0], __uint_as_float(rs[0])};
        top2_merge(x, __uint_as_float(rb[1]), (int)ri[1], __uint_as_float(rs[1]));
        t = x;
    };
    swap_merge(true);
    swap_merge(false);
    top2_merge(t, dppf<kDppRor8>(t.best), dppi<kDppRor8>(t.idx), dppf<kDppRor8>(t.second));
    top2_merge(t, dppf<kDppRor4>(t.best), dppi<kDppRor4>(t.idx), dppf<kDppRor4>(t.second));
    top2_merge(t, dppf<kDppXor2>(t.best), dppi<kDppXor2>(t.idx), dppf<kDppXor2>(t.second));
    top2_merge(t, dppf<kDppXor1>(t.best), dppi<kDppXor1>(t.idx), dppf<kDppXor1>(t.second));
}

// ------------------------------------------------------------------ grid barrier
// Workgroup w arrives on counter w % 16 (16 counters on separate 256-byte lines, so
// arrivals do not serialize on one address); the control wave then polls all 16
// counters at once (lane i reads counter i) until each holds its group's arrivals of
// this epoch. One atomic and one poll round trip: a second level of counters and a
// published epoch cost ~0.5 us more at 256 workgroups, one shared counter ~2 us more
// (256 atomics on one address). Run by the whole control wave after the workgroup
// barrier that follows every worker's own store drain; it drains its own stores
// first. A poll that outlives kSpinLimit sets *err and returns, so no wave can wait
// forever. bar[]: counter k at 64*k, the exit counter at 64*kBarGroups; all zero when a
// launch starts (zeroed at allocation, and each launch leaves them zero: see ctl_exit).
constexpr unsigned kSpinLimit = 1u << 16;   // polls (~1 us each) before a barrier gives up
constexpr int kBarGroups = 16;
constexpr int kBarWords = 64 * (kBarGroups + 2);
// per-launch barrier state of one control wave (computed once: no integer divides on
// the barrier path)
struct GridBar {
    uint32_t* arrive;          // this workgroup's group counter
    const uint32_t* poll;      // the word this lane polls (lanes >= groups: counter 0; lane 63: the error flag)
    unsigned per;              // arrivals per epoch on the polled counter (0: always met)
    unsigned need;             // this lane's target of the current epoch
    unsigned dead;             // a barrier of this launch failed: the rest do not wait
};
constexpr int kErrLane = 63;   // > kBarGroups: the lane that polls the error flag
__device__ __forceinline__ GridBar bar_init(uint32_t* bar, const int32_t* err) {
    const int lane = threadIdx.x & 63, ng = min(kBarGroups, (int)gridDim.x);
    const bool mine = lane < ng;
    GridBar b;
    b.arrive = bar + 64 * ((int)blockIdx.x % ng);
    b.poll = lane == kErrLane ? reinterpret_cast<const uint32_t*>(err) : bar + 64 * (mine ? lane : 0);
    b.per = mine ? gridDim.x / ng + ((int)(gridDim.x % ng) > lane ? 1u : 0u) : 0u;
    b.need = 0;
    b.dead = 0;
    return b;
}
// after(): work issued right after this workgroup's arrival, before the polls (loads
// issued there complete before the first poll's result: loads retire in order)
struct NoWork { __device__ void operator()() const {} };
template <class F = NoWork>
__device__ __forceinline__ void ctl_barrier(GridBar& b, int32_t* err, F after = F{}) {
    drain_vm();
    if (b.dead) { after(); return; }
    const int lane = threadIdx.x & 63;
    b.need += b.per;
    if (lane == 0) __hip_atomic_fetch_add(b.arrive, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    after();
    // every lane loads and the exit tests are ballots: the loop is scalar control flow.
    // Lane kErrLane reads *err in the same round trip: once any barrier of this launch
    // (or of an earlier launch in the stream) has failed, or the host raised the flag,
    // nobody waits any more. A poll that runs kSpinLimit rounds raises it.
    for (unsigned spins = 1;; spins++) {
        const unsigned v = ldc(b.poll);
        const bool is_err = lane == kErrLane;
        if (__builtin_amdgcn_ballot_w64(is_err && v != 0) != 0 || spins >= kSpinLimit) {
            if (lane == 0) stc(reinterpret_cast<uint32_t*>(err), 1u);
            b.dead = 1;
            break;
        }
        if (__builtin_amdgcn_ballot_w64(!is_err && (int)(v - b.need) < 0) == 0) break;
    }
}
// after the launch's last barrier: each control wave counts itself out; the last one
// (every workgroup has then finished polling) zeroes the counters for the next launch
// in the stream, which saves a memset dispatch per token
__device__ __forceinline__ void ctl_exit(uint32_t* bar) {
    const int lane = threadIdx.x & 63, ng = min(kBarGroups, (int)gridDim.x);
    unsigned last = 0;
    if (lane == 0)
        last = __hip_atomic_fetch_add(bar + 64 * kBarGroups, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) == gridDim.x - 1;
    if (__shfl(last, 0)) {
        if (lane < ng) stc(bar + 64 * lane, 0u);
        if (lane == 0) stc(bar + 64 * kBarGroups, 0u);
    }
}

// ------------------------------------------------------------------ per-layer buffers
__device__ __forceinline__ size_t hin(int l, int E) { return (size_t)(2 * l) * E; }
__device__ __forceinline__ size_t hmid(int l, int E) { return (size_t)(2 * l + 1) * E; }
__device__ __forceinline__ float* qkv_part(MPtr M, int l) { return M->qkv_part + lay::qkv_part(LY(M, 0)->qkv.ks, M->QKV, l); }
__device__ __forceinline__ float* o_part(MPtr M, int l) { return M->o_part + lay::o_part(LY(M, 0)->o.ks, M->E, l); }
__device__ __forceinline__ float* d_part(MPtr M, int l) { return M->d_part + lay::d_part(LY(M, 0)->d.ks, M->E, l); }
__device__ __forceinline__ float* att_rec(MPtr M, int l) { return M->att + lay::att(M->NH, M->maxch, M->arec, l); }
__device__ __forceinline__ uint8_t* act_rec(MPtr M, int l) { return M->act + lay::act(M->FF, l); }

// device wall clock (100 MHz) of one profile slot, one row per workgroup, written by
// thread `who` (0: the control wave, 64: the first worker)
__device__ __forceinline__ void stamp(MPtr M, int slot, int who = 0) {
    if (threadIdx.x == who && M->prof)
        M->prof[(size_t)blockIdx.x * prof_slots(M->NL) + slot] = __builtin_amdgcn_s_memrealtime();
}
// Stamps inside a phase's prologue (profile slots 5-7 of a phase) cost the step ~2% even
// when it is not profiled (code placement in the phase loop): built only with
// -DMI_PROFILE_FINE; the default build leaves those slots at 0.
#ifdef MI_PROFILE_FINE
#define FINE_STAMP(...) stamp(__VA_ARGS__)
#else
#define FINE_STAMP(...) ((void)0)
#endif
// inside k_step<HD, PROF>: stamps only in the profiling instance (the checks of M->prof
// in every phase cost the production step ~2%)
#define STAMP_IF(...)                        \
    do {                                     \
        if constexpr (PROF) stamp(M, __VA_ARGS__); \
    } while (0)
#define FINE_STAMP_IF(...)                        \
    do {                                          \
        if constexpr (PROF) FINE_STAMP(M, __VA_ARGS__); \
    } while (0)

// ------------------------------------------------------------------ control-wave prologues
// the phases of a layer, then lm_head
enum { PH_QKV = 0, PH_ATTN = 1, PH_O = 2, PH_GU = 3, PH_DOWN = 4, PH_LM = 5 };
// Vectors live in LDS; a lane handles the float4 at element 256j + 4*lane for
// j = 0, 1, ... (loops are not unrolled: the control wave's registers are shared
// with the workers' tiles in one kernel, so it keeps little in registers).
__device__ __forceinline__ float4 f4add(float4 a, float4 b) {
    return make_float4(__fadd_rn(a.x, b.x), __fadd_rn(a.y, b.y), __fadd_rn(a.z, b.z), __fadd_rn(a.w, b.w));
}
__device__ __forceinline__ float4 ld4(const float* p) { return *reinterpret_cast<const float4*>(p); }
__device__ __forceinline__ void st4(float* p, float4 v) { *reinterpret_cast<float4*>(p) = v; }
__device__ __forceinline__ void st4(float* p, int i, float4 v) { *reinterpret_cast<float4*>(p + i) = v; }

// Phase prologue, in two steps. ctl_stage (control wave, right after the grid
// barrier): one DMA batch brings the phase's inputs into LDS. wg_prologue (all
// eight waves): wave j handles the 256-element slice j of the input vector (the
// float4 at 256j + 4*lane), so the residual add, RMSNorm and int8 quantisation run
// on all four SIMDs; a single wave64 needs ~4 cycles per instruction and ~2.5 us
// for the same work.
//
// U staging of the norm phases: [w: n][h: n, when not resident][part: ks*n]

// quantise slice j (already scaled) into block records X; a 32-element block is
// 8 lanes x 4 elements
// X is LDS (P false) or a global record array that P selects the stores for
template <bool P = false>
__device__ __forceinline__ void quant_slice(float4 y, bool own, int e0, uint8_t* X, int lane, int rs = kXRec) {
    if (!own) y = make_float4(0.f, 0.f, 0.f, 0.f);
    const float a = max8(fmaxf(fmaxf(fabsf(y.x), fabsf(y.y)), fmaxf(fabsf(y.z), fabsf(y.w))));
    const float inv = a > 0.f ? __fdiv_rn(127.f, a) : 0.f;
    const int q0 = __float2int_rn(__fmul_rn(y.x, inv)), q1 = __float2int_rn(__fmul_rn(y.y, inv));
    const int q2 = __float2int_rn(__fmul_rn(y.z, inv)), q3 = __float2int_rn(__fmul_rn(y.w, inv));
    const int s = sum8(q0 + q1 + q2 + q3);
    if (own) {
        uint8_t* rec = X + (e0 >> 5) * rs;
        st_x<P>(reinterpret_cast<uint32_t*>(rec + (e0 & 31)),
                (uint32_t)(q0 & 0xFF) | ((uint32_t)(q1 & 0xFF) << 8) | ((uint32_t)(q2 & 0xFF) << 16) | ((uint32_t)q3 << 24));
        if ((lane & 7) == 0) {
            st_x<P>(reinterpret_cast<float*>(rec + 32), fp16_round(__fdiv_rn(a, 127.f)));
            st_x<P>(reinterpret_cast<uint32_t*>(rec + 36), (uint32_t)(8 * s));
        }
    }
}

// 1/sqrt(mean(x^2) + eps) of the n-vector x in LDS, the same on every lane of every
// wave: lane l sums x[256j + 4l + i]^2 over j, then i, by fma; xor butterfly
__device__ __forceinline__ float rms_scale(const float* x, int n, float eps, int lane) {
    // whole 256-element slices two at a time, both loads ahead of their part of the chain
    // (n is uniform: a scalar loop), then a last partial slice read as zeros past n
    // (fma(0, 0, a) = a for a >= +0)
    float a = 0.f;
    const int nj = n >> 8;
    int j = 0;
    for (; j + 1 < nj; j += 2) {
        const float4 u = ld4(x + 256 * j + 4 * lane), w = ld4(x + 256 * (j + 1) + 4 * lane);
        a = __fmaf_rn(u.x, u.x, a); a = __fmaf_rn(u.y, u.y, a); a = __fmaf_rn(u.z, u.z, a); a = __fmaf_rn(u.w, u.w, a);
        a = __fmaf_rn(w.x, w.x, a); a = __fmaf_rn(w.y, w.y, a); a = __fmaf_rn(w.z, w.z, a); a = __fmaf_rn(w.w, w.w, a);
    }
    for (; 256 * j < n; j++) {
        const float4 u = 256 * j + 4 * lane < n ? ld4(x + 256 * j + 4 * lane) : make_float4(0.f, 0.f, 0.f, 0.f);
        a = __fmaf_rn(u.x, u.x, a); a = __fmaf_rn(u.y, u.y, a); a = __fmaf_rn(u.z, u.z, a); a = __fmaf_rn(u.w, u.w, a);
    }
    a = bfly_sum64(a);
    return __fdiv_rn(1.0f, __builtin_sqrtf(__fadd_rn(__fdiv_rn(a, (float)n), eps)));   // correctly rounded sqrt
}

// the previous GEMV of a norm phase: down of layer l-1 (qkv), o of layer l
// (gate/up), down of the last layer (lm_head)
__device__ __forceinline__ int norm_src_layer(MPtr M, int l, int kind) {
    return kind == PH_QKV ? l - 1 : kind == PH_LM ? M->NL - 1 : l;
}

// One wave's share of a workgroup's DMA: the transfers of a staging step are cut into
// 1-KB units numbered across calls, and wave `wave` of `nw` issues units wave, wave +
// nw, ... (a single wave issuing ~50 units back to back was most of the staging time).
struct DmaShare { int wave, nw, unit; };
__device__ __forceinline__ void dma_share(const void* g, void* lds, int bytes, DmaShare& d, int lane) {
    const int n = (bytes + 1023) >> 10;
    for (int k = ((d.wave - d.unit) % d.nw + d.nw) % d.nw; k < n; k += d.nw) {
        const int off = k << 10;
        if (off + lane * 16 < bytes)
            __builtin_amdgcn_global_load_lds(static_cast<const uint8_t*>(g) + off + lane * 16,
                                             (lds_ptr)(static_cast<uint8_t*>(lds) + off), 16, 0, 0);
    }
    d.unit += n;
}

// DMA the inputs of phase (l, kind) into LDS, shared by waves wave = 0..nw-1 (all of
// them call it), each of which waits for its own transfers; a workgroup barrier then
// publishes them
__device__ __forceinline__ void stage(MPtr M, int l, int kind, int pos, const Lds& S, int wave, int nw, int lane,
                                      bool resident) {
    const int n = M->E;
    DmaShare d{wave, nw, 0};
    if (kind == PH_DOWN) {
        dma_share(act_rec(M, l), S.U, (M->FF / 32) * kActRec, d, lane);
    } else if (kind == PH_O) {
        const int nch = (pos + 1 + kAttnChunk - 1) / kAttnChunk, arec = M->arec;
        if (nch <= kInlineComb) {
            const float* att = att_rec(M, l);
            const int hb = nch * arec;
            for (int h = 0; h < M->NH; h++)
                dma_share(att + (size_t)h * M->maxch * arec, reinterpret_cast<float*>(S.U) + h * hb, hb * 4, d, lane);
        } else {
            dma_share(M->att_out + (size_t)l * n, S.T, n * 4, d, lane);
        }
    } else if (kind != PH_ATTN) {
        float* w = reinterpret_cast<float*>(S.U);
        dma_share(kind == PH_LM ? M->out_norm : kind == PH_QKV ? LY(M, l)->an : LY(M, l)->fn, w, n * 4, d, lane);
        if (kind == PH_QKV && l == 0) {
            dma_share(M->emb + (size_t)M->tokbuf[pos] * n, resident ? S.R : S.T, n * 4, d, lane);
        } else {
            const int pl = norm_src_layer(M, l, kind);
            const bool dsrc = kind != PH_GU;
            if (!resident) dma_share(M->hbuf + (dsrc ? hmid(pl, n) : hin(l, n)), w + n, n * 4, d, lane);
            dma_share(dsrc ? d_part(M, pl) : o_part(M, pl), w + (resident ? n : 2 * n),
                      (dsrc ? LY(M, pl)->d.ks : LY(M, pl)->o.ks) * n * 4, d, lane);
        }
    }
    drain_vm();     // (attention stages nothing; this completes the unit's K/V tile its waves prefetched)
}
// the control wave alone (the per-phase kernels, whose workers prefetch meanwhile)
__device__ __forceinline__ void ctl_stage(MPtr M, int l, int kind, int pos, const Lds& S, int lane, bool resident) {
    stage(M, l, kind, pos, S, 0, 1, lane, resident);
}

// all waves: the phase input records X from the staged data (see ctl_stage)
__device__ __forceinline__ void wg_prologue(MPtr M, int l, int kind, int pos, int wg, const Lds& S, int wave,
                                            int lane, bool resident, int slot = -1) {
    const int n = M->E, e0 = 256 * wave + 4 * lane;
    const bool has = 256 * wave < n, own = e0 < n;
    if (kind == PH_O) {
        const int nch = (pos + 1 + kAttnChunk - 1) / kAttnChunk;
        if (!has) return;
        float4 y = make_float4(0.f, 0.f, 0.f, 0.f);
        if (own && nch <= kInlineComb) {
            // merge of the head's chunk records by max rescaling in chunk order
            // (cuda_infer.cu:688-702), the per-chunk weights computed per lane
            const int HD = M->HD, arec = M->arec, hb = nch * arec;
            const int hh = e0 / HD, d = e0 - hh * HD;        // 4 | HD: one head
            const float* r = reinterpret_cast<const float*>(S.U) + hh * hb;
            // every record's (m, l, o) read first (nch is uniform), then the chains
            float mc[kInlineComb], lc[kInlineComb];
            float4 oc[kInlineComb];
#pragma unroll
            for (int c = 0; c < kInlineComb; c++)
                if (c < nch) { mc[c] = r[c * arec + HD]; lc[c] = r[c * arec + HD + 1]; oc[c] = ld4(r + c * arec + d); }
            float mx = -__builtin_inff();
#pragma unroll
            for (int c = 0; c < kInlineComb; c++)
                if (c < nch) mx = fmaxf(mx, mc[c]);
            float den = 0.f;
            float4 acc = make_float4(0.f, 0.f, 0.f, 0.f);
#pragma unroll
            for (int c = 0; c < kInlineComb; c++)
                if (c < nch) {
                    const float wc = mi_expf(__fsub_rn(mc[c], mx));
                    den = __fmaf_rn(lc[c], wc, den);
                    const float4 o = oc[c];
                    acc = make_float4(__fmaf_rn(o.x, wc, acc.x), __fmaf_rn(o.y, wc, acc.y), __fmaf_rn(o.z, wc, acc.z),
                                      __fmaf_rn(o.w, wc, acc.w));
                }
            y = make_float4(__fdiv_rn(acc.x, den), __fdiv_rn(acc.y, den), __fdiv_rn(acc.z, den), __fdiv_rn(acc.w, den));
        } else if (own) {
            y = ld4(S.T + e0);
        }
        quant_slice(y, own, e0, S.X, lane);
        return;
    }
    if (kind == PH_DOWN || kind == PH_ATTN) return;
    // norm phases: residual add of slice `wave`, then RMSNorm + int8 of it
    const float* w = reinterpret_cast<const float*>(S.U);
    float* h = resident && kind != PH_LM ? S.R : S.T;
    if (has && own && !(kind == PH_QKV && l == 0)) {
        const int pl = norm_src_layer(M, l, kind);
        const int ks = kind != PH_GU ? LY(M, pl)->d.ks : LY(M, pl)->o.ks;
        const float* hs = resident ? S.R : w + n;
        const float* ps = w + (resident ? n : 2 * n);
        // the partials in order, four loads ahead of their adds (ks is uniform: a scalar
        // loop; an unrolled loop over kMaxKsRes with a condition per partial branched and
        // reloaded spilled scalars around every load)
        float4 v = ld4(ps + e0);
        int s = 1;
        for (; s + 3 < ks; s += 4) {
            const float4 a = ld4(ps + s * n + e0), b = ld4(ps + (s + 1) * n + e0);
            const float4 c = ld4(ps + (s + 2) * n + e0), d = ld4(ps + (s + 3) * n + e0);
            v = f4add(f4add(f4add(f4add(v, a), b), c), d);
        }
        for (; s < ks; s++) v = f4add(v, ld4(ps + s * n + e0));
        const float4 x = f4add(ld4(hs + e0), v);
        st4(h, e0, x);
        if (!resident && wg == 0 && kind != PH_LM) {
            float* dst = M->hbuf + (kind == PH_QKV ? hin(l, n) : hmid(l, n)) + e0;
            stc(dst, x.x); stc(dst + 1, x.y); stc(dst + 2, x.z); stc(dst + 3, x.w);
        }
    } else if (has && own && kind == PH_QKV && l == 0 && !resident && wg == 0) {
        const float4 x = ld4(h + e0);
        float* dst = M->hbuf + hin(0, n) + e0;
        stc(dst, x.x); stc(dst + 1, x.y); stc(dst + 2, x.z); stc(dst + 3, x.w);
    }
    __syncthreads();
    if (slot >= 0) FINE_STAMP(M, slot);
    const float sc = rms_scale(h, n, M->eps, lane);
    if (!has) return;
    float4 y = make_float4(0.f, 0.f, 0.f, 0.f);
    if (own) {
        const float4 x = ld4(h + e0), wv = ld4(w + e0);
        y = make_float4(__fmul_rn(__fmul_rn(x.x, sc), wv.x), __fmul_rn(__fmul_rn(x.y, sc), wv.y),
                        __fmul_rn(__fmul_rn(x.z, sc), wv.z), __fmul_rn(__fmul_rn(x.w, sc), wv.w));
    }
    quant_slice(y, own, e0, S.X, lane);
}

// ------------------------------------------------------------------ gate/up epilogue
// A 64-row group = 32 gate rows + their 32 up rows (ks = 1: the segment is the whole
// row): silu(g)*u = g/(1+exp(-g))*u (cpu_infer.cpp:144-147) on lanes 0..31, quantized
// to one int8 act block record (32 codes, scale, 8*sum) on its own 128-byte line.
__device__ __forceinline__ void gu_store(const PMat W, int wg, int nwg, int kw, const float* P, uint8_t* act, int lane) {
    wg_segments(W, wg_place(W, wg, nwg), nwg, kw, [&](int g, int s, int k0, int k1) {
        (void)s;
        const float v = seg_sum(P, k0, k1, lane);
        const float u = __shfl(v, (lane & 31) + 32);
        const float t = mi_expf(-v);
        const float a = __fmul_rn(__fdiv_rn(v, __fadd_rn(1.0f, t)), u);
        int q, s8;
        float d;
        quant32_vals(a, q, d, s8);
        const uint32_t b = (uint32_t)(q & 0xFF);
        const uint32_t wd = b | (__shfl_down(b, 1) << 8) | (__shfl_down(b, 2) << 16) | (__shfl_down(b, 3) << 24);
        if (lane < 32) {
            uint32_t* r = reinterpret_cast<uint32_t*>(act + (size_t)g * kActRec);
            if ((lane & 3) == 0) stc(r + lane / 4, wd);
            if (lane == 0) { stc(r + 8, __float_as_uint(d)); stc(r + 9, (uint32_t)s8); }
        }
    });
}

// ------------------------------------------------------------------ lm_head epilogue
// workers: row values of the workgroup's vocab groups (logits when requested),
// per-lane top-2, wave top-2 -> misc; control wave: the workgroup's candidate, and in
// word 3 whether one of this launch's grid barriers gave up on this workgroup (`dead`,
// the control wave's; its inputs may then be stale)
__device__ __forceinline__ void lm_epilogue(MPtr M, int wg, int nwg, const Lds& S, int wave, int lane,
                                            unsigned dead = 0) {
    if (wave > 0) {
        Top2 t{-__builtin_inff(), INT_MAX, -__builtin_inff()};
        const PMat Wl = ldmat(&M->lm);
        wg_segments(Wl, wg_place(Wl, wg, nwg), nwg, wave - 1, [&](int g, int s, int k0, int k1) {
            (void)s;
            const float v = seg_sum(S.P, k0, k1, lane);
            const int row = g * 64 + lane;
            if (M->logits) M->logits[row] = v;
            top2_push(t, v, row);
        });
        top2_wave(t);
        if (lane == 0) reinterpret_cast<float4*>(S.misc)[wave] = make_float4(t.best, __int_as_float(t.idx), t.second, 0.f);
    }
    __syncthreads();
    if (threadIdx.x == 0) {
        const float4* red = reinterpret_cast<const float4*>(S.misc);
        Top2 a{red[1].x, __float_as_int(red[1].y), red[1].z};
        for (int w = 2; w <= kWorkers; w++) top2_merge(a, red[w].x, __float_as_int(red[w].y), red[w].z);
        float* cd = M->cand + (size_t)wg * 32;
        stc(cd, a.best);
        stc(reinterpret_cast<uint32_t*>(cd + 1), (uint32_t)a.idx);
        stc(cd + 2, a.second);
        stc(reinterpret_cast<uint32_t*>(cd + 3), dead);
    }
}

// merge of the workgroups' candidates by one wave (top-2 merging is associative and
// commutative, so any order gives the same token and margin); result on every lane;
// *failed: whether any workgroup reported a failed barrier
// a lane's candidate records i = lane, lane + 64, ... (record i: 4 floats at cand + i *
// stride, 16-byte aligned), four loads in flight at a time, merged in that order
template <class F>
__device__ __forceinline__ void merge_cand_recs(const float* cand, int stride, int n, int lane, F f) {
    for (int i0 = lane; i0 < n; i0 += 256) {
        float4 c[4];
#pragma unroll
        for (int u = 0; u < 4; u++)
            if (i0 + 64 * u < n) c[u] = *reinterpret_cast<const float4*>(cand + (size_t)(i0 + 64 * u) * stride);
#pragma unroll
        for (int u = 0; u < 4; u++)
            if (i0 + 64 * u < n) f(c[u]);
    }
}
__device__ __forceinline__ Top2 wave_merge_cands(const float* cand, int n, int lane, unsigned* failed = nullptr) {
    Top2 t{-__builtin_inff(), INT_MAX, -__builtin_inff()};
    unsigned f = 0;
    merge_cand_recs(cand, 32, n, lane, [&](float4 c) {
        top2_merge(t, c.x, __float_as_int(c.y), c.z);
        f |= __float_as_uint(c.w);
    });
    top2_wave(t);
    if (failed) *failed = __builtin_amdgcn_ballot_w64(f != 0) != 0;
    return t;
}
// The token of a merged top-2. Only when no logit compares greater than -inf (all NaN
// or -inf) is no row taken and idx left at INT_MAX; the first-max argmax of
// cpu_infer.cpp:153-154 returns row 0 then, and so does this. (It also keeps the next
// step's embedding gather, which reads row tokbuf[pos + 1], inside the table.)
__device__ __forceinline__ int top2_token(const Top2& a, int V) { return (unsigned)a.idx < (unsigned)V ? a.idx : 0; }
__device__ __forceinline__ void emit_token(MPtr M, const Top2& a, int pos, int gen, unsigned failed = 0) {
    const int tok = top2_token(a, M->V);
    const float margin = __fsub_rn(a.best, a.second);
    M->out_tok[pos] = tok;
    M->out_margin[pos] = margin;
    if (gen) M->tokbuf[pos + 1] = tok;
    if (gen == kGenRing) {
        // one 64-bit vector store at system scope, through to the host's memory; a launch
        // whose barrier failed reports that instead of its token
        const uint64_t w = failed ? kRingFail : ((uint64_t)__float_as_uint(margin) << 32) | (uint32_t)tok;
        __hip_atomic_store(M->ring + pos, w, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
    }
}

// ------------------------------------------------------------------ attention
// per-wave LDS: K [64][HD/8] 16-byte vectors, row-major with the vectors of row t
// permuted (kslot) | V [64][HD] | q partials [2][HD] | k, v partials [2][2][HD] | q [HD]
// (+ spare)

// K tile slot of 16-byte vector v of position t: t * NV + (v ^ kswz(t)). The XOR makes the
// lane-per-position read of one vector conflict-free (each 16-lane pass of a 16-byte LDS
// read touches 16 different 4-bank groups) while each row stays in its own 256 B (128 B
// at hd 64), so the DMA that fills it reads whole rows: coalesced.
template <int HD>
__device__ __forceinline__ int kswz(int t) { return HD == 128 ? (t & 15) : ((t >> 1) & 7); }
template <int HD>
__device__ __forceinline__ int kslot(int t, int v) { return t * (HD / 8) + (v ^ kswz<HD>(t)); }

// one wave's DMA of the K rows krows[0..64) of a chunk into the swizzled tile, and of its
// V rows row-major (rows past n repeat row n-1), as attn_issue_kv below does both
template <int HD>
__device__ __forceinline__ void attn_issue_k(const __half* krows, int n, uint4* kls, int lane) {
    constexpr int NV = HD / 8, RPI = 64 / NV;
    const int u = lane % NV;
#pragma unroll
    for (int i = 0; i < NV; i++) {
        const int t = i * RPI + lane / NV;
        __builtin_amdgcn_global_load_lds(krows + (size_t)min(t, n - 1) * HD + 8 * (u ^ kswz<HD>(t)),
                                         (lds_ptr)(kls + i * 64), 16, 0, 0);
    }
}
template <int HD>
__device__ __forceinline__ void attn_issue_v(const __half* vrows, int n, __half* vls, int lane) {
    constexpr int NV = HD / 8, RPI = 64 / NV;
    const int r = lane / NV, col = (lane % NV) * 8;
#pragma unroll
    for (int i = 0; i < 64 / RPI; i++)
        __builtin_amdgcn_global_load_lds(vrows + (size_t)min(i * RPI + r, n - 1) * HD + col,
                                         (lds_ptr)(vls + i * RPI * HD), 16, 0, 0);
}

// DMA the chunk's K rows (swizzled tile) and V rows; rows past n repeat row n-1. K load i
// fills tile slots 64i..64i+63, i.e. rows (64/NV)i.. whole: lane l takes slot 64i + l =
// (row t, place u) and fetches vector u ^ kswz(t) of row t, 1 KB of consecutive rows per
// instruction (one row per lane touched 64 lines per instruction and was the slow part).
template <int HD>
__device__ __forceinline__ void attn_issue_kv(const __half* krows, const __half* vrows, int t0, int n, uint4* kls,
                                              __half* vls, int lane) {
    constexpr int NV = HD / 8, RPI = 64 / NV;
    const int u = lane % NV;
#pragma unroll
    for (int i = 0; i < NV; i++) {
        const int t = i * RPI + lane / NV;
        const __half* src = krows + (size_t)(t0 + min(t, n - 1)) * HD + 8 * (u ^ kswz<HD>(t));
        __builtin_amdgcn_global_load_lds(src, (lds_ptr)(kls + i * 64), 16, 0, 0);
    }
    const int r = lane / NV, col = (lane % NV) * 8;
#pragma unroll
    for (int i = 0; i < 64 / RPI; i++) {
        const int row = min(i * RPI + r, n - 1);
        __builtin_amdgcn_global_load_lds(vrows + (size_t)(t0 + row) * HD + col, (lds_ptr)(vls + i * RPI * HD), 16, 0, 0);
    }
}

// scores (lane = position), chunk softmax, p.v (lane = dims; p of position t
// broadcast from lane t by readlane). The chunk max and sum end on every lane, the
// lane's outputs in acc.
template <int HD>
__device__ __forceinline__ void attn_core(const uint4* kls, const float* qs, const __half* vls, int n, float scale, int lane,
                                          float& m, float& lsum, float (&acc)[HD / 64]) {
    constexpr int NV = HD / 8, DPL = HD / 64;
    float a0 = 0.f, a1 = 0.f, a2 = 0.f, a3 = 0.f;
#pragma unroll 4
    for (int j = 0; j < NV; j++) {
        const uint4 w = kls[kslot<HD>(lane, j)];
        const float4 q0 = *reinterpret_cast<const float4*>(qs + 8 * j);
        const float4 q1 = *reinterpret_cast<const float4*>(qs + 8 * j + 4);
        a0 = __fmaf_rn(q0.x, h2f_lo(w.x), a0); a1 = __fmaf_rn(q0.y, h2f_hi(w.x), a1);
        a2 = __fmaf_rn(q0.z, h2f_lo(w.y), a2); a3 = __fmaf_rn(q0.w, h2f_hi(w.y), a3);
        a0 = __fmaf_rn(q1.x, h2f_lo(w.z), a0); a1 = __fmaf_rn(q1.y, h2f_hi(w.z), a1);
        a2 = __fmaf_rn(q1.z, h2f_lo(w.w), a2); a3 = __fmaf_rn(q1.w, h2f_hi(w.w), a3);
    }
    const bool valid = lane < n;
    const float sc = __fmul_rn(__fadd_rn(__fadd_rn(a0, a1), __fadd_rn(a2, a3)), scale);
    const float s = valid ? sc : -__builtin_inff();
    m = wave_max(s);
    const float p = valid ? mi_expf(__fsub_rn(s, m)) : 0.f;
    lsum = bfly_sum64(p);
#pragma unroll
    for (int e = 0; e < DPL; e++) acc[e] = 0.f;
    const int pb = __float_as_int(p);
    // V rows in batches of 8: the LDS reads of a batch are issued together, then the
    // fma chain (positions in order) consumes them; n is wave-uniform (scalar loop)
    constexpr int B = 8;
    using VT = typename std::conditional<DPL == 2, uint32_t, uint16_t>::type;
    const int ns = __builtin_amdgcn_readfirstlane(n);
    auto step = [&](VT w, int t) {
        const float pt = __int_as_float(__builtin_amdgcn_readlane(pb, t));
        if constexpr (DPL == 2) {
            acc[0] = __fmaf_rn(pt, h2f_lo(w), acc[0]);
            acc[1] = __fmaf_rn(pt, h2f_hi(w), acc[1]);
        } else {
            acc[0] = __fmaf_rn(pt, __half2float(__ushort_as_half(w)), acc[0]);
        }
    };
    int t0 = 0;
    for (; t0 + B <= ns; t0 += B) {
        VT w[B];
#pragma unroll
        for (int u = 0; u < B; u++) w[u] = *reinterpret_cast<const VT*>(vls + (t0 + u) * HD + DPL * lane);
#pragma unroll
        for (int u = 0; u < B; u++) step(w[u], t0 + u);
    }
    for (; t0 < ns; t0 += 4) {       // the tail, four rows per batch
        VT w[4];
#pragma unroll
        for (int u = 0; u < 4; u++) w[u] = *reinterpret_cast<const VT*>(vls + min(t0 + u, ns - 1) * HD + DPL * lane);
#pragma unroll
        for (int u = 0; u < 4; u++)
            if (t0 + u < ns) step(w[u], t0 + u);
    }
}

// attn_core for H query heads of one kv head at once (q rows at qs, qs + HD, ...; rows
// past nq - 1 repeat row nq - 1): each head's arithmetic is attn_core's, the same chains
// in the same order, so the results carry the same bits; the K and V values are read
// from LDS once for the H heads and the heads' chains interleave (attn_core alone is a
// chain of dependent fmas and LDS waits). The probabilities reach the p.v lanes through
// the wave's LDS row pl[H][64] (one 16-byte broadcast read gives four positions; a
// readlane per position and head cost more than the fmas it feeds).
template <int HD, int H>
__device__ __forceinline__ void attn_core_h(const uint4* kls, const float* qs, int nq, const __half* vls, int n,
                                            float scale, int lane, float* pl, float (&m)[H], float (&lsum)[H],
                                            float (&acc)[H][HD / 64]) {
    constexpr int NV = HD / 8, DPL = HD / 64;
    const float* qr[H];
#pragma unroll
    for (int h = 0; h < H; h++) qr[h] = qs + min(h, nq - 1) * HD;
    float a[H][4];
#pragma unroll
    for (int h = 0; h < H; h++) a[h][0] = a[h][1] = a[h][2] = a[h][3] = 0.f;
#pragma unroll 4
    for (int j = 0; j < NV; j++) {
        const uint4 w = kls[kslot<HD>(lane, j)];
#pragma unroll
        for (int h = 0; h < H; h++) {
            const float4 q0 = *reinterpret_cast<const float4*>(qr[h] + 8 * j);
            const float4 q1 = *reinterpret_cast<const float4*>(qr[h] + 8 * j + 4);
            a[h][0] = __fmaf_rn(q0.x, h2f_lo(w.x), a[h][0]); a[h][1] = __fmaf_rn(q0.y, h2f_hi(w.x), a[h][1]);
            a[h][2] = __fmaf_rn(q0.z, h2f_lo(w.y), a[h][2]); a[h][3] = __fmaf_rn(q0.w, h2f_hi(w.y), a[h][3]);
            a[h][0] = __fmaf_rn(q1.x, h2f_lo(w.z), a[h][0]); a[h][1] = __fmaf_rn(q1.y, h2f_hi(w.z), a[h][1]);
            a[h][2] = __fmaf_rn(q1.z, h2f_lo(w.w), a[h][2]); a[h][3] = __fmaf_rn(q1.w, h2f_hi(w.w), a[h][3]);
        }
    }
    const bool valid = lane < n;
#pragma unroll
    for (int h = 0; h < H; h++) {
        const float sc = __fmul_rn(__fadd_rn(__fadd_rn(a[h][0], a[h][1]), __fadd_rn(a[h][2], a[h][3])), scale);
        const float s = valid ? sc : -__builtin_inff();
        m[h] = wave_max(s);
        const float p = valid ? mi_expf(__fsub_rn(s, m[h])) : 0.f;
        lsum[h] = bfly_sum64(p);
        pl[h * 64 + lane] = p;                       // positions past n hold 0
#pragma unroll
        for (int e = 0; e < DPL; e++) acc[h][e] = 0.f;
    }
    wave_lds_sync();
    using VT = typename std::conditional<DPL == 2, uint32_t, uint16_t>::type;
    const int ns = __builtin_amdgcn_readfirstlane(n);
    auto step = [&](VT w, const float (&pt)[H]) {
#pragma unroll
        for (int h = 0; h < H; h++) {
            if constexpr (DPL == 2) {
                acc[h][0] = __fmaf_rn(pt[h], h2f_lo(w), acc[h][0]);
                acc[h][1] = __fmaf_rn(pt[h], h2f_hi(w), acc[h][1]);
            } else {
                acc[h][0] = __fmaf_rn(pt[h], __half2float(__ushort_as_half(w)), acc[h][0]);
            }
        }
    };
    // batches of 8 positions: the V values and the p broadcasts of a batch are read
    // together, then the chains run over the positions in order; past the last whole
    // batch, one position at a time up to n
    int t0 = 0;
    for (; t0 + 8 <= ns; t0 += 8) {
        VT w[8];
        float4 pv[H][2];
#pragma unroll
        for (int u = 0; u < 8; u++) w[u] = *reinterpret_cast<const VT*>(vls + (t0 + u) * HD + DPL * lane);
#pragma unroll
        for (int h = 0; h < H; h++) {
            pv[h][0] = *reinterpret_cast<const float4*>(pl + h * 64 + t0);
            pv[h][1] = *reinterpret_cast<const float4*>(pl + h * 64 + t0 + 4);
        }
#pragma unroll
        for (int u = 0; u < 8; u++) {
            float pt[H];
#pragma unroll
            for (int h = 0; h < H; h++) {
                const float4& v4 = pv[h][u >> 2];
                pt[h] = (u & 3) == 0 ? v4.x : (u & 3) == 1 ? v4.y : (u & 3) == 2 ? v4.z : v4.w;
            }
            step(w[u], pt);
        }
    }
    for (; t0 < ns; t0++) {
        const VT w = *reinterpret_cast<const VT*>(vls + t0 * HD + DPL * lane);
        float pt[H];
#pragma unroll
        for (int h = 0; h < H; h++) pt[h] = pl[h * 64 + t0];
        step(w, pt);
    }
}

// Attention units (kv head kvh, 64-position chunk c) of positions 0..pos, unit u =
// kvh * nch + c on workgroup u % nwg, u + nwg, ... . The unit's K and V rows come into
// one LDS tile (workers 0 and 1 DMA them during the grid barrier before the phase); wave
// hh of the workgroup (the control wave included) then computes query head kvh * G + hh
// against it, so the tile is read from memory once for the G heads.
template <int HD>
__device__ __forceinline__ void attn_issue_unit(MPtr M, int l, int pos, int u, int nch, uint8_t* U, int wave, int lane) {
    const int kvh = u / nch, t0 = (u - kvh * nch) * kAttnChunk, n = min(kAttnChunk, pos + 1 - t0);
    const size_t rowbase = lay::kv(M->NKV, M->maxseq, 1, l, kvh, t0);
    // the tile address through a VGPR: with a uniform (SGPR) generic pointer, the LDS
    // cast's aperture check hits an instruction-selection error in this compiler; and an
    // opaque lane, so the DMA addresses are not hoisted out of the step's phase loop
    int zero = 0;
    asm volatile("" : "+v"(zero));
    asm volatile("" : "+v"(lane));
    uint8_t* Uv = U + zero;
    if (wave == 1) attn_issue_k<HD>(M->kc + rowbase * HD, n, reinterpret_cast<uint4*>(Uv), lane);
    if (wave == 2) attn_issue_v<HD>(M->vc + rowbase * HD, n, reinterpret_cast<__half*>(Uv + 64 * HD * 2), lane);
}

// One head of a unit whose K/V tile is in LDS: the QKV partials of the head's q rows and,
// in the chunk that holds position pos, of its kv head's k and v rows; q = segments +
// bias + NEOX RoPE (cpu_infer.cpp:49-61); the last chunk finishes k/v of pos, rounds them
// to fp16, writes them into the tile's row for pos (every head wave of the unit writes the
// same values; each reads the row only after its own write) and head 0 appends them to
// the cache. The record o[HD], max, sum goes to att[l][h][c] (agent-coherent stores).
template <int HD>
__device__ __forceinline__ void attn_finish(MPtr M, int l, int pos, int h, int c, uint8_t* U, uint8_t* area, int lane) {
    constexpr int half = HD / 2, DPL = HD / 64;
    uint4* kls = reinterpret_cast<uint4*>(U);
    __half* vls = reinterpret_cast<__half*>(U + 64 * HD * 2);
    float* qp = reinterpret_cast<float*>(area);                                   // [ks][HD]
    float* kvp = qp + kMaxKsQkv * HD;                                            // [ks][HD] k then [ks][HD] v
    float* qs = qp + 3 * kMaxKsQkv * HD;
    const LPtr Ly = LY(M, l);
    const int ks = Ly->qkv.ks, kvh = h / M->G;
    const int L = pos + 1, nch = (L + kAttnChunk - 1) / kAttnChunk, t0 = c * kAttnChunk;
    const int n = min(kAttnChunk, L - t0);
    const bool last = c == nch - 1;
    const int cur = last ? pos - t0 : -1;
    const size_t rowbase = lay::kv(M->NKV, M->maxseq, 1, l, kvh, 0);
    const float* part = qkv_part(M, l);
    const int rq = h * HD, rk = M->NH * HD + kvh * HD, rv = M->NH * HD + M->KVD + kvh * HD;
    // bias and RoPE table values are loaded in the same batch as the partials
    const int ip = lane % half;
    const float* bq = Ly->bqkv;
    const float2 cz = M->rope[(size_t)pos * half + ip];
    const float bq0 = bq[rq + ip], bq1 = bq[rq + ip + half];
    float bk0 = 0.f, bk1 = 0.f, bv0 = 0.f, bv1 = 0.f;
    if (last) { bk0 = bq[rk + ip]; bk1 = bq[rk + ip + half]; bv0 = bq[rv + ip]; bv1 = bq[rv + ip + half]; }
    for (int s = 0; s < ks; s++) {
        dma_wave(part + (size_t)s * M->QKV + rq, qp + s * HD, HD * 4, lane);
        if (last) {
            dma_wave(part + (size_t)s * M->QKV + rk, kvp + s * HD, HD * 4, lane);
            dma_wave(part + (size_t)s * M->QKV + rv, kvp + (kMaxKsQkv + s) * HD, HD * 4, lane);
        }
    }
    drain_vm();
    wave_lds_sync();
    auto fin = [&](const float* p, int i, float bias) {
        float v = p[i];
        for (int s = 1; s < ks; s++) v = __fadd_rn(v, p[s * HD + i]);
        return __fadd_rn(v, bias);
    };
    if (lane < half) {
        const float x0 = fin(qp, ip, bq0), x1 = fin(qp, ip + half, bq1);
        qs[ip] = __fsub_rn(__fmul_rn(x0, cz.x), __fmul_rn(x1, cz.y));
        qs[ip + half] = __fadd_rn(__fmul_rn(x0, cz.y), __fmul_rn(x1, cz.x));
        if (last) {
            const float k0 = fin(kvp, ip, bk0), k1 = fin(kvp, ip + half, bk1);
            const __half y0 = __float2half(__fsub_rn(__fmul_rn(k0, cz.x), __fmul_rn(k1, cz.y)));
            const __half y1 = __float2half(__fadd_rn(__fmul_rn(k0, cz.y), __fmul_rn(k1, cz.x)));
            const __half v0 = __float2half(fin(kvp + kMaxKsQkv * HD, ip, bv0));
            const __half v1 = __float2half(fin(kvp + kMaxKsQkv * HD, ip + half, bv1));
            __half* kh = reinterpret_cast<__half*>(kls);      // position cur's K row into the swizzled tile
            kh[kslot<HD>(cur, ip >> 3) * 8 + (ip & 7)] = y0;
            kh[kslot<HD>(cur, (ip + half) >> 3) * 8 + ((ip + half) & 7)] = y1;
            vls[cur * HD + ip] = v0;
            vls[cur * HD + ip + half] = v1;
            if (h % M->G == 0) {                    // one of the kv head's G query heads appends to the cache
                __half* kd = M->kc + (rowbase + pos) * HD;
                __half* vd = M->vc + (rowbase + pos) * HD;
                kd[ip] = y0; kd[ip + half] = y1;
                vd[ip] = v0; vd[ip + half] = v1;
            }
        }
    }
    wave_lds_sync();
    float m[1], lsum[1], acc[1][DPL];
    attn_core_h<HD, 1>(kls, qs, 1, vls, n, M->scale, lane, qs + HD, m, lsum, acc);
    float* rec = att_rec(M, l) + ((size_t)h * M->maxch + c) * M->arec;
#pragma unroll
    for (int e = 0; e < DPL; e++) stc(rec + DPL * lane + e, acc[0][e]);
    if (lane == 0) { stc(rec + HD, m[0]); stc(rec + HD + 1, lsum[0]); }
}

// Workgroups per (kv head, chunk): the unit's G query heads go to S workgroups, S = 2
// while the grid holds every such unit in one round. A unit's heads then run one per
// SIMD (waves 0..2 for G = 6) instead of two on each of two SIMDs (waves w and w + 4
// share one): the scores and p.v are VALU-bound chains, 1.86 us per unit at 64 positions
// with six heads on four SIMDs. Each head's arithmetic is unchanged; only the chunk's K/V
// tile is read twice. Unit u covers (kv head, chunk) u / S and head group u % S.
__device__ __forceinline__ int attn_splits(MPtr M, int nch, int nwg) {
    return M->G > 1 && 2 * M->NKV * nch <= nwg ? 2 : 1;
}
// the workgroup's first unit: K/V DMA only, by workers 0 and 1 (issued before the grid
// barrier; the phase's staging step drains it)
template <int HD>
__device__ __forceinline__ void attn_prefetch(MPtr M, int l, int pos, int wg, int nwg, uint8_t* U, int wave, int lane) {
    const int nch = (pos + 1 + kAttnChunk - 1) / kAttnChunk, S = attn_splits(M, nch, nwg);
    if (wg < M->NKV * nch * S) attn_issue_unit<HD>(M, l, pos, wg / S, nch, U, wave, lane);
}
// all of the workgroup's units, every wave taking part (the first unit's tile is in LDS;
// later units reload it between workgroup barriers)
template <int HD>
__device__ __forceinline__ void attn_run(MPtr M, int l, int pos, int wg, int nwg, uint8_t* U, int wave, int lane) {
    // opaque lane: its addresses are not hoisted out of the step's phase loop
    asm volatile("" : "+v"(lane));
    const int nch = (pos + 1 + kAttnChunk - 1) / kAttnChunk, S = attn_splits(M, nch, nwg), units = M->NKV * nch * S;
    const int hpw = (M->G + S - 1) / S;                 // heads per workgroup
    uint8_t* area = U + 2 * 64 * HD * 2 + wave * attn_head_lds<HD>();
    for (int u = wg; u < units; u += nwg) {
        const int uc = u / S, part = u - uc * S;
        if (u != wg) {
            __syncthreads();                        // every head is done with the tile
            attn_issue_unit<HD>(M, l, pos, uc, nch, U, wave, lane);
            drain_vm();
            __syncthreads();
        }
        const int kvh = uc / nch, hh = part * hpw + wave;
        if (wave < hpw && hh < M->G) attn_finish<HD>(M, l, pos, kvh * M->G + hh, uc - kvh * nch, U, area, lane);
    }
}

// The canonical merge of chunk records (o[HD], m, l) by max rescaling (cuda_infer.cu:
// 688-702 attn_combine), as the oracle restates it: one wave merges the nch chunk
// records of one head (records r[c * arec], lane = dims 64e + lane); the max over all
// chunks first when there are
// more than kAttnSplit; each split of kAttnSplit chunks with all its loads issued at
// once (M_s = split max, w = exp(m - M_s), den and o as fma chains in chunk order),
// then the splits in order scaled by exp(M_s - M). Returns o / den per lane and dim.
// Up to two splits (nch <= 2 kAttnSplit) every record's loads go out before any of the
// arithmetic (one memory round trip instead of three); the arithmetic is the same.
template <int HD>
__device__ __forceinline__ void comb_wave2(const float* r, int arec, int nch, int lane, float (&out)[HD / 64]) {
    constexpr int DPL = HD / 64, NS = kAttnSplit;
    // lane c holds chunk c's (m, l); ov[i][e] is chunk i's o at dim 64e + lane
    const bool in = lane < nch;
    const float mv = in ? r[lane * arec + HD] : -__builtin_inff();
    const float lv = in ? r[lane * arec + HD + 1] : 0.f;
    float ov[2 * NS][DPL];
#pragma unroll
    for (int i = 0; i < 2 * NS; i++)
#pragma unroll
        for (int e = 0; e < DPL; e++) ov[i][e] = i < nch ? r[i * arec + 64 * e + lane] : 0.f;
    const int len0 = min(NS, nch), len1 = nch - len0;
    const float Ms0 = wave_max(lane < len0 ? mv : -__builtin_inff());
    const float Ms1 = wave_max(lane >= NS ? mv : -__builtin_inff());
    // chunk c of split s: w = exp(m_c - M_s) (each lane's chunk is in one split)
    const float wv = in ? mi_expf(__fsub_rn(mv, lane < NS ? Ms0 : Ms1)) : 0.f;
    float ds0 = 0.f, ds1 = 0.f, as0[DPL], as1[DPL];
#pragma unroll
    for (int e = 0; e < DPL; e++) as0[e] = as1[e] = 0.f;
#pragma unroll
    for (int i = 0; i < NS; i++)
        if (i < len0) {
            const float wi = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(wv), i));
            const float li = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(lv), i));
            ds0 = __fmaf_rn(li, wi, ds0);
#pragma unroll
            for (int e = 0; e < DPL; e++) as0[e] = __fmaf_rn(ov[i][e], wi, as0[e]);
        }
    if (len1 <= 0) {
#pragma unroll
        for (int e = 0; e < DPL; e++) out[e] = __fdiv_rn(as0[e], ds0);
        return;
    }
#pragma unroll
    for (int i = 0; i < NS; i++)
        if (i < len1) {
            const float wi = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(wv), NS + i));
            const float li = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(lv), NS + i));
            ds1 = __fmaf_rn(li, wi, ds1);
#pragma unroll
            for (int e = 0; e < DPL; e++) as1[e] = __fmaf_rn(ov[NS + i][e], wi, as1[e]);
        }
    const float Mx = fmaxf(Ms0, Ms1);
    const float w0 = mi_expf(__fsub_rn(Ms0, Mx)), w1 = mi_expf(__fsub_rn(Ms1, Mx));
    float den = __fmaf_rn(ds0, w0, 0.f);
    den = __fmaf_rn(ds1, w1, den);
#pragma unroll
    for (int e = 0; e < DPL; e++) out[e] = __fdiv_rn(__fmaf_rn(as1[e], w1, __fmaf_rn(as0[e], w0, 0.f)), den);
}
template <int HD>
__device__ __forceinline__ void comb_wave(const float* r, int arec, int nch, int lane, float (&out)[HD / 64]) {
    constexpr int DPL = HD / 64;
    if (nch <= 2 * kAttnSplit) {
        comb_wave2<HD>(r, arec, nch, lane, out);
        return;
    }
    float Mx = -__builtin_inff();
    if (nch > kAttnSplit) {
        for (int c = lane; c < nch; c += 64) Mx = fmaxf(Mx, r[c * arec + HD]);
        Mx = wave_max(Mx);
    }
    float den = 0.f, acc[DPL];
#pragma unroll
    for (int e = 0; e < DPL; e++) acc[e] = 0.f;
    for (int c0 = 0; c0 < nch; c0 += kAttnSplit) {
        const int len = min(kAttnSplit, nch - c0);
        const float* rs = r + (size_t)c0 * arec;
        const float mv = lane < len ? rs[lane * arec + HD] : -__builtin_inff();
        const float lv = lane < len ? rs[lane * arec + HD + 1] : 0.f;
        float ov[kAttnSplit][DPL];
#pragma unroll
        for (int i = 0; i < kAttnSplit; i++)
#pragma unroll
            for (int e = 0; e < DPL; e++) ov[i][e] = i < len ? rs[i * arec + 64 * e + lane] : 0.f;
        const float Ms = wave_max(mv);
        const float wv = lane < len ? mi_expf(__fsub_rn(mv, Ms)) : 0.f;
        float ds = 0.f, as[DPL];
#pragma unroll
        for (int e = 0; e < DPL; e++) as[e] = 0.f;
#pragma unroll
        for (int i = 0; i < kAttnSplit; i++)
            if (i < len) {
                const float wi = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(wv), i));
                const float li = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(lv), i));
                ds = __fmaf_rn(li, wi, ds);
#pragma unroll
                for (int e = 0; e < DPL; e++) as[e] = __fmaf_rn(ov[i][e], wi, as[e]);
            }
        if (nch <= kAttnSplit) {
            den = ds;
#pragma unroll
            for (int e = 0; e < DPL; e++) acc[e] = as[e];
        } else {
            const float ws = mi_expf(__fsub_rn(Ms, Mx));
            den = __fmaf_rn(ds, ws, den);
#pragma unroll
            for (int e = 0; e < DPL; e++) acc[e] = __fmaf_rn(as[e], ws, acc[e]);
        }
    }
#pragma unroll
    for (int e = 0; e < DPL; e++) out[e] = __fdiv_rn(acc[e], den);
}

// The canonical merge (the oracle's, the standalone k_attn_merge's) of one head's chunk
// records for 32 of its dims (one 128-byte line of each record): records r[c * arec]
// (o[hd], m, l), nch of them, out[0..32) = the merged o / den for dims d0 .. d0 + 31.
// All eight waves of the workgroup take part (it synchronizes the workgroup): wave w takes
// the split pairs (2g, 2g + 1) for g = w, w + 8, ...: the pair's 32 o lines come into the
// wave's LDS by DMA (8 records per instruction), lane 16j + c loads m, l of chunk c of
// split 2g + j meanwhile, M_s is the max over its 16 lanes and w_c = exp(m_c - M_s) goes
// to LDS; lane 32j + d then runs den_s (d = 0) and acc_s as fma chains in chunk order.
// Wave 0 merges the splits the same way in split order (lane s: w_s; lane d: the chains)
// and writes out with agent-coherent stores. The loops stay rolled (the step kernel's
// phase loop holds this code; an unrolled register version cost ~1% at short contexts,
// where the phase never runs). lds: 8 * (1024 + 64) + nsp * 34 floats.
constexpr int kCombSR = 34;
constexpr int kCombMaxSplits = 512;           // splits of 16 chunks the per-phase merge kernel holds in LDS
constexpr int kCombWaveFloats = 1024 + 64;      // per wave: o lines [2][16][32], weights [2][w | l][16]
template <int HD>
__device__ __forceinline__ void comb_slice(const float* r, int arec, int nch, int d0, int wave, int lane, float* lds,
                                           float* out) {
    // opaque lane and wave: their addresses are not hoisted out of the step's phase loop
    asm volatile("" : "+v"(lane));
    asm volatile("" : "+v"(wave));
    const int nsp = (nch + kAttnSplit - 1) / kAttnSplit;
    float* ol = lds + wave * kCombWaveFloats;
    float* wls = ol + 1024;
    float* sres = lds + 8 * kCombWaveFloats;                            // [split][M, den, acc[32]]
    for (int g = wave; 2 * g < nsp; g += 8) {
#pragma unroll 1
        for (int k = 0; k < 4; k++) {                                   // o lines of chunks 8(k&1) .. +7 of split 2g + k/2
            const int sp = min(2 * g + (k >> 1), nsp - 1);
            const int c = min(sp * kAttnSplit + (k & 1) * 8 + (lane >> 3), nch - 1);
            __builtin_amdgcn_global_load_lds(r + (size_t)c * arec + d0 + 4 * (lane & 7),
                                             (lds_ptr)(ol + ((k >> 1) * 16 + (k & 1) * 8) * 32), 16, 0, 0);
        }
        const int wj = (lane >> 4) & 1, wc = lane & 15, wsp = 2 * g + wj, cc = wsp * kAttnSplit + wc;
        const bool ok = lane < 32 && wsp < nsp && cc < nch;
        const float m = ok ? r[(size_t)cc * arec + HD] : -__builtin_inff();
        const float l = ok ? r[(size_t)cc * arec + HD + 1] : 0.f;
        float M = fmaxf(m, dppf<kDppRor8>(m));                          // max over the 16 lanes of the row
        M = fmaxf(M, dppf<kDppRor4>(M));
        M = fmaxf(M, dppf<kDppXor2>(M));
        M = fmaxf(M, dppf<kDppXor1>(M));
        if (lane < 32) {
            wls[wj * 32 + wc] = ok ? mi_expf(__fsub_rn(m, M)) : 0.f;
            wls[wj * 32 + 16 + wc] = l;
            if (wc == 0 && wsp < nsp) sres[wsp * kCombSR] = M;
        }
        drain_vm();
        wave_lds_sync();
        const int j = lane >> 5, d = lane & 31, sp = 2 * g + j;
        if (sp < nsp) {
            const int n = min(kAttnSplit, nch - sp * kAttnSplit);
            float den = 0.f, acc = 0.f;
#pragma unroll 4
            for (int i = 0; i < n; i++) {
                const float w = wls[j * 32 + i];
                den = __fmaf_rn(wls[j * 32 + 16 + i], w, den);
                acc = __fmaf_rn(ol[(j * 16 + i) * 32 + d], w, acc);
            }
            float* sr = sres + sp * kCombSR;
            if (d == 0) sr[1] = den;
            sr[2 + d] = acc;
        }
        wave_lds_sync();                                                // ol and wls are reused by the next pair
    }
    __syncthreads();
    if (wave == 0) {
        const int d = lane & 31;
        float den, acc;
        if (nsp == 1) {
            den = sres[1];
            acc = sres[2 + d];
        } else {
            float M = -__builtin_inff();
            for (int sp = lane; sp < nsp; sp += 64) M = fmaxf(M, sres[sp * kCombSR]);
            M = wave_max(M);
            for (int sp = lane; sp < nsp; sp += 64) sres[sp * kCombSR] = mi_expf(__fsub_rn(sres[sp * kCombSR], M));
            wave_lds_sync();
            den = 0.f;
            acc = 0.f;
            for (int sp = 0; sp < nsp; sp++) {
                den = __fmaf_rn(sres[sp * kCombSR + 1], sres[sp * kCombSR], den);
                acc = __fmaf_rn(sres[sp * kCombSR + 2 + d], sres[sp * kCombSR], acc);
            }
        }
        if (lane < 32) stc(out + d0 + lane, __fdiv_rn(acc, den));
    }
    __syncthreads();                                                    // lds is free again
}
// chunk merge as its own phase (more than kInlineComb chunks): workgroup t < NH * HD/32
// merges head t / (HD/32) for 32 dims (comb_slice), all of the workgroup's waves taking
// part; the merged vectors go to att_out for the O prologue
template <int HD>
__device__ __forceinline__ void phase_comb(MPtr M, int l, int pos, int wg, int nwg, int wave, int lane, float* lds) {
    const int nch = (pos + 1 + kAttnChunk - 1) / kAttnChunk;
    for (int t = wg; t < M->NH * (HD / 32); t += nwg) {
        const int h = t / (HD / 32), d0 = (t - h * (HD / 32)) * 32;
        comb_slice<HD>(att_rec(M, l) + (size_t)h * M->maxch * M->arec, M->arec, nch, d0, wave, lane, lds,
                       M->att_out + (size_t)l * M->E + (size_t)h * HD);
    }
}

// ------------------------------------------------------------------ the persistent step
// One cooperative launch of one 512-thread workgroup per CU runs the whole token:
// five phases per layer separated by grid barriers (the reference's mega kernel has
// the same count, mega.cu:695-833) + one for the chunk merge past kInlineComb
// chunks, then lm_head, one barrier and workgroup 0 merges the candidates.
// The phases run as one loop over the flattened sequence (layer, kind), so each
// piece of code exists once: the whole kernel stays within the instruction cache
// (an unrolled body of ~115 KB missed it on every layer).
// Per phase: [all waves: staging DMA shares] sync [prologue] sync [workers: tiles]
// sync [workers: segment sums, stores, store drain] sync [control: grid barrier |
// workers: next phase's prefetch] sync.
// Profile slots (every workgroup): 0 = start; then kProfPerPhase per phase in the
// sequence (qkv, attention, o, gate/up, down per layer, then lm_head): prologue end,
// first worker's tiles done, its stores drained (lm: the control wave's candidate
// written), phase end, barrier exit; with MI_PROFILE_FINE also the control wave's
// staging landed, the first worker's staging landed (with its prefetched tiles), the
// residual add done (norm phases).
__device__ __forceinline__ PMat phase_mat(MPtr M, int l, int kind) {
    if (kind == PH_LM) return ldmat(&M->lm);
    const LPtr L = LY(M, l);
    return ldmat(kind == PH_QKV ? &L->qkv : kind == PH_O ? &L->o : kind == PH_GU ? &L->gu : &L->d);
}
// the phase after (l, kind)
__device__ __forceinline__ void phase_next(MPtr M, int l, int kind, int& nl, int& nk) {
    if (kind == PH_DOWN) { nl = l + 1; nk = nl < M->NL ? PH_QKV : PH_LM; }
    else { nl = l; nk = kind + 1; }
}
// workers: the tiles of GEMV phase (l, kind)
template <int HD>
__device__ __forceinline__ void phase_work(MPtr M, int l, int kind, int pos, int wg, int nwg, const Lds& S,
                                           int kw, Tile (&tl)[2], int lane) {
    const bool down = kind == PH_DOWN;
    gemv_tiles(phase_mat(M, l, kind), wg, nwg, kw, tl, down ? S.U : S.X, down ? kActRec : kXRec, S.P, lane);
}
// workers: the stores of phase (l, kind) (lm_head has its own epilogue)
__device__ __forceinline__ void phase_store(MPtr M, int l, int kind, int wg, int nwg, const Lds& S, int kw, int lane) {
    if (kind == PH_ATTN) return;
    const PMat W = phase_mat(M, l, kind);
    if (kind == PH_GU) {
        gu_store(W, wg, nwg, kw, S.P, act_rec(M, l), lane);
    } else {
        float* part = kind == PH_QKV ? qkv_part(M, l) : kind == PH_O ? o_part(M, l) : d_part(M, l);
        seg_store(W, wg, nwg, kw, S.P, part, lane);
    }
}
// workers: the prefetch of phase (l, kind)'s first tiles (the attention K/V of the
// first items are brought in by the control wave during the QKV phase)
__device__ __forceinline__ void phase_prefetch(MPtr M, int l, int kind, int wg, int nwg, int kw, Tile (&tl)[2], int lane) {
    if (kind != PH_ATTN) {
        prefetch(phase_mat(M, l, kind), wg, nwg, kw, tl, lane);
    } else {
        tl[0] = Tile{};        // written on every path: the tiles are never live across the attention phase
        tl[1] = Tile{};
    }
}

// a workgroup with no O segment skips the O phase's staging and prologue (the records'
// merge and quantisation feed only the O GEMV; the residual is not touched there)
__device__ __forceinline__ bool phase_idle(MPtr M, int l, int kind, int wg, int nwg) {
    if (kind != PH_O) return false;
    const PMat W = phase_mat(M, l, kind);
    return wg_place(W, wg, nwg) >= (W.rows >> 6) * W.ks;
}

template <int HD, bool PROF>
__global__ __launch_bounds__(kPThreads) void k_step(const DModel* Mp, int pos, int gen) {
    const MPtr M = (MPtr)Mp;
    __shared__ __align__(16) uint8_t smem[step_lds<HD>()];
    const Lds S(smem);
    const int wg = blockIdx.x, nwg = gridDim.x, wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    const bool ctl = wave == 0;
    const int kw = wave - 1;
    const int nch = (pos + 1 + kAttnChunk - 1) / kAttnChunk;
    if (gen == kGenRing) {
        // a streaming generation that stopped at eos: every workgroup sees the same input
        // token and returns before any barrier; the eos is passed on, so the launches
        // queued behind this one return too
        const int in = M->tokbuf[pos];
        if (in == M->eos) {
            if (wg == 0 && threadIdx.x == 0) M->tokbuf[pos + 1] = in;
            return;
        }
    }
    GridBar gb = bar_init(M->bar, M->err);
    Tile tl[2];
    STAMP_IF(0);
    stage(M, 0, PH_QKV, pos, S, wave, kPWaves, lane, true);
    FINE_STAMP_IF(1 + 5);
    if (!ctl) phase_prefetch(M, 0, PH_QKV, wg, nwg, kw, tl, lane);
    int l = 0, kind = PH_QKV;
    for (int sb = 1;; sb += kProfPerPhase) {
        __syncthreads();
#ifdef MI_PROFILE_FINE
        if (!phase_idle(M, l, kind, wg, nwg)) wg_prologue(M, l, kind, pos, wg, S, wave, lane, true, PROF ? sb + 7 : -1);
#else
        if (!phase_idle(M, l, kind, wg, nwg)) wg_prologue(M, l, kind, pos, wg, S, wave, lane, true);
#endif
        __syncthreads();
        STAMP_IF(sb);
        if (kind == PH_ATTN) {
            attn_run<HD>(M, l, pos, wg, nwg, S.U, wave, lane);      // every wave: one query head each
        } else if (!ctl) {
            phase_work<HD>(M, l, kind, pos, wg, nwg, S, kw, tl, lane);
        }
        tl[0] = Tile{};            // consumed: dead (and not in registers) until the next prefetch
        tl[1] = Tile{};
        if (kind == PH_ATTN && nch > kInlineComb) {           // the chunk merge as a phase of its own
            drain_vm();
            __syncthreads();
            if (ctl) ctl_barrier(gb, M->err);
            __syncthreads();
            phase_comb<HD>(M, l, pos, wg, nwg, wave, lane, reinterpret_cast<float*>(S.U));
        }
        __syncthreads();
        STAMP_IF(sb + 1, 64);
        if (kind == PH_LM) {
            lm_epilogue(M, wg, nwg, S, wave, lane, gb.dead);
            STAMP_IF(sb + 2);
            __syncthreads();
            STAMP_IF(sb + 3);
            if (ctl) {
                ctl_barrier(gb, M->err);
                ctl_exit(M->bar);
                STAMP_IF(sb + 4);
                if (wg == 0) {
                    unsigned failed;
                    const Top2 a = wave_merge_cands(M->cand, nwg, lane, &failed);
                    if (lane == 0) emit_token(M, a, pos, gen, failed);
                }
            }
            return;
        }
        int nl, nk;
        phase_next(M, l, kind, nl, nk);
        if (!ctl) {
            phase_store(M, l, kind, wg, nwg, S, kw, lane);
            drain_vm();
            STAMP_IF(sb + 2, 64);
        } else {
            drain_vm();
            tl[0] = Tile{};
            tl[1] = Tile{};
        }
        __syncthreads();
        STAMP_IF(sb + 3);
        if (ctl) {
            ctl_barrier(gb, M->err);
            STAMP_IF(sb + 4);
        } else if (nk == PH_ATTN) {
            // the attention waves' first items: their K/V rows into LDS (U is free once
            // the QKV prologue is done); attn_finish waits for them
            tl[0] = Tile{};
            tl[1] = Tile{};
            attn_prefetch<HD>(M, nl, pos, wg, nwg, S.U, wave, lane);
        } else {
            // the next phase's first tiles, issued while the control wave waits at the
            // grid barrier (issuing ~60-120 KB per CU takes the texture unit ~1 us)
            phase_prefetch(M, nl, nk, wg, nwg, kw, tl, lane);
        }
        __syncthreads();
        if (!phase_idle(M, nl, nk, wg, nwg)) stage(M, nl, nk, pos, S, wave, kPWaves, lane, true);
        else drain_vm();
        FINE_STAMP_IF(sb + kProfPerPhase + 5);           // this wave's staging landed (control, first worker)
        FINE_STAMP_IF(sb + kProfPerPhase + 6, 64);
        l = nl;
        kind = nk;
    }
}

// barrier cost: n grid barriers and nothing else
__global__ __launch_bounds__(kPThreads) void k_barriers(uint32_t* bar, int32_t* err, int n) {
    GridBar gb = bar_init(bar, err);
    for (int i = 0; i < n; i++) {
        __syncthreads();
        if (threadIdx.x < 64) ctl_barrier(gb, err);
    }
}

// ------------------------------------------------------------------ per-phase kernels
// The same phases as one launch each (same grid and roles; the residual stream goes
// through hbuf, workgroup 0 writes it): the non-persistent reference path.
constexpr int kPhaseLds = step_lds<128>();
#define PHASE_PRELUDE                                                                        \
    __shared__ __align__(16) uint8_t smem[kPhaseLds];                                        \
    const Lds S(smem);                                                                       \
    const int wg = blockIdx.x, nwg = gridDim.x, wave = threadIdx.x >> 6, lane = threadIdx.x & 63; \
    const bool ctl = wave == 0;                                                              \
    const int kw = wave - 1;                                                                 \
    Tile tl[2];

__global__ __launch_bounds__(kPThreads) void k_qkv(const DModel* Mp, int l, int pos) {
    const MPtr M = (MPtr)Mp;
    PHASE_PRELUDE
    const PMat W = ldmat(&LY(M, l)->qkv);
    if (ctl) ctl_stage(M, l, PH_QKV, pos, S, lane, false);
    else prefetch(W, wg, nwg, kw, tl, lane);
    __syncthreads();
    wg_prologue(M, l, PH_QKV, pos, wg, S, wave, lane, false);
    __syncthreads();
    if (!ctl) gemv_tiles(W, wg, nwg, kw, tl, S.X, kXRec, S.P, lane);
    __syncthreads();
    if (!ctl) seg_store(W, wg, nwg, kw, S.P, qkv_part(M, l), lane);
}
template <int HD>
__global__ __launch_bounds__(kPThreads) void k_attn(const DModel* Mp, int l, int pos) {
    const MPtr M = (MPtr)Mp;
    __shared__ __align__(16) uint8_t smem[step_lds<HD>()];
    const Lds S(smem);
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    attn_prefetch<HD>(M, l, pos, blockIdx.x, gridDim.x, S.U, wave, lane);
    drain_vm();
    __syncthreads();
    attn_run<HD>(M, l, pos, blockIdx.x, gridDim.x, S.U, wave, lane);
}
template <int HD>
__global__ __launch_bounds__(kPThreads) void k_attn_comb(const DModel* Mp, int l, int pos) {
    const MPtr M = (MPtr)Mp;
    __shared__ __align__(16) float lds[8 * kCombWaveFloats + kCombMaxSplits * kCombSR];
    phase_comb<HD>(M, l, pos, blockIdx.x, gridDim.x, threadIdx.x >> 6, threadIdx.x & 63, lds);
}
__global__ __launch_bounds__(kPThreads) void k_o(const DModel* Mp, int l, int pos) {
    const MPtr M = (MPtr)Mp;
    PHASE_PRELUDE
    const PMat W = ldmat(&LY(M, l)->o);
    if (ctl) ctl_stage(M, l, PH_O, pos, S, lane, false);
    else prefetch(W, wg, nwg, kw, tl, lane);
    __syncthreads();
    wg_prologue(M, l, PH_O, pos, wg, S, wave, lane, false);
    __syncthreads();
    if (!ctl) gemv_tiles(W, wg, nwg, kw, tl, S.X, kXRec, S.P, lane);
    __syncthreads();
    if (!ctl) seg_store(W, wg, nwg, kw, S.P, o_part(M, l), lane);
}
__global__ __launch_bounds__(kPThreads) void k_gu(const DModel* Mp, int l) {
    const MPtr M = (MPtr)Mp;
    PHASE_PRELUDE
    const PMat W = ldmat(&LY(M, l)->gu);
    if (ctl) ctl_stage(M, l, PH_GU, 0, S, lane, false);
    else prefetch(W, wg, nwg, kw, tl, lane);
    __syncthreads();
    wg_prologue(M, l, PH_GU, 0, wg, S, wave, lane, false);
    __syncthreads();
    if (!ctl) gemv_tiles(W, wg, nwg, kw, tl, S.X, kXRec, S.P, lane);
    __syncthreads();
    if (!ctl) gu_store(W, wg, nwg, kw, S.P, act_rec(M, l), lane);
}
__global__ __launch_bounds__(kPThreads) void k_down(const DModel* Mp, int l) {
    const MPtr M = (MPtr)Mp;
    PHASE_PRELUDE
    const PMat W = ldmat(&LY(M, l)->d);
    if (ctl) ctl_stage(M, l, PH_DOWN, 0, S, lane, false);
    else prefetch(W, wg, nwg, kw, tl, lane);
    __syncthreads();
    if (!ctl) gemv_tiles(W, wg, nwg, kw, tl, S.U, kActRec, S.P, lane);
    __syncthreads();
    if (!ctl) seg_store(W, wg, nwg, kw, S.P, d_part(M, l), lane);
}
__global__ __launch_bounds__(kPThreads) void k_lm(const DModel* Mp) {
    const MPtr M = (MPtr)Mp;
    PHASE_PRELUDE
    if (ctl) ctl_stage(M, M->NL - 1, PH_LM, 0, S, lane, false);
    else prefetch(ldmat(&M->lm), wg, nwg, kw, tl, lane);
    __syncthreads();
    wg_prologue(M, M->NL - 1, PH_LM, 0, wg, S, wave, lane, false);
    __syncthreads();
    if (!ctl) gemv_tiles(ldmat(&M->lm), wg, nwg, kw, tl, S.X, kXRec, S.P, lane);
    __syncthreads();
    lm_epilogue(M, wg, nwg, S, wave, lane);
}
__global__ __launch_bounds__(64) void k_argmax(const DModel* Mp, int ncand, int pos, int gen) {
    const MPtr M = (MPtr)Mp;
    const Top2 a = wave_merge_cands(M->cand, ncand, threadIdx.x);
    if (threadIdx.x == 0) emit_token(M, a, pos, gen);
}

// ================================================================== multi-token steps
// T <= kMaxT tokens at positions pos..pos+T-1 in one pass over the weights: the
// verify step of speculative decoding (forward_batch, cuda_infer.cu:990-1026; mega.cu
// gemv_part T>1 :259-265, tile_dot :197-244). One launch per phase. Every value
// equals the single-token step's bit for bit: the per-block integer dot of q4 nibbles
// and int8 activations comes from int8 MFMA (exact), and the float work keeps the same
// plan (block fma chain per chunk, chunk sums left to right, segment sums left to
// right), the same norm/quant arithmetic and the same attention items.
// The GEMM phases read their input as int8 block records from xT, written once per
// token by kT_in (residual + RMSNorm + quant, one workgroup per token) or kT_comb
// (chunk merge + quant), so no workgroup repeats the per-token prologue.
constexpr int kTChunks = 16;       // chunk sums of one segment held in LDS
// LDS stride of one token's records: nblk * kTRec rounded up to 16 mod 128, so that the
// eight tokens' records of one block sit in different LDS banks (at a stride that is a
// multiple of 128 bytes, the MFMA operand reads of the eight token slots all hit the same
// bank group: an 8-way conflict). The xT slots in memory use the same stride
// (lay::xT_tok), so a slot's T tokens come into LDS as one copy.
__device__ __forceinline__ int xt_stride(int nblk) { return (int)lay::xT_tok(32 * nblk); }
constexpr int kTXeBytes = kMaxT * ((kMaxE / 32) * kTRec + 128);
constexpr int kTXfBytes = kMaxT * ((kMaxFF / 32) * kTRec + 128);
constexpr int kTPBytes = kTChunks * kMaxT * 64 * 4;
constexpr int kTGemvLds = kTXeBytes + kTPBytes;    // qkv, o, gate/up, lm_head
constexpr int kTDownLds = kTXfBytes + kTPBytes;    // down

typedef int v4i __attribute__((ext_vector_type(4)));
typedef unsigned int u32x2 __attribute__((ext_vector_type(2)));

__device__ __forceinline__ size_t hT_at(MPtr M, int slot, int t) { return lay::hT(M->E, slot, t); }
__device__ __forceinline__ float4 ldg4(const float* p) { return *reinterpret_cast<const float4*>(p); }
__device__ __forceinline__ uint2 ntload8(const uint8_t* p) {
    const u32x2 v = __builtin_nontemporal_load(reinterpret_cast<const u32x2*>(p));
    return make_uint2(v.x, v.y);
}

// One chunk (64 rows x CB blocks) as one lane holds it for v_mfma_i32_16x16x64_i8.
// One MFMA covers row group q (rows 16q..16q+15) and block pair p (blocks 2p, 2p+1):
// the 16 x 64 "A" side is 8 token slots per block (slot m < 8: token m, block 2p, its
// codes in the K lanes of groups kg = 0, 1 and zeros in kg = 2, 3; slot m >= 8: token
// m-8, block 2p+1, codes in kg = 2, 3), the "B" side is the rows' nibbles (block 2p in
// kg = 0, 1, block 2p+1 in kg = 2, 3). So D[m][row] is the integer dot of one token
// and one block, and all 16 x 16 outputs are used at T = 8. Within a block, lane group
// h = kg%2 carries elements 8h..8h+7 (low nibbles of bytes 8h..8h+7) and 16+8h..+7
// (their high nibbles); any pairing of K indices gives the same exact dot as long as
// both sides use it.
// w[q][p]: 8 nibble bytes of row 16q + l%16, block 2p + kg/2, bytes 8h..8h+7.
// s[j][.]: the fp16 scale line (CB halves) of row 16(2*(kg/2) + j) + l%16.
template <int CB>
struct TTile {
    uint2 w[4][CB / 2];
    uint32_t s[2][CB / 2];
};

template <int CB>
__device__ __forceinline__ void ttile_load(TTile<CB>& t, const uint8_t* tile, int lane) {
    const int col = lane & 15, kg = lane >> 4;
#pragma unroll
    for (int q = 0; q < 4; q++)
#pragma unroll
        for (int p = 0; p < CB / 2; p++)
            t.w[q][p] = ntload8(tile + (2 * p + (kg >> 1)) * 1024 + (q * 16 + col) * 16 + 8 * (kg & 1));
#pragma unroll
    for (int j = 0; j < 2; j++) {
        const uint8_t* sp = tile + CB * 1024 + ((2 * (kg >> 1) + j) * 16 + col) * CB * 2;
        if constexpr (CB == 8) {
            const uint4 v = ntload16(sp);
            t.s[j][0] = v.x; t.s[j][1] = v.y; t.s[j][2] = v.z; t.s[j][3] = v.w;
        } else {
            const uint2 v = ntload8(sp);
            t.s[j][0] = v.x; t.s[j][1] = v.y;
        }
    }
}

// chunk sums of one tile for the T tokens whose block records (kTRec bytes: 32 codes,
// fp32 scale, 8*sum) are in LDS at XT + token * rs + block * kTRec (rs = xt_stride).
// acc[j][i]: row 16(2*(kg/2) + j) + l%16, token 4*(kg%2) + i. Per (row, token) the
// float work is the single-token chain: acc = fma(dw*dx, float(dot - 8*sum), acc) over
// the CB blocks in order, from 0.
// The MFMA's C operand subtracts 8*sum (exact int32): lane kg's output slots are tokens
// 4*(kg%2) + i of block 2p + kg/2. It leaves block 2p's results in lanes kg < 2 and block
// 2p+1's in kg >= 2 for each row group; v_permlane32_swap of groups (q, q+2) hands each
// lane both blocks of one row group (q = 2*(kg/2) + j), so every lane runs two chains per
// token. Token slots T..kMaxT-1 read whatever their LDS records hold (XT has room for
// kMaxT tokens, so the reads stay in bounds); their sums are never read.
template <int CB>
__device__ __forceinline__ void ttile_sums(const TTile<CB>& W, const uint8_t* XT, int rs, int b0,
                                           float (&acc)[2][4], int lane) {
    const int col = lane & 15, kg = lane >> 4, h = kg & 1, hb = kg >> 1;
    const int am = ((col < 8) == (kg < 2)) ? -1 : 0;
    const uint8_t* xa = XT + (col & 7) * rs + (b0 + (col >> 3)) * kTRec + 8 * h;
    const uint8_t* xr = XT + (4 * h) * rs + b0 * kTRec + 32;
#pragma unroll
    for (int j = 0; j < 2; j++)
#pragma unroll
        for (int i = 0; i < 4; i++) acc[j][i] = 0.f;
#pragma unroll
    for (int p = 0; p < CB / 2; p++) {
        const uint2 lo = *reinterpret_cast<const uint2*>(xa + 2 * p * kTRec);
        const uint2 hi = *reinterpret_cast<const uint2*>(xa + 2 * p * kTRec + 16);
        const v4i a = v4i{(int)lo.x & am, (int)lo.y & am, (int)hi.x & am, (int)hi.y & am};
        float dx0[4], dx1[4];
        v4i c;
#pragma unroll
        for (int i = 0; i < 4; i++) {
            const float2 e0 = *reinterpret_cast<const float2*>(xr + i * rs + 2 * p * kTRec);
            const float2 e1 = *reinterpret_cast<const float2*>(xr + i * rs + (2 * p + 1) * kTRec);
            dx0[i] = e0.x;
            dx1[i] = e1.x;
            c[i] = (int)(0u - (uint32_t)__float_as_int(hb ? e1.y : e0.y));
        }
        int d[4][4];
#pragma unroll
        for (int q = 0; q < 4; q++) {
            const uint2 w = W.w[q][p];
            const v4i b = v4i{(int)(w.x & 0x0F0F0F0Fu), (int)(w.y & 0x0F0F0F0Fu), (int)((w.x >> 4) & 0x0F0F0F0Fu),
                              (int)((w.y >> 4) & 0x0F0F0F0Fu)};
            const v4i r = __builtin_amdgcn_mfma_i32_16x16x64_i8(a, b, c, 0, 0, 0);
#pragma unroll
            for (int i = 0; i < 4; i++) d[q][i] = r[i];
        }
#pragma unroll
        for (int i = 0; i < 4; i++) {
#pragma unroll
            for (int j = 0; j < 2; j++) {
                const auto r = __builtin_amdgcn_permlane32_swap((unsigned)d[j][i], (unsigned)d[j + 2][i], false, false);
                const uint32_t sw = W.s[j][p];
                acc[j][i] = __fmaf_rn(__fmul_rn(h2f_lo(sw), dx0[i]), __int2float_rn((int)r[0]), acc[j][i]);
                acc[j][i] = __fmaf_rn(__fmul_rn(h2f_hi(sw), dx1[i]), __int2float_rn((int)r[1]), acc[j][i]);
            }
        }
    }
}

// segment (row group g, K segment s) of work item t
__device__ __forceinline__ void tseg(const PMat W, int t, int& g, int& s, int& c0, int& c1) {
    g = W.ks == 1 ? t : div_small(t, W.ks);
    s = t - g * W.ks;
    c0 = seg_c0(W, s);
    c1 = seg_c0(W, s + 1);
}
// this wave's next chunk: k (index inside segment t) + kPWaves, else chunk `wave` of the
// workgroup's next segment (t + nwg, ...) that has one. Start with t = wg, k = wave - kPWaves.
__device__ __forceinline__ bool tnext(const PMat W, int nseg, int nwg, int wave, int& t, int& k) {
    k += kPWaves;
    for (; t < nseg; t += nwg, k = wave) {
        int g, s, c0, c1;
        tseg(W, t, g, s, c0, c1);
        if (k < c1 - c0) return true;
    }
    return false;
}

// A wave's first chunk of a T-token GEMM: (segment t, chunk k) and its tile loads.
// The GEMM issues it itself before staging its input, or kT_step issues it during the
// grid barrier before the phase (issued = true).
template <int CB>
struct TFirst {
    TTile<CB> tile;
    int t, k;
    bool have, issued;
};
template <int CB>
__device__ __forceinline__ void tgemm_first(const PMat W, int wg, int nwg, int wave, int lane, TFirst<CB>& f) {
    const int nseg = (W.rows >> 6) * W.ks;
    f.t = wg;
    f.k = wave - kPWaves;
    f.have = tnext(W, nseg, nwg, wave, f.t, f.k);
    if (f.have) {
        int g, s, c0, c1;
        tseg(W, f.t, g, s, c0, c1);
        ttile_load<CB>(f.tile, tile_ptr(W, g, c0 + f.k), lane);
    }
    f.issued = true;
}

// T-token GEMM over this workgroup's segments (t = wg, wg + nwg, ...). Each wave takes
// chunks wave, wave + 8, ... of every segment and holds the next chunk's loads in
// flight while it computes one (the first is issued before `stage` fills XT, unless
// it already is). Chunk sums go to P[chunk][token][row]; after a segment, wave t adds
// token t's chunk sums left to right and hands out(g, s, t, value) the row g*64 + lane.
template <int CB, class S, class F>
__device__ __forceinline__ void tgemm_cb(const PMat W, int wg, int nwg, const uint8_t* XT, int nblk, int T, float* P,
                                         int wave, int lane, S stage, F out, TFirst<CB>& f) {
    const int nseg = (W.rows >> 6) * W.ks, rs = xt_stride(nblk);
    if (!f.issued) tgemm_first<CB>(W, wg, nwg, wave, lane, f);
    f.issued = false;
    int t = f.t, k = f.k;
    bool have = f.have;
    TTile<CB>& cur = f.tile;
    TTile<CB> nx;
    if (wg < nseg) stage();                          // a workgroup with no segment stages nothing
    __syncthreads();
    int nt = t, nk = k;
    bool hn = have && tnext(W, nseg, nwg, wave, nt, nk);
    bool odd = false;   // the current tile is in nx
    for (int ts = wg; ts < nseg; ts += nwg) {
        int g, s, c0, c1;
        tseg(W, ts, g, s, c0, c1);
        // the tiles alternate between cur and nx (no register copy per chunk)
        auto chunk = [&](const TTile<CB>& a, TTile<CB>& b) {
            if (hn) {
                int g2, s2, a0, a1;
                tseg(W, nt, g2, s2, a0, a1);
                ttile_load<CB>(b, tile_ptr(W, g2, a0 + nk), lane);
            }
            float acc[2][4];
            ttile_sums<CB>(a, XT, rs, (c0 + k) * CB, acc, lane);
            const int col = lane & 15, kg = lane >> 4;
            float* pc = P + (size_t)k * kMaxT * 64;
#pragma unroll
            for (int j = 0; j < 2; j++)
#pragma unroll
                for (int i = 0; i < 4; i++) pc[(4 * (kg & 1) + i) * 64 + (2 * (kg >> 1) + j) * 16 + col] = acc[j][i];
            t = nt;
            k = nk;
            have = hn;
            if (hn) hn = tnext(W, nseg, nwg, wave, nt, nk);
        };
        while (have && t == ts) {
            if (!odd) chunk(cur, nx);
            else chunk(nx, cur);
            odd = !odd;
        }
        __syncthreads();
        if (wave < T) {
            float v = P[(size_t)wave * 64 + lane];
            for (int c = 1; c < c1 - c0; c++) v = __fadd_rn(v, P[((size_t)c * kMaxT + wave) * 64 + lane]);
            out(g, s, wave, v);
        }
        __syncthreads();
    }
}
// pre: the first chunks of this GEMM when kT_step issued them ahead (cb = 8 only);
// issued = false otherwise
template <class S, class F>
__device__ __forceinline__ void tgemm(const PMat W, int wg, int nwg, const uint8_t* XT, int nblk, int T, float* P, int wave,
                                      int lane, S stage, F out, TFirst<8>& pre) {
    if (W.cb == 8) {
        tgemm_cb<8>(W, wg, nwg, XT, nblk, T, P, wave, lane, stage, out, pre);
    } else {
        TFirst<4> own;
        own.issued = false;
        tgemm_cb<4>(W, wg, nwg, XT, nblk, T, P, wave, lane, stage, out, own);
    }
}

// The thread index is made opaque per phase body: inside kT_step's layer loop its derived
// addresses would otherwise be hoisted out of the loop and stay live across every phase.
__device__ __forceinline__ int opaque_tid() {
    int t = threadIdx.x;
    asm volatile("" : "+v"(t));
    return t;
}
// The GEMM inputs' int8 records, one slot per (layer, input) so that every line is
// written once per step (the persistent step reads them with plain loads; layout.hpp)
using lay::kXtQkv;
using lay::kXtO;
using lay::kXtGu;
__device__ __forceinline__ int xt_slot(MPtr M, int l, int which) { return lay::xt_slot(M->NL, l, which); }
__device__ __forceinline__ uint8_t* xT_at(MPtr M, int slot) { return M->xT + lay::xT(M->E, slot); }
// T tokens' records of an E-wide GEMM input: its xT slot -> LDS (all threads)
// the T tokens' input records of a GEMM (contiguous, 1-KB units shared over the waves)
// into LDS by DMA, all in flight at once (a thread-per-8-bytes copy loop waited for
// each load before its store)
__device__ __forceinline__ void tstage_x(MPtr M, int slot, int T, uint8_t* XT) {
    const int tid = opaque_tid();
    DmaShare d{tid >> 6, (int)(blockDim.x >> 6), 0};
    dma_share(xT_at(M, slot), XT, T * xt_stride(M->E / 32), d, tid & 63);
    drain_vm();
}

// O in the per-phase multi-token launches: one K segment per chunk (ks = nc; 2.18 ->
// 2.14 ms per 8-token S3 step); the persistent kT_step keeps the plan's split, which is
// faster there. oT is laid out for nc partials either way.
__device__ __forceinline__ PMat omatT(MPtr M, int l, bool persistent) {
    PMat W = ldmat(&LY(M, l)->o);
    if (!persistent) W.ks = W.nc;
    return W;
}
__device__ __forceinline__ float* oT_at(MPtr M, int l) { return M->oT + lay::oT(LY(M, 0)->o.nc, M->E, l); }
// phase input of token t for the qkv (kind PH_QKV), gate/up (PH_GU) and
// lm_head (PH_LM) GEMMs: x = h + split-K partials in order (layer 0 of qkv: the
// token's embedding row) -> hT -> RMSNorm -> int8 records in xT. The same arithmetic
// as the single-token step's norm prologue (cuda_infer.cu:43-60 rmsnorm, 80-89 quant).
template <bool P>
__device__ __forceinline__ void kT_in_body(MPtr M, int l, int kind, int t, float* x, int pos) {
    const int wave = threadIdx.x >> 6, lane = opaque_tid() & 63, n = M->E, nblk = n / 32;
    const bool qkv = kind == PH_QKV, lm = kind == PH_LM, dsrc = kind != PH_GU;
    const int pl = qkv ? l - 1 : lm ? M->NL - 1 : l;
    float* hdst = M->hT + hT_at(M, qkv ? 2 * l : 2 * l + 1, t);
    // wave j quantizes slice j (n <= kMaxE: one slice per wave at most); its norm
    // weights are loaded with the inputs, not after the sum of squares
    static_assert(kMaxE <= 256 * kPWaves, "one 256-element slice per wave");
    const float* w = lm ? M->out_norm : qkv ? LY(M, l)->an : LY(M, l)->fn;
    const int ew = 256 * wave + 4 * lane;
    const float4 wv = ew < n ? ldg4(w + ew) : make_float4(0.f, 0.f, 0.f, 0.f);
    for (int e0 = ew; e0 < n; e0 += 256 * kPWaves) {
        float4 v;
        if (qkv && l == 0) {
            v = ldg4(M->emb + (size_t)M->tokbuf[pos + t] * n + e0);
        } else {
            const int ks = dsrc ? LY(M, pl)->d.ks : omatT(M, pl, P).ks;
            const float* part = dsrc ? M->dT + (size_t)pl * LY(M, 0)->d.ks * kMaxT * n : oT_at(M, pl);
            const float* h = M->hT + hT_at(M, dsrc ? 2 * pl + 1 : 2 * l, t);
            float4 p[kMaxKsRes];
#pragma unroll
            for (int s = 0; s < kMaxKsRes; s++)
                if (s < ks) p[s] = ldg4(part + ((size_t)s * kMaxT + t) * n + e0);
            float4 sum = p[0];
#pragma unroll
            for (int s = 1; s < kMaxKsRes; s++)
                if (s < ks) sum = f4add(sum, p[s]);
            v = f4add(ldg4(h + e0), sum);
        }
        st4(x, e0, v);
        if (!lm) {
            if constexpr (P) {
                stc(hdst + e0, v.x); stc(hdst + e0 + 1, v.y); stc(hdst + e0 + 2, v.z); stc(hdst + e0 + 3, v.w);
            } else {
                *reinterpret_cast<float4*>(hdst + e0) = v;
            }
        }
    }
    __syncthreads();
    const float sc = rms_scale(x, n, M->eps, lane);
    uint8_t* xr = xT_at(M, lm ? xt_slot(M, M->NL, 0) : xt_slot(M, l, qkv ? kXtQkv : kXtGu)) + (size_t)t * xt_stride(nblk);
    if (256 * wave < n) {
        const bool own = ew < n;
        float4 y = make_float4(0.f, 0.f, 0.f, 0.f);
        if (own) {
            const float4 xv = ld4(x + ew);
            y = make_float4(__fmul_rn(__fmul_rn(xv.x, sc), wv.x), __fmul_rn(__fmul_rn(xv.y, sc), wv.y),
                            __fmul_rn(__fmul_rn(xv.z, sc), wv.z), __fmul_rn(__fmul_rn(xv.w, sc), wv.w));
        }
        quant_slice<P>(y, own, ew, xr, lane, kTRec);
    }
}
__global__ __launch_bounds__(kPThreads) void kT_in(const DModel* Mp, int l, int kind) {
    __shared__ __align__(16) float x[kMaxE];
    kT_in_body<false>((MPtr)Mp, l, kind, blockIdx.x, x, *((MPtr)Mp)->posT);
}

__device__ __forceinline__ float* qkvT_at(MPtr M, int l) { return M->qkvT + lay::qkvT(LY(M, 0)->qkv.ks, M->QKV, l); }
__device__ __forceinline__ float* dT_at(MPtr M, int l) { return M->dT + lay::dT(LY(M, 0)->d.ks, M->E, l); }
__device__ __forceinline__ float* attT_at(MPtr M, int l, int t) { return M->attT + lay::attT(M->NH, M->maxch, M->arec, l, t); }
__device__ __forceinline__ uint8_t* actT_at(MPtr M, int l, int t) { return M->actT + lay::actT(M->FF, l, t); }

// The phase bodies take the workgroup's LDS, its index and the grid size; P selects the
// stores (and xT loads) for phases that run inside one persistent launch (kT_step).
#define TBODY const int wave = threadIdx.x >> 6, lane = opaque_tid() & 63;
#define TWRAP(BYTES, CALL)                                                                       \
    __shared__ __align__(16) uint8_t smem[BYTES];                                                \
    CALL;
// the GEMM kernels' wrapper: their first chunks issued by the GEMM itself
#define TWRAP_G(BYTES, CALL)                                                                     \
    __shared__ __align__(16) uint8_t smem[BYTES];                                                \
    TFirst<8> pre;                                                                               \
    pre.issued = false;                                                                          \
    CALL;

template <bool PS>
__device__ __forceinline__ void kT_qkv_body(MPtr M, int l, int T, uint8_t* smem, int wg, int nwg, TFirst<8>& pre) {
    TBODY
    uint8_t* XT = smem;
    float* P = reinterpret_cast<float*>(smem + kTXeBytes);
    const PMat W = ldmat(&LY(M, l)->qkv);
    float* part = qkvT_at(M, l);
    tgemm(W, wg, nwg, XT, M->E / 32, T, P, wave, lane, [&] { tstage_x(M, xt_slot(M, l, kXtQkv), T, XT); },
          [&](int g, int s, int t, float v) { st_x<PS>(&part[((size_t)s * kMaxT + t) * W.rows + g * 64 + lane], v); }, pre);
}
__global__ __launch_bounds__(kPThreads) void kT_qkv(const DModel* Mp, int l, int T) {
    TWRAP_G(kTGemvLds, kT_qkv_body<false>((MPtr)Mp, l, T, smem, blockIdx.x, gridDim.x, pre))
}

// Multi-token attention. Item = (kv head, 64-position chunk c, group of tg consecutive
// tokens): the workgroup stages the chunk's K/V once (cached rows by DMA; the rows of
// this step's positions pos..pos+T-1 finished from the QKV rows: bias, RoPE, fp16, as
// the single-token step does for its own position) and its waves run the (token, query
// head) pairs of the group against it, one attn_core each (the single-token chunk
// arithmetic), writing record (t, h, c). Token t uses the chunk's rows up to pos + t.
// The item holding token T-1 appends the step's rows of the chunk to the cache.
// LDS: the chunk's K tile and V rows, then per wave two q rows and two probability rows
template <int HD>
constexpr int kt_attn_lds() { return 2 * 64 * HD * 2 + kPWaves * (2 * HD + 2 * 64) * 4; }

// The items of a T-token attention phase: tokens per item tg is the smallest power of
// two that keeps the items within one per workgroup (more tokens per item: fewer K/V
// stagings, more pairs per wave). Item it runs on workgroup nwg - 1 - it (+ k nwg), so
// that the first items sit on the last workgroups, which have no QKV rows.
struct KtAttnPlan { int nchx, tg, ngrp, total; };
__device__ __forceinline__ KtAttnPlan kt_attn_plan(int NKV, int pos, int T, int nwg) {
    KtAttnPlan P;
    P.nchx = (pos + T - 1 + kAttnChunk) / kAttnChunk;
    P.tg = 1;
    while (P.tg < T && NKV * P.nchx * ((T + P.tg - 1) / P.tg) > nwg) P.tg *= 2;
    P.ngrp = (T + P.tg - 1) / P.tg;
    P.total = NKV * P.nchx * P.ngrp;
    return P;
}
// item it: kv head, chunk, its tokens ta..tb; false when the chunk starts past them
__device__ __forceinline__ bool kt_attn_item(const KtAttnPlan& P, int it, int T, int pos, int& kvh, int& c, int& ta,
                                             int& tb) {
    const int grp = it % P.ngrp, rest = it / P.ngrp;
    c = rest % P.nchx;
    kvh = rest / P.nchx;
    ta = grp * P.tg;
    tb = min(T, ta + P.tg) - 1;
    return c * kAttnChunk <= pos + tb;
}
// The cached K/V rows (positions before pos) of this workgroup's first attention item
// into LDS, issued by wave 0 during the QKV phase by a workgroup without QKV rows: the
// cache rows do not depend on this step. True (on every wave) when issued.
template <int HD>
__device__ __forceinline__ bool kt_attn_prefetch(MPtr M, int l, int T, int pos, int wg, int nwg, uint8_t* smem) {
    const KtAttnPlan P = kt_attn_plan(M->NKV, pos, T, nwg);
    const int it = nwg - 1 - wg;
    int kvh, c, ta, tb;
    if (it >= P.total || !kt_attn_item(P, it, T, pos, kvh, c, ta, tb)) return false;
    const int t0 = c * kAttnChunk, ncached = min(kAttnChunk, max(0, pos - t0));
    if (ncached <= 0) return false;
    if ((threadIdx.x >> 6) == 0) {
        const size_t rowbase = lay::kv(M->NKV, M->maxseq, 1, l, kvh, 0);
        attn_issue_kv<HD>(M->kc + rowbase * HD, M->vc + rowbase * HD, t0, ncached, reinterpret_cast<uint4*>(smem),
                          reinterpret_cast<__half*>(smem + 64 * HD * 2), opaque_tid() & 63);
    }
    return true;
}

// kv_pre: kt_attn_prefetch issued this workgroup's first item's cached rows
template <int HD, bool PS>
__device__ __forceinline__ void kT_attn_body(MPtr M, int l, int T, uint8_t* smem, int wg, int nwg, int pos,
                                             bool kv_pre = false) {
    TBODY
    constexpr int half = HD / 2, DPL = HD / 64;
    uint4* kls = reinterpret_cast<uint4*>(smem);
    __half* vls = reinterpret_cast<__half*>(smem + 64 * HD * 2);
    float* qs = reinterpret_cast<float*>(smem + 2 * 64 * HD * 2) + wave * (2 * HD + 2 * 64);
    float* pl = qs + 2 * HD;
    const LPtr Ly = LY(M, l);
    const int G = M->G, NKV = M->NKV, ks = Ly->qkv.ks, QKV = M->QKV;
    const KtAttnPlan AP = kt_attn_plan(NKV, pos, T, nwg);
    const int total = AP.total, ip = lane % half;
    const float* part = qkvT_at(M, l);
    const float* bq = Ly->bqkv;
    auto fin = [&](int tok, int row) {
        float v = part[(size_t)tok * QKV + row];
        for (int s = 1; s < ks; s++) v = __fadd_rn(v, part[((size_t)s * kMaxT + tok) * QKV + row]);
        return __fadd_rn(v, bq[row]);
    };
    // q of (token t, head h), rotated at position pos + t, into the wave's q row j
    auto load_q = [&](int t, int h, int j) {
        if (lane < half) {
            const int rq = h * HD;
            const float2 cz = M->rope[(size_t)(pos + t) * half + ip];
            const float x0 = fin(t, rq + ip), x1 = fin(t, rq + ip + half);
            qs[j * HD + ip] = __fsub_rn(__fmul_rn(x0, cz.x), __fmul_rn(x1, cz.y));
            qs[j * HD + ip + half] = __fadd_rn(__fmul_rn(x0, cz.y), __fmul_rn(x1, cz.x));
        }
    };
    for (int it = nwg - 1 - wg; it < total; it += nwg) {
        int kvh, c, ta, tb;
        if (!kt_attn_item(AP, it, T, pos, kvh, c, ta, tb)) continue;   // uniform over the workgroup
        const int t0 = c * kAttnChunk, ncached = min(kAttnChunk, max(0, pos - t0));
        const size_t rowbase = lay::kv(NKV, M->maxseq, 1, l, kvh, 0);     // row index of position 0
        if (wave == 0 && ncached > 0 && !(kv_pre && it == nwg - 1 - wg))
            attn_issue_kv<HD>(M->kc + rowbase * HD, M->vc + rowbase * HD, t0, ncached, kls, vls, lane);
        // this step's row pos + wave, if the chunk holds it and a token of the group sees it
        const int p = pos + wave;
        const bool mine = wave <= tb && p >= t0 && p < t0 + kAttnChunk;
        __half y0 = __float2half(0.f), y1 = y0, v0 = y0, v1 = y0;
        if (mine && lane < half) {
            const int rk = M->NH * HD + kvh * HD, rv = M->NH * HD + M->KVD + kvh * HD;
            const float2 cu = M->rope[(size_t)p * half + ip];
            const float k0 = fin(wave, rk + ip), k1 = fin(wave, rk + ip + half);
            y0 = __float2half(__fsub_rn(__fmul_rn(k0, cu.x), __fmul_rn(k1, cu.y)));
            y1 = __float2half(__fadd_rn(__fmul_rn(k0, cu.y), __fmul_rn(k1, cu.x)));
            v0 = __float2half(fin(wave, rv + ip));
            v1 = __float2half(fin(wave, rv + ip + half));
        }
        // (token, head) pairs i = ta.., in token-major order: wave w takes pairs w*ppw ..
        // w*ppw + ppw - 1, two at a time (the q rows of both loaded together, and two
        // heads of one token run as one attn_core_h<HD, 2>: the same chains per head as
        // attn_core, the K and V values read once for both). The first two q rows load
        // while the chunk's rows come in.
        const int npair = (tb - ta + 1) * G, ppw = (npair + kPWaves - 1) / kPWaves;
        auto pair_th = [&](int i, int& t, int& h) {
            t = ta + i / G;
            h = kvh * G + i % G;
        };
        {
            const int i0 = wave * ppw;
            int t, h;
            if (i0 < npair) { pair_th(i0, t, h); load_q(t, h, 0); }
            if (ppw > 1 && i0 + 1 < npair) { pair_th(i0 + 1, t, h); load_q(t, h, 1); }
        }
        if (wave == 0) drain_vm();
        __syncthreads();                                           // cached rows landed
        if (mine && lane < half) {
            const int r = p - t0;
            __half* kh = reinterpret_cast<__half*>(kls);
            kh[kslot<HD>(r, ip >> 3) * 8 + (ip & 7)] = y0;
            kh[kslot<HD>(r, (ip + half) >> 3) * 8 + ((ip + half) & 7)] = y1;
            vls[r * HD + ip] = v0;
            vls[r * HD + ip + half] = v1;
            if (tb == T - 1) {                                     // one item per (kv head, chunk) appends
                __half* kd = M->kc + (rowbase + p) * HD;
                __half* vd = M->vc + (rowbase + p) * HD;
                kd[ip] = y0; kd[ip + half] = y1;
                vd[ip] = v0; vd[ip + half] = v1;
            }
        }
        __syncthreads();                                           // the chunk's rows complete
        auto store_rec = [&](int t, int h, float m, float lsum, const float (&acc)[DPL]) {
            float* rec = attT_at(M, l, t) + ((size_t)h * M->maxch + c) * M->arec;
#pragma unroll
            for (int e = 0; e < DPL; e++) st_x<PS>(rec + DPL * lane + e, acc[e]);
            if (lane == 0) { st_x<PS>(rec + HD, m); st_x<PS>(rec + HD + 1, lsum); }
        };
        for (int j0 = 0; j0 < ppw; j0 += 2) {
            const int i0 = wave * ppw + j0;
            if (i0 >= npair) break;
            const bool two = j0 + 1 < ppw && i0 + 1 < npair;
            int ta0, ha, tb0 = -1, hb = 0;
            pair_th(i0, ta0, ha);
            if (two) pair_th(i0 + 1, tb0, hb);
            if (j0 > 0) {
                wave_lds_sync();                                   // the last round's q rows are read
                load_q(ta0, ha, 0);
                if (two) load_q(tb0, hb, 1);
            }
            wave_lds_sync();
            if (two && tb0 == ta0) {
                if (t0 > pos + ta0) continue;                      // the chunk is past this token
                float m[2], lsum[2], acc[2][DPL];
                attn_core_h<HD, 2>(kls, qs, 2, vls, min(kAttnChunk, pos + ta0 + 1 - t0), M->scale, lane, pl, m, lsum, acc);
                store_rec(ta0, ha, m[0], lsum[0], acc[0]);
                store_rec(ta0, hb, m[1], lsum[1], acc[1]);
            } else {
                for (int k = 0; k < (two ? 2 : 1); k++) {
                    const int t = k ? tb0 : ta0, h = k ? hb : ha;
                    if (t0 > pos + t) continue;                    // the chunk is past this token
                    if (k) wave_lds_sync();                        // pl is reused
                    float m[1], lsum[1], acc[1][DPL];
                    attn_core_h<HD, 1>(kls, qs + k * HD, 1, vls, min(kAttnChunk, pos + t + 1 - t0), M->scale, lane, pl, m,
                                       lsum, acc);
                    store_rec(t, h, m[0], lsum[0], acc[0]);
                }
            }
        }
        __syncthreads();                                           // LDS is reused by the next item
    }
}
template <int HD>
__global__ __launch_bounds__(kPThreads) void kT_attn(const DModel* Mp, int l, int T) {
    TWRAP(kt_attn_lds<HD>(), (kT_attn_body<HD, false>((MPtr)Mp, l, T, smem, blockIdx.x, gridDim.x, *((MPtr)Mp)->posT)))
}

// chunk merge of token t's records for query head h (one wave per (t, h); lane = dims
// lane + 64j) into the O phase's int8 records in xT. The merge is comb_wave's, the
// step's merge phase uses the same function.
template <int HD, bool PS>
__device__ __forceinline__ void kT_comb_item(MPtr M, int l, int item, int lane, int pos) {
    constexpr int DPL = HD / 64;
    const int t = item / M->NH, hh = item - t * M->NH, nch = (pos + t + kAttnChunk) / kAttnChunk, arec = M->arec;
    const float* r = attT_at(M, l, t) + (size_t)hh * M->maxch * arec;
    float o[DPL];
    comb_wave<HD>(r, arec, nch, lane, o);
    const int nblk = M->E / 32;
#pragma unroll
    for (int e = 0; e < DPL; e++) {
        int q, s8;
        float d;
        quant32_vals(o[e], q, d, s8);
        const int el = hh * HD + 64 * e + lane;       // lanes 4k..4k+3 fill code word k of the block
        uint8_t* rec = xT_at(M, xt_slot(M, l, kXtO)) + (size_t)t * xt_stride(nblk) + (el >> 5) * kTRec;
        const uint32_t b = (uint32_t)(q & 0xFF);
        const uint32_t wd = b | (__shfl_down(b, 1) << 8) | (__shfl_down(b, 2) << 16) | (__shfl_down(b, 3) << 24);
        if ((lane & 3) == 0) st_x<PS>(reinterpret_cast<uint32_t*>(rec + (el & 31)), wd);
        if ((lane & 31) == 0) {
            st_x<PS>(reinterpret_cast<float*>(rec + 32), d);
            st_x<PS>(reinterpret_cast<uint32_t*>(rec + 36), (uint32_t)s8);
        }
    }
}
template <int HD>
__global__ __launch_bounds__(256) void kT_comb(const DModel* Mp, int l, int T) {
    const MPtr M = (MPtr)Mp;
    const int item = blockIdx.x * 4 + (threadIdx.x >> 6);
    if (item < T * M->NH) kT_comb_item<HD, false>(M, l, item, threadIdx.x & 63, *M->posT);
}

template <bool PS>
__device__ __forceinline__ void kT_o_body(MPtr M, int l, int T, uint8_t* smem, int wg, int nwg, TFirst<8>& pre) {
    TBODY
    uint8_t* XT = smem;
    float* P = reinterpret_cast<float*>(smem + kTXeBytes);
    const PMat W = omatT(M, l, PS);
    float* part = oT_at(M, l);
    tgemm(W, wg, nwg, XT, M->E / 32, T, P, wave, lane, [&] { tstage_x(M, xt_slot(M, l, kXtO), T, XT); },
          [&](int g, int s, int t, float v) { st_x<PS>(&part[((size_t)s * kMaxT + t) * W.rows + g * 64 + lane], v); }, pre);
}
__global__ __launch_bounds__(kPThreads) void kT_o(const DModel* Mp, int l, int T) {
    TWRAP_G(kTGemvLds, kT_o_body<false>((MPtr)Mp, l, T, smem, blockIdx.x, gridDim.x, pre))
}

template <bool PS>
__device__ __forceinline__ void kT_gu_body(MPtr M, int l, int T, uint8_t* smem, int wg, int nwg, TFirst<8>& pre) {
    TBODY
    uint8_t* XT = smem;
    float* P = reinterpret_cast<float*>(smem + kTXeBytes);
    const PMat W = ldmat(&LY(M, l)->gu);
    tgemm(W, wg, nwg, XT, M->E / 32, T, P, wave, lane, [&] { tstage_x(M, xt_slot(M, l, kXtGu), T, XT); }, [&](int g, int s, int t, float v) {
        (void)s;
        const float u = __shfl(v, (lane & 31) + 32);
        const float e = mi_expf(-v);
        const float a = __fmul_rn(__fdiv_rn(v, __fadd_rn(1.0f, e)), u);
        int q, s8;
        float d;
        quant32_vals(a, q, d, s8);
        const uint32_t b = (uint32_t)(q & 0xFF);
        const uint32_t wd = b | (__shfl_down(b, 1) << 8) | (__shfl_down(b, 2) << 16) | (__shfl_down(b, 3) << 24);
        if (lane < 32) {
            uint32_t* r = reinterpret_cast<uint32_t*>(actT_at(M, l, t) + (size_t)g * kActRec);
            if ((lane & 3) == 0) st_x<PS>(r + lane / 4, wd);
            if (lane == 0) { st_x<PS>(r + 8, __float_as_uint(d)); st_x<PS>(r + 9, (uint32_t)s8); }
        }
    }, pre);
}
__global__ __launch_bounds__(kPThreads) void kT_gu(const DModel* Mp, int l, int T) {
    TWRAP_G(kTGemvLds, kT_gu_body<false>((MPtr)Mp, l, T, smem, blockIdx.x, gridDim.x, pre))
}

template <bool PS>
__device__ __forceinline__ void kT_down_body(MPtr M, int l, int T, uint8_t* smem, int wg, int nwg, TFirst<8>& pre) {
    TBODY
    uint8_t* XT = smem;
    float* P = reinterpret_cast<float*>(smem + kTXfBytes);
    const int nblk = M->FF / 32;
    const PMat W = ldmat(&LY(M, l)->d);
    float* part = dT_at(M, l);
    // act records of the T tokens over the blocks this workgroup's segments cover,
    // compacted to kTRec bytes per block
    auto stage = [&] {
        const int nseg = (W.rows >> 6) * W.ks;
        int blo = nblk, bhi = 0;
        for (int t = wg; t < nseg; t += nwg) {
            int g, s, c0, c1;
            tseg(W, t, g, s, c0, c1);
            blo = min(blo, c0 * W.cb);
            bhi = max(bhi, c1 * W.cb);
        }
        const int nb = max(0, bhi - blo), n8 = T * nb * (kTRec / 8), rs = xt_stride(nblk);
        // every load of a round in flight before its stores
        constexpr int U = 4;
        for (int i0 = opaque_tid(); i0 < n8; i0 += U * (int)blockDim.x) {
            uint2 v[U];
            int at[U];
#pragma unroll
            for (int u = 0; u < U; u++) {
                const int i = i0 + u * (int)blockDim.x;
                at[u] = -1;
                if (i < n8) {
                    const int rcd = i / (kTRec / 8), k = i - rcd * (kTRec / 8), t = div_small(rcd, max(nb, 1));
                    const int b = blo + rcd - t * nb;
                    v[u] = reinterpret_cast<const uint2*>(actT_at(M, l, t) + (size_t)b * kActRec)[k];
                    at[u] = t * rs + b * kTRec + 8 * k;
                }
            }
#pragma unroll
            for (int u = 0; u < U; u++)
                if (at[u] >= 0) *reinterpret_cast<uint2*>(XT + at[u]) = v[u];
        }
    };
    tgemm(W, wg, nwg, XT, nblk, T, P, wave, lane, stage, [&](int g, int s, int t, float v) {
        st_x<PS>(&part[((size_t)s * kMaxT + t) * W.rows + g * 64 + lane], v);
    }, pre);
}
__global__ __launch_bounds__(kPThreads) void kT_down(const DModel* Mp, int l, int T) {
    TWRAP_G(kTDownLds, kT_down_body<false>((MPtr)Mp, l, T, smem, blockIdx.x, gridDim.x, pre))
}

template <bool PS>
__device__ __forceinline__ void kT_lm_body(MPtr M, int T, uint8_t* smem, int wg, int nwg, TFirst<8>& pre) {
    TBODY
    uint8_t* XT = smem;
    float* P = reinterpret_cast<float*>(smem + kTXeBytes);
    const PMat W = ldmat(&M->lm);
    Top2 tp{-__builtin_inff(), INT_MAX, -__builtin_inff()};
    tgemm(W, wg, nwg, XT, M->E / 32, T, P, wave, lane, [&] { tstage_x(M, xt_slot(M, M->NL, 0), T, XT); }, [&](int g, int s, int t, float v) {
        (void)s;
        const int row = g * 64 + lane;
        if (M->logitsT) M->logitsT[(size_t)t * M->V + row] = v;
        top2_push(tp, v, row);
    }, pre);
    if (wave < T) {
        top2_wave(tp);
        if (lane == 0) {
            float* cd = M->candT + lay::candT(wg, wave);
            st_x<PS>(cd, tp.best);
            st_x<PS>(reinterpret_cast<uint32_t*>(cd + 1), (uint32_t)tp.idx);
            st_x<PS>(cd + 2, tp.second);
        }
    }
}
__global__ __launch_bounds__(kPThreads) void kT_lm(const DModel* Mp, int T) {
    TWRAP_G(kTGemvLds, kT_lm_body<false>((MPtr)Mp, T, smem, blockIdx.x, gridDim.x, pre))
}

__device__ __forceinline__ void kT_argmax_body(MPtr M, int ncand, int T, int pos) {
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    if (wave >= T) return;
    Top2 tp{-__builtin_inff(), INT_MAX, -__builtin_inff()};
    merge_cand_recs(M->candT + lay::candT(0, wave), (int)lay::candT(1, 0), ncand, lane,
                    [&](float4 c) { top2_merge(tp, c.x, __float_as_int(c.y), c.z); });
    top2_wave(tp);
    if (lane == 0) {
        M->out_tok[pos + wave] = top2_token(tp, M->V);
        M->out_margin[pos + wave] = __fsub_rn(tp.best, tp.second);
    }
}
__global__ __launch_bounds__(kPThreads) void kT_argmax(const DModel* Mp, int ncand, int T) {
    kT_argmax_body((MPtr)Mp, ncand, T, *((MPtr)Mp)->posT);
}

// The multi-token step as one persistent launch (mega.cu:621-623 runs prompt chunks and
// verify steps inside its persistent loop): one workgroup per CU runs the phase bodies
// above in order, the step kernel's grid barrier between them (each workgroup drains its
// stores first; a barrier that gives up sets M.err, and the later ones do not wait).
// Values that cross workgroups inside the launch are stored agent-coherent (P = true)
// into buffers whose lines are each written once per launch before any workgroup reads
// them (per-layer partials, records and xT slots), so plain loads never meet a stale
// line. The same arithmetic as the per-phase launches, so the same bits.
// ---- speculative generation on the device (the host loop's steps, engine.hip
// generate_spec, in the same float arithmetic)
// mi_best_draft_len (spec.cpp; mega.cu:581-589): the k in 0..tmax-1 with the best expected
// tokens per unit of step cost
__device__ __forceinline__ int spec_best_k(float alpha, float slope, int tmax) {
    int best_k = 0;
    float best_rate = 1.f, all_accepted = alpha;
    for (int k = 1; k < tmax; ++k) {
        all_accepted = __fmul_rn(all_accepted, alpha);
        const float expected = __fdiv_rn(__fsub_rn(1.f, all_accepted), __fsub_rn(1.f, alpha));
        const float rate = __fdiv_rn(expected, __fadd_rn(1.f, __fmul_rn(slope, (float)k)));
        if (rate > best_rate) {
            best_rate = rate;
            best_k = k;
        }
    }
    return best_k;
}
// mi_ngram_draft (spec.cpp; mega.cu:561-578) by one wave: for n = ngmax..1 the latest
// earlier j whose h[j..j+n) equals the last n tokens of h[0..len), lanes testing 64
// candidates j at a time from the top; its following tokens go to out. Returns K. The
// history is read with agent-coherent loads (this wave has just written its tail).
__device__ __forceinline__ int spec_draft(int32_t* h, int len, int ngmax, int kmax, int32_t* out, int lane) {
    if (kmax <= 0) return 0;
    auto hv = [&](int i) { return (int32_t)ldc(reinterpret_cast<const uint32_t*>(h + i)); };
    for (int n = ngmax; n >= 1; n--) {
        if (len < n + 1) continue;
        for (int base = len - n - 1; base >= 0; base -= 64) {
            const int j = base - lane;
            bool match = j >= 0;
            for (int k = 0; k < n && match; k++) match = hv(j + k) == hv(len - n + k);
            const uint64_t b = __builtin_amdgcn_ballot_w64(match);
            if (b) {
                const int jj = base - (int)__builtin_ctzll(b);      // the largest matching j
                const int K = min(kmax, len - (jj + n));
                if (lane < K) out[lane] = hv(jj + n + lane);
                return K;
            }
        }
    }
    return 0;
}
// after the verify step of T tokens at pos: the commit and the next draft (one wave).
// When a grid barrier of this launch gave up (*err set), workgroups may still be running
// this step with its T and pos, and the step's outputs are not trustworthy: the state is
// left as it was except done = 1, so the launches queued behind this one return at once
// and the host recomputes the whole generation with cooperative launches.
__device__ __forceinline__ void spec_commit(MPtr M, SpecDev* sp, int lane, int pos) {
    if (ldc(reinterpret_cast<const uint32_t*>(M->err)) != 0) {
        if (lane == 0) sp->done = 1;
        return;
    }
    const int K = sp->T - 1;
    int32_t* h = M->tokbuf;
    int a = 0;
    while (a < K && h[pos + 1 + a] == M->out_tok[pos + a]) a++;
    int emitted = sp->emitted, last = sp->last_pos;
    bool done = false;
    for (int i = 0; i <= a && !done; i++) {
        const int32_t y = M->out_tok[pos + i];
        if (lane == 0) h[pos + 1 + i] = y;
        emitted++;
        last = pos + 1 + i;
        done = emitted >= sp->n_gen || (sp->eos >= 0 && y == sp->eos);
    }
    const int np = pos + a + 1;                              // h[np] = the new current token (written above)
    float an = sp->acc_num, ad = sp->acc_den;
    if (K > 0) {
        an = __fadd_rn(__fmul_rn(0.85f, an), __fmul_rn(0.15f, (float)a));
        ad = __fadd_rn(__fmul_rn(0.85f, ad), __fmul_rn(0.15f, (float)(a + (a < K ? 1 : 0))));
    }
    int T = 1;
    if (!done) {
        drain_vm();                                          // the history writes above, before the search reads them
        const float alpha = fminf(fmaxf(__fdiv_rn(an, ad), 0.01f), 0.99f);
        const int kmax = min(spec_best_k(alpha, sp->slope, sp->tmax), min(sp->n_gen - emitted - 1, sp->maxseq - 1 - np));
        T = 1 + spec_draft(h, np + 1, sp->ngmax, kmax, h + np + 1, lane);
    }
    if (lane == 0) {
        sp->T = T;
        sp->done = done;
        sp->emitted = emitted;
        sp->last_pos = last;
        sp->steps += 1;
        sp->drafted += K;
        sp->accepted += a;
        sp->acc_num = an;
        sp->acc_den = ad;
        if (!done) *M->posT = np;
    }
}

constexpr int kTStepLds = kTDownLds > kTGemvLds ? kTDownLds : kTGemvLds;
static_assert(kTStepLds >= kt_attn_lds<128>() && kTStepLds >= 4 * kMaxE, "every phase's LDS fits");
// SPEC: T comes from M->spec (a speculative generation driven on the device): a launch
// after the generation finished returns at once, and workgroup 0 ends the step with
// spec_commit.
template <int HD, bool SPEC>
__global__ __launch_bounds__(kPThreads) void kT_step(const DModel* Mp, int T) {
    const MPtr M = (MPtr)Mp;
    if constexpr (SPEC) {
        if (M->spec->done) return;                           // every workgroup reads the same word
        T = M->spec->T;
    }
    // the step's position, read once: with SPEC, workgroup 0's spec_commit rewrites posT
    // (and T) for the next launch at the end of this one
    const int pos = *M->posT;
    __shared__ __align__(16) uint8_t smem[kTStepLds];
    const int wg = blockIdx.x, nwg = gridDim.x, wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    float* xs = reinterpret_cast<float*>(smem);
    // the light phases (kT_in: token t; the chunk merge items) run on the last
    // workgroups, rw = nwg - 1 - wg: the GEMM segments start at workgroup 0, so these
    // have the least GEMM work in the phase after (their first tiles are issued late,
    // when they reach the barrier last)
    const int rw = nwg - 1 - wg;
    GridBar gb = bar_init(M->bar, M->err);
    auto barrier = [&] {
        drain_vm();
        __syncthreads();
        if (wave == 0) ctl_barrier(gb, M->err);
        __syncthreads();
    };
    // the barrier before a GEMM phase also issues the phase's first tile loads: waves
    // 1-7 after this workgroup's stores have drained, wave 0 once it has passed the
    // barrier (its arrival and polls would otherwise wait for them); they land while
    // the grid waits
    TFirst<8> pre;
    pre.issued = false;
    auto barrier_pre = [&](const AS4 PMat* Wp) {
        const PMat W = ldmat(Wp);
        drain_vm();
        __syncthreads();
        auto first = [&] {
            if (W.cb == 8) tgemm_first<8>(W, wg, nwg, wave, opaque_tid() & 63, pre);
        };
        if (wave == 0) ctl_barrier(gb, M->err, first);
        else first();
        __syncthreads();
    };
    for (int l = 0; l < M->NL; l++) {
        if (rw < T) kT_in_body<true>(M, l, PH_QKV, rw, xs, pos);
        barrier_pre(&LY(M, l)->qkv);
        const PMat Wq = ldmat(&LY(M, l)->qkv);
        const bool kv_pre = wg >= (Wq.rows >> 6) * Wq.ks && kt_attn_prefetch<HD>(M, l, T, pos, wg, nwg, smem);
        kT_qkv_body<true>(M, l, T, smem, wg, nwg, pre);
        barrier();
        kT_attn_body<HD, true>(M, l, T, smem, wg, nwg, pos, kv_pre);
        barrier();
        for (int it = rw * kPWaves + wave; it < T * M->NH; it += nwg * kPWaves) kT_comb_item<HD, true>(M, l, it, lane, pos);
        barrier_pre(&LY(M, l)->o);
        kT_o_body<true>(M, l, T, smem, wg, nwg, pre);
        barrier();
        if (rw < T) kT_in_body<true>(M, l, PH_GU, rw, xs, pos);
        barrier_pre(&LY(M, l)->gu);
        kT_gu_body<true>(M, l, T, smem, wg, nwg, pre);
        barrier_pre(&LY(M, l)->d);
        kT_down_body<true>(M, l, T, smem, wg, nwg, pre);
        barrier();
    }
    if (rw < T) kT_in_body<true>(M, M->NL - 1, PH_LM, rw, xs, pos);
    barrier_pre(&M->lm);
    kT_lm_body<true>(M, T, smem, wg, nwg, pre);
    barrier();
    if (wave == 0) ctl_exit(M->bar);
    if (wg == 0) {
        kT_argmax_body(M, nwg, T, pos);
        if constexpr (SPEC) {
            __syncthreads();                                 // the step's out_tok / out_margin
            if (wave == 0) spec_commit(M, M->spec, lane, pos);
        }
    }
}

// ------------------------------------------------------------------ standalone kernels
__global__ __launch_bounds__(kThreads) void k_quant(const float* x, int n, int8_t* xq, float* xd, int32_t* xs8) {
    const int lane = threadIdx.x & 63;
    const int e = blockIdx.x * kThreads + threadIdx.x;
    const bool own = e < n;
    int q, s8;
    float d;
    quant32_vals(own ? x[e] : 0.f, q, d, s8);
    if (own) {
        xq[e] = (int8_t)q;
        if ((lane & 31) == 0) { xd[e >> 5] = d; xs8[e >> 5] = s8; }
    }
}

// split-K partials part[s][row] of a packed matrix: one wave per (group, segment),
// its chunks in order (chunk sums added left to right)
// Standalone GEMV (q4 tiles x int8 records -> split-K partials): one wave per segment
// (64-row group g, K segment s); chunk sums add left to right. Three launch shapes (the
// launcher picks): with at most kGemvWgsPerCu segments per CU, a segment of several
// chunks gets a workgroup whose waves share its chunks (k_gemv_seg below), and a
// one-chunk segment a workgroup of its own (SPREAD), so the matrix spreads over as many
// CUs as it has segments; the wave keeps its next chunk's loads in flight while it
// computes one (the first is issued before the activation records are staged).
// Otherwise four segments per workgroup, one chunk in flight per wave: the lower
// register use keeps ~20 waves per CU resident, which is what feeds HBM for large
// matrices.
constexpr int kGemvWgsPerCu = 2;
template <bool SPREAD>
__global__ __launch_bounds__(kThreads) void k_gemv(PMat W, const int8_t* xq, const float* xd, const int32_t* xs8, float* part) {
    __shared__ __align__(16) uint8_t X[(kMaxFF / 32) * kXRec];
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int ntask = (W.rows / 64) * W.ks;
    auto stage = [&] {
        for (int b = threadIdx.x; b < W.nb; b += kThreads) {
            uint8_t* r = X + b * kXRec;
            const uint4* src = reinterpret_cast<const uint4*>(xq + 32 * b);
            reinterpret_cast<uint4*>(r)[0] = src[0];
            reinterpret_cast<uint4*>(r)[1] = src[1];
            *reinterpret_cast<float*>(r + 32) = xd[b];
            *reinterpret_cast<int32_t*>(r + 36) = xs8[b];
        }
        __syncthreads();
    };
    if constexpr (!SPREAD) {
        stage();
        for (int task = blockIdx.x * kWaves + wave; task < ntask; task += gridDim.x * kWaves) {
            int g, s, c0, c1;
            tseg(W, task, g, s, c0, c1);
            float seg = 0.f;
            for (int c = c0; c < c1; c++) {
                Tile t;
                tile_load(t, tile_ptr(W, g, c), W.cb, lane);
                const float p = chunk_dot(t, W.cb, X, kXRec, c * W.cb);
                seg = c == c0 ? p : __fadd_rn(seg, p);
            }
            part[(size_t)s * W.rows + g * 64 + lane] = seg;
        }
    } else {
        const int task = blockIdx.x;
        const bool have = wave == 0 && task < ntask;
        int g = 0, s = 0, c0 = 0, c1 = 0;
        Tile cur, nxt;
        if (have) {
            tseg(W, task, g, s, c0, c1);
            tile_load(cur, tile_ptr(W, g, c0), W.cb, lane);
        }
        stage();
        if (!have) return;
        float seg = 0.f;
        for (int c = c0; c < c1; c++) {
            if (c + 1 < c1) tile_load(nxt, tile_ptr(W, g, c + 1), W.cb, lane);
            const float p = chunk_dot(cur, W.cb, X, kXRec, c * W.cb);
            seg = c == c0 ? p : __fadd_rn(seg, p);
            cur = nxt;
        }
        part[(size_t)s * W.rows + g * 64 + lane] = seg;
    }
}

// Segment-per-workgroup GEMV (segments of at most kSegMaxChunks chunks): workgroup t owns
// segment t; wave j takes its chunks j, j + NW, ... (the next one's loads in flight while
// it computes one), so all of a short segment's loads are issued at once. Chunk sums go
// to LDS; wave 0 adds them left to right, as the one-wave loop does. Only the segment's
// activation blocks are staged.
constexpr int kSegMaxChunks = 48;
template <int NW>
__global__ __launch_bounds__(64 * NW) void k_gemv_seg(PMat W, const int8_t* xq, const float* xd, const int32_t* xs8,
                                                      float* part) {
    __shared__ __align__(16) uint8_t X[kSegMaxChunks * 8 * kXRec];
    __shared__ float sums[kSegMaxChunks][64];
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    int g, s, c0, c1;
    tseg(W, blockIdx.x, g, s, c0, c1);
    int c = c0 + wave;
    Tile cur, nxt;
    if (c < c1) tile_load(cur, tile_ptr(W, g, c), W.cb, lane);
    const int b0 = c0 * W.cb, nblk = (c1 - c0) * W.cb;
    for (int b = threadIdx.x; b < nblk; b += 64 * NW) {
        uint8_t* r = X + b * kXRec;
        const uint4* src = reinterpret_cast<const uint4*>(xq + 32 * (b0 + b));
        reinterpret_cast<uint4*>(r)[0] = src[0];
        reinterpret_cast<uint4*>(r)[1] = src[1];
        *reinterpret_cast<float*>(r + 32) = xd[b0 + b];
        *reinterpret_cast<int32_t*>(r + 36) = xs8[b0 + b];
    }
    __syncthreads();
    for (; c < c1; c += NW) {
        if (c + NW < c1) tile_load(nxt, tile_ptr(W, g, c + NW), W.cb, lane);
        sums[c - c0][lane] = chunk_dot(cur, W.cb, X, kXRec, (c - c0) * W.cb);
        cur = nxt;
    }
    __syncthreads();
    if (wave == 0) {
        float seg = sums[0][lane];
        for (int k = 1; k < c1 - c0; k++) seg = __fadd_rn(seg, sums[k][lane]);
        part[(size_t)s * W.rows + g * 64 + lane] = seg;
    }
}

// Wave-per-segment GEMV: grid wave w owns segment w (row group g, K segment s). Each
// lane first loads its share of the segment's activation block records (codes, scale,
// 8*sum) into registers, then the wave issues its first chunk's tile, then it writes the
// records into its own LDS area: a wave's loads complete in issue order, so the records
// land before the weights and no workgroup barrier waits on anyone's tiles. The chunks
// follow with the next chunk's loads in flight while one is summed; chunk sums are added
// left to right, the step's order, into one split-K partial.
constexpr int kWaveMaxBlocks = 64;   // activation blocks of one wave's segment
template <int NW, int CB>
__global__ __launch_bounds__(64 * NW) void k_gemv_wave(PMat W, const int8_t* xq, const float* xd, const int32_t* xs8,
                                                       float* part) {
    __shared__ __align__(16) uint8_t X[NW][kWaveMaxBlocks * kXRec];
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int task = blockIdx.x * NW + wave;
    if (task >= (W.rows / 64) * W.ks) return;          // no workgroup barrier below
    int g, s, c0, c1;
    tseg(W, task, g, s, c0, c1);
    const int b0 = c0 * CB, nblk = (c1 - c0) * CB;
    // this lane's pieces of the records: code halves lane and lane + 64, block lane's scale and sum
    uint4 q0 = make_uint4(0u, 0u, 0u, 0u), q1 = q0;
    float d = 0.f;
    int s8 = 0;
    const uint4* xq4 = reinterpret_cast<const uint4*>(xq + 32 * b0);
    if (lane < 2 * nblk) q0 = xq4[lane];
    if (lane + 64 < 2 * nblk) q1 = xq4[lane + 64];
    if (lane < nblk) { d = xd[b0 + lane]; s8 = xs8[b0 + lane]; }
    Tile cur, nxt;
    tile_load_cb<CB>(cur, tile_ptr(W, g, c0), lane);
    uint8_t* x = X[wave];
    if (lane < 2 * nblk) *reinterpret_cast<uint4*>(x + (lane >> 1) * kXRec + 16 * (lane & 1)) = q0;
    if (lane + 64 < 2 * nblk) *reinterpret_cast<uint4*>(x + ((lane + 64) >> 1) * kXRec + 16 * (lane & 1)) = q1;
    if (lane < nblk) {
        *reinterpret_cast<float*>(x + lane * kXRec + 32) = d;
        *reinterpret_cast<int32_t*>(x + lane * kXRec + 36) = s8;
    }
    wave_lds_sync();
    float seg = 0.f;
    for (int c = c0; c < c1; c++) {
        if (c + 1 < c1) tile_load_cb<CB>(nxt, tile_ptr(W, g, c + 1), lane);
        const float p = chunk_dot<CB>(cur, x, kXRec, (c - c0) * CB);
        seg = c == c0 ? p : __fadd_rn(seg, p);
        cur = nxt;
    }
    part[(size_t)s * W.rows + g * 64 + lane] = seg;
}

__global__ void k_seg_sum(const float* part, int rows, int ks, float* y) {
    const int r = blockIdx.x * blockDim.x + threadIdx.x;
    if (r >= rows) return;
    float v = part[r];
    for (int s = 1; s < ks; s++) v = __fadd_rn(v, part[(size_t)s * rows + r]);
    y[r] = v;
}

// isum[row][block] of the packed matrix, lane = row of a 64-row group
__global__ __launch_bounds__(64) void k_isums(PMat W, const int8_t* xq, int32_t* isum) {
    const int g = blockIdx.x, b = blockIdx.y, lane = threadIdx.x;
    const int c = W.cb == 8 ? b >> 3 : b >> 2, k = b & (W.cb - 1);      // cb is 8 or 4
    const uint8_t* t = tile_ptr(W, g, c);
    const uint4 w = *reinterpret_cast<const uint4*>(t + k * 1024 + lane * 16);
    const int4* xp = reinterpret_cast<const int4*>(xq + 32 * b);
    isum[(size_t)(g * 64 + lane) * W.nb + b] = dot_q4(w, xp[0], xp[1]);
}

// ------------------------------------------------------------------ standalone attention
// q[nh][hd] fp32 and an fp16 cache [nkv][ctx][hd]; two launches do the whole
// attention: k_attn_rec writes a record (o[hd], m, l) per head and 64-position chunk,
// k_attn_merge merges them in the canonical order. scratch: chunk records o
// [nh][nch][hd], m [nh][nch], l [nh][nch].
constexpr int kAttnMaxG = 8;        // query heads per kv head

// Standalone attention, part 1: the chunk records. A unit is (kv head, 64-position
// chunk). A workgroup takes S units per round (units SP .. SP + S - 1 for P = w,
// w + grid, ...) with W = ceil(G / H) compute waves per unit (H heads each) and one data
// wave. The data wave DMAs a round's K rows (coalesced, 1 KB of consecutive rows per
// instruction, into the step kernel's swizzled tile: kslot), V rows and the G query rows
// of each unit's kv head into one of two sets of LDS buffers, and issues the next
// round's DMA into the other set as soon as the compute waves start on this one, so
// every CU keeps loads in flight while it computes (all units' DMA issued at once, as a
// one-workgroup-per-unit launch does, lands everywhere at about the same time and
// leaves the compute after it). A compute wave runs its H heads together
// (attn_core_h: each head's arithmetic is attn_core's, so the records carry its bits).
// Records go to recs as o[h][chunk][hd], then m[h][chunk], then l[h][chunk] (the merge
// of 16 dims reads every m and l of a head: contiguous); the merge kernel reads them
// after this launch ends (the kernel boundary orders the plain stores before it).
template <int HD>
constexpr int attn_rec_buf() { return 2 * 64 * HD * 2 + kAttnMaxG * HD * 4; }
template <int H>
constexpr int attn_rec_wmax() { return (kAttnMaxG + H - 1) / H; }          // compute waves per unit, at most
template <int HD, int H, int S>
constexpr int attn_rec_lds() { return 2 * S * attn_rec_buf<HD>() + S * attn_rec_wmax<H>() * H * 64 * 4; }

// the DMA of unit u (kv head, chunk) into buffer B: K tile, V rows, the kv head's q rows
template <int HD>
__device__ __forceinline__ void attn_rec_issue(const float* q, const __half* kc, const __half* vc, int G, int nch, int L,
                                               int ctx, int u, uint8_t* B, int lane) {
    const int kvh = u / nch, t0 = (u - kvh * nch) * kAttnChunk, n = min(kAttnChunk, L - t0);
    dma_wave(q + (size_t)kvh * G * HD, B + 2 * 64 * HD * 2, G * HD * 4, lane);
    attn_issue_kv<HD>(kc + (size_t)kvh * ctx * HD, vc + (size_t)kvh * ctx * HD, t0, n, reinterpret_cast<uint4*>(B),
                      reinterpret_cast<__half*>(B + 64 * HD * 2), lane);
}

template <int HD, int H, int S>
__global__ __launch_bounds__(64 * (S * ((kAttnMaxG + H - 1) / H) + 1)) void k_attn_rec(const float* q, const __half* kc,
                                                                      const __half* vc, int nh, int nkv, int L, int ctx,
                                                                      float scale, float* recs) {
    constexpr int DPL = HD / 64, KV = 2 * 64 * HD * 2, BUF = attn_rec_buf<HD>();
    __shared__ __align__(16) uint8_t smem[attn_rec_lds<HD, H, S>()];
    const int lane = threadIdx.x & 63, wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int G = nh / nkv, W = (G + H - 1) / H, dw = S * W;          // wave dw moves the data
    const int nch = (L + kAttnChunk - 1) / kAttnChunk, units = nkv * nch;
    float* pls = reinterpret_cast<float*>(smem + 2 * S * BUF) + wave * H * 64;   // the wave's [H][64] probabilities
    int P = blockIdx.x;
    if (wave == dw) {
#pragma unroll
        for (int j = 0; j < S; j++)
            if (S * P + j < units) attn_rec_issue<HD>(q, kc, vc, G, nch, L, ctx, S * P + j, smem + j * BUF, lane);
    }
    for (int k = 0; S * P < units; k++, P += gridDim.x) {
        if (wave == dw) drain_vm();                     // round P is in buffer set k & 1
        __syncthreads();                                // (and the compute waves are done with the other set)
        if (wave == dw) {
            const int Pn = P + gridDim.x;
            uint8_t* Bn = smem + ((k + 1) & 1) * S * BUF;
#pragma unroll
            for (int j = 0; j < S; j++)
                if (S * Pn + j < units) attn_rec_issue<HD>(q, kc, vc, G, nch, L, ctx, S * Pn + j, Bn + j * BUF, lane);
            continue;
        }
        const int j = wave / W, u = S * P + j;
        const int hb = (wave - j * W) * H, hn = min(H, G - hb);
        if (u >= units) continue;
        const int kvh = u / nch, c = u - kvh * nch, n = min(kAttnChunk, L - c * kAttnChunk);
        const uint8_t* B = smem + ((k & 1) * S + j) * BUF;
        float m[H], ls[H], acc[H][DPL];
        attn_core_h<HD, H>(reinterpret_cast<const uint4*>(B), reinterpret_cast<const float*>(B + KV) + hb * HD, hn,
                           reinterpret_cast<const __half*>(B + 64 * HD * 2), n, scale, lane, pls, m, ls, acc);
#pragma unroll
        for (int h = 0; h < H; h++) {
            if (h < hn) {
                const size_t hc = (size_t)(kvh * G + hb + h) * nch + c;
#pragma unroll
                for (int e = 0; e < DPL; e++) recs[hc * HD + DPL * lane + e] = acc[h][e];
                if (lane == 0) {
                    recs[(size_t)nh * nch * HD + hc] = m[h];
                    recs[(size_t)nh * nch * (HD + 1) + hc] = ls[h];
                }
            }
        }
    }
}

// Standalone attention, part 2: the canonical merge (orc_attention_canon's order, the
// step's merge phase's) of one head's chunk records, for 32 of its dims (one 128-byte
// line of each o record) per workgroup. Wave w takes the split pairs (2g, 2g + 1) for
// g = w, w + 16, ... (all of a pair's loads in one batch): lane 16j + c (j < 2) loads m and l of chunk c of split 2g + j,
// takes M_s as the max over its 16 lanes and w_c = exp(m_c - M_s), both into LDS; lane
// 32j + d then runs acc_s (and, for d = 0, den_s) as fma chains in chunk order over o of
// dim d. The split results meet in LDS; wave 0 merges the splits the same way (lane s:
// w_s; lane d: the chains in split order) and divides (one split: acc / den directly).
constexpr int kAttnMaxSplits = 512;
constexpr int kMergeWaves = 16;
template <int HD>
__global__ __launch_bounds__(64 * kMergeWaves) void k_attn_merge(const float* recs, int nh, int L, float* out) {
    constexpr int SR = 34;
    __shared__ float sres[kAttnMaxSplits * SR];                        // [split][M, den, acc[32]]
    __shared__ float wls[kMergeWaves][2][2][16];                        // per wave: [split j][w | l][chunk]
    const int h = blockIdx.x / (HD / 32), d0 = (blockIdx.x - h * (HD / 32)) * 32;
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int nch = (L + kAttnChunk - 1) / kAttnChunk, nsp = (nch + kAttnSplit - 1) / kAttnSplit;
    const float* ro = recs + (size_t)h * nch * HD;
    const float* rm = recs + (size_t)nh * nch * HD + (size_t)h * nch;
    const float* rl = rm + (size_t)nh * nch;
    for (int g = wave; 2 * g < nsp; g += kMergeWaves) {
        // the pair's o values (lane 32j + d) and chunk (m, l) (lane 16j + c) in one batch
        const int j = lane >> 5, d = lane & 31, sp = 2 * g + j;
        const int c0 = sp * kAttnSplit, n = sp < nsp ? min(kAttnSplit, nch - c0) : 1;
        float oo[kAttnSplit];
#pragma unroll
        for (int i = 0; i < kAttnSplit; i++) oo[i] = sp < nsp ? ro[(size_t)(c0 + min(i, n - 1)) * HD + d0 + d] : 0.f;
        const int wj = (lane >> 4) & 1, wc = lane & 15, wsp = 2 * g + wj, cc = wsp * kAttnSplit + wc;
        const bool ok = lane < 32 && wsp < nsp && cc < nch;
        const float m = ok ? rm[cc] : -__builtin_inff();
        const float l = ok ? rl[cc] : 0.f;
        // chunk weights: M_s = max over the split's 16 lanes, w_c = exp(m_c - M_s)
        float M = fmaxf(m, dppf<kDppRor8>(m));
        M = fmaxf(M, dppf<kDppRor4>(M));
        M = fmaxf(M, dppf<kDppXor2>(M));
        M = fmaxf(M, dppf<kDppXor1>(M));
        if (lane < 32) {
            wls[wave][wj][0][wc] = ok ? mi_expf(__fsub_rn(m, M)) : 0.f;
            wls[wave][wj][1][wc] = l;
            if (wc == 0 && wsp < nsp) sres[wsp * SR] = M;
        }
        wave_lds_sync();
        if (sp < nsp) {
            float den = 0.f, acc = 0.f;
#pragma unroll
            for (int i = 0; i < kAttnSplit; i++) {
                if (i < n) {
                    const float w = wls[wave][j][0][i];
                    den = __fmaf_rn(wls[wave][j][1][i], w, den);
                    acc = __fmaf_rn(oo[i], w, acc);
                }
            }
            float* sr = sres + sp * SR;
            if (d == 0) sr[1] = den;
            sr[2 + d] = acc;
        }
        wave_lds_sync();                                                // wls is reused by the wave's next pair
    }
    __syncthreads();
    if (wave != 0) return;
    const int d = lane & 31;
    float den, acc;
    if (nsp == 1) {
        den = sres[1];
        acc = sres[2 + d];
    } else {
        // M over the splits, then lane s computes w_s = exp(M_s - M) (splits s, s + 64, ...
        // into sres's M column), then the lanes run the chains in split order
        float M = -__builtin_inff();
        for (int sp = lane; sp < nsp; sp += 64) M = fmaxf(M, sres[sp * SR]);
        M = wave_max(M);
        for (int sp = lane; sp < nsp; sp += 64) sres[sp * SR] = mi_expf(__fsub_rn(sres[sp * SR], M));
        wave_lds_sync();
        den = 0.f;
        acc = 0.f;
        int sp = 0;
        for (; sp + 4 <= nsp; sp += 4) {
            float w[4], dn[4], ac[4];
#pragma unroll
            for (int i = 0; i < 4; i++) {
                w[i] = sres[(sp + i) * SR];
                dn[i] = sres[(sp + i) * SR + 1];
                ac[i] = sres[(sp + i) * SR + 2 + d];
            }
#pragma unroll
            for (int i = 0; i < 4; i++) {
                den = __fmaf_rn(dn[i], w[i], den);
                acc = __fmaf_rn(ac[i], w[i], acc);
            }
        }
        for (; sp < nsp; sp++) {
            den = __fmaf_rn(sres[sp * SR + 1], sres[sp * SR], den);
            acc = __fmaf_rn(sres[sp * SR + 2 + d], sres[sp * SR], acc);
        }
    }
    if (lane < 32) out[(size_t)h * HD + d0 + lane] = __fdiv_rn(acc, den);
}

// ------------------------------------------------------------------ standalone attention on MFMA
// The chunk records of k_attn_rec (same units, same record layout, merged by the same
// k_attn_merge), with a unit's scores and p.v as fp16 MFMA contractions instead of one
// fp32 fma chain per head and lane. Per unit (kv head, 64-position chunk):
//   S[pos][head] = K[pos][:] . q[head][:]   v_mfma_f32_16x16x32_f16, A = K rows (as
//                                           stored, fp16, exact), B = q split in two
//                                           fp16 parts q' = hi + lo (q' = q * 2^kq per
//                                           kv head, so the parts stay in fp16 range)
//   O^T[dim][head] = sum_pos V[pos][dim] p[head][pos]   A = V gathered from LDS, B = p
//                                           split hi + lo the same way
// The hi/lo split keeps ~22 significant bits of q and p, the products are exact and the
// MFMA accumulates in fp32, so a record agrees with attn_core's to ~1e-6 relative, but
// not bit for bit (the summation order inside an MFMA is the hardware's). The G <= 8
// query heads of a kv head are the 16 MFMA columns (8 used). Lane l = 16g + c owns
// column c (head c) and, in the D layout, rows 4g .. 4g + 3 of each tile: the scores of
// positions 16mt + 4g + r, which are exactly the p values its B operand of the p.v
// product needs (position 32ks + 16(e/4) + 4g + e%4 for element e of K step ks), so p
// never leaves the registers; only V is gathered (8 halves per operand).
// A workgroup is two compute waves and one data wave with one unit buffer (four
// workgroups per CU at hd 128): the data wave DMAs the unit's K tile, then its V rows;
// the compute waves meanwhile load q and build its operands, and compute wave w takes
// positions 32w .. 32w + 31 (scores, its half of the chunk softmax, its half of p.v).
// The maxima and sums of the two halves meet in LDS, and each wave adds the other's
// partial tiles for half of the record. The next unit's DMA waits for the compute; the
// CU's other workgroups fill the gap. The chunk probabilities use the hardware exp2
// (v_exp_f32, ~1 ulp) rather than mi_expf: the records are not bit-canonical anyway,
// and the polynomial was a third of a wave's instructions.
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
constexpr int kVPad = 32;          // bytes after each 1-KB block of V rows (conflict-free gathers)
template <int HD>
constexpr int amx_vbytes() { return (64 * HD * 2 / 1024) * (1024 + kVPad); }
template <int HD>
constexpr int amx_buf() { return 64 * HD * 2 + amx_vbytes<HD>(); }
template <int HD>
constexpr int amx_lds() { return amx_buf<HD>() + 64 * 4; }
// s_waitcnt with vmcnt(n) and no wait on the other counters
constexpr int waitcnt_vm(int n) { return 0x0F70 | (n & 15) | (((n >> 4) & 3) << 14); }

// the DMA of unit u into buffer B: K rows (swizzled tile, kslot), V rows in 1-KB blocks
// of RPI rows each followed by kVPad bytes; rows past n repeat row n-1 (finite: their
// p is 0)
template <int HD>
__device__ __forceinline__ void amx_issue(const __half* kc, const __half* vc, int nch, int L, int ctx, int u,
                                          uint8_t* B, int lane) {
    constexpr int NV = HD / 8, RPI = 64 / NV;
    const int kvh = u / nch, t0 = (u - kvh * nch) * kAttnChunk, n = min(kAttnChunk, L - t0);
    const __half* vr = vc + ((size_t)kvh * ctx + t0) * HD;
    const __half* kr = kc + ((size_t)kvh * ctx + t0) * HD;
    const int u8 = lane % NV;
#pragma unroll
    for (int i = 0; i < NV; i++) {         // K load i: tile slots 64i .. 64i + 63 (rows RPI*i ..)
        const int t = i * RPI + lane / NV;
        __builtin_amdgcn_global_load_lds(kr + (size_t)min(t, n - 1) * HD + 8 * (u8 ^ kswz<HD>(t)),
                                         (lds_ptr)(B + i * 1024), 16, 0, 0);
    }
    const int r = lane / NV, col = (lane % NV) * 8;
#pragma unroll
    for (int i = 0; i < 64 / RPI; i++)
        __builtin_amdgcn_global_load_lds(vr + (size_t)min(i * RPI + r, n - 1) * HD + col,
                                         (lds_ptr)(B + 64 * HD * 2 + i * (1024 + kVPad)), 16, 0, 0);
}

__device__ __forceinline__ void split_f16(float x, _Float16& hi, _Float16& lo) {
    hi = (_Float16)x;                                   // round to nearest even
    lo = (_Float16)__fsub_rn(x, (float)hi);             // the remainder is exact in fp32
}

// both waves' halves of a lane value combined: max or sum over lanes l, l ^ 16, l ^ 32
// and l ^ 48 (the lanes of one MFMA column)
__device__ __forceinline__ float col_max(float v) {
    float a, b;
    pair16(v, a, b);
    v = fmaxf(a, b);
    pair32(v, a, b);
    return fmaxf(a, b);
}
__device__ __forceinline__ float col_sum(float v) {
    float a, b;
    pair16(v, a, b);
    v = __fadd_rn(a, b);
    pair32(v, a, b);
    return __fadd_rn(a, b);
}

template <int HD>
__global__ __launch_bounds__(192) __attribute__((amdgpu_waves_per_eu(3))) void k_attn_mx(const float* q, const __half* kc, const __half* vc, int nh, int nkv,
                                                 int L, int ctx, float scale, float* recs) {
    constexpr int KS = HD / 32, NT = HD / 16, NV = HD / 8, RPI = 64 / NV, VB = 1024 + kVPad, BUF = amx_buf<HD>();
    __shared__ __align__(16) uint8_t smem[amx_lds<HD>()];
    const int lane = threadIdx.x & 63, w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);    // wave 2 moves data
    const int G = nh / nkv, nch = (L + kAttnChunk - 1) / kAttnChunk, units = nkv * nch;
    const int col = lane & 15, g = lane >> 4;
    float* xch = reinterpret_cast<float*>(smem + BUF);              // [m w0 | m w1 | l w0 | l w1][16]
    int P = blockIdx.x;
    if (w == 2) amx_issue<HD>(kc, vc, nch, L, ctx, P, smem, lane);
    // lane's part of a V gather address: row 4g + (e & 3) of a group of rows starting at a
    // multiple of 16 lies in block (row / RPI), at (row % RPI) rows into it
    const int vlane = (RPI == 4 ? g * VB : (g >> 1) * VB + (g & 1) * 4 * HD * 2) + 2 * col;
    for (int k = 0; P < units; k++, P += gridDim.x) {
        if (k > 0) {
            __syncthreads();                            // the compute waves are done with the buffer
            if (w == 2) amx_issue<HD>(kc, vc, nch, L, ctx, P, smem, lane);
        }
        const int kvh = P / nch, c = P - kvh * nch, n = min(kAttnChunk, L - c * kAttnChunk);
        // the kv head's q operands, built while the unit's DMA is in flight: lane (g,
        // col) holds head col, dims 32ks + 8g .. + 7, scaled by 2^kq (the largest |q| of
        // the G heads just under 2^15) and split hi + lo
        f16x8 qh[KS], ql[KS];
        float sc = 0.f;
        if (w < 2) {
            float qv[KS][8];
#pragma unroll
            for (int ks = 0; ks < KS; ks++) {
                float4 a = make_float4(0.f, 0.f, 0.f, 0.f), b = a;
                if (col < G) {
                    const float* qr = q + (size_t)(kvh * G + col) * HD + 32 * ks + 8 * g;
                    a = ld4(qr);
                    b = ld4(qr + 4);
                }
                qv[ks][0] = a.x; qv[ks][1] = a.y; qv[ks][2] = a.z; qv[ks][3] = a.w;
                qv[ks][4] = b.x; qv[ks][5] = b.y; qv[ks][6] = b.z; qv[ks][7] = b.w;
            }
            float mx = 0.f;
#pragma unroll
            for (int ks = 0; ks < KS; ks++)
#pragma unroll
                for (int e = 0; e < 8; e++) mx = fmaxf(mx, fabsf(qv[ks][e]));
            mx = wave_max(mx);
            int ex = 0;
            (void)frexpf(mx, &ex);
            const int kq = mx > 0.f ? min(max(15 - ex, -100), 100) : 0;
            sc = ldexpf(scale, -kq);
#pragma unroll
            for (int ks = 0; ks < KS; ks++)
#pragma unroll
                for (int e = 0; e < 8; e++) {
                    _Float16 hi, lo;
                    split_f16(ldexpf(qv[ks][e], kq), hi, lo);
                    qh[ks][e] = hi;
                    ql[ks][e] = lo;
                }
        }
        // K is DMA'd before V: the scores start once K has landed, and V is waited for
        // at the first exchange
        if (w == 2) __builtin_amdgcn_s_waitcnt(waitcnt_vm(NV));
        __syncthreads();                                // unit P's K tile is in LDS
        if (w == 2) {
            drain_vm();
            __syncthreads();                            // (A) V too
            __syncthreads();                            // (B)
            __syncthreads();                            // (C)
            continue;
        }
        // scores of this wave's positions 32w .. 32w + 31: tiles mt = 2w + j
        const uint4* kls = reinterpret_cast<const uint4*>(smem);
        f32x4 S[2] = {f32x4{0.f, 0.f, 0.f, 0.f}, f32x4{0.f, 0.f, 0.f, 0.f}};
#pragma unroll
        for (int ks = 0; ks < KS; ks++)
#pragma unroll
            for (int j = 0; j < 2; j++) {
                const f16x8 a = __builtin_bit_cast(f16x8, kls[kslot<HD>(16 * (2 * w + j) + col, 4 * ks + g)]);
                S[j] = __builtin_amdgcn_mfma_f32_16x16x32_f16(a, qh[ks], S[j], 0, 0, 0);
                S[j] = __builtin_amdgcn_mfma_f32_16x16x32_f16(a, ql[ks], S[j], 0, 0, 0);
            }
        // chunk softmax per head (column) over both waves' positions
        float p[2][4];
        float m = -__builtin_inff();
#pragma unroll
        for (int j = 0; j < 2; j++)
#pragma unroll
            for (int r = 0; r < 4; r++) {
                const bool ok = col < G && 32 * w + 16 * j + 4 * g + r < n;
                p[j][r] = ok ? __fmul_rn(S[j][r], sc) : -__builtin_inff();
                m = fmaxf(m, p[j][r]);
            }
        m = col_max(m);
        if (g == 0) xch[16 * w + col] = m;
        __syncthreads();                                // (A) both maxima and V; K is no longer read
        m = fmaxf(xch[col], xch[16 + col]);
        float ls = 0.f;
#pragma unroll
        for (int j = 0; j < 2; j++)
#pragma unroll
            for (int r = 0; r < 4; r++) {
                const bool ok = col < G && 32 * w + 16 * j + 4 * g + r < n;
                p[j][r] = ok ? __builtin_amdgcn_exp2f(__fmul_rn(__fsub_rn(p[j][r], m), 0x1.715476p+0f)) : 0.f;
                ls = __fadd_rn(ls, p[j][r]);
            }
        ls = col_sum(ls);
        if (g == 0) xch[32 + 16 * w + col] = ls;
        f16x8 ph, pl;
#pragma unroll
        for (int e = 0; e < 8; e++) {
            _Float16 hi, lo;
            split_f16(p[e / 4][e & 3], hi, lo);
            ph[e] = hi;
            pl[e] = lo;
        }
        // p.v over this wave's 32 positions (K step w of the unit); tile nt = dims
        // 16nt .. 16nt + 15
        const uint8_t* vb = smem + 64 * HD * 2 + vlane;
        f32x4 O[NT];
#pragma unroll
        for (int nt = 0; nt < NT; nt++) {
            f16x8 a;
#pragma unroll
            for (int e = 0; e < 8; e++) {
                const int c0 = 32 * w + 16 * (e / 4) + (e & 3);             // row of lane group 0
                a[e] = *reinterpret_cast<const _Float16*>(vb + (c0 / RPI) * VB + (c0 % 4) * HD * 2 + 32 * nt);
            }
            O[nt] = __builtin_amdgcn_mfma_f32_16x16x32_f16(a, ph, f32x4{0.f, 0.f, 0.f, 0.f}, 0, 0, 0);
            O[nt] = __builtin_amdgcn_mfma_f32_16x16x32_f16(a, pl, O[nt], 0, 0, 0);
        }
        // wave w finishes tiles [w NT/2, (w + 1) NT/2): the other half of its partials
        // go through the (free) K tile
        float4* xo = reinterpret_cast<float4*>(smem);
#pragma unroll
        for (int i = 0; i < NT / 2; i++) {
            const f32x4 o = O[(1 - w) * (NT / 2) + i];
            xo[(w * (NT / 2) + i) * 64 + lane] = make_float4(o[0], o[1], o[2], o[3]);
        }
        __syncthreads();                                // (B) the sums and the partials
        ls = __fadd_rn(xch[32 + col], xch[48 + col]);
        if (col < G) {
            const size_t hc = (size_t)(kvh * G + col) * nch + c;
#pragma unroll
            for (int i = 0; i < NT / 2; i++) {
                const int nt = w * (NT / 2) + i;
                const float4 o = xo[((1 - w) * (NT / 2) + i) * 64 + lane];
                const f32x4 mine = O[nt];
                // wave 0's part + wave 1's part, the same order for both halves
                const float4 s = w == 0 ? make_float4(__fadd_rn(mine[0], o.x), __fadd_rn(mine[1], o.y),
                                                      __fadd_rn(mine[2], o.z), __fadd_rn(mine[3], o.w))
                                        : make_float4(__fadd_rn(o.x, mine[0]), __fadd_rn(o.y, mine[1]),
                                                      __fadd_rn(o.z, mine[2]), __fadd_rn(o.w, mine[3]));
                st4(recs + hc * HD + 16 * nt + 4 * g, s);
            }
            if (w == 0 && g == 0) {
                recs[(size_t)nh * nch * HD + hc] = m;
                recs[(size_t)nh * nch * (HD + 1) + hc] = ls;
            }
        }
        __syncthreads();                                // (C) the exchange area is read
    }
}

__global__ __launch_bounds__(kThreads) void k_stream(const u32x4* __restrict__ p, size_t n4, uint32_t* sink) {
    const size_t nth = (size_t)gridDim.x * blockDim.x;
    size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    uint32_t acc = 0;
    constexpr int U = 4;
    for (; i + (U - 1) * nth < n4; i += U * nth) {
        u32x4 v[U];
#pragma unroll
        for (int u = 0; u < U; u++) v[u] = __builtin_nontemporal_load(p + i + u * nth);
#pragma unroll
        for (int u = 0; u < U; u++) acc ^= v[u].x ^ v[u].y ^ v[u].z ^ v[u].w;
    }
    for (; i < n4; i += nth) { const u32x4 v = p[i]; acc ^= v.x ^ v.y ^ v.z ^ v.w; }
    if (acc == 0x9E3779B9u) sink[threadIdx.x] = acc;   // never true in practice; keeps the loads
}

// ------------------------------------------------------------------ host side
#define LAUNCH(kern, grid, block, stream, ...) hipLaunchKernelGGL(kern, dim3(grid), dim3(block), 0, stream, __VA_ARGS__)

bool kernels_support(int G, int HD) { return (HD == 64 || HD == 128) && G >= 1 && G <= kPWaves; }
// 64-position chunks the merge phase holds (its split results live in the step's LDS union)
int kernels_max_ctx_chunks(int HD) {
    const int ub = HD == 128 ? union_bytes<128>() : union_bytes<64>();
    return min(kCombMaxSplits, (ub / 4 - 8 * kCombWaveFloats) / kCombSR) * kAttnSplit;
}
int attn_record_floats(int HD) { return HD + 32; }

template <class F>
static void with_hd(int HD, F f) {
    if (HD == 64) f(std::integral_constant<int, 64>());
    else f(std::integral_constant<int, 128>());
}

// Reduction plan: chunk size by row length (8 blocks, 4 when the block count is not
// a multiple of 8); one K segment per row except the down matrix, whose rows are
// split into as many segments as leave one per workgroup of a 256-CU device (more
// segments = shorter ones, and the down phase is a one-round latency chain; past one
// per workgroup some workgroups take two), within what the phase prologue stages (the
// norm weights, the h vector and ks partials in kCtlBytes). The plan depends only on
// the shape, so the float order is device-independent.
constexpr int kPlanWgs = 256;
bool kernels_plan(int E, int FF, int cb[5], int ks[5]) {
    const int nbE = E / 32, nbF = FF / 32;
    const int cbE = nbE % 8 == 0 ? 8 : 4, cbF = nbF % 8 == 0 ? 8 : 4;
    cb[0] = cb[1] = cb[2] = cb[4] = cbE;
    cb[3] = cbF;
    ks[0] = ks[1] = ks[2] = ks[4] = 1;
    const int ncF = nbF / cbF, cap = std::min(kMaxKsRes, kCtlBytes / (4 * E) - 2);
    if (cap < 1) return false;
    ks[3] = std::max(1, std::min(std::min(cap, ncF), kPlanWgs / (E / 64)));
    if (nbE / cbE > kMaxKsRes) return false;      // the per-phase multi-token O's partials (one per chunk)
    return (FF / 32) * kActRec <= kCtlBytes;
}

// chunk sums a workgroup stages for one matrix (rows x nb blocks, plan cb/ks) over nwg workgroups
int kernels_tiles_per_wg(int rows, int nb, int cb, int ks, int nwg) {
    const int nseg = (rows / 64) * ks, nc = nb / cb;
    return ((nseg + nwg - 1) / nwg) * ((nc + ks - 1) / ks);
}
int kernels_max_tiles_per_wg() { return kPartTiles; }

void launch_phase(const DModel& M, const DModel* dM, int nwg, int phase, int l, int pos, int gen, hipStream_t s) {
    const int nch = (pos + 1 + kAttnChunk - 1) / kAttnChunk;
    switch (phase) {
        case 0: LAUNCH(k_qkv, nwg, kPThreads, s, dM, l, pos); break;
        case 1: with_hd(M.HD, [&](auto hd) { LAUNCH((k_attn<decltype(hd)::value>), nwg, kPThreads, s, dM, l, pos); }); break;
        case 2:
            if (nch > kInlineComb)
                with_hd(M.HD, [&](auto hd) { LAUNCH((k_attn_comb<decltype(hd)::value>), nwg, kPThreads, s, dM, l, pos); });
            break;
        case 3: LAUNCH(k_o, nwg, kPThreads, s, dM, l, pos); break;
        case 4: LAUNCH(k_gu, nwg, kPThreads, s, dM, l); break;
        case 5: LAUNCH(k_down, nwg, kPThreads, s, dM, l); break;
        case 6: LAUNCH(k_lm, nwg, kPThreads, s, dM); break;
        default: LAUNCH(k_argmax, 1, 64, s, dM, nwg, pos, gen); break;
    }
}

void launch_step_phases(const DModel& M, const DModel* dM, int nwg, int pos, int gen, hipStream_t s) {
    for (int l = 0; l < M.NL; l++)
        for (int ph = 0; ph < 6; ph++) launch_phase(M, dM, nwg, ph, l, pos, gen, s);
    launch_phase(M, dM, nwg, 6, 0, pos, gen, s);
    launch_phase(M, dM, nwg, 7, 0, pos, gen, s);
}

hipError_t launch_step_persistent(const DModel& M, const DModel* dM, int nwg, int pos, int gen, bool coop,
                                  hipStream_t s) {
    hipError_t err = hipSuccess;
    with_hd(M.HD, [&](auto hd) {
        const DModel* m = dM;
        void* args[] = {&m, &pos, &gen};
        // the profiling instance only when the model description carries a stamp buffer
        const void* f = M.prof ? reinterpret_cast<const void*>(&k_step<decltype(hd)::value, true>)
                               : reinterpret_cast<const void*>(&k_step<decltype(hd)::value, false>);
        err = coop ? hipLaunchCooperativeKernel(f, dim3(nwg), dim3(kPThreads), args, 0, s)
                   : hipLaunchKernel(f, dim3(nwg), dim3(kPThreads), args, 0, s);
    });
    return err;
}

void launch_step_multi(const DModel& M, const DModel* dM, int nwg, int T, hipStream_t s) {
    const int ncomb = (T * M.NH + 3) / 4;
    for (int l = 0; l < M.NL; l++) {
        LAUNCH(kT_in, T, kPThreads, s, dM, l, (int)PH_QKV);
        LAUNCH(kT_qkv, nwg, kPThreads, s, dM, l, T);
        with_hd(M.HD, [&](auto hd) {
            LAUNCH((kT_attn<decltype(hd)::value>), nwg, kPThreads, s, dM, l, T);
            LAUNCH((kT_comb<decltype(hd)::value>), ncomb, 256, s, dM, l, T);
        });
        LAUNCH(kT_o, nwg, kPThreads, s, dM, l, T);
        LAUNCH(kT_in, T, kPThreads, s, dM, l, (int)PH_GU);
        LAUNCH(kT_gu, nwg, kPThreads, s, dM, l, T);
        LAUNCH(kT_down, nwg, kPThreads, s, dM, l, T);
    }
    LAUNCH(kT_in, T, kPThreads, s, dM, M.NL - 1, (int)PH_LM);
    LAUNCH(kT_lm, nwg, kPThreads, s, dM, T);
    LAUNCH(kT_argmax, 1, kPThreads, s, dM, nwg, T);
}
hipError_t launch_step_multi_persistent(const DModel& M, const DModel* dM, int nwg, int T, bool coop, hipStream_t s) {
    hipError_t err = hipSuccess;
    with_hd(M.HD, [&](auto hd) {
        const DModel* m = dM;
        void* args[] = {&m, &T};
        const void* f = reinterpret_cast<const void*>(&kT_step<decltype(hd)::value, false>);
        err = coop ? hipLaunchCooperativeKernel(f, dim3(nwg), dim3(kPThreads), args, 0, s)
                   : hipLaunchKernel(f, dim3(nwg), dim3(kPThreads), args, 0, s);
    });
    return err;
}
hipError_t launch_spec_step(const DModel& M, const DModel* dM, int nwg, bool coop, hipStream_t s) {
    hipError_t err = hipSuccess;
    with_hd(M.HD, [&](auto hd) {
        const DModel* m = dM;
        int T = 0;
        void* args[] = {&m, &T};
        const void* f = reinterpret_cast<const void*>(&kT_step<decltype(hd)::value, true>);
        err = coop ? hipLaunchCooperativeKernel(f, dim3(nwg), dim3(kPThreads), args, 0, s)
                   : hipLaunchKernel(f, dim3(nwg), dim3(kPThreads), args, 0, s);
    });
    return err;
}
int multi_persistent_max_grid(int HD) {
    int per_cu = 0;
    with_hd(HD, [&](auto hd) {
        if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, reinterpret_cast<const void*>(&kT_step<decltype(hd)::value, true>),
                                                         kPThreads, 0) != hipSuccess)
            per_cu = 0;
    });
    return per_cu;
}
int kernels_max_tokens() { return kMaxT; }
int kernels_max_chunks_multi() { return kTChunks; }

hipError_t launch_barriers(uint32_t* bar, int32_t* err, int nwg, int n, hipStream_t s) {
    hipError_t e = hipMemsetAsync(bar, 0, sizeof(uint32_t) * kBarWords, s);
    if (e != hipSuccess) return e;
    void* args[] = {&bar, &err, &n};
    return hipLaunchCooperativeKernel(reinterpret_cast<const void*>(&k_barriers), dim3(nwg), dim3(kPThreads), args, 0, s);
}
int barrier_words() { return kBarWords; }

int persistent_max_grid(int G, int HD) {
    (void)G;
    int per_cu = 0;
    with_hd(HD, [&](auto hd) {
        if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, reinterpret_cast<const void*>(&k_step<decltype(hd)::value, false>),
                                                         kPThreads, 0) != hipSuccess)
            per_cu = 0;
    });
    return per_cu;
}

void launch_quant(const float* x, int n, int8_t* xq, float* xd, int32_t* xs8, hipStream_t s) {
    LAUNCH(k_quant, (n + kThreads - 1) / kThreads, kThreads, s, x, n, xq, xd, xs8);
}
// Kernel choice by segment count and length (sweep on the box, config-1 shapes, µs per
// launch from graph replay; every choice gives the same bits):
// * one-chunk segments (qkv, o, gate/up at ks 6): one wave per segment, 1-wave workgroups
//   (gate/up 5.38 -> 4.89, qkv 3.12 -> 2.88);
// * many short segments (lm_head at ks 2: 4748 segments of 3 chunks): the same kernel, 4
//   waves per workgroup (22.0 vs 24.4 for the dense loop at ks 1);
// * few segments of several chunks (down): a workgroup per segment, a wave per chunk, so
//   that all of a segment's loads go out at once (the wave kernel walks them in turn).
void launch_gemv(const PMat& W, const int8_t* xq, const float* xd, const int32_t* xs8, float* part, float* y,
                 int n_cu, hipStream_t s) {
    const int tasks = (W.rows / 64) * W.ks;
    const int maxc = (W.nc + W.ks - 1) / W.ks;          // chunks of the longest segment
    const bool wave1 = maxc == 1, wave4 = tasks > kGemvWgsPerCu * n_cu && maxc * W.cb <= kWaveMaxBlocks;
    if (wave1 || wave4) {
        auto go = [&](auto cbv) {
            constexpr int CB = decltype(cbv)::value;
            if (wave1) LAUNCH((k_gemv_wave<1, CB>), tasks, 64, s, W, xq, xd, xs8, part);
            else LAUNCH((k_gemv_wave<4, CB>), (tasks + 3) / 4, 256, s, W, xq, xd, xs8, part);
        };
        if (W.cb == 8) go(std::integral_constant<int, 8>());
        else go(std::integral_constant<int, 4>());
    } else if (tasks <= kGemvWgsPerCu * n_cu && maxc >= 2 && maxc <= kSegMaxChunks) {
        switch (std::min(maxc, 8)) {
        case 2: LAUNCH(k_gemv_seg<2>, tasks, 128, s, W, xq, xd, xs8, part); break;
        case 3: LAUNCH(k_gemv_seg<3>, tasks, 192, s, W, xq, xd, xs8, part); break;
        case 4: LAUNCH(k_gemv_seg<4>, tasks, 256, s, W, xq, xd, xs8, part); break;
        case 5: LAUNCH(k_gemv_seg<5>, tasks, 320, s, W, xq, xd, xs8, part); break;
        case 6: LAUNCH(k_gemv_seg<6>, tasks, 384, s, W, xq, xd, xs8, part); break;
        case 7: LAUNCH(k_gemv_seg<7>, tasks, 448, s, W, xq, xd, xs8, part); break;
        default: LAUNCH(k_gemv_seg<8>, tasks, 512, s, W, xq, xd, xs8, part); break;
        }
    } else if (tasks <= kGemvWgsPerCu * n_cu)
        LAUNCH(k_gemv<true>, tasks, kThreads, s, W, xq, xd, xs8, part);
    else
        LAUNCH(k_gemv<false>, std::min(4 * n_cu, (tasks + kWaves - 1) / kWaves), kThreads, s, W, xq, xd, xs8, part);
    if (y) LAUNCH(k_seg_sum, (W.rows + 255) / 256, 256, s, part, W.rows, W.ks, y);
}
void launch_isums(const PMat& W, const int8_t* xq, int32_t* isum, hipStream_t s) {
    hipLaunchKernelGGL(k_isums, dim3(W.rows / 64, W.nb), dim3(64), 0, s, W, xq, isum);
}
size_t attn_scratch_floats(int nh, int hd, int L) {
    const int nch = (L + kAttnChunk - 1) / kAttnChunk;
    return (size_t)nh * nch * (hd + 2);
}
static int device_cus() {
    static int n_cu = 0;
    if (!n_cu) {
        int dev = 0, n = 0;
        if (hipGetDevice(&dev) != hipSuccess || hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || n < 1)
            n = 256;
        n_cu = n;
    }
    return n_cu;
}
template <int HD, int H, int S>
static void launch_attn_rec(const float* q, const __half* kc, const __half* vc, int nh, int nkv, int L, int ctx,
                            float scale, float* recs, hipStream_t s) {
    const int G = nh / nkv, units = nkv * ((L + kAttnChunk - 1) / kAttnChunk);
    const int per_cu = max(1, (160 * 1024) / attn_rec_lds<HD, H, S>());
    const int grid = min((units + S - 1) / S, device_cus() * per_cu);
    LAUNCH((k_attn_rec<HD, H, S>), grid, 64 * (S * ((G + H - 1) / H) + 1), s, q, kc, vc, nh, nkv, L, ctx, scale, recs);
}
bool launch_attn_decode(const float* q, const __half* kc, const __half* vc, int nh, int nkv, int hd, int L, int ctx,
                        float scale, float* scratch, float* out, hipStream_t s) {
    if (nh % nkv || !kernels_support(nh / nkv, hd) || nh / nkv > kAttnMaxG || L < 1) return false;
    const int nch = (L + kAttnChunk - 1) / kAttnChunk, nsp = (nch + kAttnSplit - 1) / kAttnSplit;
    if (nsp > kAttnMaxSplits) return false;
    with_hd(hd, [&](auto h) {
        constexpr int HD = decltype(h)::value;
        // one head per compute wave, one unit per round (two workgroups per CU at hd 128):
        // the fastest of H = 1..3, S = 1..2 at L = 512..32768 on the box
        launch_attn_rec<HD, 1, 1>(q, kc, vc, nh, nkv, L, ctx, scale, scratch, s);
        LAUNCH((k_attn_merge<HD>), nh * (HD / 32), 64 * kMergeWaves, s, scratch, nh, L, out);
    });
    return true;
}
// the same two-launch attention with the chunk records from k_attn_mx (MFMA scores and
// p.v): one compute and one data wave per workgroup, as many workgroups per CU as the
// double-buffered LDS allows (two at hd 128)
bool launch_attn_decode_mfma(const float* q, const __half* kc, const __half* vc, int nh, int nkv, int hd, int L,
                             int ctx, float scale, float* scratch, float* out, hipStream_t s) {
    if (nh % nkv || !kernels_support(nh / nkv, hd) || nh / nkv > kAttnMaxG || L < 1) return false;
    const int nch = (L + kAttnChunk - 1) / kAttnChunk, nsp = (nch + kAttnSplit - 1) / kAttnSplit;
    if (nsp > kAttnMaxSplits) return false;
    with_hd(hd, [&](auto h) {
        constexpr int HD = decltype(h)::value;
        const int units = nkv * nch, per_cu = max(1, (160 * 1024) / amx_lds<HD>());
        const int grid = min(units, device_cus() * per_cu);
        LAUNCH((k_attn_mx<HD>), grid, 192, s, q, kc, vc, nh, nkv, L, ctx, scale, scratch);
        LAUNCH((k_attn_merge<HD>), nh * (HD / 32), 64 * kMergeWaves, s, scratch, nh, L, out);
    });
    return true;
}
// ------------------------------------------------------------------ allocation-free attention
// Scratch of mi_attn_decode_noalloc: a file-scope device array (each GPU the library
// runs on holds its own copy until the process ends), laid out as the workspace of
// launch_attn_decode: the chunk records, every one written before it is read in each
// call, so nothing needs clearing. Host code never passes the array's name to a kernel
// (on the host it is a stand-in, not a device address): the per-device address comes
// from hipGetSymbolAddress at the first call on each device. Calls on one device share
// the array, so calls that overlap on one GPU race.
static __device__ __align__(256) float scratch[kNoAllocScratchFloats];

namespace {
constexpr int kMaxDevices = 64;
std::mutex g_scratch_mu;
float* g_scratch_ptr[kMaxDevices] = {};
}  // namespace

// the device address of the current device's scratch array (looked up at the first
// call on a device)
hipError_t noalloc_scratch(hipStream_t s, float** out) {
    (void)s;
    int dev = 0;
    hipError_t e = hipGetDevice(&dev);
    if (e != hipSuccess) return e;
    if (dev < 0 || dev >= kMaxDevices) return hipErrorInvalidDevice;
    std::lock_guard<std::mutex> lk(g_scratch_mu);
    if (!g_scratch_ptr[dev]) {
        void* p = nullptr;
        e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
        if (e != hipSuccess) return e;
        g_scratch_ptr[dev] = static_cast<float*>(p);
    }
    *out = g_scratch_ptr[dev];
    return hipSuccess;
}

void launch_stream(const void* buf, size_t bytes, uint32_t* sink, int n_cu, hipStream_t s) {
    LAUNCH(k_stream, 8 * n_cu, kThreads, s, reinterpret_cast<const u32x4*>(buf), bytes / 16, sink);
}

}  // namespace mi
