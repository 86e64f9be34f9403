/* q8act.c -- the GPU engine's numerics restated as plain C (ORC_MODE_Q8ACT).
 * TEST INFRASTRUCTURE ONLY (see oracle.h). Compiled with -ffp-contract=off:
 * every fused multiply-add below is an explicit fmaf(), every other product and
 * sum is rounded on its own, exactly as the HIP kernels issue them.
 *
 * What follows the reference (file:line) and what is fixed here:
 *   quantization      cuda_infer.cu:80-89, mega.cu:303-325 (amax, 127/amax, round
 *                     half even, d = fp16(amax/127), 8*sum(q) kept per block)
 *   q4 x int8 block   cuda_infer.cu:108-121, mega.cu:157-165 (nibble n in 0..15
 *                     times x, minus 8*sum(x))
 *   block accumulate  mega.cu:153-155: acc = fma(dw*dx, float(isum - 8*sum x), acc)
 *   row order         fixed here: cb-block chunks, each an fma chain from 0; ks
 *                     contiguous segments of chunks, chunk sums added left to
 *                     right; segments added left to right (the reference's mega
 *                     sums splits in order, :665-673)
 *   RMSNorm           cpu_infer.cpp:40-46 formula; the sum of squares is a fixed
 *                     64-lane fma partial (lane l: elements 256j+4l+i) + xor
 *                     butterfly instead of a double loop
 *   RoPE              cpu_infer.cpp:49-61 pairs (i, i+hd/2), cos/sin from the same
 *                     float powf/cosf/sinf values; products rounded separately
 *   attention         cpu_infer.cpp:121-140 softmax(q.k/sqrt(hd)) v, computed as
 *                     split-KV partials of 64 positions merged by max rescaling
 *                     (cuda_infer.cu:650-702), in the order written below
 *   SiLU              cpu_infer.cpp:147: g / (1 + exp(-g)) * u
 *   exp               orc_expf: Cody-Waite reduction by ln2 + degree-7 Taylor
 *                     polynomial (Horner), replaces libm expf on both sides
 */
#include "internal.h"
#include <math.h>
#include <stdlib.h>
#include <string.h>

/* exp(x): n = rint(x*log2e); r = x - n*ln2 (two-constant Cody-Waite, ln2_hi has 16
 * trailing zero bits); exp(r) by the Taylor polynomial of degree 7 on |r| <= ln2/2
 * (truncation < 6e-9 relative); result p * 2^n. Inputs below -87 give 0, above
 * ln(FLT_MAX) give +inf, so every finite result is a normal float.
 * Parity: pinned against libm expf (tests/test_oracle_numerics.py, <= 2 ulp). */
float orc_expf(float x) {
    if (x != x) return x;
    if (x > 88.72283f) return INFINITY;
    if (x < -87.0f) return 0.0f;
    const float n = rintf(x * 0x1.715476p+0f);
    float r = fmaf(n, -0x1.62e4p-1f, x);
    r = fmaf(n, -0x1.7f7d1cp-20f, r);
    float p = 0x1.a01a02p-13f;
    p = fmaf(p, r, 0x1.6c16c2p-10f);
    p = fmaf(p, r, 0x1.111112p-7f);
    p = fmaf(p, r, 0x1.555556p-5f);
    p = fmaf(p, r, 0x1.555556p-3f);
    p = fmaf(p, r, 0x1p-1f);
    p = fmaf(p, r, 1.0f);
    p = fmaf(p, r, 1.0f);
    return ldexpf(p, (int)n);
}

/* cuda_infer.cu:80-89 / mega.cu:303-325. Parity: closed form + brute force
 * (tests/test_oracle_numerics.py). */
void orc_quant_q8(const float* x, int n, int8_t* xq, float* xd, int32_t* xs8) {
    for (int b = 0; b < n / 32; b++) {
        const float* v = x + 32 * b;
        float a = 0.f;
        for (int j = 0; j < 32; j++) a = fmaxf(a, fabsf(v[j]));
        const float inv = a > 0.f ? 127.f / a : 0.f;
        int32_t s = 0;
        for (int j = 0; j < 32; j++) {
            const int q = (int)rintf(v[j] * inv);
            xq[32 * b + j] = (int8_t)q;
            s += q;
        }
        xd[b] = orc_f16_to_f32(orc_f32_to_f16(a / 127.f));
        xs8[b] = 8 * s;
    }
}

/* mega.cu:157-165 (dp4a over masked nibble words): sum_j (lo_j * x_j + hi_j * x_{j+16}).
 * Parity: brute force over all nibble x int8 pairs (tests/test_oracle_numerics.py). */
int32_t orc_q4_block_isum(const uint8_t* blk, const int8_t* x) {
    const uint8_t* qs = blk + 2;
    int32_t s = 0;
    for (int j = 0; j < 16; j++) s += (qs[j] & 15) * x[j] + (qs[j] >> 4) * x[j + 16];
    return s;
}

/* mega.cu:153-155 accumulate; the order is fixed here (the reference's mega adds its
 * splits in order, :665-673): every chunk of cb blocks is an fma chain from 0, the
 * chunks of a segment are added left to right, then the segments left to right.
 * Parity: closed form (exact int) + float tolerance vs fp64 dot of dequantized rows. */
float orc_q4_row_dot(const uint8_t* row, int nb, int cb, int ks,
                     const int8_t* xq, const float* xd, const int32_t* xs8) {
    const int nc = nb / cb;
    float tot = 0.f;
    for (int s = 0; s < ks; s++) {
        const int c0 = s * nc / ks, c1 = (s + 1) * nc / ks;
        float seg = 0.f;
        for (int c = c0; c < c1; c++) {
            float acc = 0.f;
            for (int b = c * cb; b < (c + 1) * cb; b++) {
                const uint8_t* blk = row + (size_t)b * 18;
                uint16_t hd; memcpy(&hd, blk, 2);
                const float dw = orc_f16_to_f32(hd);
                const int32_t isum = orc_q4_block_isum(blk, xq + 32 * b);
                acc = fmaf(dw * xd[b], (float)(isum - xs8[b]), acc);
            }
            seg = c == c0 ? acc : seg + acc;
        }
        tot = s == 0 ? seg : tot + seg;
    }
    return tot;
}

float orc_butterfly64(const float* v) {
    float a[64], b[64];
    memcpy(a, v, sizeof a);
    for (int off = 32; off >= 1; off >>= 1) {
        for (int i = 0; i < 64; i++) b[i] = a[i] + a[i ^ off];
        memcpy(a, b, sizeof a);
    }
    return a[0];
}

/* cpu_infer.cpp:40-46 with the sum of squares as 64 lane partials folded by the xor
 * butterfly: lane l takes the elements 256j + 4l + i (i = 0..3) for j = 0, 1, ... in
 * that order (one float4 per lane per 256 elements). Parity: tolerance vs the
 * double-accumulated cpu_infer form (tests/test_oracle_numerics.py). */
void orc_rmsnorm_canon(const float* x, const float* w, int n, float eps, float* out) {
    float p[64];
    for (int l = 0; l < 64; l++) {
        float a = 0.f;
        for (int j = 0; 256 * j < n; j++)
            for (int i = 0; i < 4; i++) {
                const int e = 256 * j + 4 * l + i;
                if (e < n) a = fmaf(x[e], x[e], a);
            }
        p[l] = a;
    }
    const float ss = orc_butterfly64(p);
    const float mean = ss / (float)n;
    const float scale = 1.0f / sqrtf(mean + eps);
    for (int i = 0; i < n; i++) out[i] = (x[i] * scale) * w[i];
}

/* max-first merge of chunk records [c0, c1) (cuda_infer.cu:688-702 attn_combine):
 * M = max m_c, w_c = exp(m_c - M), den and acc[d] as fma-chains over the chunks in
 * order; writes M, den and the weighted sums acc[hd] (not yet divided by den) */
static void merge_records(const float* mc, const float* lc, const float* oc, int c0, int c1, int hd,
                          float* Mo, float* deno, float* acc) {
    float M = -INFINITY;
    for (int c = c0; c < c1; c++) M = fmaxf(M, mc[c]);
    float den = 0.f;
    for (int d = 0; d < hd; d++) acc[d] = 0.f;
    for (int c = c0; c < c1; c++) {
        const float w = orc_expf(mc[c] - M);
        den = fmaf(lc[c], w, den);
        for (int d = 0; d < hd; d++) acc[d] = fmaf(oc[(size_t)c * hd + d], w, acc[d]);
    }
    *Mo = M;
    *deno = den;
}

/* cpu_infer.cpp:121-140 as split-KV partials (cuda_infer.cu:650-702):
 *   chunk c = positions [64c, 64c+64) of 0..L-1
 *   score  = (a0 + a1) + (a2 + a3) with a_j = fma-chain over dims d = 4i + j; times scale
 *   m_c    = max score; p_t = exp(score - m_c); l_c = butterfly64 over the chunk's lanes
 *   o_c[d] = fma-chain over positions in order of p_t * v_t[d]
 *   merge  : up to ORC_ATTN_SPLIT chunks: M = max m_c, w_c = exp(m_c - M), den and o as
 *            fma-chains over chunks in order, out = o / den. More chunks merge as a
 *            two-level tree: each split of ORC_ATTN_SPLIT consecutive chunks that way
 *            (giving M_s, den_s, o_s), then the splits in order the same way with
 *            (M_s, den_s, o_s) in place of (m_c, l_c, o_c), out = o / den.
 * Parity: tolerance vs fp64 brute-force softmax and vs orc_attention_fp32. */
void orc_attention_canon(const float* q, const float* k, const float* v, int L, int hd,
                         int stride, float scale, int chunk, float* out) {
    (void)chunk;  /* the canonical order is defined for 64-position chunks */
    const int nch = (L + 63) / 64;
    const int nsp = nch > ORC_ATTN_SPLIT ? (nch + ORC_ATTN_SPLIT - 1) / ORC_ATTN_SPLIT : 0;
    float* mc = (float*)malloc(sizeof(float) * (nch + nsp));
    float* lc = (float*)malloc(sizeof(float) * (nch + nsp));
    float* oc = (float*)malloc(sizeof(float) * (size_t)(nch + nsp) * hd);
    for (int c = 0; c < nch; c++) {
        const int t0 = 64 * c, n = L - t0 < 64 ? L - t0 : 64;
        float sc[64], p[64];
        float mx = -INFINITY;
        for (int t = 0; t < n; t++) {
            const float* kt = k + (size_t)(t0 + t) * stride;
            float a[4] = {0.f, 0.f, 0.f, 0.f};
            for (int i = 0; i < hd / 4; i++)
                for (int j = 0; j < 4; j++) a[j] = fmaf(q[4 * i + j], kt[4 * i + j], a[j]);
            sc[t] = ((a[0] + a[1]) + (a[2] + a[3])) * scale;
            mx = fmaxf(mx, sc[t]);
        }
        for (int t = 0; t < 64; t++) p[t] = t < n ? orc_expf(sc[t] - mx) : 0.f;
        lc[c] = orc_butterfly64(p);
        mc[c] = mx;
        for (int d = 0; d < hd; d++) {
            float a = 0.f;
            for (int t = 0; t < n; t++) a = fmaf(p[t], v[(size_t)(t0 + t) * stride + d], a);
            oc[(size_t)c * hd + d] = a;
        }
    }
    float M, den;
    if (nsp == 0) {
        merge_records(mc, lc, oc, 0, nch, hd, &M, &den, out);
    } else {
        for (int s = 0; s < nsp; s++) {
            const int c0 = s * ORC_ATTN_SPLIT, c1 = c0 + ORC_ATTN_SPLIT < nch ? c0 + ORC_ATTN_SPLIT : nch;
            merge_records(mc, lc, oc, c0, c1, hd, mc + nch + s, lc + nch + s, oc + (size_t)(nch + s) * hd);
        }
        merge_records(mc, lc, oc, nch, nch + nsp, hd, &M, &den, out);
    }
    for (int d = 0; d < hd; d++) out[d] = out[d] / den;
    free(mc); free(lc); free(oc);
}

static float f16r(float x) { return orc_f16_to_f32(orc_f32_to_f16(x)); }

/* rows [0, out) of a q4_0 matrix in the canonical order */
static int rows_q8(const orc_tensor* W, const orc_plan* P, int kind, const struct orc_model* m, float* y) {
    if (W->type != ORC_Q4_0) return -1;
    const int nb = (int)(W->ne[0] / 32), out = (int)(W->ne[1] * W->ne[2]);
    const int cb = P->cb[kind], ks = P->ks[kind];
    if (cb <= 0 || nb % cb || ks < 1 || ks > nb / cb) return -1;
    const uint8_t* base = W->data;
    #pragma omp parallel for schedule(static) num_threads(m->n_threads)
    for (int j = 0; j < out; j++)
        y[j] = orc_q4_row_dot(base + (size_t)j * nb * 18, nb, cb, ks, m->xq, m->xd, m->xs8);
    return 0;
}

/* NEOX RoPE of n_head heads (cpu_infer.cpp:49-61): pair (i, i + hd/2) rotated by the
 * angle whose cos/sin are c[i], s[i]: (x0, x1) -> (x0 c - x1 s, x0 s + x1 c), the four
 * products rounded separately (no fma). Exported as orc_rope_rotate. Parity: known
 * answers (a quarter turn maps (x, y) to (-y, x)) and a float64 rotation
 * (tests/test_oracle_numerics.py), and the attention-sensitive golden model, where a
 * flipped sign moves the logits by ~2x their range (tests/test_oracle_golden.py). */
static void rope_q8(float* v, int n_head, int hd, const float* c, const float* s) {
    const int half = hd / 2;
    for (int h = 0; h < n_head; h++) {
        float* p = v + (size_t)h * hd;
        for (int i = 0; i < half; i++) {
            const float x0 = p[i], x1 = p[i + half];
            const float a = x0 * c[i], b = x1 * s[i], e = x0 * s[i], f = x1 * c[i];
            p[i] = a - b;
            p[i + half] = e + f;
        }
    }
}

void orc_rope_rotate(float* v, int n_head, int hd, const float* c, const float* s) { rope_q8(v, n_head, hd, c, s); }

/* one decode step in the GPU engine's numerics; see the table at the top */
int32_t orc_forward_q8act(struct orc_model* m, int32_t token, int32_t pos) {
    const orc_config* c = &m->c;
    const orc_plan* P = &m->plan;
    const int E = c->n_embd, HD = c->head_dim, kvd = c->n_head_kv * HD, gqa = c->n_head / c->n_head_kv;
    const float inv = 1.f / sqrtf((float)HD);
    orc_dequant_row(m->tok_emb, token, m->h);
    const float* rc = m->rope_c + (size_t)pos * (HD / 2);
    const float* rs = m->rope_s + (size_t)pos * (HD / 2);
    for (int l = 0; l < c->n_layer; l++) {
        const orc_layer* ly = &m->L[l];
        orc_rmsnorm_canon(m->h, (const float*)ly->an->data, E, c->rms_eps, m->xb);
        orc_quant_q8(m->xb, E, m->xq, m->xd, m->xs8);
        if (rows_q8(ly->wq, P, ORC_MAT_QKV, m, m->q) || rows_q8(ly->wk, P, ORC_MAT_QKV, m, m->k) ||
            rows_q8(ly->wv, P, ORC_MAT_QKV, m, m->v)) return -1;
        const float *bq = (const float*)ly->bq->data, *bk = (const float*)ly->bk->data, *bv = (const float*)ly->bv->data;
        for (int i = 0; i < c->n_head * HD; i++) m->q[i] = m->q[i] + bq[i];
        for (int i = 0; i < kvd; i++) { m->k[i] = m->k[i] + bk[i]; m->v[i] = m->v[i] + bv[i]; }
        rope_q8(m->q, c->n_head, HD, rc, rs);
        rope_q8(m->k, c->n_head_kv, HD, rc, rs);
        float* kc = m->kc + ((size_t)l * m->max_seq + pos) * kvd;
        float* vc = m->vc + ((size_t)l * m->max_seq + pos) * kvd;
        for (int i = 0; i < kvd; i++) {
            kc[i] = P->kv_f16 ? f16r(m->k[i]) : m->k[i];
            vc[i] = P->kv_f16 ? f16r(m->v[i]) : m->v[i];
        }
        #pragma omp parallel for schedule(static) num_threads(m->n_threads)
        for (int hh = 0; hh < c->n_head; hh++) {
            const int kvh = hh / gqa;
            orc_attention_canon(m->q + (size_t)hh * HD, m->kc + (size_t)l * m->max_seq * kvd + kvh * HD,
                                m->vc + (size_t)l * m->max_seq * kvd + kvh * HD, pos + 1, HD, kvd, inv,
                                P->attn_chunk, m->att + (size_t)hh * HD);
        }
        orc_quant_q8(m->att, E, m->xq, m->xd, m->xs8);
        if (rows_q8(ly->wo, P, ORC_MAT_O, m, m->proj)) return -1;
        for (int i = 0; i < E; i++) m->h[i] = m->h[i] + m->proj[i];
        orc_rmsnorm_canon(m->h, (const float*)ly->fn->data, E, c->rms_eps, m->xb);
        orc_quant_q8(m->xb, E, m->xq, m->xd, m->xs8);
        if (rows_q8(ly->wg, P, ORC_MAT_GU, m, m->gbuf) || rows_q8(ly->wu, P, ORC_MAT_GU, m, m->ubuf)) return -1;
        for (int i = 0; i < c->n_ff; i++) {
            const float g = m->gbuf[i];
            const float t = orc_expf(-g);
            const float den = 1.0f + t;
            const float sg = g / den;
            m->gbuf[i] = sg * m->ubuf[i];
        }
        orc_quant_q8(m->gbuf, c->n_ff, m->xq, m->xd, m->xs8);
        if (rows_q8(ly->wd, P, ORC_MAT_DOWN, m, m->proj)) return -1;
        for (int i = 0; i < E; i++) m->h[i] = m->h[i] + m->proj[i];
    }
    orc_rmsnorm_canon(m->h, (const float*)m->out_norm->data, E, c->rms_eps, m->xb);
    orc_quant_q8(m->xb, E, m->xq, m->xd, m->xs8);
    if (rows_q8(m->out_w, P, ORC_MAT_LM, m, m->logits)) return -1;
    return 0;
}
