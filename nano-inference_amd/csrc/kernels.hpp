// kernels.hpp -- host-side launchers of the gfx950 kernels (kernels.hip).
#pragma once
#include "common.hpp"

namespace mi {

// Kernels read the model description through a pointer to a device copy (dM) of the
// host DModel M: a kernel-argument struct would be treated as invariant and kept in
// scalar registers for the whole persistent step, which runs out of them.
bool kernels_support(int G, int HD);
int kernels_max_ctx_chunks(int HD);   // attention chunks (64 positions) a context may hold
// reduction plan (blocks per chunk, K segments) of qkv, o, gate/up, down, lm_head;
// false when the shape does not fit the kernels' LDS staging
bool kernels_plan(int E, int FF, int cb[5], int ks[5]);
// chunk sums one workgroup stages for a matrix under the plan, and the limit
int kernels_tiles_per_wg(int rows, int nb, int cb, int ks, int nwg);
int kernels_max_tiles_per_wg();
// one decode step at position pos as one launch per phase (nwg workgroups each);
// gen != 0 stores the prediction as the token of position pos + 1
void launch_step_phases(const DModel& M, const DModel* dM, int nwg, int pos, int gen, hipStream_t s);
// the same step as one launch of nwg workgroups that must all be resident at once
// (grid barriers). coop: a cooperative launch, which the runtime only starts when
// they are; otherwise a plain launch (~18 us less per token on MI355X: no cooperative
// queue hand-off), which relies on an idle device and reports a failed barrier through
// M.err. M.bar must be zero (it is after allocation, and every launch leaves it zero).
hipError_t launch_step_persistent(const DModel& M, const DModel* dM, int nwg, int pos, int gen, bool coop,
                                  hipStream_t s);
// T tokens (2 <= T <= kernels_max_tokens()) at positions p..p+T-1, p = *M.posT (device
// memory: the launch sequence depends on T only, so it can be captured once and
// replayed), in one pass over the weights (int8 MFMA tiles), one launch per phase;
// the predictions land in out_tok/out_margin[p..p+T-1], logits in logitsT if set
void launch_step_multi(const DModel& M, const DModel* dM, int nwg, int T, hipStream_t s);
// the same multi-token step as one persistent launch of nwg workgroups, all resident at
// once (grid barriers; coop and M.bar / M.err as for launch_step_persistent)
hipError_t launch_step_multi_persistent(const DModel& M, const DModel* dM, int nwg, int T, bool coop, hipStream_t s);
// one verify step of a speculative generation driven on the device (M.spec holds T, the
// position is *M.posT; a launch after the generation finished does nothing)
hipError_t launch_spec_step(const DModel& M, const DModel* dM, int nwg, bool coop, hipStream_t s);
// co-resident workgroups per CU of the persistent multi-token kernels (0: cannot launch)
int multi_persistent_max_grid(int HD);
int kernels_max_tokens();
int kernels_max_chunks_multi();   // chunks per K segment the multi-token kernels stage
// co-resident workgroups per CU of the persistent kernel (0: cannot launch)
int persistent_max_grid(int G, int HD);
hipError_t launch_barriers(uint32_t* bar, int32_t* err, int nwg, int n, hipStream_t s);
int barrier_words();        // uint32 words the grid barrier uses
int attn_record_floats(int HD);   // floats per attention chunk record
constexpr int kProfPerPhase = 8;
constexpr int prof_slots(int n_layer) { return 1 + (5 * n_layer + 1) * kProfPerPhase; }

// one phase kernel of the step at pos: 0 qkv, 1 attention, 2 chunk merge (only
// launched past kInlineComb chunks), 3 o, 4 gate/up+act, 5 down, 6 lm_head, 7 argmax
void launch_phase(const DModel& M, const DModel* dM, int nwg, int phase, int l, int pos, int gen, hipStream_t s);

void launch_quant(const float* x, int n, int8_t* xq, float* xd, int32_t* xs8, hipStream_t s);
void launch_gemv(const PMat& W, const int8_t* xq, const float* xd, const int32_t* xs8, float* part, float* y,
                 int n_cu, hipStream_t s);
void launch_isums(const PMat& W, const int8_t* xq, int32_t* isum, hipStream_t s);
size_t attn_scratch_floats(int nh, int hd, int L);
// floats of the file-scope scratch array behind mi_attn_decode_noalloc (16 MiB per device)
constexpr size_t kNoAllocScratchFloats = size_t(4) << 20;
// device address of the current device's scratch array (looked up on the host at the
// first call on each device; s is not used)
hipError_t noalloc_scratch(hipStream_t s, float** out);
bool launch_attn_decode(const float* q, const __half* kc, const __half* vc, int nh, int nkv, int hd, int L, int ctx,
                        float scale, float* scratch, float* out, hipStream_t s);
// the same attention with MFMA chunk records (k_attn_mx): ~1e-6 relative of the
// canonical records, not bit-identical
bool launch_attn_decode_mfma(const float* q, const __half* kc, const __half* vc, int nh, int nkv, int hd, int L,
                             int ctx, float scale, float* scratch, float* out, hipStream_t s);
void launch_stream(const void* buf, size_t bytes, uint32_t* sink, int n_cu, hipStream_t s);

}  // namespace mi
