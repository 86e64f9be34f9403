// kernels.hpp -- host-side launchers of the gfx950 kernels (kernels.hip).
#pragma once
#include "common.hpp"

namespace mi {

struct PhaseGrid { int qkv, fin, comb, o, gu, act, down, lm; };

bool kernels_support(int G, int HD);
PhaseGrid plan_phase_grid(const DModel& M, const DLayer& L0, int n_cu);
// one decode step at position pos as one launch per phase; gen != 0 stores the
// prediction as the token of position pos + 1
void launch_step_phases(const DModel& M, const PhaseGrid& pg, int pos, int gen, hipStream_t s);
// the same step as one cooperative launch of nwg workgroups (zeroes the barrier counter first)
hipError_t launch_step_persistent(const DModel& M, int nwg, int pos, int gen, hipStream_t s);
// co-resident workgroups per CU of the persistent kernel (0: cannot launch)
int persistent_max_grid(int G, int HD);
hipError_t launch_barriers(uint32_t* bar, int32_t* err, int nwg, int n, hipStream_t s);
int barrier_words();        // uint32 words the grid barrier uses
int kernels_max_ks();       // largest K-segment count the phases stage in LDS
int attn_record_floats(int HD);   // floats per attention chunk record
constexpr int kProfSlotsPerLayer = 15;
// profile slots of one workgroup: start, 15 per layer, lm prologue, lm end, last barrier
constexpr int prof_slots(int n_layer) { return n_layer * kProfSlotsPerLayer + 4; }

// one phase kernel of the step at pos: 0 qkv, 1 attention, 2 chunk merge (only
// launched past kInlineComb chunks), 3 o, 4 gate/up+act, 5 down, 6 lm_head, 7 argmax
void launch_phase(const DModel& M, const PhaseGrid& pg, int phase, int l, int pos, int gen, hipStream_t s);

void launch_quant(const float* x, int n, int8_t* xq, float* xd, int32_t* xs8, hipStream_t s);
void launch_gemv(const PMat& W, const int8_t* xq, const float* xd, const int32_t* xs8, float* part, float* y,
                 int n_cu, hipStream_t s);
void launch_isums(const PMat& W, const int8_t* xq, int32_t* isum, hipStream_t s);
bool launch_attn_decode(const float* q, const __half* kc, const __half* vc, int nh, int nkv, int hd, int L, int ctx,
                        float scale, float* scratch, float* out, hipStream_t s);
void launch_stream(const void* buf, size_t bytes, uint32_t* sink, int n_cu, hipStream_t s);

}  // namespace mi
