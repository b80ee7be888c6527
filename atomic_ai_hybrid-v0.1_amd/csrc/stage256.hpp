// Stage-level entries at the reference's Pallas block of 256 rows: the GDN2
// kernels A, B, C, D (kernel_a_scores.py:15-17 BT = 256) and the Mamba2 M3,
// M4 stages at chunk_size 256, over float32 per-chunk arrays in the
// reference's layout.  Launchers; kernels in stage256.hip.
#pragma once
#include <hip/hip_runtime.h>

#include "gdn2.hpp"
#include "launch.hpp"
#include "mamba2.hpp"

namespace ah {

constexpr int kStageBlock = 256;

// GDN2 (dims with C = 256, NT = T / 256; K = V in {64, 128}); dtype is the
// operand type of q, k, v, w, b (ATOMIC_BF16 / ATOMIC_F32), arrays fp32.
int g256_scores(const Gdn2Dims& d, int dtype, const void* q, const void* k, const void* b, const float* g,
                float* aqk, float* akk, Launch& L);
int g256_solve(const Gdn2Dims& d, const float* akk, float* a, Launch& L);
int g256_recompute(const Gdn2Dims& d, int dtype, const void* q, const void* k, const void* v, const void* w,
                   const void* b, const float* g, const float* a, float* wt, float* u, float* kg, float* qg,
                   float* gcl, Launch& L);
int g256_combine(const Gdn2Dims& d, const float* aqk, const float* wt, const float* u, const float* kg,
                 const float* qg, const float* gcl, const float* h0, float* o, float* h_final, float* h_pre,
                 float* v_new, Launch& L);

// Mamba2 (dims with C = 256): M3 (y_diag [B][T][H][P], state_end
// [B][H][NT][P][N]) and M4 (y, state_final; the states entering each chunk
// go to ws, [B][NT][H][P][N] fp32).
int m256_intra(const Mamba2Dims& d, const void* dt, const void* x, const void* Bm, const void* Cm,
               const float* cum, float* y_diag, float* state_end, Launch& L);
int m256_combine(const Mamba2Dims& d, const float* y_diag, const float* state_end, const float* cum,
                 const void* Cm, const float* state0, float* y, float* state_final, float* ws, Launch& L);
size_t m256_combine_ws(const Mamba2Dims& d);

}  // namespace ah
