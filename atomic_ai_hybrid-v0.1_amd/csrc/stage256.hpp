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

// A read-only operand of either element type: the stage kernels read bf16
// or fp32 inputs and compute in fp32.
struct StageIn {
  const void* p;
  int bf;  // 1: bf16, 0: fp32
};
__device__ __forceinline__ float ld(const StageIn& a, size_t i) {
  return a.bf ? to_f(reinterpret_cast<const bf16*>(a.p)[i]) : reinterpret_cast<const float*>(a.p)[i];
}

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

// Mamba2 (dims with C = 64, 128 or 256; dt, x, B, C of dtype, bf16 or
// fp32): M3 (y_diag [B][T][H][P], state_end [B][H][NT][P][N]) over the
// reference's min(128, C)-row sub-blocks, with the chunks' CB = sanitize(C
// B^T) formed once per (batch, chunk) into cb ([B][NT][C][C] fp32, m_cb_ws
// bytes), and M4 (y, state_final; the states entering each chunk go to ws,
// [B][NT][H][P][N] fp32).
int m256_intra(const Mamba2Dims& d, int dtype, const void* dt, const void* x, const void* Bm, const void* Cm,
               const float* cum, float* y_diag, float* state_end, float* cb, Launch& L);
// CB = sanitize(C B^T) per (batch, chunk) on the float32 GEMM (stage256_bwd.hip)
int m_cb(const Mamba2Dims& d, int dtype, const void* Bm, const void* Cm, float* cb, Launch& L);
size_t m_cb_ws(const Mamba2Dims& d);
int m256_combine(const Mamba2Dims& d, int dtype, const float* y_diag, const float* state_end, const float* cum,
                 const void* Cm, const float* state0, float* y, float* state_final, float* ws, Launch& L);
size_t m256_combine_ws(const Mamba2Dims& d);

// Backward stages (stage256_bwd.hip), GDN2 dims as above; dO is of type
// do_dtype, q, k, b, w, v of type dtype, every other array fp32:
//   B2  dAqk [B][H][NT][256][256], dv_new [B][H][NT][256][V]
//   B1  dh_all [B][H][NT][K][V], dh0 [B][H][K][V], dv_all like dv_new
//   B3  per-block q, k, b, w, v, gc, dO, dv [B][H][NT][256][D], A
//       [B][H][NT][256][256], h_pre / dh_next [B][H][NT][K][V]; workspace
//       g256_b3_ws bytes
//   B4  q, k, b, g [B][T][H][K] (row strides of the dims), outputs per block
//   B5  dg of a [blocks][rows][cols] array
int g256_dav_bwd(const Gdn2Dims& d, int do_dtype, const float* aqk, const float* v_new, const void* dO,
                 float* daqk, float* dvn, Launch& L);
int g256_dhu_bwd(const Gdn2Dims& d, int do_dtype, const void* dO, const float* dvp, const float* wp,
                 const float* qg, const float* kg, const float* gcl, const float* dht, float* dh_all, float* dh0,
                 float* dv_all, Launch& L);
size_t g256_b3_ws(const Gdn2Dims& d);
int g256_b3_bwd(const Gdn2Dims& d, int dtype, int do_dtype, const void* q, const void* k, const void* b,
                const void* w, const void* v, const float* gc, const float* A, const float* h_pre,
                const float* v_new, const void* dO, const float* dv, const float* dh_next, float* dq, float* dk,
                float* db, float* dw, float* dvr, float* dgc, float* dakk, float* ws, Launch& L);
int g256_intra_bwd(const Gdn2Dims& d, int dtype, const float* daqk, const float* dakk, const void* q,
                   const void* k, const void* b, const float* g, float* dq, float* dk, float* db, float* dgc,
                   Launch& L);
int rev_cumsum_bwd(const float* dgc, float* dg, long long blocks, int rows, int cols, Launch& L);

// Mamba2 MB2 (chunk d.C of 64, 128 or 256): dt, x, B, C bf16, dy of
// dy_dtype; cumdecay [B][H][NT][C][P] and dstate_end_grad [B][H][NT][P][N]
// fp32.  ddt, dx [B][T][H][P], dB, dC [B][T][N] (summed over the heads),
// dcum [B][H][NT][C][P], fp32; workspace m_intra_bwd_ws bytes.
size_t m_intra_bwd_ws(const Mamba2Dims& d);
int m_intra_bwd(const Mamba2Dims& d, int dtype, int dy_dtype, const void* dt, const void* x, const void* Bm,
                const void* Cm, const float* cum, const void* dy, const float* dse, float* ddt, float* dx, float* dB,
                float* dC, float* dcum, float* ws, Launch& L);

// Mamba2 MB1 + MB3 (mamba2_bwd_scan): workspace m_bwd_scan_ws bytes, whose
// first B H NT C P floats hold the cumdecay (M2's output, written by the
// caller; ws doubles as cum).  Outputs fp32: ddt (the dBx part), dx [B][T][H][P],
// dB, dC [B][T][N], dstate0 [B][H][P][N], dcum [B][H][NT][C][P].  P a
// multiple of 32, N 64 or 128.
size_t m_bwd_scan_ws(const Mamba2Dims& d);
int m_bwd_scan(const Mamba2Dims& d, int dtype, int dy_dtype, const void* dt, const void* x, const void* Bm,
               const void* Cm, const float* cum, const void* dy, const float* dsf, const float* state0, float* ddt,
               float* dB, float* dC, float* dx, float* ds0, float* dcum, float* ws, Launch& L);
// Mamba2 MB4 (mamba2_dA_backward): dt of dt_dtype per chunk [B][H][NT][C][P], or
// in the token layout [B][T][H][P] (row stride d.rdt) with tok,
// A [H], dcum [B][H][NT][C][P]; ddt2 like dt (fp32), dA [H]; workspace
// m_da_bwd_ws bytes; C <= 256.
size_t m_da_bwd_ws(const Mamba2Dims& d);

// Mamba2 with fp32 operands (dt, x, B, C): M2 for any chunk and operand type,
// and the whole forward / backward as the staged chain of the reference's
// trainable op (M2 -> M3 -> M4; MB1 + MB3 -> MB4, final sanitise), dims at the
// caller's chunk.  Outputs and gradients fp32; workspaces m_f32_*_ws bytes.
int m_cumdecay(const Mamba2Dims& d, int dtype, const void* dt, const float* A, float* cum, Launch& L);
size_t m_f32_fwd_ws(const Mamba2Dims& d);
int m_f32_fwd(const Mamba2Dims& d, const void* dt, const void* x, const void* Bm, const void* Cm, const float* A,
              const float* state0, float* y, float* state_final, float* ws, Launch& L);
size_t m_f32_bwd_ws(const Mamba2Dims& d);
int m_f32_bwd(const Mamba2Dims& d, int dy_dtype, const void* dt, const void* x, const void* Bm, const void* Cm,
              const float* A, const float* state0, const void* dy, const float* dsf, float* ddt, float* dx,
              float* dB, float* dC, float* dA, float* ds0, float* ws, Launch& L);
int m_da_bwd(const Mamba2Dims& d, int dt_dtype, int tok, const void* dtp, const float* A, const float* dcum,
             float* ddt2, float* dA, float* ws, Launch& L);

}  // namespace ah
