// GDN2 WY chunk pipeline: shapes and the per-chunk intermediate buffers shared
// by the forward and backward kernels.
#pragma once
#include "common.hpp"

namespace ah {

struct Gdn2Dims {
  int B, T, H, K, V, C, NT;
  float scale;
  // row strides of the [B, T, H, D] inputs in elements (token t of batch b
  // starts at (b T + t) * stride): q, k, v, w, b, g, dO
  long long rq, rk, rv, rw, rb, rg, rdo;
};

// Per-(batch, head, chunk) intermediates, each a contiguous block indexed by
// bhn = (b * H + h) * NT + n.  Element type T is the operand type (bf16 for
// bf16 inputs, fp32 for fp32 inputs).
template <typename T>
struct Gdn2Chunks {
  T* qg;      // [C][K]  q * exp(gc)
  T* kg;      // [C][K]  k * exp(gc_last - gc)
  T* wt;      // [C][K]  w_pseudo = A (b k exp(gc))
  T* u;       // [C][V]  A (w v)
  T* aqk;     // [C][C]  scale * sum_d q k exp(gc_i - gc_j), causal
  T* ainv;    // [C][C]  A = (I + Akk)^-1
  T* akk;     // [C][C]  strict Akk (written or read by the stage-level kernels A / B only)
  float* gcl; // [K]     gc of the chunk's last row
  T* hT;      // [V][K]  state entering the chunk, transposed (saved for backward)
  T* vnT;     // [V][C]  v_new = u - w_pseudo h, transposed (saved for backward)
};

// Backward scratch.
template <typename T>
struct Gdn2Grads {
  T* dvn;       // [C][V]  dv_new (B1 output; an MFMA operand downstream)
  T* dhT;       // [V][K]  dh carried into the chunk from the next one, transposed
  T* dqg;       // [C][K]  scale dO h_pre^T
  T* dwt;       // [C][K]  -dv_new h_pre^T (an MFMA operand of the WY step)
  T* dkb;       // [C][K]  A^T dwt
  T* dkg;       // [C][K]  v_new dh_next^T
  T* daqk;      // [C][C]  scale (dO v_new^T) * causal
  T* dakk;      // [C][C]  -A^T (dA A^T) * strict
  float* rlast; // [K]     exp(gc_last) * sum_v dh_next * h_pre
};

}  // namespace ah
