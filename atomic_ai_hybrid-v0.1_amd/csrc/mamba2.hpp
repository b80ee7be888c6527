// Mamba2 SSD chunk scan: shapes and per-chunk buffers shared by the forward
// and backward kernels.
#pragma once
#include "common.hpp"

namespace ah {

struct Mamba2Dims {
  int B, T, H, P, N, C, NT;
  // row strides of the inputs in elements (token t of batch b starts at
  // (b T + t) * stride): dt, x, B, C, dy
  long long rdt, rx, rB, rC, rdy;
  // the forward state pass sanitises state0 (clip +-1e4, nan_to_num) before
  // its first chunk, as the reference's staged combine does
  // (kernel_mamba2_c_interchunk.py:58)
  int sanitize_state0;
};

template <typename T>
struct Mamba2Chunks {
  T* cb;         // [B][NT][C][C]      sanitize(C_i . B_j), shared by every head
  T* state_pre;  // [B][NT][H][P][N]   state entering each chunk
  float* cl;     // [B][NT][H][P]      cumulative log decay at the chunk's last row
  float* src;    // [B][NT][H][P][N]   the two-pass form's per-chunk state_end, then
                 //                    the backward's (dy decay_h)^T C (NULL when the
                 //                    state loops form them); stage-level entries:
                 //                    the caller's state_end [B][H][NT][P][N]
  // stage-level entries only (NULL on the whole path):
  const float* cum;    // [B][H][NT][C][P]  the caller's cumdecay
  const float* ydiag;  // [B][T][H][P]      the caller's y_diag (the combine)
};

}  // namespace ah
