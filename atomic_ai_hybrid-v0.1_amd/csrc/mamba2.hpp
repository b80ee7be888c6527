// Mamba2 SSD chunk scan: shapes and per-chunk buffers shared by the forward
// and backward kernels.
#pragma once
#include "common.hpp"

namespace ah {

struct Mamba2Dims {
  int B, T, H, P, N, C, NT;
};

template <typename T>
struct Mamba2Chunks {
  T* cb;         // [B][NT][C][C]   sanitize(C_i . B_j), shared by every head
  T* state_pre;  // [B][H][NT][P][N] state entering each chunk (saved for backward)
};

}  // namespace ah
