// Optional per-stage reports (the atomic_stage_report entries of an args
// struct's `diag`): a reduction of a stage's buffer to its non-finite count
// and the largest |x| over its finite entries.  Launched only when the
// caller asked for reports, after the path's own kernels, on the same stream.
#pragma once
#include "../../include/atomic_hybrid.h"
#include "common.hpp"
#include "launch.hpp"

namespace ah {

// Clears reports [first, first + n) (a kernel, not a memset: safe under graph
// capture).  A template so that each translation unit's copy merges at link.
template <typename R>
__global__ __launch_bounds__(64) void stage_report_clear(R* r, int first, int n) {
  const int i = threadIdx.x;
  if (i < n) {
    r[first + i].n_nonfinite = 0u;
    r[first + i].max_abs = 0.f;
  }
}

// Folds one thread's (count, max) into the report: wave reduction, then one
// atomic per wave.  max_abs is non-negative, so its bit pattern orders as an
// unsigned integer.
__device__ __forceinline__ void stage_report_fold(uint32_t bad, float mx, atomic_stage_report* r) {
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) {
    bad += (uint32_t)__shfl_xor((int)bad, off);
    mx = fmaxf(mx, __shfl_xor(mx, off));
  }
  if (lane_id() == 0) {
    if (bad) atomicAdd(&r->n_nonfinite, bad);
    atomicMax(reinterpret_cast<unsigned int*>(&r->max_abs), __float_as_uint(mx));
  }
}

template <typename T>
__global__ __launch_bounds__(256) void stage_report_reduce(const T* __restrict__ x, size_t n,
                                                           atomic_stage_report* r) {
  uint32_t bad = 0;
  float mx = 0.f;
  const size_t stride = (size_t)gridDim.x * 256;
  for (size_t i = (size_t)blockIdx.x * 256 + threadIdx.x; i < n; i += stride) {
    const float v = to_f(x[i]);
    if (__builtin_isfinite(v)) mx = fmaxf(mx, fabsf(v));
    else ++bad;
  }
  stage_report_fold(bad, mx, r);
}

struct StageDiag {
  atomic_stage_report* r;  // the caller's report array (NULL: no reports)
  Launch& L;
  explicit operator bool() const { return r != nullptr; }
  int clear(int first, int n) {
    return L("stage_report_clear", [&] {
      hipLaunchKernelGGL(stage_report_clear<atomic_stage_report>, dim3(1), dim3(64), 0, L.st, r, first, n);
    });
  }
  template <typename T>
  int reduce(int stage, const T* x, size_t n) {
    if (!x || n == 0) return ATOMIC_OK;
    size_t blocks = (n + 255) / 256;
    if (blocks > 2048) blocks = 2048;
    return L("stage_report_reduce", [&] {
      hipLaunchKernelGGL((stage_report_reduce<T>), dim3((unsigned)blocks), dim3(256), 0, L.st, x, n,
                         r + stage);
    });
  }
};

}  // namespace ah
