// Fused output epilogue of the two mixer blocks (the path's downstream
// caller): RMSNorm over the model dimension and the SiLU gate, forward and
// backward, for gfx950.
//
//   GDN2   (reference model.py:612-613,650-653):
//     out = bf16( bf16(RMSNorm(o)) * silu(clip(gate, -1e2, 1e2)) )
//   Mamba2 (reference model.py:516-525):
//     out = clip( bf16( bf16(RMSNorm(bf16(y))) * silu(res) ), -3e2, 3e2 )
// RMSNorm(x) = x * (rsqrt(mean_c x^2 + eps) * weight) in fp32, as flax
// linen RMSNorm computes it (statistics in fp32, scale folded into the
// multiplier).  The bf16 products and the SiLU round once to bf16, as an
// XLA elementwise op on bf16 operands does.
//
// One wave per row: the row's sum of squares is a wave reduction (no LDS,
// no barrier); each lane holds NPL pieces of 8 consecutive channels
// (channel 8 (lane + 64 s) + j), so every global access is a 16- or 32-byte
// vector.  The backward keeps each wave's weight-gradient partial sums in
// registers over its rows, combines the four waves through LDS and writes
// one partial row per workgroup; a second kernel sums them column-wise.
#include "../../include/atomic_hybrid.h"
#include "common.hpp"
#include "launch.hpp"
#include "ws_tag.hpp"

namespace ah {

enum { kNgGdn2 = 0, kNgMamba2 = 1 };

struct NgDims {
  int rows, d;
  float eps;
};

__device__ __forceinline__ float bf16r(float x) { return (float)(bf16)x; }
// logistic with the hardware reciprocal (about 1 ulp; every use rounds to bf16)
__device__ __forceinline__ float sigmoidf_(float x) { return __builtin_amdgcn_rcpf(1.f + __expf(-x)); }

template <int CTRL>
__device__ __forceinline__ float dpp_add(float v) {
  return v + __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), CTRL, 0xF, 0xF, false));
}
// Sum over the wave, every lane getting the total: DPP steps inside each
// 16-lane row (swap neighbours, swap pairs, mirror halves, mirror the row),
// then the four rows through two lane exchanges.  Each step adds a lane
// pair's values in both lanes, so every lane holds the identical sum.
__device__ __forceinline__ float wave_sum(float v) {
  v = dpp_add<0xB1>(v);   // quad_perm [1, 0, 3, 2]
  v = dpp_add<0x4E>(v);   // quad_perm [2, 3, 0, 1]
  v = dpp_add<0x141>(v);  // row_half_mirror
  v = dpp_add<0x140>(v);  // row_mirror
  v += __shfl_xor(v, 16);
  v += __shfl_xor(v, 32);
  return v;
}

// One row's input, gate and (backward) upstream gradient in registers.
template <int VAR, int NPL>
struct NgRow {
  float x[NPL][8];   // o (GDN2) or bf16(y) (Mamba2)
  float g[NPL][8];   // gate pre-activation
  __device__ __forceinline__ void load(const float* __restrict__ xr, const bf16* __restrict__ gr) {
    const int lane = lane_id();
#pragma unroll
    for (int s = 0; s < NPL; ++s) {
      const int c = 8 * (lane + 64 * s);
      load8(xr + c, x[s]);
      load8(gr + c, g[s]);
    }
    if (VAR == kNgMamba2) {
#pragma unroll
      for (int s = 0; s < NPL; ++s)
#pragma unroll
        for (int j = 0; j < 8; ++j) x[s][j] = bf16r(x[s][j]);
    }
  }
  // rsqrt(mean x^2 + eps) of the row
  __device__ __forceinline__ float inv_rms(int d, float eps) const {
    float ss = 0.f;
#pragma unroll
    for (int s = 0; s < NPL; ++s)
#pragma unroll
      for (int j = 0; j < 8; ++j) ss += x[s][j] * x[s][j];
    ss = wave_sum(ss);
    return rsqrtf(ss / (float)d + eps);
  }
};

// Cotangent factor of clip(v, -c, c) = min(max(v, -c), c): 1 inside, 0
// outside, 1/2 on the bound (the max / min VJP splits ties evenly).
__device__ __forceinline__ float clip_grad(float v, float c) {
  const float a = fabsf(v);
  return a < c ? 1.f : (a == c ? 0.5f : 0.f);
}

// gate value entering the SiLU: GDN2 clips the gate to +-1e2 (model.py:613)
template <int VAR>
__device__ __forceinline__ float gate_in(float g) {
  return VAR == kNgGdn2 ? fminf(fmaxf(g, -1e2f), 1e2f) : g;
}

template <int VAR, int NPL>
__global__ __launch_bounds__(256) void norm_gate_fwd(NgDims dm, const float* __restrict__ x,
                                                     const bf16* __restrict__ gate,
                                                     const float* __restrict__ weight,
                                                     bf16* __restrict__ out) {
  const int row = blockIdx.x * 4 + wave_id();
  if (row >= dm.rows) return;  // wave-uniform
  const size_t ro = (size_t)row * dm.d;
  NgRow<VAR, NPL> r;
  r.load(x + ro, gate + ro);
  const float inv = r.inv_rms(dm.d, dm.eps);
  const int lane = lane_id();
#pragma unroll
  for (int s = 0; s < NPL; ++s) {
    const int c = 8 * (lane + 64 * s);
    float w8[8], o8[8];
    load8(weight + c, w8);
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      const float nb = bf16r(r.x[s][j] * (inv * w8[j]));
      const float gc = gate_in<VAR>(r.g[s][j]);
      const float sl = bf16r(gc * sigmoidf_(gc));
      float v = bf16r(nb * sl);
      if (VAR == kNgMamba2) v = fminf(fmaxf(v, -3e2f), 3e2f);
      o8[j] = v;
    }
    store8(out + ro + c, o8);
  }
}

// Gradients of the epilogue for dout = d loss / d out (bf16):
//   dx (fp32), dgate (bf16), and per-wave partial sums of dweight.
// The VJPs follow the forward's dtype flow: the bf16 products give bf16
// cotangents, the bf16 casts pass the cotangent through, the clips mask it.
template <int VAR, int NPL>
__global__ __launch_bounds__(256) void norm_gate_bwd(NgDims dm, const float* __restrict__ x,
                                                     const bf16* __restrict__ gate,
                                                     const float* __restrict__ weight,
                                                     const bf16* __restrict__ dout,
                                                     float* __restrict__ dx, bf16* __restrict__ dgate,
                                                     float* __restrict__ part) {
  const int lane = lane_id();
  const int wg = blockIdx.x * 4 + wave_id(), nwave = gridDim.x * 4;
  float dw[NPL][8];
#pragma unroll
  for (int s = 0; s < NPL; ++s)
#pragma unroll
    for (int j = 0; j < 8; ++j) dw[s][j] = 0.f;
  for (int row = wg; row < dm.rows; row += nwave) {
    const size_t ro = (size_t)row * dm.d;
    NgRow<VAR, NPL> r;
    r.load(x + ro, gate + ro);
    float du[NPL][8];
#pragma unroll
    for (int s = 0; s < NPL; ++s) load8(dout + ro + 8 * (lane + 64 * s), du[s]);
    const float inv = r.inv_rms(dm.d, dm.eps);
    // d_n = dout * silu (bf16), dgate from dout * n; the row sum for the
    // rsqrt term: sum_c d_n w x
    float dn[NPL][8];
    float dot = 0.f;
#pragma unroll
    for (int s = 0; s < NPL; ++s) {
      const int c = 8 * (lane + 64 * s);
      float w8[8], dg8[8];
      load8(weight + c, w8);
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        const float mul = inv * w8[j];
        const float nb = bf16r(r.x[s][j] * mul);
        const float g = r.g[s][j];
        const float gc = gate_in<VAR>(g);
        const float sg = sigmoidf_(gc);
        const float sl = bf16r(gc * sg);
        float u = du[s][j];
        if (VAR == kNgMamba2) {  // clip(+-3e2) of the product (model.py:524)
          const float pr = bf16r(nb * sl);
          u *= clip_grad(pr, 3e2f);
        }
        const float d_nb = bf16r(u * sl);
        const float d_sl = bf16r(u * nb);
        float d_g = bf16r(d_sl * (sg * (1.f + gc * (1.f - sg))));
        if (VAR == kNgGdn2) d_g *= clip_grad(g, 1e2f);  // clip(+-1e2) (model.py:613)
        dg8[j] = d_g;
        dn[s][j] = d_nb;
        dot += d_nb * w8[j] * r.x[s][j];
        dw[s][j] += d_nb * r.x[s][j] * inv;
      }
      store8(dgate + ro + c, dg8);
    }
    dot = wave_sum(dot);
    // x * inv * w:  dx = d_n w inv - x inv^3 / d * sum_c d_n w x
    const float k3 = inv * inv * inv * dot / (float)dm.d;
#pragma unroll
    for (int s = 0; s < NPL; ++s) {
      const int c = 8 * (lane + 64 * s);
      float w8[8], o8[8];
      load8(weight + c, w8);
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        o8[j] = dn[s][j] * w8[j] * inv - r.x[s][j] * k3;
        // Mamba2: the fp32 promotion of bf16(y) returns a bf16 cotangent
        if (VAR == kNgMamba2) o8[j] = bf16r(o8[j]);
      }
      store8(dx + ro + c, o8);
    }
  }
  // the four waves' partial sums combined through LDS, one 512-column piece
  // at a time, into this workgroup's partial row
  __shared__ __attribute__((aligned(16))) float red[4][512];
  float* pw = part + (size_t)blockIdx.x * dm.d;
  const int wv = wave_id();
#pragma unroll
  for (int s = 0; s < NPL; ++s) {
    store8(&red[wv][8 * lane], dw[s]);
    __syncthreads();
    if (wv == 0) {
      float a[8], t[8];
      load8(&red[0][8 * lane], a);
#pragma unroll
      for (int u = 1; u < 4; ++u) {
        load8(&red[u][8 * lane], t);
#pragma unroll
        for (int j = 0; j < 8; ++j) a[j] += t[j];
      }
      store8(pw + 8 * (lane + 64 * s), a);
    }
    __syncthreads();
  }
}

// The same gradients for wide rows (d >= 4096): one row at a time per
// workgroup, wave w holding pieces [w NPW, (w + 1) NPW) of it (channel
// 8 (lane + 64 s)), so a lane keeps NPL / 4 pieces of each array instead of
// NPL.  The row's two sums (x^2 and d_n w x) cross the four waves through
// LDS, alternating buffers, one barrier each; every wave's weight-gradient
// partial sums cover its own channels, so the workgroup's partial row needs
// no combine.
template <int VAR, int NPL>
__global__ __launch_bounds__(256) void norm_gate_bwd_wide(NgDims dm, const float* __restrict__ x,
                                                          const bf16* __restrict__ gate,
                                                          const float* __restrict__ weight,
                                                          const bf16* __restrict__ dout,
                                                          float* __restrict__ dx, bf16* __restrict__ dgate,
                                                          float* __restrict__ part) {
  constexpr int NPW = NPL / 4;
  static_assert(NPL % 4 == 0, "whole pieces per wave");
  __shared__ float red[2][4];
  const int lane = lane_id(), wv = wave_id();
  float dw[NPW][8];
#pragma unroll
  for (int s = 0; s < NPW; ++s)
#pragma unroll
    for (int j = 0; j < 8; ++j) dw[s][j] = 0.f;
  for (int row = blockIdx.x; row < dm.rows; row += gridDim.x) {
    const size_t ro = (size_t)row * dm.d;
    float xr[NPW][8], gr[NPW][8], du[NPW][8];
    float ss = 0.f;
#pragma unroll
    for (int s = 0; s < NPW; ++s) {
      const int c = 8 * (lane + 64 * (wv * NPW + s));
      load8(x + ro + c, xr[s]);
      load8(gate + ro + c, gr[s]);
      load8(dout + ro + c, du[s]);
    }
#pragma unroll
    for (int s = 0; s < NPW; ++s)
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        if (VAR == kNgMamba2) xr[s][j] = bf16r(xr[s][j]);
        ss += xr[s][j] * xr[s][j];
      }
    ss = wave_sum(ss);
    if (lane == 0) red[0][wv] = ss;
    __syncthreads();
    const float inv = rsqrtf((red[0][0] + red[0][1] + red[0][2] + red[0][3]) / (float)dm.d + dm.eps);
    float dn[NPW][8];
    float dot = 0.f;
#pragma unroll
    for (int s = 0; s < NPW; ++s) {
      const int c = 8 * (lane + 64 * (wv * NPW + s));
      float w8[8], dg8[8];
      load8(weight + c, w8);
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        const float mul = inv * w8[j];
        const float nb = bf16r(xr[s][j] * mul);
        const float g = gr[s][j];
        const float gc = gate_in<VAR>(g);
        const float sg = sigmoidf_(gc);
        const float sl = bf16r(gc * sg);
        float u = du[s][j];
        if (VAR == kNgMamba2) {  // clip(+-3e2) of the product (model.py:524)
          const float pr = bf16r(nb * sl);
          u *= clip_grad(pr, 3e2f);
        }
        const float d_nb = bf16r(u * sl);
        const float d_sl = bf16r(u * nb);
        float d_g = bf16r(d_sl * (sg * (1.f + gc * (1.f - sg))));
        if (VAR == kNgGdn2) d_g *= clip_grad(g, 1e2f);  // clip(+-1e2) (model.py:613)
        dg8[j] = d_g;
        dn[s][j] = d_nb;
        dot += d_nb * w8[j] * xr[s][j];
        dw[s][j] += d_nb * xr[s][j] * inv;
      }
      store8(dgate + ro + c, dg8);
    }
    dot = wave_sum(dot);
    if (lane == 0) red[1][wv] = dot;
    __syncthreads();
    const float dsum = red[1][0] + red[1][1] + red[1][2] + red[1][3];
    const float k3 = inv * inv * inv * dsum / (float)dm.d;
#pragma unroll
    for (int s = 0; s < NPW; ++s) {
      const int c = 8 * (lane + 64 * (wv * NPW + s));
      float w8[8], o8[8];
      load8(weight + c, w8);
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        o8[j] = dn[s][j] * w8[j] * inv - xr[s][j] * k3;
        if (VAR == kNgMamba2) o8[j] = bf16r(o8[j]);
      }
      store8(dx + ro + c, o8);
    }
  }
  float* pw = part + (size_t)blockIdx.x * dm.d;
#pragma unroll
  for (int s = 0; s < NPW; ++s) store8(pw + 8 * (lane + 64 * (wv * NPW + s)), dw[s]);
}

// dweight[c] = sum over the partial rows: 64 columns per workgroup of 16
// waves; wave w takes the rows w, w + 16, ... with eight loads in flight,
// then LDS combines the 16 sums.
__global__ __launch_bounds__(1024) void norm_gate_dweight(int d, int nparts, const float* __restrict__ part,
                                                          float* __restrict__ dweight) {
  constexpr int NWV = 16, U = 8;
  __shared__ float red[NWV][64];
  const int c = blockIdx.x * 64 + lane_id(), w = wave_id();
  float acc[U];
#pragma unroll
  for (int u = 0; u < U; ++u) acc[u] = 0.f;
  int k = w;
  for (; k + (U - 1) * NWV < nparts; k += U * NWV) {
#pragma unroll
    for (int u = 0; u < U; ++u) acc[u] += part[(size_t)(k + u * NWV) * d + c];
  }
  for (; k < nparts; k += NWV) acc[0] += part[(size_t)k * d + c];
  float t = 0.f;
#pragma unroll
  for (int u = 0; u < U; ++u) t += acc[u];
  red[w][lane_id()] = t;
  __syncthreads();
  if (w == 0) {
    float s = 0.f;
#pragma unroll
    for (int u = 0; u < NWV; ++u) s += red[u][lane_id()];
    dweight[c] = s;
  }
}

// ------------------------------------------------------------------ host
static int ng_check(const atomic_norm_gate_args* a) {
  if (!a) return ATOMIC_ERR_NULL;
  if (a->variant != ATOMIC_NORM_GATE_GDN2 && a->variant != ATOMIC_NORM_GATE_MAMBA2) return ATOMIC_ERR_SHAPE;
  if (a->rows <= 0 || a->dim <= 0 || a->dim % 512 != 0 || a->dim > 8192) return ATOMIC_ERR_SHAPE;
  // the instantiated row widths (ng_dispatch): 512 x {1, 2, 3, 4, 6, 8, 12, 16}
  switch (a->dim / 512) {
    case 1: case 2: case 3: case 4: case 6: case 8: case 12: case 16: break;
    default: return ATOMIC_ERR_SHAPE;
  }
  if (!(a->eps >= 0.f)) return ATOMIC_ERR_SHAPE;
  return ATOMIC_OK;
}

// backward workgroups (four rows at a time each), one weight-gradient
// partial row per workgroup
static int ng_parts(const atomic_norm_gate_args* a) {
  const int wgs = (a->rows + 3) / 4;
  return wgs < 512 ? wgs : 512;
}

template <typename F>
static int ng_dispatch(int dim, F&& f) {
  switch (dim / 512) {
    case 1: return f(IntC<1>{});
    case 2: return f(IntC<2>{});
    case 3: return f(IntC<3>{});
    case 4: return f(IntC<4>{});
    case 6: return f(IntC<6>{});
    case 8: return f(IntC<8>{});
    case 12: return f(IntC<12>{});
    case 16: return f(IntC<16>{});
    default: return ATOMIC_ERR_SHAPE;
  }
}

}  // namespace ah

using namespace ah;

extern "C" size_t atomic_norm_gate_workspace_size(const atomic_norm_gate_args* a) {
  if (ng_check(a) != ATOMIC_OK) return 0;
  return (size_t)ng_parts(a) * (size_t)a->dim * sizeof(float);
}

extern "C" int atomic_norm_gate_fwd(const atomic_norm_gate_args* a, const float* x, const void* gate,
                                    const float* weight, void* out, void* stream) {
  int rc = ng_check(a);
  if (rc) return rc;
  if (!x || !gate || !weight || !out) return ATOMIC_ERR_NULL;
  hipStream_t st = (hipStream_t)stream;
  const NgDims dm{a->rows, a->dim, a->eps};
  const unsigned nwg = (unsigned)((a->rows + 3) / 4);
  Launch L{a->profile, st};
  return ng_dispatch(a->dim, [&](auto Nc) {
    constexpr int NPL = decltype(Nc)::value;
    return L("norm_gate_fwd", [&] {
      if (a->variant == ATOMIC_NORM_GATE_GDN2)
        hipLaunchKernelGGL((norm_gate_fwd<kNgGdn2, NPL>), dim3(nwg), dim3(256), 0, st, dm, x,
                           (const bf16*)gate, weight, (bf16*)out);
      else
        hipLaunchKernelGGL((norm_gate_fwd<kNgMamba2, NPL>), dim3(nwg), dim3(256), 0, st, dm, x,
                           (const bf16*)gate, weight, (bf16*)out);
    });
  });
}

extern "C" int atomic_norm_gate_bwd(const atomic_norm_gate_args* a, const float* x, const void* gate,
                                    const float* weight, const void* dout, float* dx, void* dgate,
                                    float* dweight, void* workspace, size_t workspace_bytes,
                                    void* stream) {
  int rc = ng_check(a);
  if (rc) return rc;
  if (!x || !gate || !weight || !dout || !dx || !dgate || !dweight) return ATOMIC_ERR_NULL;
  if (!workspace || workspace_bytes < atomic_norm_gate_workspace_size(a)) return ATOMIC_ERR_WORKSPACE;
  ws_tag_clobber(workspace, atomic_norm_gate_workspace_size(a));
  hipStream_t st = (hipStream_t)stream;
  const NgDims dm{a->rows, a->dim, a->eps};
  const int nparts = ng_parts(a);
  float* part = (float*)workspace;
  Launch L{a->profile, st};
  rc = ng_dispatch(a->dim, [&](auto Nc) {
    constexpr int NPL = decltype(Nc)::value;
    return L("norm_gate_bwd", [&] {
      // rows of d >= 4096 take a workgroup each (the per-lane arrays of one
      // wave per row would not fit the registers)
      if constexpr (NPL >= 8) {
        if (a->variant == ATOMIC_NORM_GATE_GDN2)
          hipLaunchKernelGGL((norm_gate_bwd_wide<kNgGdn2, NPL>), dim3((unsigned)nparts), dim3(256), 0, st,
                             dm, x, (const bf16*)gate, weight, (const bf16*)dout, dx, (bf16*)dgate, part);
        else
          hipLaunchKernelGGL((norm_gate_bwd_wide<kNgMamba2, NPL>), dim3((unsigned)nparts), dim3(256), 0, st,
                             dm, x, (const bf16*)gate, weight, (const bf16*)dout, dx, (bf16*)dgate, part);
      } else {
        if (a->variant == ATOMIC_NORM_GATE_GDN2)
          hipLaunchKernelGGL((norm_gate_bwd<kNgGdn2, NPL>), dim3((unsigned)nparts), dim3(256), 0, st,
                             dm, x, (const bf16*)gate, weight, (const bf16*)dout, dx, (bf16*)dgate, part);
        else
          hipLaunchKernelGGL((norm_gate_bwd<kNgMamba2, NPL>), dim3((unsigned)nparts), dim3(256), 0, st,
                             dm, x, (const bf16*)gate, weight, (const bf16*)dout, dx, (bf16*)dgate, part);
      }
    });
  });
  if (rc) return rc;
  return L("norm_gate_dweight", [&] {
    hipLaunchKernelGGL(norm_gate_dweight, dim3((unsigned)(a->dim / 64)), dim3(1024), 0, st, a->dim, nparts,
                       part, dweight);
  });
}
