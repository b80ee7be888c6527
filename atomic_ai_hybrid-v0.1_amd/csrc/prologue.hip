// Fused prologue of the GDN2 block (the path's upstream caller), forward and
// backward, for gfx950.  From the projection outputs (bf16 [B, L, d],
// d = H dh) it produces the path's inputs q, k, v, w, b (bf16) and g (fp32)
// in the [B, L, H, dh] layout the chunk pipeline reads, with the semantics of
// GatedDeltaNet2J.__call__ (reference model.py:574-619):
//   q, k: normalize(silu(conv(lin) + bias)) per head    v: clip(silu(conv + bias), +-50)
//   b, w: sigmoid(pre)     g: nan_to_num(-exp(clip(a, +-20)) softplus(f))
//   every output: nan_to_num(clip(., +-1e3))
// conv is the causal depthwise convolution (d_conv = 4 taps) with the fp32
// parameters cast to bf16; normalize(t) = t rsqrt(sum_head t^2 + eps^2).
// bf16 roundings follow the reference's dtypes: each bf16 elementwise op
// rounds once, the conv taps and the head's sum of squares accumulate in
// fp32 and round once.
//
// Mapping: one wave per (batch, token tile, 512 channels); lane l holds the
// 8 consecutive channels 8 l .. 8 l + 7 of the block, so a head's channels
// sit in dh / 8 consecutive lanes (its sum of squares is a lane-group
// reduction) and every access is a 16-byte vector.  The convolution slides a
// register window over the tile's tokens (the forward walks time upwards
// with the three previous inputs, the backward walks it downwards with the
// three following cotangents, recomputed past the tile's end).  Parameter
// gradients: each workgroup (four consecutive tiles) combines its waves'
// sums through LDS into one partial row; a final kernel sums the rows.
#include "../../include/atomic_hybrid.h"
#include "common.hpp"
#include "launch.hpp"
#include "ws_tag.hpp"
#include "proj_gemm.hpp"

namespace ah {

constexpr int kDc = 4;         // d_conv of the model config
constexpr int kTileF = 16;     // tokens per wave, forward
constexpr int kTileB = 32;     // tokens per wave, backward

struct PlDims {
  int B, L, H, dh, d;
  float eps;
  int ldi;  // elements between consecutive tokens of the convolutions' input (>= d)
};

__device__ __forceinline__ float bfr(float x) { return (float)(bf16)x; }
// logistic with the hardware reciprocal (about 1 ulp; every use rounds to bf16)
__device__ __forceinline__ float sigm(float x) { return __builtin_amdgcn_rcpf(1.f + __expf(-x)); }
// jax.nn.softplus(x) = logaddexp(x, 0) = max(x, 0) + log(1 + e^{-|x|}); the
// fast log of 1 + e (in [1, 2]) drops only terms below 1e-7 of max(x, 0)
__device__ __forceinline__ float softplus_(float x) { return fmaxf(x, 0.f) + __logf(1.f + __expf(-fabsf(x))); }

// 8 bf16 of a row as floats, from a raw 16-byte piece
__device__ __forceinline__ void unpack8(const u32x4& r, float (&o)[8]) {
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    o[2 * i] = __uint_as_float(r[i] << 16);
    o[2 * i + 1] = __uint_as_float(r[i] & 0xffff0000u);
  }
}
// the row piece of token t, or zeros for t < 0 (the conv's left padding); the
// load itself is unconditional (clamped row) so loads can be issued early
__device__ __forceinline__ u32x4 row_or_zero(const bf16* p, int t, int ld) {
  const u32x4 v = *reinterpret_cast<const u32x4*>(p + (size_t)(t < 0 ? 0 : t) * ld);
  const u32x4 z = {0u, 0u, 0u, 0u};
  return t < 0 ? z : v;
}
// cotangent factor of clip(v, -c, c) = min(max(v, -c), c): ties split evenly
__device__ __forceinline__ float clip_g(float v, float c) {
  const float a = fabsf(v);
  return a < c ? 1.f : (a == c ? 0.5f : 0.f);
}
// nan_to_num(clip(x, -c, c)) (model.py:615-617)
__device__ __forceinline__ float sanit(float x, float c) {
  if (__builtin_isnan(x)) return 0.f;
  return fminf(fmaxf(x, -c), c);
}

// v + v of the lane that the DPP control CTRL selects (within a 16-lane row)
template <int CTRL>
__device__ __forceinline__ float dpp_add(float v) {
  return v + __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), CTRL, 0xF, 0xF, false));
}
// Sum over the lanes of one head (G = dh / 8 consecutive lanes, 8 or 16),
// every lane getting the total, by DPP steps inside a 16-lane row: swap
// neighbours, swap pairs (quad_perm 1032, 2301), mirror the 8-lane halves,
// mirror the row.  Each step adds a lane pair's values in both lanes (the
// same sum), so the lanes of a head end with identical totals.
template <int G>
__device__ __forceinline__ float head_sum(float v) {
  static_assert(G == 8 || G == 16 || G == 32, "8, 16 or 32 lanes per head");
  v = dpp_add<0xB1>(v);   // quad_perm [1, 0, 3, 2]
  v = dpp_add<0x4E>(v);   // quad_perm [2, 3, 0, 1]
  v = dpp_add<0x141>(v);  // row_half_mirror
  if (G >= 16) v = dpp_add<0x140>(v);  // row_mirror
  if (G == 32) v += __shfl_xor(v, 16);  // the neighbouring row
  return v;
}

// the lane's conv weights (bf16-rounded, [tap][CPL channels]) and biases
template <int CPL = 8>
struct ConvW {
  float w[kDc][CPL], b[CPL];
  __device__ __forceinline__ void load(const float* __restrict__ cw, const float* __restrict__ cb, int c) {
#pragma unroll
    for (int j = 0; j < CPL; ++j) {
      const float4 t = *reinterpret_cast<const float4*>(cw + (size_t)(c + j) * kDc);
      w[0][j] = bfr(t.x); w[1][j] = bfr(t.y); w[2][j] = bfr(t.z); w[3][j] = bfr(t.w);
      b[j] = bfr(cb[c + j]);
    }
  }
};

// silu(conv + bias) at one token from the window u[t-3..t] (tap order)
template <int CPL>
__device__ __forceinline__ void conv_silu(const ConvW<CPL>& W, const float (&win)[kDc][CPL], float (&pre)[CPL],
                                          float (&s)[CPL]) {
#pragma unroll
  for (int j = 0; j < CPL; ++j) {
    float acc = 0.f;
#pragma unroll
    for (int tp = 0; tp < kDc; ++tp) acc += win[tp][j] * W.w[tp][j];
    pre[j] = bfr(bfr(acc) + W.b[j]);
    s[j] = bfr(pre[j] * sigm(pre[j]));
  }
}

// ---------------------------------------------------------------- forward
// Output of a conv path (MODE): kNorm (GDN2 q, k: per-head normalisation),
// kClip50 (GDN2 v: clip +-50), kPlain (Mamba2 x); every one is sanitised +-1e3.
enum { kNorm = 0, kClip50 = 1, kPlain = 2 };

template <int MODE, int DH>
__global__ __launch_bounds__(256) void prologue_conv_fwd(PlDims dm, const bf16* __restrict__ lin,
                                                         const float* __restrict__ conv_w,
                                                         const float* __restrict__ conv_b,
                                                         bf16* __restrict__ out) {
  constexpr int G = DH / 8;
  const int lane = lane_id();
  const int nblk = dm.d / 512, ntile = dm.L / kTileF;
  const int wv = blockIdx.x * 4 + wave_id();
  if (wv >= dm.B * ntile * nblk) return;  // wave-uniform
  const int cb = wv % nblk, tile = (wv / nblk) % ntile, b = wv / (nblk * ntile);
  const int c = cb * 512 + 8 * lane, t0 = tile * kTileF;
  ConvW<8> W;
  W.load(conv_w, conv_b, c);
  const bf16* u = lin + (size_t)b * dm.L * dm.ldi + c;
  bf16* o = out + (size_t)b * dm.L * dm.d + c;
  // every input row of the tile (three before it) requested at once
  u32x4 rows[kTileF + kDc - 1];
#pragma unroll
  for (int r = 0; r < kTileF + kDc - 1; ++r) rows[r] = row_or_zero(u, t0 - (kDc - 1) + r, dm.ldi);
  float win[kDc][8];
#pragma unroll
  for (int tp = 0; tp < kDc - 1; ++tp) unpack8(rows[tp], win[tp]);
#pragma unroll
  for (int i = 0; i < kTileF; ++i) {
    const int t = t0 + i;
    unpack8(rows[i + kDc - 1], win[kDc - 1]);
    float pre[8], s[8], y[8];
    conv_silu(W, win, pre, s);
    if (MODE == kClip50) {
#pragma unroll
      for (int j = 0; j < 8; ++j) y[j] = sanit(fminf(fmaxf(s[j], -50.f), 50.f), 1e3f);
    } else if (MODE == kPlain) {
#pragma unroll
      for (int j = 0; j < 8; ++j) y[j] = sanit(s[j], 1e3f);
    } else {
      float ss = 0.f;
#pragma unroll
      for (int j = 0; j < 8; ++j) ss += bfr(s[j] * s[j]);
      ss = bfr(head_sum<G>(ss));
      const float r = bfr(rsqrtf(bfr(ss + dm.eps * dm.eps)));
#pragma unroll
      for (int j = 0; j < 8; ++j) y[j] = sanit(bfr(s[j] * r), 1e3f);
    }
    store8(o + (size_t)t * dm.d, y);
#pragma unroll
    for (int tp = 0; tp < kDc - 1; ++tp)
#pragma unroll
      for (int j = 0; j < 8; ++j) win[tp][j] = win[tp + 1][j];
  }
}

// b, w = sigmoid(pre); g = nan_to_num(-exp(clip(a)) softplus(f)); 8 channels per thread
template <int DH>
__global__ __launch_bounds__(256) void prologue_gates_fwd(PlDims dm, const bf16* __restrict__ b_pre,
                                                          const bf16* __restrict__ w_pre,
                                                          const bf16* __restrict__ f_pre,
                                                          const float* __restrict__ a_param,
                                                          bf16* __restrict__ bo, bf16* __restrict__ wo,
                                                          float* __restrict__ go) {
  const size_t e = ((size_t)blockIdx.x * 256 + threadIdx.x) * 8;
  if (e >= (size_t)dm.B * dm.L * dm.d) return;
  const int h = (int)((e % dm.d) / DH);
  const float ea = __expf(fminf(fmaxf(a_param[h], -20.f), 20.f));
  float bv[8], wv[8], fv[8], gv[8];
  load8(b_pre + e, bv);
  load8(w_pre + e, wv);
  load8(f_pre + e, fv);
#pragma unroll
  for (int j = 0; j < 8; ++j) {
    bv[j] = sanit(bfr(sigm(bv[j])), 1e3f);
    wv[j] = sanit(bfr(sigm(wv[j])), 1e3f);
    float g = -ea * softplus_(fv[j]);
    if (__builtin_isnan(g)) g = 0.f;
    else if (__builtin_isinf(g)) g = g > 0.f ? 0.f : -20.f;
    gv[j] = sanit(g, 1e3f);
  }
  store8(bo + e, bv);
  store8(wo + e, wv);
  store8(go + e, gv);
}

// ---------------------------------------------------------------- backward
// Per token of the reverse sweep: the cotangent of the conv accumulator
// (e = d(conv + bias)), from the output cotangent dy and the forward values.
template <int MODE, int G, int CPL>
__device__ __forceinline__ void conv_out_vjp(const ConvW<CPL>& W, const float (&win)[kDc][CPL],
                                             const float (&dy)[CPL], float eps, float (&e)[CPL]) {
  float pre[CPL], s[CPL], ds[CPL];
  conv_silu(W, win, pre, s);
  if (MODE == kClip50) {
#pragma unroll
    for (int j = 0; j < CPL; ++j) {
      const float v = fminf(fmaxf(s[j], -50.f), 50.f);
      ds[j] = bfr(dy[j] * clip_g(v, 1e3f) * clip_g(s[j], 50.f));
    }
  } else if (MODE == kPlain) {
#pragma unroll
    for (int j = 0; j < CPL; ++j) ds[j] = bfr(dy[j] * clip_g(s[j], 1e3f));
  } else {
    float ss = 0.f;
#pragma unroll
    for (int j = 0; j < CPL; ++j) ss += bfr(s[j] * s[j]);
    ss = bfr(head_sum<G>(ss));
    const float r = bfr(rsqrtf(bfr(ss + eps * eps)));
    // output clip (|y| <= 1 passes), then the gradient sanitiser (model.py:206-214)
    float gy[CPL], dot = 0.f;
#pragma unroll
    for (int j = 0; j < CPL; ++j) {
      const float y = bfr(s[j] * r);
      float g = dy[j] * clip_g(y, 1e3f);
      g = __builtin_isnan(g) ? 0.f : fminf(fmaxf(g, -1e3f), 1e3f);
      gy[j] = g;
      dot += g * s[j];
    }
    dot = head_sum<G>(dot);
    const float r3 = r * r * r;
#pragma unroll
    for (int j = 0; j < CPL; ++j) ds[j] = bfr(gy[j] * r - s[j] * r3 * dot);
  }
#pragma unroll
  for (int j = 0; j < CPL; ++j) {
    const float sg = sigm(pre[j]);
    e[j] = bfr(ds[j] * (sg * (1.f + pre[j] * (1.f - sg))));
  }
}

// 4 bf16 of a row as floats, from a raw 8-byte piece
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));
__device__ __forceinline__ void unpack4(const u32x2& r, float (&o)[4]) {
#pragma unroll
  for (int i = 0; i < 2; ++i) {
    o[2 * i] = __uint_as_float(r[i] << 16);
    o[2 * i + 1] = __uint_as_float(r[i] & 0xffff0000u);
  }
}
__device__ __forceinline__ u32x2 row4_or_zero(const bf16* p, int t, int ld) {
  const u32x2 v = *reinterpret_cast<const u32x2*>(p + (size_t)(t < 0 ? 0 : t) * ld);
  const u32x2 z = {0u, 0u};
  return t < 0 ? z : v;
}
__device__ __forceinline__ void store4f(bf16* p, const float (&v)[4]) {
  bf16x4 o;
#pragma unroll
  for (int i = 0; i < 4; ++i) o[i] = (bf16)v[i];
  *reinterpret_cast<bf16x4*>(p) = o;
}

// Partial sums of one workgroup (4 waves, 64 CPL channels each) combined
// through LDS and written as one row of NV floats per channel ([d][NV] at dst).
template <int NV, int CPL>
__device__ __forceinline__ void combine_partials(float (&v)[NV][CPL], float* __restrict__ dst, int c) {
  __shared__ __attribute__((aligned(16))) float red[4][64 * CPL];
  const int w = wave_id(), lane = lane_id();
#pragma unroll
  for (int k = 0; k < NV; ++k) {
#pragma unroll
    for (int j = 0; j < CPL; ++j) red[w][CPL * lane + j] = v[k][j];
    __syncthreads();
    if (w == 0) {
#pragma unroll
      for (int j = 0; j < CPL; ++j)
        dst[(size_t)(c + j) * NV + k] = red[0][CPL * lane + j] + red[1][CPL * lane + j] +
                                        red[2][CPL * lane + j] + red[3][CPL * lane + j];
    }
    __syncthreads();
  }
}

// Four channels per lane (a wave covers 256 channels): half the registers of
// the 8-channel mapping, so four waves fit per SIMD.  The four waves of a
// workgroup take four consecutive tiles of one (batch, 256-channel block);
// partial row index = (batch, tile group).
constexpr int kCplB = 4;
template <int MODE, int DH>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(4, 4))) void prologue_conv_bwd(
    PlDims dm, const bf16* __restrict__ lin, const float* __restrict__ conv_w, const float* __restrict__ conv_b,
    const bf16* __restrict__ dout, bf16* __restrict__ dlin, float* __restrict__ part) {
  constexpr int CPL = kCplB, G = DH / CPL, NV = kDc + 1;  // partials: the 4 taps, then the bias
  const int lane = lane_id();
  const int nblk = dm.d / (64 * CPL), ngrp = dm.L / (4 * kTileB);
  const int cb = blockIdx.x % nblk, grp = (blockIdx.x / nblk) % ngrp, b = blockIdx.x / (nblk * ngrp);
  const int tile = grp * 4 + wave_id();
  const int c = cb * 64 * CPL + CPL * lane, t0 = tile * kTileB;
  ConvW<CPL> W;
  W.load(conv_w, conv_b, c);
  const bf16* u = lin + (size_t)b * dm.L * dm.ldi + c;
  const bf16* dy = dout + (size_t)b * dm.L * dm.d + c;
  bf16* du = dlin + (size_t)b * dm.L * dm.d + c;
  float acc[NV][CPL];
#pragma unroll
  for (int k = 0; k < NV; ++k)
#pragma unroll
    for (int j = 0; j < CPL; ++j) acc[k][j] = 0.f;
  // reverse sweep from the last halo token: window u[t-3..t] and the conv
  // cotangents e[t+1..t+3] of the tokens above
  const int t_hi = min(t0 + kTileB + kDc - 2, dm.L - 1);
  float win[kDc][CPL], en[kDc - 1][CPL];
#pragma unroll
  for (int tp = 0; tp < kDc; ++tp) unpack4(row4_or_zero(u, t_hi - (kDc - 1) + tp, dm.ldi), win[tp]);
#pragma unroll
  for (int k = 0; k < kDc - 1; ++k)
#pragma unroll
    for (int j = 0; j < CPL; ++j) en[k][j] = 0.f;
#pragma unroll 4
  for (int t = t_hi; t >= t0; --t) {
    float g4[CPL], e[CPL];
    const u32x2 rdy = *reinterpret_cast<const u32x2*>(dy + (size_t)t * dm.d);
    const u32x2 rnext = row4_or_zero(u, t - kDc, dm.ldi);
    unpack4(rdy, g4);
    conv_out_vjp<MODE, G, CPL>(W, win, g4, dm.eps, e);
    if (t < t0 + kTileB) {
      // d lin[t] = sum_s e[t + s] w[3 - s]; the parameter sums
      float o4[CPL];
#pragma unroll
      for (int j = 0; j < CPL; ++j) {
        float v = e[j] * W.w[kDc - 1][j];
#pragma unroll
        for (int s2 = 1; s2 < kDc; ++s2) v += en[s2 - 1][j] * W.w[kDc - 1 - s2][j];
        o4[j] = v;
#pragma unroll
        for (int tp = 0; tp < kDc; ++tp) acc[tp][j] += e[j] * win[tp][j];
        acc[kDc][j] += e[j];
      }
      store4f(du + (size_t)t * dm.d, o4);
    }
    // slide: e[t] becomes the nearest token above; the window moves down
#pragma unroll
    for (int k = kDc - 2; k >= 1; --k)
#pragma unroll
      for (int j = 0; j < CPL; ++j) en[k][j] = en[k - 1][j];
#pragma unroll
    for (int j = 0; j < CPL; ++j) en[0][j] = e[j];
#pragma unroll
    for (int tp = kDc - 1; tp >= 1; --tp)
#pragma unroll
      for (int j = 0; j < CPL; ++j) win[tp][j] = win[tp - 1][j];
    unpack4(rnext, win[0]);
  }
  combine_partials<NV, CPL>(acc, part + ((size_t)b * ngrp + grp) * dm.d * NV, c);
}

// b, w, g gradients; per-head partial sums of da
template <int DH>
__global__ __launch_bounds__(256) void prologue_gates_bwd(PlDims dm, const bf16* __restrict__ b_pre,
                                                          const bf16* __restrict__ w_pre,
                                                          const bf16* __restrict__ f_pre,
                                                          const float* __restrict__ a_param,
                                                          const bf16* __restrict__ db, const bf16* __restrict__ dw,
                                                          const float* __restrict__ dg, bf16* __restrict__ dbp,
                                                          bf16* __restrict__ dwp, bf16* __restrict__ dfp,
                                                          float* __restrict__ part_a) {
  constexpr int G = DH / 8;
  const int lane = lane_id();
  const int nblk = dm.d / 512, ntile = dm.L / kTileB;
  const int wv = blockIdx.x * 4 + wave_id();
  if (wv >= dm.B * ntile * nblk) return;  // wave-uniform
  const int cb = wv % nblk, tile = (wv / nblk) % ntile, b = wv / (nblk * ntile);
  const int c = cb * 512 + 8 * lane, h = c / DH;
  const float araw = a_param[h];
  const float ea = __expf(fminf(fmaxf(araw, -20.f), 20.f)), ga = clip_g(araw, 20.f);
  float da = 0.f;
#pragma unroll 4
  for (int t = tile * kTileB; t < (tile + 1) * kTileB; ++t) {
    const size_t e = ((size_t)b * dm.L + t) * dm.d + c;
    float bv[8], wv8[8], fv[8], gb[8], gw[8], gg[8], o1[8], o2[8], o3[8];
    load8(b_pre + e, bv);
    load8(w_pre + e, wv8);
    load8(f_pre + e, fv);
    load8(db + e, gb);
    load8(dw + e, gw);
    load8(dg + e, gg);
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      const float sb = bfr(sigm(bv[j])), sw = bfr(sigm(wv8[j]));
      o1[j] = bfr(gb[j] * clip_g(sb, 1e3f) * sb * (1.f - sb));
      o2[j] = bfr(gw[j] * clip_g(sw, 1e3f) * sw * (1.f - sw));
      const float sp = softplus_(fv[j]);
      const float g = -ea * sp;
      // nan_to_num passes the cotangent of finite values; then the +-1e3 clip
      const float dgi = (__builtin_isfinite(g) ? gg[j] : 0.f) * clip_g(g, 1e3f);
      o3[j] = bfr(dgi * (-ea) * sigm(fv[j]));
      da += dgi * g * ga;
    }
    store8(dbp + e, o1);
    store8(dwp + e, o2);
    store8(dfp + e, o3);
  }
  da = head_sum<G>(da);
  // one partial per (wave, head of the block): lane 0 of each head group writes
  if ((lane % G) == 0) part_a[(size_t)wv * (512 / DH) + lane / G] = da;
}

// Column sums of the partial rows: out[c] = sum_r part[r][c] for c < ncol
// (64 columns per workgroup of 16 waves, eight loads in flight per lane).
__global__ __launch_bounds__(1024) void prologue_colsum(int ncol, int nrows, const float* __restrict__ part,
                                                        float* __restrict__ out) {
  constexpr int NWV = 16, U = 8;
  __shared__ float red[NWV][64];
  const int c = blockIdx.x * 64 + lane_id(), w = wave_id();
  const bool ok = c < ncol;
  float acc[U];
#pragma unroll
  for (int u = 0; u < U; ++u) acc[u] = 0.f;
  int k = w;
  if (ok) {
    for (; k + (U - 1) * NWV < nrows; k += U * NWV) {
#pragma unroll
      for (int u = 0; u < U; ++u) acc[u] += part[(size_t)(k + u * NWV) * ncol + c];
    }
    for (; k < nrows; k += NWV) acc[0] += part[(size_t)k * ncol + c];
  }
  float t = 0.f;
#pragma unroll
  for (int u = 0; u < U; ++u) t += acc[u];
  red[w][lane_id()] = t;
  __syncthreads();
  if (w == 0 && ok) {
    float s = 0.f;
#pragma unroll
    for (int u = 0; u < NWV; ++u) s += red[u][lane_id()];
    out[c] = s;
  }
}

// conv weight / bias gradients from the summed [3][d][5] block, bf16-rounded
// like the reference's bf16 conv-parameter cotangents
__global__ __launch_bounds__(256) void prologue_param_split(int d, const float* __restrict__ sums,
                                                            float* __restrict__ dconv_w,
                                                            float* __restrict__ dconv_b) {
  const int i = blockIdx.x * 256 + threadIdx.x;  // (which, channel)
  if (i >= 3 * d) return;
#pragma unroll
  for (int tp = 0; tp < kDc; ++tp) dconv_w[(size_t)i * kDc + tp] = bfr(sums[(size_t)i * (kDc + 1) + tp]);
  dconv_b[i] = bfr(sums[(size_t)i * (kDc + 1) + kDc]);
}

// ---------------------------------------------------------- Mamba2 prologue
// dt = clip(softplus(dt_pre), bf16(1e-2), 1) and B, C, x, dt sanitised
// (reference model.py:426-433): the element-wise part; x's convolution is
// prologue_conv_* in kPlain mode.  A = -exp(clip(A_log, +-20)) (:420-422).
__device__ __forceinline__ float dt_lo() { return bfr(1e-2f); }

__global__ __launch_bounds__(256) void m2_prologue_elem_fwd(size_t n_dt, size_t n_bc, int H,
                                                            const bf16* __restrict__ dt_pre,
                                                            const bf16* __restrict__ b_pre,
                                                            const bf16* __restrict__ c_pre,
                                                            const float* __restrict__ a_log,
                                                            bf16* __restrict__ dt, bf16* __restrict__ bo,
                                                            bf16* __restrict__ co, float* __restrict__ a_out) {
  const size_t e = ((size_t)blockIdx.x * 256 + threadIdx.x) * 8;
  if (e < n_dt) {
    float v[8];
    load8(dt_pre + e, v);
#pragma unroll
    for (int j = 0; j < 8; ++j) v[j] = sanit(fminf(fmaxf(bfr(softplus_(v[j])), dt_lo()), 1.f), 1e3f);
    store8(dt + e, v);
  }
  if (e < n_bc) {
    float b8[8], c8[8];
    load8(b_pre + e, b8);
    load8(c_pre + e, c8);
#pragma unroll
    for (int j = 0; j < 8; ++j) { b8[j] = sanit(b8[j], 1e3f); c8[j] = sanit(c8[j], 1e3f); }
    store8(bo + e, b8);
    store8(co + e, c8);
  }
  if (blockIdx.x == 0)
    for (int h = threadIdx.x; h < H; h += 256) a_out[h] = -__expf(fminf(fmaxf(a_log[h], -20.f), 20.f));
}

// cotangent factor of clip(x, lo, hi) = min(max(x, lo), hi)
__device__ __forceinline__ float clip_range_g(float x, float lo, float hi) {
  const float a = x > lo ? 1.f : (x == lo ? 0.5f : 0.f);
  const float b = x < hi ? 1.f : (x == hi ? 0.5f : 0.f);
  return a * b;
}

__global__ __launch_bounds__(256) void m2_prologue_elem_bwd(size_t n_dt, size_t n_bc, int H,
                                                            const bf16* __restrict__ dt_pre,
                                                            const bf16* __restrict__ b_pre,
                                                            const bf16* __restrict__ c_pre,
                                                            const float* __restrict__ a_log,
                                                            const bf16* __restrict__ ddt, const bf16* __restrict__ dbo,
                                                            const bf16* __restrict__ dco, const float* __restrict__ da,
                                                            bf16* __restrict__ ddt_pre, bf16* __restrict__ db_pre,
                                                            bf16* __restrict__ dc_pre, float* __restrict__ da_log) {
  const size_t e = ((size_t)blockIdx.x * 256 + threadIdx.x) * 8;
  if (e < n_dt) {
    float v[8], g[8], o[8];
    load8(dt_pre + e, v);
    load8(ddt + e, g);
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      const float sp = bfr(softplus_(v[j]));
      const float c = fminf(fmaxf(sp, dt_lo()), 1.f);
      const float dsp = bfr(g[j] * clip_g(c, 1e3f) * clip_range_g(sp, dt_lo(), 1.f));
      o[j] = bfr(dsp * sigm(v[j]));   // softplus' = logistic
    }
    store8(ddt_pre + e, o);
  }
  if (e < n_bc) {
    float b8[8], c8[8], gb[8], gc[8];
    load8(b_pre + e, b8);
    load8(c_pre + e, c8);
    load8(dbo + e, gb);
    load8(dco + e, gc);
#pragma unroll
    for (int j = 0; j < 8; ++j) { gb[j] = bfr(gb[j] * clip_g(b8[j], 1e3f)); gc[j] = bfr(gc[j] * clip_g(c8[j], 1e3f)); }
    store8(db_pre + e, gb);
    store8(dc_pre + e, gc);
  }
  if (blockIdx.x == 0)
    for (int h = threadIdx.x; h < H; h += 256) {
      const float al = a_log[h];
      da_log[h] = da[h] * (-__expf(fminf(fmaxf(al, -20.f), 20.f))) * clip_g(al, 20.f);
    }
}

// one conv's weight / bias gradients from its summed [d][5] block
__global__ __launch_bounds__(256) void prologue_param_split1(int d, const float* __restrict__ sums,
                                                             float* __restrict__ dconv_w,
                                                             float* __restrict__ dconv_b) {
  const int i = blockIdx.x * 256 + threadIdx.x;
  if (i >= d) return;
#pragma unroll
  for (int tp = 0; tp < kDc; ++tp) dconv_w[(size_t)i * kDc + tp] = bfr(sums[(size_t)i * (kDc + 1) + tp]);
  dconv_b[i] = bfr(sums[(size_t)i * (kDc + 1) + kDc]);
}

// ------------------------------------------------------------------ host
static int pl_check(const atomic_gdn2_prologue_args* a) {
  if (!a) return ATOMIC_ERR_NULL;
  if (a->batch <= 0 || a->seqlen <= 0 || a->heads <= 0) return ATOMIC_ERR_SHAPE;
  if (a->dhead != 64 && a->dhead != 128) return ATOMIC_ERR_SHAPE;
  if (a->dconv != kDc) return ATOMIC_ERR_SHAPE;
  if ((a->heads * a->dhead) % 512 != 0) return ATOMIC_ERR_SHAPE;
  if (a->seqlen % (4 * kTileB) != 0) return ATOMIC_ERR_SHAPE;
  if (!(a->eps >= 0.f)) return ATOMIC_ERR_SHAPE;
  return ATOMIC_OK;
}

static PlDims pl_dims(const atomic_gdn2_prologue_args* a) {
  return PlDims{a->batch, a->seqlen, a->heads, a->dhead, a->heads * a->dhead, a->eps, a->heads * a->dhead};
}

// workspace: conv partial rows [3][B][L / 128][d][5], then the da partials
// [B][L / 32][d / 512][512 / dh], then the summed [3][d][5] block
struct PlWs {
  size_t conv, da, sums, total;
  int conv_rows, da_rows;
};
static PlWs pl_ws(const PlDims& d) {
  PlWs w;
  const size_t ngrp = (size_t)d.L / (4 * kTileB);
  w.conv_rows = (int)(3 * d.B * ngrp);
  w.da_rows = (int)((size_t)d.B * (d.L / kTileB) * (d.d / 512));
  auto al = [](size_t x) { return (x + 255) & ~size_t(255); };
  w.conv = 0;
  w.da = al((size_t)w.conv_rows * d.d * (kDc + 1) * 4);
  w.sums = w.da + al((size_t)w.da_rows * (512 / d.dh) * 4);
  w.total = w.sums + al((size_t)3 * d.d * (kDc + 1) * 4);
  return w;
}

}  // namespace ah

using namespace ah;

extern "C" size_t atomic_gdn2_prologue_workspace_size(const atomic_gdn2_prologue_args* a) {
  if (pl_check(a) != ATOMIC_OK) return 0;
  return pl_ws(pl_dims(a)).total;
}

extern "C" int atomic_gdn2_prologue_fwd(const atomic_gdn2_prologue_args* a, const void* q_lin,
                                        const void* k_lin, const void* v_lin, const float* conv_w,
                                        const float* conv_b, const void* b_pre, const void* w_pre,
                                        const void* f_pre, const float* a_param, void* q, void* k,
                                        void* v, void* w, void* b, float* g, void* stream) {
  int rc = pl_check(a);
  if (rc) return rc;
  if (!q_lin || !k_lin || !v_lin || !conv_w || !conv_b || !b_pre || !w_pre || !f_pre || !a_param || !q ||
      !k || !v || !w || !b || !g)
    return ATOMIC_ERR_NULL;
  hipStream_t st = (hipStream_t)stream;
  const PlDims dm = pl_dims(a);
  Launch L{a->profile, st};
  const unsigned nconv = (unsigned)(((size_t)dm.B * (dm.L / kTileF) * (dm.d / 512) + 3) / 4);
  const unsigned ngate = (unsigned)(((size_t)dm.B * dm.L * dm.d / 8 + 255) / 256);
  const bf16* lins[3] = {(const bf16*)q_lin, (const bf16*)k_lin, (const bf16*)v_lin};
  bf16* outs[3] = {(bf16*)q, (bf16*)k, (bf16*)v};
  auto run = [&](auto Dc) {
    constexpr int DH = decltype(Dc)::value;
    int r = L("prologue_conv_fwd", [&] {
      const size_t ow = (size_t)dm.d * kDc, ob = (size_t)dm.d;
      hipLaunchKernelGGL((prologue_conv_fwd<kNorm, DH>), dim3(nconv), dim3(256), 0, st, dm, lins[0], conv_w,
                         conv_b, outs[0]);
      hipLaunchKernelGGL((prologue_conv_fwd<kNorm, DH>), dim3(nconv), dim3(256), 0, st, dm, lins[1],
                         conv_w + ow, conv_b + ob, outs[1]);
      hipLaunchKernelGGL((prologue_conv_fwd<kClip50, DH>), dim3(nconv), dim3(256), 0, st, dm, lins[2],
                         conv_w + 2 * ow, conv_b + 2 * ob, outs[2]);
    });
    if (r) return r;
    return L("prologue_gates_fwd", [&] {
      hipLaunchKernelGGL((prologue_gates_fwd<DH>), dim3(ngate), dim3(256), 0, st, dm, (const bf16*)b_pre,
                         (const bf16*)w_pre, (const bf16*)f_pre, a_param, (bf16*)b, (bf16*)w, g);
    });
  };
  return dm.dh == 64 ? run(IntC<64>{}) : run(IntC<128>{});
}

extern "C" int atomic_gdn2_prologue_bwd(const atomic_gdn2_prologue_args* a, const void* q_lin,
                                        const void* k_lin, const void* v_lin, const float* conv_w,
                                        const float* conv_b, const void* b_pre, const void* w_pre,
                                        const void* f_pre, const float* a_param, const void* dq,
                                        const void* dk, const void* dv, const void* dw, const void* db,
                                        const float* dg, void* dq_lin, void* dk_lin, void* dv_lin,
                                        float* dconv_w, float* dconv_b, void* db_pre, void* dw_pre,
                                        void* df_pre, float* da_param, void* workspace,
                                        size_t workspace_bytes, void* stream) {
  int rc = pl_check(a);
  if (rc) return rc;
  if (!q_lin || !k_lin || !v_lin || !conv_w || !conv_b || !b_pre || !w_pre || !f_pre || !a_param || !dq ||
      !dk || !dv || !dw || !db || !dg || !dq_lin || !dk_lin || !dv_lin || !dconv_w || !dconv_b || !db_pre ||
      !dw_pre || !df_pre || !da_param)
    return ATOMIC_ERR_NULL;
  const PlDims dm = pl_dims(a);
  const PlWs ws = pl_ws(dm);
  if (!workspace || workspace_bytes < ws.total) return ATOMIC_ERR_WORKSPACE;
  ws_tag_clobber(workspace, ws.total);
  unsigned char* wsb = (unsigned char*)workspace;
  float* pconv = (float*)(wsb + ws.conv);
  float* pda = (float*)(wsb + ws.da);
  float* sums = (float*)(wsb + ws.sums);
  hipStream_t st = (hipStream_t)stream;
  Launch L{a->profile, st};
  const int ngrp = dm.L / (4 * kTileB);
  const unsigned nconv = (unsigned)((size_t)dm.B * ngrp * (dm.d / (64 * kCplB)));
  const unsigned ngate = (unsigned)(((size_t)dm.B * (dm.L / kTileB) * (dm.d / 512) + 3) / 4);
  const bf16* lins[3] = {(const bf16*)q_lin, (const bf16*)k_lin, (const bf16*)v_lin};
  const bf16* dys[3] = {(const bf16*)dq, (const bf16*)dk, (const bf16*)dv};
  bf16* dls[3] = {(bf16*)dq_lin, (bf16*)dk_lin, (bf16*)dv_lin};
  auto run = [&](auto Dc) {
    constexpr int DH = decltype(Dc)::value;
    int r = L("prologue_conv_bwd", [&] {
      const size_t ow = (size_t)dm.d * kDc, ob = (size_t)dm.d;
      const size_t op = (size_t)dm.B * ngrp * dm.d * (kDc + 1);  // one conv's partial rows
      hipLaunchKernelGGL((prologue_conv_bwd<kNorm, DH>), dim3(nconv), dim3(256), 0, st, dm, lins[0], conv_w,
                         conv_b, dys[0], dls[0], pconv);
      hipLaunchKernelGGL((prologue_conv_bwd<kNorm, DH>), dim3(nconv), dim3(256), 0, st, dm, lins[1],
                         conv_w + ow, conv_b + ob, dys[1], dls[1], pconv + op);
      hipLaunchKernelGGL((prologue_conv_bwd<kClip50, DH>), dim3(nconv), dim3(256), 0, st, dm, lins[2],
                         conv_w + 2 * ow, conv_b + 2 * ob, dys[2], dls[2], pconv + 2 * op);
    });
    if (r) return r;
    return L("prologue_gates_bwd", [&] {
      hipLaunchKernelGGL((prologue_gates_bwd<DH>), dim3(ngate), dim3(256), 0, st, dm, (const bf16*)b_pre,
                         (const bf16*)w_pre, (const bf16*)f_pre, a_param, (const bf16*)db, (const bf16*)dw, dg,
                         (bf16*)db_pre, (bf16*)dw_pre, (bf16*)df_pre, pda);
    });
  };
  rc = dm.dh == 64 ? run(IntC<64>{}) : run(IntC<128>{});
  if (rc) return rc;
  // parameter gradients: conv partial rows per `which`, then the da partials
  rc = L("prologue_colsum", [&] {
    const int ncol = dm.d * (kDc + 1), rows = dm.B * ngrp;
    for (int wch = 0; wch < 3; ++wch)
      hipLaunchKernelGGL(prologue_colsum, dim3((unsigned)((ncol + 63) / 64)), dim3(1024), 0, st, ncol, rows,
                         pconv + (size_t)wch * rows * ncol, sums + (size_t)wch * ncol);
    // da: the partial rows are [B][L / 32] x [d / 512][heads per block] = [rows][H]
    hipLaunchKernelGGL(prologue_colsum, dim3((unsigned)((dm.H + 63) / 64)), dim3(1024), 0, st, dm.H,
                       dm.B * (dm.L / kTileB), pda, da_param);
  });
  if (rc) return rc;
  return L("prologue_param_split", [&] {
    hipLaunchKernelGGL(prologue_param_split, dim3((unsigned)((3 * dm.d + 255) / 256)), dim3(256), 0, st, dm.d,
                       sums, dconv_w, dconv_b);
  });
}

// ------------------------------------------------------------ Mamba2 entry points
static int m2p_check(const atomic_mamba2_prologue_args* a) {
  if (!a) return ATOMIC_ERR_NULL;
  if (a->batch <= 0 || a->seqlen <= 0 || a->heads <= 0 || a->headdim <= 0 || a->dstate <= 0)
    return ATOMIC_ERR_SHAPE;
  if (a->dconv != kDc || (a->heads * a->headdim) % 512 != 0 || a->seqlen % (4 * kTileB) != 0 ||
      a->dstate % 8 != 0)
    return ATOMIC_ERR_SHAPE;
  return ATOMIC_OK;
}
static PlDims m2p_dims(const atomic_mamba2_prologue_args* a) {
  return PlDims{a->batch, a->seqlen, a->heads, 128, a->heads * a->headdim, 0.f, a->heads * a->headdim};
}
// workspace: x's conv partial rows [B][L / 128][d][5], then the summed [d][5]
static size_t m2p_ws(const PlDims& d, size_t* sums_off) {
  auto al = [](size_t x) { return (x + 255) & ~size_t(255); };
  const size_t rows = (size_t)d.B * (d.L / (4 * kTileB));
  *sums_off = al(rows * d.d * (kDc + 1) * 4);
  return *sums_off + al((size_t)d.d * (kDc + 1) * 4);
}

extern "C" size_t atomic_mamba2_prologue_workspace_size(const atomic_mamba2_prologue_args* a) {
  if (m2p_check(a) != ATOMIC_OK) return 0;
  size_t so;
  return m2p_ws(m2p_dims(a), &so);
}

extern "C" int atomic_mamba2_prologue_fwd(const atomic_mamba2_prologue_args* a, const void* x_bc,
                                          const float* conv_w, const float* conv_b, const void* dt_pre,
                                          const void* b_pre, const void* c_pre, const float* a_log, void* x,
                                          void* dt, void* B, void* C, float* A, void* stream) {
  int rc = m2p_check(a);
  if (rc) return rc;
  if (!x_bc || !conv_w || !conv_b || !dt_pre || !b_pre || !c_pre || !a_log || !x || !dt || !B || !C || !A)
    return ATOMIC_ERR_NULL;
  hipStream_t st = (hipStream_t)stream;
  const PlDims dm = m2p_dims(a);
  Launch L{a->profile, st};
  const unsigned nconv = (unsigned)(((size_t)dm.B * (dm.L / kTileF) * (dm.d / 512) + 3) / 4);
  rc = L("prologue_conv_fwd", [&] {
    hipLaunchKernelGGL((prologue_conv_fwd<kPlain, 128>), dim3(nconv), dim3(256), 0, st, dm, (const bf16*)x_bc,
                       conv_w, conv_b, (bf16*)x);
  });
  if (rc) return rc;
  const size_t n_dt = (size_t)dm.B * dm.L * dm.d, n_bc = (size_t)dm.B * dm.L * a->dstate;
  const size_t n = n_dt > n_bc ? n_dt : n_bc;
  return L("m2_prologue_elem_fwd", [&] {
    hipLaunchKernelGGL(m2_prologue_elem_fwd, dim3((unsigned)((n / 8 + 255) / 256)), dim3(256), 0, st, n_dt, n_bc,
                       dm.H, (const bf16*)dt_pre, (const bf16*)b_pre, (const bf16*)c_pre, a_log, (bf16*)dt,
                       (bf16*)B, (bf16*)C, A);
  });
}

extern "C" int atomic_mamba2_prologue_bwd(const atomic_mamba2_prologue_args* a, const void* x_bc,
                                          const float* conv_w, const float* conv_b, const void* dt_pre,
                                          const void* b_pre, const void* c_pre, const float* a_log,
                                          const void* dx, const void* ddt, const void* dB, const void* dC,
                                          const float* dA, void* dx_bc, float* dconv_w, float* dconv_b,
                                          void* ddt_pre, void* db_pre, void* dc_pre, float* da_log,
                                          void* workspace, size_t workspace_bytes, void* stream) {
  int rc = m2p_check(a);
  if (rc) return rc;
  if (!x_bc || !conv_w || !conv_b || !dt_pre || !b_pre || !c_pre || !a_log || !dx || !ddt || !dB || !dC || !dA ||
      !dx_bc || !dconv_w || !dconv_b || !ddt_pre || !db_pre || !dc_pre || !da_log)
    return ATOMIC_ERR_NULL;
  const PlDims dm = m2p_dims(a);
  size_t so;
  if (!workspace || workspace_bytes < m2p_ws(dm, &so)) return ATOMIC_ERR_WORKSPACE;
  ws_tag_clobber(workspace, m2p_ws(dm, &so));
  float* part = (float*)workspace;
  float* sums = (float*)((unsigned char*)workspace + so);
  hipStream_t st = (hipStream_t)stream;
  Launch L{a->profile, st};
  const int ngrp = dm.L / (4 * kTileB);
  rc = L("prologue_conv_bwd", [&] {
    hipLaunchKernelGGL((prologue_conv_bwd<kPlain, 128>), dim3((unsigned)((size_t)dm.B * ngrp * (dm.d / (64 * kCplB)))),
                       dim3(256), 0, st, dm, (const bf16*)x_bc, conv_w, conv_b, (const bf16*)dx, (bf16*)dx_bc, part);
  });
  if (rc) return rc;
  const size_t n_dt = (size_t)dm.B * dm.L * dm.d, n_bc = (size_t)dm.B * dm.L * a->dstate;
  const size_t n = n_dt > n_bc ? n_dt : n_bc;
  rc = L("m2_prologue_elem_bwd", [&] {
    hipLaunchKernelGGL(m2_prologue_elem_bwd, dim3((unsigned)((n / 8 + 255) / 256)), dim3(256), 0, st, n_dt, n_bc,
                       dm.H, (const bf16*)dt_pre, (const bf16*)b_pre, (const bf16*)c_pre, a_log, (const bf16*)ddt,
                       (const bf16*)dB, (const bf16*)dC, dA, (bf16*)ddt_pre, (bf16*)db_pre, (bf16*)dc_pre, da_log);
  });
  if (rc) return rc;
  rc = L("prologue_colsum", [&] {
    const int ncol = dm.d * (kDc + 1);
    hipLaunchKernelGGL(prologue_colsum, dim3((unsigned)((ncol + 63) / 64)), dim3(1024), 0, st, ncol,
                       dm.B * ngrp, part, sums);
  });
  if (rc) return rc;
  return L("prologue_param_split", [&] {
    // one conv: the split kernel's (which, channel) range is just the channels
    hipLaunchKernelGGL(prologue_param_split1, dim3((unsigned)((dm.d + 255) / 256)), dim3(256), 0, st, dm.d, sums,
                       dconv_w, dconv_b);
  });
}

// ------------------------------------------------- Mamba2 prologue with its projections
static int m2x_check(const atomic_mamba2_proj_args* a) {
  if (!a) return ATOMIC_ERR_NULL;
  if (a->batch <= 0 || a->seqlen <= 0 || a->heads <= 0 || a->headdim <= 0 || a->dstate <= 0)
    return ATOMIC_ERR_SHAPE;
  const long long d = (long long)a->heads * a->headdim;
  if (a->dconv != kDc || d % 512 != 0 || a->seqlen % (4 * kTileB) != 0 || a->dstate % 64 != 0)
    return ATOMIC_ERR_SHAPE;
  if (a->in_stride < d || a->in_stride % 8 != 0 || a->in_stride > (1LL << 30)) return ATOMIC_ERR_SHAPE;
  return ATOMIC_OK;
}

// Workspace: the packed bf16 weights [W_dt | W_B | W_C] (either layout); for
// the backward also dPre [M][d + 2n] bf16, the convolution path's dx [M][d]
// bf16, the weight-gradient partials [splits][d][d + 2n] fp32, the b_dt
// partials [M / 32][d] and sums [d] fp32, and the convolution's partial rows.
struct M2xPlan {
  PlDims dm;
  int M, d, n, nt, splits;
  size_t o_w, o_dpre, o_dxc, o_dw, o_dbp, o_dbs, o_conv, o_convsum, total;
};
static M2xPlan m2x_plan(const atomic_mamba2_proj_args* a, bool bwd) {
  M2xPlan p;
  p.d = a->heads * a->headdim;
  p.n = a->dstate;
  p.nt = p.d + 2 * p.n;
  p.M = a->batch * a->seqlen;
  p.dm = PlDims{a->batch, a->seqlen, a->heads, 128, p.d, 0.f, (int)a->in_stride};
  // row splits of the weight-gradient GEMM: enough workgroups to fill the chip,
  // each split a multiple of 64 rows
  const int tiles = (p.d / kGT) * (p.nt / (p.nt % 256 == 0 ? 256 : 128));
  int s = 1;
  while (s * tiles < 1024 && p.M % (2 * s * kGK) == 0) s *= 2;
  p.splits = s;
  auto al = [](size_t x) { return (x + 255) & ~size_t(255); };
  size_t off = 0;
  auto take = [&](size_t bytes) { const size_t o = off; off += al(bytes); return o; };
  const size_t M = p.M, d = p.d, nt = p.nt;
  p.o_w = take(d * nt * 2);
  p.o_dpre = p.o_dxc = p.o_dw = p.o_dbp = p.o_dbs = p.o_conv = p.o_convsum = 0;
  if (bwd) {
    p.o_dpre = take(M * nt * 2);
    p.o_dxc = take(M * d * 2);
    p.o_dw = take((size_t)p.splits * d * nt * 4);
    p.o_dbp = take((M / 32) * d * 4);
    p.o_dbs = take(d * 4);
    size_t so;
    const size_t cb = m2p_ws(p.dm, &so);
    p.o_conv = take(cb);
    p.o_convsum = p.o_conv + so;
  }
  p.total = off;
  return p;
}

extern "C" size_t atomic_mamba2_proj_workspace_size(const atomic_mamba2_proj_args* a, int backward) {
  if (m2x_check(a) != ATOMIC_OK) return 0;
  return m2x_plan(a, backward != 0).total;
}

extern "C" int atomic_mamba2_proj_fwd(const atomic_mamba2_proj_args* a, const void* x_bc, const float* conv_w,
                                      const float* conv_b, const float* w_dt, const float* b_dt,
                                      const float* w_b, const float* w_c, const float* a_log, void* x,
                                      void* dt, void* B, void* C, float* A, void* dt_pre, void* b_pre,
                                      void* c_pre, void* workspace, size_t workspace_bytes, void* stream) {
  int rc = m2x_check(a);
  if (rc) return rc;
  if (!x_bc || !conv_w || !conv_b || !w_dt || !b_dt || !w_b || !w_c || !a_log || !x || !dt || !B || !C || !A)
    return ATOMIC_ERR_NULL;
  const M2xPlan p = m2x_plan(a, false);
  if (!workspace || workspace_bytes < p.total) return ATOMIC_ERR_WORKSPACE;
  ws_tag_clobber(workspace, p.total);
  bf16* wt = reinterpret_cast<bf16*>(static_cast<unsigned char*>(workspace) + p.o_w);
  hipStream_t st = (hipStream_t)stream;
  Launch L{a->profile, st};
  rc = L("m2p_pack_t", [&] {
    hipLaunchKernelGGL(m2p_pack_t, dim3((unsigned)((p.nt / 64) * (p.d / 64))), dim3(256), 0, st, p.d, p.n, w_dt,
                       w_b, w_c, wt);
  });
  if (rc) return rc;
  rc = L("prologue_conv_fwd", [&] {
    const unsigned nconv = (unsigned)(((size_t)p.dm.B * (p.dm.L / kTileF) * (p.d / 512) + 3) / 4);
    hipLaunchKernelGGL((prologue_conv_fwd<kPlain, 128>), dim3(nconv), dim3(256), 0, st, p.dm, (const bf16*)x_bc,
                       conv_w, conv_b, (bf16*)x);
  });
  if (rc) return rc;
  rc = L("m2p_proj_gemm", [&] {
    const GemmNT g{(const bf16*)x_bc, (long long)a->in_stride, wt, (long long)p.d, p.M, p.nt, p.d};
    const M2ProjEpi e{p.d, p.n, b_dt, (bf16*)dt, (bf16*)B, (bf16*)C, (bf16*)dt_pre, (bf16*)b_pre, (bf16*)c_pre};
    if (p.nt % 256 == 0)
      hipLaunchKernelGGL((gemm_nt<256, M2ProjEpi>), dim3((unsigned)((p.M / kGT) * (p.nt / 256))), dim3(256), 0, st, g,
                         e);
    else
      hipLaunchKernelGGL((gemm_nt<128, M2ProjEpi>), dim3((unsigned)((p.M / kGT) * (p.nt / 128))), dim3(256), 0, st, g,
                         e);
  });
  if (rc) return rc;
  return L("m2_prologue_elem_fwd", [&] {  // A only (no element ranges)
    hipLaunchKernelGGL(m2_prologue_elem_fwd, dim3(1), dim3(256), 0, st, (size_t)0, (size_t)0, a->heads,
                       (const bf16*)nullptr, (const bf16*)nullptr, (const bf16*)nullptr, a_log, (bf16*)nullptr,
                       (bf16*)nullptr, (bf16*)nullptr, A);
  });
}

extern "C" int atomic_mamba2_proj_bwd(const atomic_mamba2_proj_args* a, const void* x_bc, const float* conv_w,
                                      const float* conv_b, const float* w_dt, const float* b_dt,
                                      const float* w_b, const float* w_c, const float* a_log,
                                      const void* dt_pre, const void* b_pre, const void* c_pre, const void* dx,
                                      const void* ddt, const void* dB, const void* dC, const float* dA,
                                      void* dx_bc, float* dconv_w, float* dconv_b, float* dw_dt, float* db_dt,
                                      float* dw_b, float* dw_c, float* da_log, void* workspace,
                                      size_t workspace_bytes, void* stream) {
  int rc = m2x_check(a);
  if (rc) return rc;
  if (!x_bc || !conv_w || !conv_b || !w_dt || !b_dt || !w_b || !w_c || !a_log || !dt_pre || !b_pre || !c_pre ||
      !dx || !ddt || !dB || !dC || !dA || !dx_bc || !dconv_w || !dconv_b || !dw_dt || !db_dt || !dw_b || !dw_c ||
      !da_log)
    return ATOMIC_ERR_NULL;
  const M2xPlan p = m2x_plan(a, true);
  if (!workspace || workspace_bytes < p.total) return ATOMIC_ERR_WORKSPACE;
  ws_tag_clobber(workspace, p.total);
  unsigned char* wsb = static_cast<unsigned char*>(workspace);
  bf16* w = reinterpret_cast<bf16*>(wsb + p.o_w);
  bf16* dpre = reinterpret_cast<bf16*>(wsb + p.o_dpre);
  bf16* dxc = reinterpret_cast<bf16*>(wsb + p.o_dxc);
  float* dwp = reinterpret_cast<float*>(wsb + p.o_dw);
  float* dbp = reinterpret_cast<float*>(wsb + p.o_dbp);
  float* dbs = reinterpret_cast<float*>(wsb + p.o_dbs);
  float* cpart = reinterpret_cast<float*>(wsb + p.o_conv);
  float* csum = reinterpret_cast<float*>(wsb + p.o_convsum);
  hipStream_t st = (hipStream_t)stream;
  Launch L{a->profile, st};
  const PlDims& dm = p.dm;
  rc = L("m2p_pack", [&] {
    hipLaunchKernelGGL(m2p_pack, dim3((unsigned)(((size_t)p.d * p.nt + 255) / 256)), dim3(256), 0, st, p.d, p.n,
                       w_dt, w_b, w_c, w);
  });
  if (rc) return rc;
  rc = L("m2p_vjp", [&] {
    const size_t nth = (size_t)(p.M / 32) * (p.nt / 8);
    hipLaunchKernelGGL(m2p_vjp, dim3((unsigned)((nth + 255) / 256)), dim3(256), 0, st, p.M, p.d, p.n, a->heads,
                       (const bf16*)dt_pre, (const bf16*)b_pre, (const bf16*)c_pre, a_log, (const bf16*)ddt,
                       (const bf16*)dB, (const bf16*)dC, dA, dpre, dbp, da_log);
  });
  if (rc) return rc;
  const int ngrp = dm.L / (4 * kTileB);
  rc = L("prologue_conv_bwd", [&] {
    hipLaunchKernelGGL((prologue_conv_bwd<kPlain, 128>), dim3((unsigned)((size_t)dm.B * ngrp * (dm.d / (64 * kCplB)))),
                       dim3(256), 0, st, dm, (const bf16*)x_bc, conv_w, conv_b, (const bf16*)dx, dxc, cpart);
  });
  if (rc) return rc;
  rc = L("m2p_dx_gemm", [&] {
    const GemmNT g{dpre, (long long)p.nt, w, (long long)p.nt, p.M, p.d, p.nt};
    const M2DxEpi e{dxc, p.d, (bf16*)dx_bc, (long long)a->in_stride};
    hipLaunchKernelGGL((gemm_nt<256, M2DxEpi>), dim3((unsigned)((p.M / kGT) * (p.d / 256))), dim3(256), 0, st, g, e);
  });
  if (rc) return rc;
  rc = L("m2p_dw_gemm", [&] {
    const GemmTN g{(const bf16*)x_bc, (long long)a->in_stride, dpre, (long long)p.nt, p.d, p.nt, p.M / p.splits, dwp};
    if (p.nt % 256 == 0)
      hipLaunchKernelGGL(gemm_tn<256>, dim3((unsigned)(p.splits * (p.d / kGT) * (p.nt / 256))), dim3(256), 0, st, g);
    else
      hipLaunchKernelGGL(gemm_tn<128>, dim3((unsigned)(p.splits * (p.d / kGT) * (p.nt / 128))), dim3(256), 0, st, g);
  });
  if (rc) return rc;
  rc = L("prologue_colsum", [&] {
    const int ncol = dm.d * (kDc + 1);
    hipLaunchKernelGGL(prologue_colsum, dim3((unsigned)((ncol + 63) / 64)), dim3(1024), 0, st, ncol, dm.B * ngrp,
                       cpart, csum);
    hipLaunchKernelGGL(prologue_colsum, dim3((unsigned)((p.d + 63) / 64)), dim3(1024), 0, st, p.d, p.M / 32, dbp,
                       dbs);
  });
  if (rc) return rc;
  rc = L("prologue_param_split", [&] {
    hipLaunchKernelGGL(prologue_param_split1, dim3((unsigned)((dm.d + 255) / 256)), dim3(256), 0, st, dm.d, csum,
                       dconv_w, dconv_b);
  });
  if (rc) return rc;
  return L("m2p_dw_finish", [&] {
    hipLaunchKernelGGL(m2p_dw_finish, dim3((unsigned)(((size_t)p.d * p.nt + 255) / 256)), dim3(256), 0, st, p.d,
                       p.n, p.splits, dwp, dbs, dw_dt, dw_b, dw_c, db_dt);
  });
}
