// bf16 MFMA GEMMs of the Mamba2 projection prologue (gfx950), with the
// kernels around them: weight packing, the element-wise VJP of the
// projection epilogue and the weight-gradient reduction.
//
//   gemm_nt   C[M][N] = A[M][K] . Bt[N][K]^T, both operands K-contiguous with
//             row strides (the in_proj half x_bc is read in place), fp32
//             accumulation, the result handed to an epilogue functor.
//   gemm_tn   P[s][K][N] = sum over the rows m of split s of X[m][K] D[m][N]
//             (the weight gradient X^T D over the tokens), fp32 partials.
//
// Tiles: one 128 x BN block of C per workgroup of four waves (2 x 2, each
// 64 x BN/2 as v_mfma_f32_16x16x32_bf16 tiles; BN = 256 where N allows, else
// 128); the reduction dimension in steps of 64 through one LDS stage: the
// next step's 16-byte pieces are loaded into registers while the current
// step's MFMAs run, and stored after a barrier.
#pragma once
#include "common.hpp"

namespace ah {

constexpr int kGT = 128;       // C tile rows (M)
constexpr int kGK = 64;        // reduction step
constexpr int kGP = kGK + 8;   // NT staging row pitch (elements): 16 rows of a fragment read hit distinct banks
constexpr int kTP = kGT + 16;  // TN staging row pitch: four rows of a transposed read hit distinct banks

__device__ __forceinline__ float bf16r(float x) { return (float)(bf16)x; }

// 4 x 4 transpose inside each lane quad: lane (4 a + j) holds v[k] = M[j][k]
// on entry and v[k] = M[k][j] on return (M the quad's 4 x 4 block), by two
// exchange steps (quad partners l ^ 2, then l ^ 1).  Applied to an MFMA
// result tile (lane: rows 4 g + k, column c) it leaves the lane with row
// 4 g + (c & 3) and the four columns (c & ~3) .. + 3, so stores are vectors.
__device__ __forceinline__ void quad_transpose(float (&v)[4]) {
  const int l = lane_id();
  {
    const bool hi = (l & 2) != 0;
    const float s0 = hi ? v[0] : v[2], s1 = hi ? v[1] : v[3];
    const float r0 = __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(s0), 0x4E, 0xF, 0xF, false));
    const float r1 = __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(s1), 0x4E, 0xF, 0xF, false));
    v[0] = hi ? r0 : v[0];
    v[1] = hi ? r1 : v[1];
    v[2] = hi ? v[2] : r0;
    v[3] = hi ? v[3] : r1;
  }
  {
    const bool odd = (l & 1) != 0;
    const float s0 = odd ? v[0] : v[1], s1 = odd ? v[2] : v[3];
    const float r0 = __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(s0), 0xB1, 0xF, 0xF, false));
    const float r1 = __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(s1), 0xB1, 0xF, 0xF, false));
    v[0] = odd ? r0 : v[0];
    v[2] = odd ? r1 : v[2];
    v[1] = odd ? v[1] : r0;
    v[3] = odd ? v[3] : r1;
  }
}

__device__ __forceinline__ void st4bf(bf16* p, const float (&v)[4]) {
  bf16x4 o;
  o[0] = (bf16)v[0]; o[1] = (bf16)v[1]; o[2] = (bf16)v[2]; o[3] = (bf16)v[3];
  *reinterpret_cast<bf16x4*>(p) = o;
}
__device__ __forceinline__ void ld4bf(const bf16* p, float (&v)[4]) {
  const bf16x4 t = *reinterpret_cast<const bf16x4*>(p);
  v[0] = (float)t[0]; v[1] = (float)t[1]; v[2] = (float)t[2]; v[3] = (float)t[3];
}

// ---------------------------------------------------------------- NT GEMM
struct GemmNT {
  const bf16* A;   // [M][K], row stride lda
  long long lda;
  const bf16* Bt;  // [N][K], row stride ldb
  long long ldb;
  int M, N, K;     // multiples of 128, BN, 64
};

// One 128 x BN tile of C per workgroup: waves in a 2 x 2 grid, each 64 x BN/2
// as 4 x (BN / 32) MFMA tiles.  One LDS stage: the next step's pieces are
// loaded into registers while the current step's MFMAs read the stage, then
// stored after a barrier.  The epilogue gets each wave's block (rows m0..,
// columns n0..) as acc[i][j], the 16 x 16 tile at rows m0 + 16 i, columns n0 + 16 j.
template <int BN, typename Epi>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(2, 2))) void gemm_nt(GemmNT g, Epi epi) {
  constexpr int NJ = BN / 32, PB = BN / 32;  // tiles per wave along N; Bt pieces per thread
  __shared__ __attribute__((aligned(16))) bf16 sA[kGT * kGP];
  __shared__ __attribute__((aligned(16))) bf16 sB[BN * kGP];
  typedef Mma<bf16>::frag frag;
  const int tid = threadIdx.x, w = wave_id();
  const int ntn = g.N / BN;
  const int tm = blockIdx.x / ntn, tn = blockIdx.x % ntn;  // consecutive workgroups share the A rows
  const bf16* Ag = g.A + (size_t)tm * kGT * g.lda;
  const bf16* Bg = g.Bt + (size_t)tn * BN * g.ldb;
  u32x4 ra[4], rb[PB];
  auto gload = [&](int k0) {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int e = tid + 256 * i, r = e >> 3, c = (e & 7) * 8;
      ra[i] = *reinterpret_cast<const u32x4*>(Ag + (size_t)r * g.lda + k0 + c);
    }
#pragma unroll
    for (int i = 0; i < PB; ++i) {
      const int e = tid + 256 * i, r = e >> 3, c = (e & 7) * 8;
      rb[i] = *reinterpret_cast<const u32x4*>(Bg + (size_t)r * g.ldb + k0 + c);
    }
  };
  auto lstore = [&]() {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int e = tid + 256 * i, r = e >> 3, c = (e & 7) * 8;
      *reinterpret_cast<u32x4*>(&sA[r * kGP + c]) = ra[i];
    }
#pragma unroll
    for (int i = 0; i < PB; ++i) {
      const int e = tid + 256 * i, r = e >> 3, c = (e & 7) * 8;
      *reinterpret_cast<u32x4*>(&sB[r * kGP + c]) = rb[i];
    }
  };
  f32x4 acc[4][NJ];
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int j = 0; j < NJ; ++j) acc[i][j] = zero4();
  const int wm = (w >> 1) * 64, wn = (w & 1) * (BN / 2);
  const int nk = g.K / kGK;
  gload(0);
  lstore();
  __syncthreads();
  for (int kt = 0; kt < nk; ++kt) {
    if (kt + 1 < nk) gload((kt + 1) * kGK);
#pragma unroll
    for (int ks = 0; ks < kGK; ks += 32) {
      frag af[4];
#pragma unroll
      for (int i = 0; i < 4; ++i) af[i] = Mma<bf16>::ld_c(sA, kGP, wm + 16 * i, ks);
#pragma unroll
      for (int j = 0; j < NJ; ++j) {
        const frag bfr = Mma<bf16>::ld_c(sB, kGP, wn + 16 * j, ks);
#pragma unroll
        for (int i = 0; i < 4; ++i) acc[i][j] = Mma<bf16>::mma(af[i], bfr, acc[i][j]);
      }
    }
    if (kt + 1 < nk) {
      __syncthreads();  // every wave is done reading the stage
      lstore();
      __syncthreads();
    }
  }
  epi(tm * kGT + wm, tn * BN + wn, acc);
}

// ---------------------------------------------------------------- TN GEMM
struct GemmTN {
  const bf16* X;  // [M][Kd], row stride ldx
  long long ldx;
  const bf16* D;  // [M][N], row stride ldd
  long long ldd;
  int Kd, N;      // multiples of 128 and BN
  int rows;       // rows per split (a multiple of 64); split s covers rows [s rows, (s + 1) rows)
  float* part;    // [splits][Kd][N]
};

// P[s] tile (128 x BN) = X^T D over the split's rows, both operands staged as
// 64-row tiles and read transposed (ds_read_b64_tr_b16) as the MFMA fragments.
template <int BN>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(2, 2))) void gemm_tn(GemmTN g) {
  constexpr int NJ = BN / 32, PD = BN / 32, LD = BN + 16;
  __shared__ __attribute__((aligned(16))) bf16 sX[kGK * kTP];
  __shared__ __attribute__((aligned(16))) bf16 sD[kGK * LD];
  typedef Mma<bf16>::frag frag;
  const int tid = threadIdx.x, w = wave_id();
  const int ntn = g.N / BN, ntk = g.Kd / kGT;
  const int s = blockIdx.x / (ntk * ntn), t = blockIdx.x % (ntk * ntn);
  const int tk = t / ntn, tn = t % ntn;
  const bf16* Xg = g.X + (size_t)s * g.rows * g.ldx + tk * kGT;
  const bf16* Dg = g.D + (size_t)s * g.rows * g.ldd + tn * BN;
  u32x4 ra[4], rb[PD];
  auto gload = [&](int m0) {  // 64 rows x 128 columns of X, 64 x BN of D
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int e = tid + 256 * i, r = e >> 4, c = (e & 15) * 8;
      ra[i] = *reinterpret_cast<const u32x4*>(Xg + (size_t)(m0 + r) * g.ldx + c);
    }
#pragma unroll
    for (int i = 0; i < PD; ++i) {
      const int e = tid + 256 * i, r = e / (BN / 8), c = (e % (BN / 8)) * 8;
      rb[i] = *reinterpret_cast<const u32x4*>(Dg + (size_t)(m0 + r) * g.ldd + c);
    }
  };
  auto lstore = [&]() {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int e = tid + 256 * i, r = e >> 4, c = (e & 15) * 8;
      *reinterpret_cast<u32x4*>(&sX[r * kTP + c]) = ra[i];
    }
#pragma unroll
    for (int i = 0; i < PD; ++i) {
      const int e = tid + 256 * i, r = e / (BN / 8), c = (e % (BN / 8)) * 8;
      *reinterpret_cast<u32x4*>(&sD[r * LD + c]) = rb[i];
    }
  };
  f32x4 acc[4][NJ];
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int j = 0; j < NJ; ++j) acc[i][j] = zero4();
  const int wm = (w >> 1) * 64, wn = (w & 1) * (BN / 2);
  const int nk = g.rows / kGK;
  gload(0);
  lstore();
  __syncthreads();
  for (int kt = 0; kt < nk; ++kt) {
    if (kt + 1 < nk) gload((kt + 1) * kGK);
#pragma unroll
    for (int ks = 0; ks < kGK; ks += 32) {
      // A(k, m) = X[m][k] and B(m, n) = D[m][n]: both read transposed from the row tiles
      frag af[4];
#pragma unroll
      for (int i = 0; i < 4; ++i) af[i] = Mma<bf16>::ld_t(sX, kTP, wm + 16 * i, ks);
#pragma unroll
      for (int j = 0; j < NJ; ++j) {
        const frag bfr = Mma<bf16>::ld_t(sD, LD, wn + 16 * j, ks);
#pragma unroll
        for (int i = 0; i < 4; ++i) acc[i][j] = Mma<bf16>::mma(af[i], bfr, acc[i][j]);
      }
    }
    if (kt + 1 < nk) {
      __syncthreads();
      lstore();
      __syncthreads();
    }
  }
  // partial tile, stored as 4-column vectors after a quad transpose
  float* P = g.part + (size_t)s * g.Kd * g.N;
  const int c = tile_col();
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int j = 0; j < NJ; ++j) {
      float v[4] = {acc[i][j][0], acc[i][j][1], acc[i][j][2], acc[i][j][3]};
      quad_transpose(v);
      const int row = tk * kGT + wm + 16 * i + tile_row(0) + (c & 3);
      const int col = tn * BN + wn + 16 * j + (c & ~3);
      *reinterpret_cast<float4*>(P + (size_t)row * g.N + col) = make_float4(v[0], v[1], v[2], v[3]);
    }
}

// ---------------------------------------------------------------- epilogues
__device__ __forceinline__ float m2p_dt_lo() { return bf16r(1e-2f); }
// jax.nn.softplus(x) = logaddexp(x, 0); every use rounds the result to bf16
__device__ __forceinline__ float m2p_softplus(float x) { return fmaxf(x, 0.f) + __logf(1.f + __expf(-fabsf(x))); }
// nan_to_num(clip(x, -c, c))
__device__ __forceinline__ float m2p_sanit(float x, float c) {
  if (__builtin_isnan(x)) return 0.f;
  return fminf(fmaxf(x, -c), c);
}

// Forward epilogue: the columns of [W_dt | W_B | W_C] give
//   dt = sanitize(clip(softplus(bf16(bf16(x W_dt) + bf16(b_dt))), bf16(1e-2), 1), 1e3)
//   B  = sanitize(bf16(x W_B), 1e3)      C = sanitize(bf16(x W_C), 1e3)
// (model.py:425-433); the pre-activations are also stored when asked for.
struct M2ProjEpi {
  int d, n;
  const float* b_dt;               // [d]
  bf16 *dt, *B, *C;                // [M][d], [M][n], [M][n]
  bf16 *dt_pre, *b_pre, *c_pre;    // the same shapes, or NULL
  template <int NJ>
  __device__ __forceinline__ void operator()(int m0, int n0, f32x4 (&acc)[4][NJ]) const {
    const int c = tile_col();
#pragma unroll
    for (int j = 0; j < NJ; ++j) {
      const int col = n0 + 16 * j + (c & ~3);  // this lane's four columns after the transpose
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int row = m0 + 16 * i + tile_row(0) + (c & 3);
        float v[4] = {acc[i][j][0], acc[i][j][1], acc[i][j][2], acc[i][j][3]};
        quad_transpose(v);
#pragma unroll
        for (int k = 0; k < 4; ++k) v[k] = bf16r(v[k]);
        if (col < d) {  // uniform over the 16-column tile
          const float4 bb = *reinterpret_cast<const float4*>(b_dt + col);
          const float bv[4] = {bb.x, bb.y, bb.z, bb.w};
          float o[4];
#pragma unroll
          for (int k = 0; k < 4; ++k) {
            v[k] = bf16r(v[k] + bf16r(bv[k]));
            o[k] = m2p_sanit(fminf(fmaxf(bf16r(m2p_softplus(v[k])), m2p_dt_lo()), 1.f), 1e3f);
          }
          st4bf(dt + (size_t)row * d + col, o);
          if (dt_pre) st4bf(dt_pre + (size_t)row * d + col, v);
        } else {
          const bool isb = col < d + n;
          const int cc = isb ? col - d : col - d - n;
          bf16* out = isb ? B : C;
          bf16* pre = isb ? b_pre : c_pre;
          float o[4];
#pragma unroll
          for (int k = 0; k < 4; ++k) o[k] = m2p_sanit(v[k], 1e3f);
          st4bf(out + (size_t)row * n + cc, o);
          if (pre) st4bf(pre + (size_t)row * n + cc, v);
        }
      }
    }
  }
};

// Backward epilogue of dX = dPre [W_dt | W_B | W_C]^T: x_bc's gradient is the
// projections' part (bf16) plus the convolution path's part, written to the
// strided view of the in_proj gradient.
struct M2DxEpi {
  const bf16* dxc;  // [M][d] the convolution path's part
  int d;
  bf16* out;        // [M] rows of stride ldo
  long long ldo;
  template <int NJ>
  __device__ __forceinline__ void operator()(int m0, int n0, f32x4 (&acc)[4][NJ]) const {
    const int c = tile_col();
#pragma unroll
    for (int j = 0; j < NJ; ++j) {
      const int col = n0 + 16 * j + (c & ~3);
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int row = m0 + 16 * i + tile_row(0) + (c & 3);
        float v[4] = {acc[i][j][0], acc[i][j][1], acc[i][j][2], acc[i][j][3]};
        quad_transpose(v);
        float cv[4];
        ld4bf(dxc + (size_t)row * d + col, cv);
#pragma unroll
        for (int k = 0; k < 4; ++k) v[k] = bf16r(v[k]) + cv[k];
        st4bf(out + (size_t)row * ldo + col, v);
      }
    }
  }
};

// ---------------------------------------------------------------- packing
// W(k, r) for the concatenated [W_dt | W_B | W_C] ([d][d + 2n], fp32 params)
__device__ __forceinline__ float m2p_w(int d, int n, const float* wdt, const float* wb, const float* wc, int k,
                                       int r) {
  return r < d ? wdt[(size_t)k * d + r] : (r < d + n ? wb[(size_t)k * n + r - d] : wc[(size_t)k * n + r - d - n]);
}
// out[k][r] = bf16(W(k, r))  (the layout of the backward's dX GEMM)
__global__ __launch_bounds__(256) void m2p_pack(int d, int n, const float* __restrict__ wdt,
                                                const float* __restrict__ wb, const float* __restrict__ wc,
                                                bf16* __restrict__ out) {
  const int nt = d + 2 * n;
  const size_t e = (size_t)blockIdx.x * 256 + threadIdx.x;
  if (e >= (size_t)d * nt) return;
  out[e] = (bf16)m2p_w(d, n, wdt, wb, wc, (int)(e / nt), (int)(e % nt));
}
// out[r][k] = bf16(W(k, r))  (the forward GEMM's Bt), 64 x 64 tiles through LDS
__global__ __launch_bounds__(256) void m2p_pack_t(int d, int n, const float* __restrict__ wdt,
                                                  const float* __restrict__ wb, const float* __restrict__ wc,
                                                  bf16* __restrict__ out) {
  __shared__ float t[64][65];
  const int nt = d + 2 * n, ntr = nt / 64;
  const int tr = blockIdx.x % ntr, tk = blockIdx.x / ntr;
  for (int e = threadIdx.x; e < 64 * 64; e += 256) {
    const int kk = e >> 6, rr = e & 63;
    t[kk][rr] = m2p_w(d, n, wdt, wb, wc, tk * 64 + kk, tr * 64 + rr);
  }
  __syncthreads();
  for (int e = threadIdx.x; e < 64 * 64; e += 256) {
    const int rr = e >> 6, kk = e & 63;
    out[(size_t)(tr * 64 + rr) * d + tk * 64 + kk] = (bf16)t[kk][rr];
  }
}

// ---------------------------------------------------------------- backward pieces
// cotangent factors of clip(v, -c, c) and of clip(x, lo, hi) (ties split evenly)
__device__ __forceinline__ float m2p_clip_g(float v, float c) {
  const float a = fabsf(v);
  return a < c ? 1.f : (a == c ? 0.5f : 0.f);
}
__device__ __forceinline__ float m2p_range_g(float x, float lo, float hi) {
  const float a = x > lo ? 1.f : (x == lo ? 0.5f : 0.f);
  const float b = x < hi ? 1.f : (x == hi ? 0.5f : 0.f);
  return a * b;
}

// The element-wise VJP of M2ProjEpi into dPre [M][d + 2n] (columns: dt, B, C
// pre-activations), one thread per 8 columns of 32 rows; column sums of the
// dt part (b_dt's gradient) per 32 rows into dbpart [M / 32][d].  Block 0
// also writes dA_log from dA (A = -exp(clip(A_log, +-20)), model.py:420-422).
__global__ __launch_bounds__(256) void m2p_vjp(int M, int d, int n, int H, const bf16* __restrict__ dt_pre,
                                               const bf16* __restrict__ b_pre, const bf16* __restrict__ c_pre,
                                               const float* __restrict__ a_log, const bf16* __restrict__ ddt,
                                               const bf16* __restrict__ dB, const bf16* __restrict__ dC,
                                               const float* __restrict__ dA, bf16* __restrict__ dpre,
                                               float* __restrict__ dbpart, float* __restrict__ da_log) {
  const int nt = d + 2 * n, ncg = nt / 8;
  const size_t gi = (size_t)blockIdx.x * 256 + threadIdx.x;
  if (gi < (size_t)(M / 32) * ncg) {
    const int cg = (int)(gi % ncg), rt = (int)(gi / ncg);
    const int col = cg * 8;
    if (col < d) {
      float acc[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
      for (int r = 0; r < 32; ++r) {
        const size_t m = (size_t)rt * 32 + r;
        float v[8], g[8], o[8];
        load8(dt_pre + m * d + col, v);
        load8(ddt + m * d + col, g);
#pragma unroll
        for (int j = 0; j < 8; ++j) {
          const float sp = bf16r(m2p_softplus(v[j]));
          const float cl = fminf(fmaxf(sp, m2p_dt_lo()), 1.f);
          const float dsp = bf16r(g[j] * m2p_clip_g(cl, 1e3f) * m2p_range_g(sp, m2p_dt_lo(), 1.f));
          o[j] = bf16r(dsp * __builtin_amdgcn_rcpf(1.f + __expf(-v[j])));  // softplus' = logistic
          acc[j] += o[j];
        }
        store8(dpre + m * nt + col, o);
      }
      store8(dbpart + (size_t)rt * d + col, acc);
    } else {
      const bool isb = col < d + n;
      const int cc = isb ? col - d : col - d - n;
      const bf16* pre = isb ? b_pre : c_pre;
      const bf16* gg = isb ? dB : dC;
      for (int r = 0; r < 32; ++r) {
        const size_t m = (size_t)rt * 32 + r;
        float v[8], g[8], o[8];
        load8(pre + m * n + cc, v);
        load8(gg + m * n + cc, g);
#pragma unroll
        for (int j = 0; j < 8; ++j) o[j] = bf16r(g[j] * m2p_clip_g(v[j], 1e3f));
        store8(dpre + m * nt + col, o);
      }
    }
  }
  if (blockIdx.x == 0)
    for (int h = threadIdx.x; h < H; h += 256) {
      const float al = a_log[h];
      da_log[h] = dA[h] * (-__expf(fminf(fmaxf(al, -20.f), 20.f))) * m2p_clip_g(al, 20.f);
    }
}

// Weight and bias gradients: dW = fp32(bf16(sum of the split partials)) split
// into [W_dt | W_B | W_C]; b_dt's gradient = fp32(bf16(dbsum)) (the bf16
// dot / bias VJPs of the reference, then the cast of the fp32 parameters).
__global__ __launch_bounds__(256) void m2p_dw_finish(int d, int n, int splits, const float* __restrict__ part,
                                                     const float* __restrict__ dbsum, float* __restrict__ dw_dt,
                                                     float* __restrict__ dw_b, float* __restrict__ dw_c,
                                                     float* __restrict__ db_dt) {
  const int nt = d + 2 * n;
  const size_t e = (size_t)blockIdx.x * 256 + threadIdx.x;
  const size_t tot = (size_t)d * nt;
  if (e < (size_t)d) db_dt[e] = bf16r(dbsum[e]);
  if (e >= tot) return;
  float s = 0.f;
  for (int sp = 0; sp < splits; ++sp) s += part[(size_t)sp * tot + e];
  const float v = bf16r(s);
  const int k = (int)(e / nt), r = (int)(e % nt);
  if (r < d) dw_dt[(size_t)k * d + r] = v;
  else if (r < d + n) dw_b[(size_t)k * n + r - d] = v;
  else dw_c[(size_t)k * n + r - d - n] = v;
}

}  // namespace ah
