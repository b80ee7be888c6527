// Stage-level kernels at the reference's 256-row Pallas block.
//
// The whole-path kernels run GDN2 at 64-row chunks and Mamba2 at 64 / 128
// rows; these kernels give the reference's staged functions at the block
// they are written for, with their float32 arrays:
//   GDN2 kernel A  build_chunk_scores_pallas  (kernel_a_scores.py:26-98)
//        kernel B  wy_solve_pallas            (kernel_b_solve.py:68-171)
//        kernel C  recompute_wy_pallas        (kernel_c_recompute.py:48-123)
//        kernel D  gdn2_inter_chunk_combine(_with_state) (kernel_d_pipeline.py:94-158)
//   Mamba2 M3    intra_chunk_ssd_pallas       (kernel_mamba2_b_intra.py:69-168)
//          M4    mamba2_inter_chunk_combine   (kernel_mamba2_c_interchunk.py:38-87)
// The Mamba2 kernels take the chunk (64, 128 or 256) at run time and serve
// every chunk for float32 operands, whose whole path is the staged chain;
// bfloat16 operands use them at 256 only.  Operands are bfloat16 or float32
// (StageIn).  Every value is computed in float32 (the reference upcasts its
// inputs on entry); the clip / nan_to_num placement is the reference's.  These are the
// drop-in stage functions, not the benchmark path: the decays are evaluated
// pair by pair (exp(clip(gc_i - gc_j, +-20)), as the reference does) on the
// vector ALUs, with the operands staged through LDS.
#include "../../include/atomic_hybrid.h"
#include "common.hpp"
#include "stage256.hpp"

namespace ah {

namespace {

constexpr int BT = kStageBlock;  // rows of a block
constexpr int RB = 64;           // row block of a workgroup
constexpr int NRB = BT / RB;     // row blocks per block

// token row of (batch bb, block n, row r) in [B][T][...]
__device__ __forceinline__ size_t tok(const Gdn2Dims& d, int bb, int n, int r) {
  return (size_t)bb * d.T + (size_t)n * BT + r;
}

// ------------------------------------------------------------ GDN2 helpers
// gc = cumsum over the block's rows of g for rows [64X, 64X + 64) and the 32
// channels [c0, c0 + 32), into sG[c][r] (row stride LT).  256 threads:
// channel c = t % 32, segment s = t / 32 of 8 rows.  sRed holds 2 x 8 x 32
// floats.  Ends with a barrier.
template <int LT>
__device__ void gc_tile(const Gdn2Dims& d, const float* __restrict__ g, size_t row0, int goff, int X,
                        float* sG, float* sRed) {
  const int t = threadIdx.x, c = t & 31, s = t >> 5;
  const float* gp = g + goff + c;
  // rows before the tile: thread s sums rows s, s + 8, ... < 64 X
  float base = 0.f;
  for (int r = s; r < RB * X; r += 8) base += gp[(row0 + r) * d.rg];
  // the tile's own 8-row segment
  float v[8];
#pragma unroll
  for (int i = 0; i < 8; ++i) v[i] = gp[(row0 + RB * X + 8 * s + i) * d.rg];
#pragma unroll
  for (int i = 1; i < 8; ++i) v[i] += v[i - 1];
  sRed[s * 32 + c] = base;
  sRed[256 + s * 32 + c] = v[7];
  __syncthreads();
  float pre = 0.f;
#pragma unroll
  for (int j = 0; j < 8; ++j) {
    pre += sRed[j * 32 + c];
    if (j < s) pre += sRed[256 + j * 32 + c];
  }
#pragma unroll
  for (int i = 0; i < 8; ++i) sG[c * LT + 8 * s + i] = pre + v[i];
  __syncthreads();
}

// A [64][32] tile (rows row0.., channels coff..) of a [B][T][H][D] input
// into sX[c][r] as float (row stride LT); with M, times the same tile of M.
template <int LT, typename T>
__device__ __forceinline__ void load_tile_t(const T* __restrict__ src, size_t stride, size_t row0, int coff,
                                            float* sX, const T* __restrict__ mul = nullptr,
                                            size_t mstride = 0) {
  const int t = threadIdx.x, c = t & 31;
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    const int r = (t >> 5) + 8 * i;
    float x = to_f(src[(row0 + r) * stride + coff + c]);
    if (mul) x *= to_f(mul[(row0 + r) * mstride + coff + c]);
    sX[c * LT + r] = x;
  }
}

// ------------------------------------------------------------ GDN2 kernel A
// One workgroup per (batch, head, block, row block I): the score blocks
// (I, J) for every J, 64 x 64 each, J > I written as zeros.  Thread (ty, tx)
// holds rows ty + 16 a and columns tx + 16 c (a, c < 4).
//   Aqk[i,j] = n2n(scale sum_d q_i,d e_ij,d k_j,d), i >= j
//   Akk[i,j] = n2n(sum_d (b k)_i,d e_ij,d k_j,d),   i > j
//   e_ij,d = exp(clip(gc_i,d - gc_j,d, +-20))   (kernel_a_scores.py:39-66)
template <typename T, int K>
__global__ __launch_bounds__(256) void g256_scores_k(Gdn2Dims d, const T* __restrict__ q, const T* __restrict__ k,
                                                     const T* __restrict__ b, const float* __restrict__ g,
                                                     float* __restrict__ aqk, float* __restrict__ akk) {
  constexpr int LT = RB + 1;
  __shared__ float sQ[32 * LT], sBK[32 * LT], sGI[32 * LT], sK[32 * LT], sGJ[32 * LT];
  __shared__ float sRed[512];
  const int bhn = blockIdx.x / NRB, I = NRB - 1 - (int)(blockIdx.x % NRB);
  const int bh = bhn / d.NT, n = bhn % d.NT, bb = bh / d.H, h = bh % d.H;
  const size_t row0 = tok(d, bb, n, 0);
  const int ty = threadIdx.x >> 4, tx = threadIdx.x & 15;
  float* oq = aqk + (size_t)bhn * BT * BT + (size_t)(RB * I) * BT;
  float* ok = akk + (size_t)bhn * BT * BT + (size_t)(RB * I) * BT;
  for (int J = 0; J <= I; ++J) {
    float aq[4][4], ak[4][4];
#pragma unroll
    for (int a = 0; a < 4; ++a)
#pragma unroll
      for (int c = 0; c < 4; ++c) aq[a][c] = ak[a][c] = 0.f;
    for (int c0 = 0; c0 < K; c0 += 32) {
      const int hc = h * K + c0;
      __syncthreads();  // the previous tiles' readers are done
      load_tile_t<LT>(q, d.rq, row0 + RB * I, hc, sQ);
      load_tile_t<LT>(b, d.rb, row0 + RB * I, hc, sBK, k, d.rk);
      load_tile_t<LT>(k, d.rk, row0 + RB * J, hc, sK);
      gc_tile<LT>(d, g, row0, hc, I, sGI, sRed);
      gc_tile<LT>(d, g, row0, hc, J, sGJ, sRed);
      for (int dd = 0; dd < 32; ++dd) {
        float qi[4], bi[4], gi[4], kj[4], gj[4];
#pragma unroll
        for (int a = 0; a < 4; ++a) {
          qi[a] = sQ[dd * LT + ty + 16 * a];
          bi[a] = sBK[dd * LT + ty + 16 * a];
          gi[a] = sGI[dd * LT + ty + 16 * a];
          kj[a] = sK[dd * LT + tx + 16 * a];
          gj[a] = sGJ[dd * LT + tx + 16 * a];
        }
#pragma unroll
        for (int a = 0; a < 4; ++a)
#pragma unroll
          for (int c = 0; c < 4; ++c) {
            const float e = __expf(fminf(fmaxf(gi[a] - gj[c], -kClipDecay), kClipDecay)) * kj[c];
            aq[a][c] += qi[a] * e;
            ak[a][c] += bi[a] * e;
          }
      }
    }
#pragma unroll
    for (int a = 0; a < 4; ++a)
#pragma unroll
      for (int c = 0; c < 4; ++c) {
        const int i = ty + 16 * a, j = tx + 16 * c;
        const bool diag = J == I;
        oq[(size_t)i * BT + RB * J + j] = (!diag || i >= j) ? n2n(d.scale * aq[a][c]) : 0.f;
        ok[(size_t)i * BT + RB * J + j] = (!diag || i > j) ? n2n(ak[a][c]) : 0.f;
      }
  }
  for (int J = I + 1; J < NRB; ++J)
#pragma unroll
    for (int a = 0; a < 4; ++a)
#pragma unroll
      for (int c = 0; c < 4; ++c) {
        const int i = ty + 16 * a, j = tx + 16 * c;
        oq[(size_t)i * BT + RB * J + j] = 0.f;
        ok[(size_t)i * BT + RB * J + j] = 0.f;
      }
}

// ------------------------------------------------------------ GDN2 kernel B
// (I + Akk)^-1 of a 256 x 256 block as the reference builds it: each
// 128-row half T_hh by forward substitution on 16 x 16 diagonal blocks
// (every new row sanitised) and the block recursion
//   A_mn = sanitize(-A_mm acc),  acc = sanitize(acc + T_mk A_kn) over k = n..m-1
// (kernel_b_solve.py:68-127), then A10 = sanitize(-A11 sanitize(T10 A00))
// (:130-148).  Only the strictly lower parts of the diagonal blocks and the
// whole lower-left T10 are read, as in the reference.
constexpr int LS = 129;  // LDS row stride of the 128 x 128 halves

// One workgroup per (batch, head, block, half): A_hh into rows of that half;
// the upper-right 128 x 128 block is written as zeros by the first half.
__global__ __launch_bounds__(256) void g256_solve_half_k(const float* __restrict__ akk, float* __restrict__ ainv) {
  __shared__ float smem[2 * 128 * LS + 8 * 16 * 17];
  float* sT = smem;               // [128][LS]
  float* sA = smem + 128 * LS;    // [128][LS]
  float* sAcc = sA + 128 * LS;    // [8][16][17]
  const int bhn = blockIdx.x >> 1, hf = blockIdx.x & 1;
  const float* T = akk + (size_t)bhn * BT * BT + (size_t)(128 * hf) * BT + 128 * hf;
  float* Ao = ainv + (size_t)bhn * BT * BT + (size_t)(128 * hf) * BT;
  const int t = threadIdx.x;
  for (int e = t; e < 128 * 128; e += 256) {
    const int r = e >> 7, c = e & 127;
    sT[r * LS + c] = T[(size_t)r * BT + c];
    sA[r * LS + c] = 0.f;
  }
  __syncthreads();
  // diagonal 16 x 16 blocks: thread (m, c) builds column c of block m
  if (t < 128) {
    const int m = t >> 4, c = t & 15, o = 16 * m;
    for (int i = 0; i < 16; ++i) {
      float s = 0.f;
      for (int j = 0; j < i; ++j) s += sT[(o + i) * LS + o + j] * sA[(o + j) * LS + o + c];
      sA[(o + i) * LS + o + c] = sanitize((i == c ? 1.f : 0.f) - s);
    }
  }
  __syncthreads();
  for (int m = 1; m < 8; ++m) {
    for (int e = t; e < m * 256; e += 256) {
      const int nb = e >> 8, r = (e >> 4) & 15, c = e & 15;
      float acc = 0.f;
      for (int kb = nb; kb < m; ++kb) {
        float s = 0.f;
#pragma unroll
        for (int l = 0; l < 16; ++l) s += sT[(16 * m + r) * LS + 16 * kb + l] * sA[(16 * kb + l) * LS + 16 * nb + c];
        acc = sanitize(acc + s);
      }
      sAcc[(nb * 16 + r) * 17 + c] = acc;
    }
    __syncthreads();
    for (int e = t; e < m * 256; e += 256) {
      const int nb = e >> 8, r = (e >> 4) & 15, c = e & 15;
      float s = 0.f;
#pragma unroll
      for (int l = 0; l < 16; ++l) s += sA[(16 * m + r) * LS + 16 * m + l] * sAcc[(nb * 16 + l) * 17 + c];
      sA[(16 * m + r) * LS + 16 * nb + c] = sanitize(-s);
    }
    __syncthreads();
  }
  for (int e = t; e < 128 * 128; e += 256) {
    const int r = e >> 7, c = e & 127;
    Ao[(size_t)r * BT + 128 * hf + c] = sA[r * LS + c];
    if (hf == 0) Ao[(size_t)r * BT + 128 + c] = 0.f;
  }
}

// One workgroup per (batch, head, block, 32-column panel of A10):
//   tmp = sanitize(T10 A00[:, panel]);  A10[:, panel] = sanitize(-A11 tmp).
// Thread t: row r = t % 128, columns 16 (t / 128) .. + 15 of the panel.
__global__ __launch_bounds__(256) void g256_solve_offdiag_k(const float* __restrict__ akk, float* __restrict__ ainv) {
  constexpr int LP = 33;
  __shared__ float sP[128 * LP], sX[128 * LP], sTmp[128 * LP];
  const int bhn = blockIdx.x >> 2, c0 = 32 * (blockIdx.x & 3);
  const float* T10 = akk + (size_t)bhn * BT * BT + (size_t)128 * BT;
  float* Ab = ainv + (size_t)bhn * BT * BT;
  const int t = threadIdx.x, r = t & 127, cc = 16 * (t >> 7);
  for (int e = t; e < 128 * 32; e += 256) {
    const int l = e >> 5, c = e & 31;
    sP[l * LP + c] = Ab[(size_t)l * BT + c0 + c];   // A00[:, panel]
  }
  float acc[16];
#pragma unroll
  for (int c = 0; c < 16; ++c) acc[c] = 0.f;
  for (int lc = 0; lc < 128; lc += 32) {
    __syncthreads();
    for (int e = t; e < 128 * 32; e += 256) {
      const int rr = e >> 5, l = e & 31;
      sX[rr * LP + l] = T10[(size_t)rr * BT + lc + l];
    }
    __syncthreads();
    for (int l = 0; l < 32; ++l) {
      const float x = sX[r * LP + l];
#pragma unroll
      for (int c = 0; c < 16; ++c) acc[c] += x * sP[(lc + l) * LP + cc + c];
    }
  }
#pragma unroll
  for (int c = 0; c < 16; ++c) {
    sTmp[r * LP + cc + c] = sanitize(acc[c]);
    acc[c] = 0.f;
  }
  for (int lc = 0; lc < 128; lc += 32) {
    __syncthreads();
    for (int e = t; e < 128 * 32; e += 256) {
      const int rr = e >> 5, l = e & 31;
      sX[rr * LP + l] = Ab[(size_t)(128 + rr) * BT + 128 + lc + l];   // A11
    }
    __syncthreads();
    for (int l = 0; l < 32; ++l) {
      const float x = sX[r * LP + l];
#pragma unroll
      for (int c = 0; c < 16; ++c) acc[c] += x * sTmp[(lc + l) * LP + cc + c];
    }
  }
#pragma unroll
  for (int c = 0; c < 16; ++c) Ab[(size_t)(128 + r) * BT + c0 + cc + c] = sanitize(-acc[c]);
}

// ------------------------------------------------------------ GDN2 kernel C
// One workgroup per (batch, head, block, row block I):
//   w_pseudo = sanitize(A (b k e^gc)),  u = sanitize(A (w v)),
//   kg = sanitize(k e^(gc_last - gc)),  qg = sanitize(q e^gc),
//   gc_last = sanitize(gc[255])         (kernel_c_recompute.py:58-82)
// with the whole 64 x 256 row block of A read (its zero upper blocks too).
// gc is built block by block (a running per-channel base); thread (c = t % K,
// segment s = t / K) scans RS = 64 K / 256 rows of channel c.
template <typename T, int K>
__global__ __launch_bounds__(256) void g256_recompute_k(Gdn2Dims d, const T* __restrict__ q, const T* __restrict__ k,
                                                        const T* __restrict__ v, const T* __restrict__ w,
                                                        const T* __restrict__ b, const float* __restrict__ g,
                                                        const float* __restrict__ ainv, float* __restrict__ wt,
                                                        float* __restrict__ u, float* __restrict__ kg,
                                                        float* __restrict__ qg, float* __restrict__ gcl) {
  constexpr int LK = K + 1, LA = RB + 1, NS = 256 / K, RS = RB / NS, NC = K / 64;
  __shared__ float smem[2 * RB * LK + RB * LA + NS * K];
  float* sKB = smem;             // [64][LK] b k e^gc of block J
  float* sWV = sKB + RB * LK;    // [64][LK] w v of block J
  float* sA = sWV + RB * LK;     // [64][LA] A[I rows][J cols]
  float* sSeg = sA + RB * LA;    // [NS][K]
  const int bhn = blockIdx.x / NRB, I = (int)(blockIdx.x % NRB);
  const int bh = bhn / d.NT, n = bhn % d.NT, bb = bh / d.H, h = bh % d.H;
  const size_t row0 = tok(d, bb, n, 0);
  const int t = threadIdx.x, c = t % K, s = t / K;
  const int gr = t >> 6, gc0 = t & 63;   // GEMM: rows gr + 4 a, columns gc0 + 64 j
  float accW[16][NC], accU[16][NC];
#pragma unroll
  for (int a = 0; a < 16; ++a)
#pragma unroll
    for (int j = 0; j < NC; ++j) accW[a][j] = accU[a][j] = 0.f;
  float base = 0.f;   // gc entering the block J, channel c
  float gI[RS];       // gc of this thread's rows of block I
  for (int J = 0; J < NRB; ++J) {
    // gc of block J, rows s RS .. s RS + RS - 1
    float gv[RS];
#pragma unroll
    for (int i = 0; i < RS; ++i) gv[i] = g[(row0 + RB * J + RS * s + i) * d.rg + h * K + c];
#pragma unroll
    for (int i = 1; i < RS; ++i) gv[i] += gv[i - 1];
    __syncthreads();  // the previous block's readers are done
    sSeg[s * K + c] = gv[RS - 1];
    __syncthreads();
    float pre = base, tot = 0.f;
#pragma unroll
    for (int j = 0; j < NS; ++j) {
      const float sv = sSeg[j * K + c];
      if (j < s) pre += sv;
      tot += sv;
    }
#pragma unroll
    for (int i = 0; i < RS; ++i) {
      const int r = RS * s + i;
      const size_t row = row0 + RB * J + r;
      gv[i] += pre;
      const float kk = to_f(k[row * d.rk + h * K + c]);
      sKB[r * LK + c] = to_f(b[row * d.rb + h * K + c]) * kk * __expf(gv[i]);
      sWV[r * LK + c] = to_f(w[row * d.rw + h * K + c]) * to_f(v[row * d.rv + h * K + c]);
      if (J == I) gI[i] = gv[i];
    }
    base += tot;
    for (int e = t; e < RB * RB; e += 256) {
      const int r = e >> 6, l = e & 63;
      sA[r * LA + l] = ainv[((size_t)bhn * BT + RB * I + r) * BT + RB * J + l];
    }
    __syncthreads();
    for (int l = 0; l < RB; ++l) {
      float xk[NC], xw[NC];
#pragma unroll
      for (int j = 0; j < NC; ++j) {
        xk[j] = sKB[l * LK + gc0 + 64 * j];
        xw[j] = sWV[l * LK + gc0 + 64 * j];
      }
#pragma unroll
      for (int a = 0; a < 16; ++a) {
        const float av = sA[(gr + 4 * a) * LA + l];
#pragma unroll
        for (int j = 0; j < NC; ++j) {
          accW[a][j] += av * xk[j];
          accU[a][j] += av * xw[j];
        }
      }
    }
  }
  const size_t ob = (size_t)bhn * BT + RB * I;   // first output row of [B][H][NT][256]
#pragma unroll
  for (int a = 0; a < 16; ++a)
#pragma unroll
    for (int j = 0; j < NC; ++j) {
      const size_t o = (ob + gr + 4 * a) * K + gc0 + 64 * j;
      wt[o] = sanitize(accW[a][j]);
      u[o] = sanitize(accU[a][j]);
    }
  // base = gc of the block's last row (every block has been scanned)
#pragma unroll
  for (int i = 0; i < RS; ++i) {
    const int r = RS * s + i;
    const size_t row = row0 + RB * I + r;
    const size_t o = (ob + r) * K + c;
    kg[o] = sanitize(to_f(k[row * d.rk + h * K + c]) * __expf(base - gI[i]));
    qg[o] = sanitize(to_f(q[row * d.rq + h * K + c]) * __expf(gI[i]));
  }
  if (I == 0 && s == 0) gcl[(size_t)bhn * K + c] = sanitize(base);
}

// ------------------------------------------------------------ GDN2 kernel D
// The sequential state loop over 256-row blocks, one workgroup per (batch,
// head, 16 state columns):
//   v_new = u - w_pseudo h;  o = n2n(scale qg h + Aqk v_new)
//   h = sanitize(h e^gc_last + kg^T v_new)     (kernel_d_pipeline.py:94-124)
// with h0 sanitised first (:54-55,101).  With h_pre / v_new given it also
// writes the state entering each block [B][H][NT][K][V] and v_new
// [B][H][NT][256][V] (gdn2_inter_chunk_combine_with_state, :127-158).
constexpr int VC = 16;  // state columns of a workgroup

template <int K>
struct CombineLds {
  static constexpr int LK = K + 1, LA = BT + 1;
  static constexpr int slab = (2 * RB * LK > RB * LA ? 2 * RB * LK : RB * LA);
  static constexpr int off_h = 0;                       // [K][VC]
  static constexpr int off_vn = off_h + K * VC;         // [256][VC]
  static constexpr int off_qh = off_vn + BT * VC;       // [256][VC] qg h
  static constexpr int off_gl = off_qh + BT * VC;       // [K]
  static constexpr int off_slab = off_gl + K;
  static constexpr int floats = off_slab + slab;
};

// Copy 64 rows of 32..256 floats (rows `sld` apart) into LDS rows `ld` apart.
template <int D>
__device__ __forceinline__ void stage_slab(float* dst, int ld, const float* __restrict__ src, size_t sld) {
  constexpr int PR = D / 4;
  for (int e = threadIdx.x; e < RB * PR; e += 256) {
    const int r = e / PR, c = 4 * (e % PR);
    const float4 x = *reinterpret_cast<const float4*>(src + (size_t)r * sld + c);
    float* o = dst + r * ld + c;
    o[0] = x.x; o[1] = x.y; o[2] = x.z; o[3] = x.w;
  }
}

template <int K>
__global__ __launch_bounds__(256) void g256_combine_k(Gdn2Dims d, const float* __restrict__ aqk,
                                                      const float* __restrict__ wt, const float* __restrict__ u,
                                                      const float* __restrict__ kgp, const float* __restrict__ qgp,
                                                      const float* __restrict__ gclp, const float* __restrict__ h0,
                                                      float* __restrict__ o, float* __restrict__ h_final,
                                                      float* __restrict__ h_pre, float* __restrict__ v_new) {
  typedef CombineLds<K> L;
  constexpr int V = K, LK = L::LK, LA = L::LA;
  constexpr int HC = 256 / K, HW = VC / HC;   // h update: thread (row t % K, columns HW (t / K) .. + HW - 1)
  __shared__ __attribute__((aligned(16))) float smem[L::floats];
  float* sH = smem + L::off_h;
  float* sVn = smem + L::off_vn;
  float* sQh = smem + L::off_qh;
  float* sGl = smem + L::off_gl;
  float* sS = smem + L::off_slab;
  const int bh = blockIdx.x / (V / VC), v0 = VC * (blockIdx.x % (V / VC));
  const int t = threadIdx.x, r = t & 63, cg = 4 * (t >> 6);   // rows r of a slab, 4 columns cg..cg+3
  const int hd = t % K, hc = HW * (t / K);
  for (int e = t; e < K * VC; e += 256) {
    const int dd = e / VC, c = e % VC;
    sH[e] = h0 ? sanitize(h0[((size_t)bh * K + dd) * V + v0 + c]) : 0.f;
  }
  __syncthreads();
  for (int n = 0; n < d.NT; ++n) {
    const size_t bhn = (size_t)bh * d.NT + n;
    if (h_pre)
      for (int e = t; e < K * VC; e += 256) h_pre[(bhn * K + e / VC) * V + v0 + e % VC] = sH[e];
    if (t < K) sGl[t] = gclp[bhn * K + t];
    // v_new and qg h, slab by slab
#pragma unroll 1
    for (int sl = 0; sl < NRB; ++sl) {
      __syncthreads();
      stage_slab<K>(sS, LK, wt + (bhn * BT + RB * sl) * K, K);
      stage_slab<K>(sS + RB * LK, LK, qgp + (bhn * BT + RB * sl) * K, K);
      __syncthreads();
      float vn[4] = {0.f, 0.f, 0.f, 0.f}, qv[4] = {0.f, 0.f, 0.f, 0.f};
#pragma unroll 4
      for (int dd = 0; dd < K; ++dd) {
        const float wv = sS[r * LK + dd], qq = sS[(RB + r) * LK + dd];
        const float4 hv = *reinterpret_cast<const float4*>(sH + dd * VC + cg);
        vn[0] += wv * hv.x; vn[1] += wv * hv.y; vn[2] += wv * hv.z; vn[3] += wv * hv.w;
        qv[0] += qq * hv.x; qv[1] += qq * hv.y; qv[2] += qq * hv.z; qv[3] += qq * hv.w;
      }
      const size_t row = bhn * BT + RB * sl + r;
      const float4 uu = *reinterpret_cast<const float4*>(u + row * V + v0 + cg);
      const float4 nv = make_float4(uu.x - vn[0], uu.y - vn[1], uu.z - vn[2], uu.w - vn[3]);
      *reinterpret_cast<float4*>(sVn + (RB * sl + r) * VC + cg) = nv;
      if (v_new) *reinterpret_cast<float4*>(v_new + row * V + v0 + cg) = nv;
      *reinterpret_cast<float4*>(sQh + (RB * sl + r) * VC + cg) = make_float4(qv[0], qv[1], qv[2], qv[3]);
    }
    // o = n2n(scale qg h + Aqk v_new), every column of Aqk summed
#pragma unroll 1
    for (int sl = 0; sl < NRB; ++sl) {
      __syncthreads();
      stage_slab<BT>(sS, LA, aqk + (bhn * BT + RB * sl) * BT, BT);
      __syncthreads();
      float acc[4] = {0.f, 0.f, 0.f, 0.f};
#pragma unroll 4
      for (int j = 0; j < BT; ++j) {
        const float a = sS[r * LA + j];
        const float4 x = *reinterpret_cast<const float4*>(sVn + j * VC + cg);
        acc[0] += a * x.x; acc[1] += a * x.y; acc[2] += a * x.z; acc[3] += a * x.w;
      }
      const float4 qh = *reinterpret_cast<const float4*>(sQh + (RB * sl + r) * VC + cg);  // own writes
      float4 ov;
      ov.x = n2n(d.scale * qh.x + acc[0]);
      ov.y = n2n(d.scale * qh.y + acc[1]);
      ov.z = n2n(d.scale * qh.z + acc[2]);
      ov.w = n2n(d.scale * qh.w + acc[3]);
      *reinterpret_cast<float4*>(o + (bhn * BT + RB * sl + r) * V + v0 + cg) = ov;
    }
    // h = sanitize(h e^gc_last + kg^T v_new)
    float wr[HW];
#pragma unroll
    for (int j = 0; j < HW; ++j) wr[j] = 0.f;
#pragma unroll 1
    for (int sl = 0; sl < NRB; ++sl) {
      __syncthreads();
      stage_slab<K>(sS, LK, kgp + (bhn * BT + RB * sl) * K, K);
      __syncthreads();
#pragma unroll 8
      for (int rr = 0; rr < RB; ++rr) {
        const float kv = sS[rr * LK + hd];
#pragma unroll
        for (int j = 0; j < HW; ++j) wr[j] += kv * sVn[(RB * sl + rr) * VC + hc + j];
      }
    }
    const float dec = __expf(sGl[hd]);
    float hn[HW];
#pragma unroll
    for (int j = 0; j < HW; ++j) hn[j] = sanitize(sH[hd * VC + hc + j] * dec + wr[j]);
    __syncthreads();   // every reader of sH (the v_new / qg h phase) is done
#pragma unroll
    for (int j = 0; j < HW; ++j) sH[hd * VC + hc + j] = hn[j];
    __syncthreads();
  }
  for (int e = t; e < K * VC; e += 256) h_final[((size_t)bh * K + e / VC) * V + v0 + e % VC] = sH[e];
}

// ------------------------------------------------------------ Mamba2 M3
// One workgroup per (batch, head, chunk, 64-row block I): y_diag of rows
// [64 I, 64 I + 64) over the reference's min(128, C)-row sub-blocks,
//   y_blk(si, sj)[i,p] = sum_j exp(clip(cum_i,p - cum_j,p, +-20)) CB_ij dBx_j,p  (j <= i)
//   y_diag[si] = sanitize(y_diag[si] + y_blk(si, sj)) for sj = 0 .. si
// (kernel_mamba2_b_intra.py:86-108), CB = sanitize(C B^T) (:83-84),
// dBx = sanitize(dt x) (:81).  Thread (p = t % 64 of a 64-channel group,
// rows 16 (t / 64) ..  + 15).
// One source block at a time (50 KB, three workgroups per CU): the CB tile
// of block I against it, then its cum_j and dBx_j, [64][LP] each.
struct M3Lds {
  static constexpr int LP = 65;
  static constexpr int off_cb = 0, off_cum = RB * LP, off_dbx = 2 * RB * LP, floats = 3 * RB * LP;
};

template <int P, int N>
__global__ __launch_bounds__(256) void m256_ydiag_k(Mamba2Dims d, StageIn dt, StageIn x, const float* __restrict__ cbg,
                                                    const float* __restrict__ cum, float* __restrict__ y_diag) {
  typedef M3Lds L;
  __shared__ float smem[L::floats];
  const int C = d.C, nrb = C / RB;
  float* sCB = smem + L::off_cb;
  float* sCum = smem + L::off_cum;
  float* sDbx = smem + L::off_dbx;
  const int bhn = blockIdx.x / nrb, I = nrb - 1 - (int)(blockIdx.x % nrb);
  const int bh = bhn / d.NT, n = bhn % d.NT, bb = bh / d.H, h = bh % d.H;
  const size_t row0 = (size_t)bb * d.T + (size_t)n * C;
  const int t = threadIdx.x;
  // row blocks per sub-block, and block I's sub-block
  const int srb = (C < 128 ? C : 128) / RB, si = I / srb;
  // CB rows of block I in the chunk's CB
  const float* cbz = cbg + (((size_t)bb * d.NT + n) * C + (size_t)RB * I) * C;
  const int p = t & 63, rg = 16 * (t >> 6);
  for (int p0 = 0; p0 < P; p0 += 64) {
    const size_t hp = (size_t)h * P + p0 + p;
    const float* cb = cum + (size_t)bhn * C * P + p0 + p;   // cum[b][h][n][row][p]
    float ci[16], acc0[16], acc1[16];
#pragma unroll
    for (int a = 0; a < 16; ++a) {
      ci[a] = cb[(size_t)(RB * I + rg + a) * P];
      acc0[a] = acc1[a] = 0.f;
    }
    for (int J = 0; J <= I; ++J) {
      __syncthreads();
      for (int e = t; e < RB * 64; e += 256) {
        const int rr = e >> 6, pp = e & 63;
        const size_t row = row0 + RB * J + rr;
        sCum[rr * L::LP + pp] = cum[((size_t)bhn * C + RB * J + rr) * P + p0 + pp];
        sDbx[rr * L::LP + pp] = sanitize(ld(dt, row * d.rdt + (size_t)h * P + p0 + pp) *
                                         ld(x, row * d.rx + (size_t)h * P + p0 + pp));
        sCB[rr * L::LP + pp] = cbz[(size_t)rr * C + RB * J + pp];   // CB(row 64 I + rr, source 64 J + pp)
      }
      __syncthreads();
      // sources of an earlier sub-block feed this sub-block's rows through
      // their own sanitised sub-block sum (acc0); C <= 256 gives at most two
      const bool cross = si > 0 && J / srb < si;
      // on the diagonal block, sources past this wave's last row add nothing
      const int jend = J == I ? rg + 16 : RB;
      for (int jj = 0; jj < jend; ++jj) {
        const int j = RB * J + jj;
        const float cj = sCum[jj * L::LP + p], xb = sDbx[jj * L::LP + p];
#pragma unroll
        for (int a = 0; a < 16; ++a) {
          const int i = RB * I + rg + a;
          const float wgt = j <= i ? __expf(fminf(fmaxf(ci[a] - cj, -kClipDecay), kClipDecay)) *
                                         sCB[(rg + a) * L::LP + jj]
                                   : 0.f;
          if (cross) acc0[a] += wgt * xb;
          else acc1[a] += wgt * xb;
        }
      }
    }
#pragma unroll
    for (int a = 0; a < 16; ++a) {
      const float y = si > 0 ? sanitize(sanitize(acc0[a]) + acc1[a]) : sanitize(acc1[a]);
      y_diag[(row0 + RB * I + rg + a) * (size_t)d.H * P + hp] = y;
    }
  }
}

// state_end[p][s] = sanitize(sum_j write_j,p B_j,s), write = sanitize(dBx
// exp(clip(cum_last - cum, +-20))) (kernel_mamba2_b_intra.py:110-116).  One
// workgroup per (batch, head, chunk, 32 channels); thread (s = t % N, channels
// 32 N / 256 from (t / N) on).
template <int P, int N>
__global__ __launch_bounds__(256) void m256_state_end_k(Mamba2Dims d, StageIn dt, StageIn x, StageIn Bm,
                                                        const float* __restrict__ cum,
                                                        float* __restrict__ state_end) {
  constexpr int PC = 32, LN = N + 1, LW = PC + 4, CPT = PC * N / 256;
  __shared__ float sB[RB * LN];
  __shared__ __attribute__((aligned(16))) float sW[RB * LW];
  const int bhn = blockIdx.x / (P / PC), p0 = PC * (int)(blockIdx.x % (P / PC));
  const int bh = bhn / d.NT, n = bhn % d.NT, bb = bh / d.H, h = bh % d.H;
  const int C = d.C;
  const size_t row0 = (size_t)bb * d.T + (size_t)n * C;
  const float* cb = cum + (size_t)bhn * C * P + p0;
  const int t = threadIdx.x, s = t % N, pc = CPT * (t / N);
  float acc[CPT];
#pragma unroll
  for (int j = 0; j < CPT; ++j) acc[j] = 0.f;
  for (int J = 0; J < C / RB; ++J) {
    __syncthreads();
    for (int e = t; e < RB * N; e += 256) {
      const int rr = e / N, ss = e % N;
      sB[rr * LN + ss] = ld(Bm, (row0 + RB * J + rr) * d.rB + ss);
    }
    for (int e = t; e < RB * PC; e += 256) {
      const int rr = e / PC, pp = e % PC;
      const size_t row = row0 + RB * J + rr;
      const float dbx = sanitize(ld(dt, row * d.rdt + (size_t)h * P + p0 + pp) *
                                 ld(x, row * d.rx + (size_t)h * P + p0 + pp));
      const float dte = __expf(fminf(fmaxf(cb[(size_t)(C - 1) * P + pp] - cb[(size_t)(RB * J + rr) * P + pp],
                                           -kClipDecay), kClipDecay));
      sW[rr * LW + pp] = sanitize(dbx * dte);
    }
    __syncthreads();
    for (int rr = 0; rr < RB; ++rr) {
      const float bv = sB[rr * LN + s];
#pragma unroll
      for (int j = 0; j < CPT; ++j) acc[j] += sW[rr * LW + pc + j] * bv;
    }
  }
#pragma unroll
  for (int j = 0; j < CPT; ++j) state_end[((size_t)bhn * P + p0 + pc + j) * N + s] = sanitize(acc[j]);
}

// ------------------------------------------------------------ Mamba2 M4
// The state entering each chunk, in float32 (kernel_mamba2_c_interchunk.py:58,75-76):
//   state = sanitize(state0); per chunk: pre[n] = state;
//   state = sanitize(state exp(clip(cum_last, -20, 0)) + state_end[n]).
// One thread per (batch, head, p, s).
template <int P, int N>
__global__ __launch_bounds__(256) void m256_state_pass_k(Mamba2Dims d, const float* __restrict__ state_end,
                                                         const float* __restrict__ cum,
                                                         const float* __restrict__ state0, float* __restrict__ pre,
                                                         float* __restrict__ state_final) {
  const size_t e = (size_t)blockIdx.x * 256 + threadIdx.x;   // (bh, p, s)
  const int s = (int)(e % N), p = (int)((e / N) % P);
  const size_t bh = e / ((size_t)P * N);
  const int bb = (int)(bh / d.H), h = (int)(bh % d.H);
  float st = state0 ? sanitize(state0[e]) : 0.f;
  for (int n = 0; n < d.NT; ++n) {
    const size_t bhn = bh * d.NT + n;
    pre[((((size_t)bb * d.NT + n) * d.H + h) * P + p) * N + s] = st;
    const float cl = cum[(bhn * d.C + d.C - 1) * P + p];
    st = sanitize(st * __expf(fminf(fmaxf(cl, -kClipDecay), 0.f)) + state_end[(bhn * P + p) * N + s]);
  }
  state_final[e] = st;
}

// y = sanitize(y_diag + sanitize((C state_prev^T) exp(clip(cum, -20, 0))))
// (kernel_mamba2_c_interchunk.py:70-78).  One workgroup per (batch, head,
// chunk, 64-row block); thread (p = t % 64 of a 64-channel group, rows
// 16 (t / 64) .. + 15).
template <int P, int N>
__global__ __launch_bounds__(256) void m256_y_k(Mamba2Dims d, const float* __restrict__ y_diag,
                                                const float* __restrict__ pre, const float* __restrict__ cum,
                                                StageIn Cm, float* __restrict__ y) {
  constexpr int LN = N + 1;
  __shared__ float sC[RB * LN], sS[64 * LN];
  const int C = d.C, nrb = C / RB;
  const int bhn = blockIdx.x / nrb, I = (int)(blockIdx.x % nrb);
  const int bh = bhn / d.NT, n = bhn % d.NT, bb = bh / d.H, h = bh % d.H;
  const size_t row0 = (size_t)bb * d.T + (size_t)n * C + RB * I;
  const int t = threadIdx.x, p = t & 63, rg = 16 * (t >> 6);
  for (int e = t; e < RB * N; e += 256) {
    const int rr = e / N, s = e % N;
    sC[rr * LN + s] = ld(Cm, (row0 + rr) * d.rC + s);
  }
  const float* sp = pre + (((size_t)bb * d.NT + n) * d.H + h) * P * N;
  for (int p0 = 0; p0 < P; p0 += 64) {
    __syncthreads();
    for (int e = t; e < 64 * N; e += 256) {
      const int pp = e / N, s = e % N;
      sS[pp * LN + s] = sp[(size_t)(p0 + pp) * N + s];
    }
    __syncthreads();
    float acc[16];
#pragma unroll
    for (int a = 0; a < 16; ++a) acc[a] = 0.f;
    for (int s = 0; s < N; ++s) {
      const float sv = sS[p * LN + s];
#pragma unroll
      for (int a = 0; a < 16; ++a) acc[a] += sC[(rg + a) * LN + s] * sv;
    }
#pragma unroll
    for (int a = 0; a < 16; ++a) {
      const int i = RB * I + rg + a;
      const float dfs = __expf(fminf(fmaxf(cum[((size_t)bhn * C + i) * P + p0 + p], -kClipDecay), 0.f));
      const size_t o = (row0 + rg + a) * (size_t)d.H * P + (size_t)h * P + p0 + p;
      y[o] = sanitize(y_diag[o] + sanitize(acc[a] * dfs));
    }
  }
}

}  // namespace

// ------------------------------------------------------------------ launchers
int g256_scores(const Gdn2Dims& d, int dtype, const void* q, const void* k, const void* b, const float* g,
                float* aqk, float* akk, Launch& L) {
  const unsigned nwg = (unsigned)((size_t)d.B * d.H * d.NT * NRB);
  return L("gdn2_scores_bt256", [&] {
    if (dtype == ATOMIC_BF16) {
      if (d.K == 128)
        hipLaunchKernelGGL((g256_scores_k<bf16, 128>), dim3(nwg), dim3(256), 0, L.st, d, (const bf16*)q,
                           (const bf16*)k, (const bf16*)b, g, aqk, akk);
      else
        hipLaunchKernelGGL((g256_scores_k<bf16, 64>), dim3(nwg), dim3(256), 0, L.st, d, (const bf16*)q,
                           (const bf16*)k, (const bf16*)b, g, aqk, akk);
    } else {
      if (d.K == 128)
        hipLaunchKernelGGL((g256_scores_k<float, 128>), dim3(nwg), dim3(256), 0, L.st, d, (const float*)q,
                           (const float*)k, (const float*)b, g, aqk, akk);
      else
        hipLaunchKernelGGL((g256_scores_k<float, 64>), dim3(nwg), dim3(256), 0, L.st, d, (const float*)q,
                           (const float*)k, (const float*)b, g, aqk, akk);
    }
  });
}

int g256_solve(const Gdn2Dims& d, const float* akk, float* a, Launch& L) {
  const size_t blocks = (size_t)d.B * d.H * d.NT;
  int rc = L("gdn2_wy_solve_bt256", [&] {
    hipLaunchKernelGGL(g256_solve_half_k, dim3((unsigned)(blocks * 2)), dim3(256), 0, L.st, akk, a);
  });
  if (rc) return rc;
  return L("gdn2_wy_solve_bt256_offdiag", [&] {
    hipLaunchKernelGGL(g256_solve_offdiag_k, dim3((unsigned)(blocks * 4)), dim3(256), 0, L.st, akk, a);
  });
}

int g256_recompute(const Gdn2Dims& d, int dtype, const void* q, const void* k, const void* v, const void* w,
                   const void* b, const float* g, const float* a, float* wt, float* u, float* kg, float* qg,
                   float* gcl, Launch& L) {
  const unsigned nwg = (unsigned)((size_t)d.B * d.H * d.NT * NRB);
  return L("gdn2_recompute_wy_bt256", [&] {
#define AH_G256C(TT, KK)                                                                                       \
  hipLaunchKernelGGL((g256_recompute_k<TT, KK>), dim3(nwg), dim3(256), 0, L.st, d, (const TT*)q,            \
                     (const TT*)k, (const TT*)v, (const TT*)w, (const TT*)b, g, a, wt, u, kg, qg, gcl)
    if (dtype == ATOMIC_BF16) {
      if (d.K == 128) AH_G256C(bf16, 128);
      else AH_G256C(bf16, 64);
    } else {
      if (d.K == 128) AH_G256C(float, 128);
      else AH_G256C(float, 64);
    }
#undef AH_G256C
  });
}

int g256_combine(const Gdn2Dims& d, const float* aqk, const float* wt, const float* u, const float* kg,
                 const float* qg, const float* gcl, const float* h0, float* o, float* h_final, float* h_pre,
                 float* v_new, Launch& L) {
  const unsigned nwg = (unsigned)((size_t)d.B * d.H * (d.V / VC));
  return L("gdn2_combine_bt256", [&] {
    if (d.K == 128)
      hipLaunchKernelGGL((g256_combine_k<128>), dim3(nwg), dim3(256), 0, L.st, d, aqk, wt, u, kg, qg, gcl, h0, o,
                         h_final, h_pre, v_new);
    else
      hipLaunchKernelGGL((g256_combine_k<64>), dim3(nwg), dim3(256), 0, L.st, d, aqk, wt, u, kg, qg, gcl, h0, o,
                         h_final, h_pre, v_new);
  });
}

template <int P, int N>
static int m256_intra_t(const Mamba2Dims& d, int dtype, const void* dt, const void* x, const void* Bm,
                        const void* Cm, const float* cum, float* y_diag, float* state_end, float* cb, Launch& L) {
  const size_t bhn = (size_t)d.B * d.H * d.NT;
  if (d.C != 64 && d.C != 128 && d.C != 256) return ATOMIC_ERR_SHAPE;
  const int bf = dtype == ATOMIC_BF16;
  const StageIn idt{dt, bf}, ix{x, bf}, iB{Bm, bf};
  int rc = m_cb(d, dtype, Bm, Cm, cb, L);
  if (rc) return rc;
  rc = L("mamba2_intra_bt256", [&] {
    hipLaunchKernelGGL((m256_ydiag_k<P, N>), dim3((unsigned)(bhn * (d.C / RB))), dim3(256), 0, L.st, d, idt, ix,
                       cb, cum, y_diag);
  });
  if (rc) return rc;
  return L("mamba2_state_end_bt256", [&] {
    hipLaunchKernelGGL((m256_state_end_k<P, N>), dim3((unsigned)(bhn * (P / 32))), dim3(256), 0, L.st, d, idt,
                       ix, iB, cum, state_end);
  });
}

template <int P, int N>
static int m256_combine_t(const Mamba2Dims& d, int dtype, const float* y_diag, const float* state_end,
                          const float* cum, const void* Cm, const float* state0, float* y, float* state_final,
                          float* ws, Launch& L) {
  if (d.C != 64 && d.C != 128 && d.C != 256) return ATOMIC_ERR_SHAPE;
  const StageIn iC{Cm, dtype == ATOMIC_BF16};
  const size_t elems = (size_t)d.B * d.H * P * N;
  int rc = L("mamba2_state_pass_bt256", [&] {
    hipLaunchKernelGGL((m256_state_pass_k<P, N>), dim3((unsigned)(elems / 256)), dim3(256), 0, L.st, d,
                       state_end, cum, state0, ws, state_final);
  });
  if (rc) return rc;
  return L("mamba2_combine_y_bt256", [&] {
    hipLaunchKernelGGL((m256_y_k<P, N>), dim3((unsigned)((size_t)d.B * d.H * d.NT * (d.C / RB))), dim3(256), 0,
                       L.st, d, y_diag, ws, cum, iC, y);
  });
}

#define AH_M256_DISPATCH(FN, ...)                                           \
  do {                                                                      \
    if (d.P == 64 && d.N == 128) return FN<64, 128>(__VA_ARGS__);           \
    if (d.P == 128 && d.N == 128) return FN<128, 128>(__VA_ARGS__);         \
    if (d.P == 192 && d.N == 128) return FN<192, 128>(__VA_ARGS__);         \
    if (d.P == 64 && d.N == 64) return FN<64, 64>(__VA_ARGS__);             \
    if (d.P == 128 && d.N == 64) return FN<128, 64>(__VA_ARGS__);           \
    return ATOMIC_ERR_SHAPE;                                                \
  } while (0)

int m256_intra(const Mamba2Dims& d, int dtype, const void* dt, const void* x, const void* Bm, const void* Cm,
               const float* cum, float* y_diag, float* state_end, float* cb, Launch& L) {
  AH_M256_DISPATCH(m256_intra_t, d, dtype, dt, x, Bm, Cm, cum, y_diag, state_end, cb, L);
}

int m256_combine(const Mamba2Dims& d, int dtype, const float* y_diag, const float* state_end, const float* cum,
                 const void* Cm, const float* state0, float* y, float* state_final, float* ws, Launch& L) {
  AH_M256_DISPATCH(m256_combine_t, d, dtype, y_diag, state_end, cum, Cm, state0, y, state_final, ws, L);
}

size_t m256_combine_ws(const Mamba2Dims& d) { return (size_t)d.B * d.NT * d.H * d.P * d.N * sizeof(float); }

}  // namespace ah
