// Stage-level backward kernels at the reference's 256-row Pallas block.
//
// The reference's trainable ops run their backward as separate staged
// functions over per-block float32 arrays (kernel_trainable_B6.py:97-181):
//   GDN2 B2  dav_backward_pallas           (kernel_bwd_b2_dav.py:17-51)
//        B1  gdn2_dhu_backward             (kernel_bwd_b1_dhu.py:14-44)
//        B3  wy_dqkg_backward_pallas       (kernel_bwd_b3_wy_dqkg.py:33-148)
//        B4  intra_backward_pallas         (kernel_bwd_b4_intra.py:57-165)
//        B5  reverse_cumsum_bwd            (kernel_bwd_b5_reverse_cumsum.py:17-24)
//   Mamba2 MB2 intra_chunk_ssd_bwd_pallas  (kernel_mamba2_bwd_b2_intra.py:32-180)
//          MB1 + MB3 mamba2_bwd_scan       (kernel_mamba2_bwd_b1_state.py:132-254)
//          MB4 mamba2_dA_backward          (mamba2_bwd_a_dA_reference.py:60-115)
// and, composed from them and the forward stage kernels, the float32 whole
// path that fp32 Mamba2 operands run (m_f32_fwd, m_f32_bwd).
// The whole path fuses these into its own kernels at 64 / 128-row chunks;
// the kernels here give each staged function with its own inputs, outputs
// and clip / nan_to_num placement.  Every value is float32 (the reference
// upcasts on entry).  They are the drop-in stage functions, not the
// benchmark path: block products run on a float32 LDS-tiled GEMM, and the
// pairwise-decay sums of B4 and MB2 are evaluated pair by pair on the vector
// ALUs with exp(clip(., +-20)) as the reference does.
#include "../../include/atomic_hybrid.h"
#include "common.hpp"
#include "stage256.hpp"

namespace ah {

namespace {

using In = StageIn;  // a read-only bf16 or fp32 operand

// Offset of batch item z = (z2 * Z1 + z1) * Z0 + z0 in an operand.
struct Bat {
  long long s2, s1, s0;
};
__device__ __forceinline__ size_t bat_off(const Bat& s, int z, int Z1, int Z0) {
  const int z0 = z % Z0, z1 = (z / Z0) % Z1, z2 = z / (Z0 * Z1);
  return (size_t)((long long)z2 * s.s2 + (long long)z1 * s.s1 + (long long)z0 * s.s0);
}

__device__ __forceinline__ float n2n_acc(float x) { return n2n(x, 1e4f); }

// ------------------------------------------------------------------ GEMM
// C(m, n) [op]= alpha sum_k A(m, k) B(k, n) per batch item, float32
// accumulation.  A(m, k) = ta ? A[k lda + m] : A[m lda + k]; likewise B.
// Epilogue: accum adds the previous C, then mask (1: keep m >= n, 2: keep
// m > n; masked entries are 0), then post (1: nan_to_num with +-1e4 for
// +-inf, 2: clip to +-1e4 and nan_to_num).
struct GemmOp {
  int M, N, K, Z1, Z0;
  In A;
  long long lda;
  Bat sa;
  int ta;
  In B;
  long long ldb;
  Bat sb;
  int tb;
  float* C;
  long long ldc;
  Bat sc;
  float alpha;
  int accum, mask, post;
};

constexpr int GT = 64, GK = 16;

__global__ __launch_bounds__(256) void sb_gemm_k(GemmOp g) {
  __shared__ __attribute__((aligned(16))) float sA[GK][GT + 4];
  __shared__ __attribute__((aligned(16))) float sB[GK][GT + 4];
  const int z = blockIdx.z;
  const int m0 = blockIdx.y * GT, n0 = blockIdx.x * GT;
  const int t = threadIdx.x, tx = t % 16, ty = t / 16;
  const size_t oa = bat_off(g.sa, z, g.Z1, g.Z0), ob = bat_off(g.sb, z, g.Z1, g.Z0);
  float acc[4][4];
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int j = 0; j < 4; ++j) acc[i][j] = 0.f;
  for (int k0 = 0; k0 < g.K; k0 += GK) {
#pragma unroll
    for (int it = 0; it < GT * GK / 256; ++it) {
      const int e = t + 256 * it;
      const int mm = g.ta ? e % GT : e / GK, kk = g.ta ? e / GT : e % GK;
      const int m = m0 + mm, k = k0 + kk;
      sA[kk][mm] = (m < g.M && k < g.K)
                       ? ld(g.A, oa + (g.ta ? (size_t)k * g.lda + m : (size_t)m * g.lda + k))
                       : 0.f;
      const int nn = g.tb ? e / GK : e % GT, kb = g.tb ? e % GK : e / GT;
      const int n = n0 + nn, kq = k0 + kb;
      sB[kb][nn] = (n < g.N && kq < g.K)
                       ? ld(g.B, ob + (g.tb ? (size_t)n * g.ldb + kq : (size_t)kq * g.ldb + n))
                       : 0.f;
    }
    __syncthreads();
#pragma unroll
    for (int kk = 0; kk < GK; ++kk) {
      float a[4], b[4];
#pragma unroll
      for (int i = 0; i < 4; ++i) a[i] = sA[kk][ty + 16 * i];
      const float4 bv = *reinterpret_cast<const float4*>(&sB[kk][4 * tx]);
      b[0] = bv.x; b[1] = bv.y; b[2] = bv.z; b[3] = bv.w;
#pragma unroll
      for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int j = 0; j < 4; ++j) acc[i][j] = fmaf(a[i], b[j], acc[i][j]);
    }
    __syncthreads();
  }
  const size_t oc = bat_off(g.sc, z, g.Z1, g.Z0);
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int m = m0 + ty + 16 * i;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int n = n0 + 4 * tx + j;
      if (m >= g.M || n >= g.N) continue;
      const size_t o = oc + (size_t)m * g.ldc + n;
      float v = g.alpha * acc[i][j];
      if (g.accum) v = g.C[o] + v;
      if ((g.mask == 1 && n > m) || (g.mask == 2 && n >= m)) v = 0.f;
      if (g.post == 1) v = n2n_acc(v);
      else if (g.post == 2) v = sanitize(v);
      g.C[o] = v;
    }
  }
}

int gemm(const GemmOp& g, int batch, const char* name, Launch& L) {
  if (batch <= 0 || batch > 65535 || g.M <= 0 || g.N <= 0 || g.K <= 0) return ATOMIC_ERR_SHAPE;
  const dim3 grid((g.N + GT - 1) / GT, (g.M + GT - 1) / GT, batch);
  return L(name, [&] { hipLaunchKernelGGL(sb_gemm_k, grid, dim3(256), 0, L.st, g); });
}

// A dense [Z][rows][cols] operand: plain batch stride rows * cols.
Bat dense(long long rows, long long cols) { return Bat{0, 0, rows * cols}; }

GemmOp gemm_op(int M, int N, int K, int Z) {
  GemmOp g{};
  g.M = M; g.N = N; g.K = K; g.Z1 = 1; g.Z0 = Z;
  g.alpha = 1.f;
  return g;
}

// ------------------------------------------------------------------ GDN2 B1
// Reverse scan per (batch, head, 32-column V tile): dh [K][32] in LDS; per
// block the rows go in 32-row pieces: dv_new = sanitize(dv_partial + kg dh),
// then from_out += qg^T (scale dO) and from_vnew += w_pseudo^T dv_new; at the
// block's end dh = sanitize(from_out + dh e^{gc_last} - from_vnew)
// (kernel_bwd_b1_dhu.py:22-39).
template <int K>
__global__ __launch_bounds__(256) void g256_dhu_k(Gdn2Dims d, In dO, const float* __restrict__ dvp,
                                                  const float* __restrict__ wp, const float* __restrict__ qg,
                                                  const float* __restrict__ kg, const float* __restrict__ gcl,
                                                  const float* __restrict__ dht, float* __restrict__ dh_all,
                                                  float* __restrict__ dh0, float* __restrict__ dv_all) {
  constexpr int VT = 32, RB = 32, KR = K / 8, LKP = K + 1;
  __shared__ float sDh[K][VT + 1];
  __shared__ float sKg[RB][LKP], sQg[RB][LKP], sWp[RB][LKP];
  __shared__ float sDo[RB][VT + 1], sDvn[RB][VT + 1];
  const int t = threadIdx.x, c = t % VT, kr = t / VT;  // this thread: column c, rows kr + 8 i of dh
  const int nvt = d.V / VT;
  const int bh = blockIdx.x / nvt, v0 = (blockIdx.x % nvt) * VT;
  const int V = d.V;
  // dht sanitised (kernel_bwd_b1_dhu.py:16-18)
  for (int i = 0; i < KR; ++i) {
    const int k = kr + 8 * i;
    sDh[k][c] = dht ? sanitize(dht[((size_t)bh * K + k) * V + v0 + c]) : 0.f;
  }
  __syncthreads();
  for (int n = d.NT - 1; n >= 0; --n) {
    const size_t blk = (size_t)bh * d.NT + n;
    float fo[KR], fv[KR];
    for (int i = 0; i < KR; ++i) { fo[i] = 0.f; fv[i] = 0.f; }
    for (int r0 = 0; r0 < kStageBlock; r0 += RB) {
      for (int e = t; e < RB * K; e += 256) {
        const int r = e / K, k = e % K;
        const size_t o = (blk * kStageBlock + r0 + r) * K + k;
        sKg[r][k] = kg[o];
        sQg[r][k] = qg[o];
        sWp[r][k] = wp[o];
      }
      for (int e = t; e < RB * VT; e += 256) {
        const int r = e / VT, cc = e % VT;
        sDo[r][cc] = d.scale * ld(dO, (blk * kStageBlock + r0 + r) * V + v0 + cc);   // :26
      }
      __syncthreads();
      for (int e = t; e < RB * VT; e += 256) {
        const int r = e / VT, cc = e % VT;
        float s = 0.f;
        for (int k = 0; k < K; ++k) s = fmaf(sKg[r][k], sDh[k][cc], s);
        const size_t o = (blk * kStageBlock + r0 + r) * V + v0 + cc;
        const float dv = sanitize(dvp[o] + s);                                      // :30-32
        sDvn[r][cc] = dv;
        dv_all[o] = dv;
      }
      __syncthreads();
      for (int r = 0; r < RB; ++r) {
        const float dov = sDo[r][c], dvv = sDvn[r][c];
        for (int i = 0; i < KR; ++i) {
          const int k = kr + 8 * i;
          fo[i] = fmaf(sQg[r][k], dov, fo[i]);                                      // :26-27
          fv[i] = fmaf(sWp[r][k], dvv, fv[i]);                                      // :34
        }
      }
      __syncthreads();
    }
    for (int i = 0; i < KR; ++i) {
      const int k = kr + 8 * i;
      const float decay = __expf(gcl[blk * K + k]);                                 // :24
      const float h = sanitize(fo[i] + sDh[k][c] * decay + (-fv[i]));               // :36-37
      sDh[k][c] = h;
      dh_all[(blk * K + k) * V + v0 + c] = h;
    }
    __syncthreads();
  }
  for (int i = 0; i < KR; ++i) {
    const int k = kr + 8 * i;
    dh0[((size_t)bh * K + k) * V + v0 + c] = sDh[k][c];
  }
}

// ------------------------------------------------------------------ GDN2 B3 element-wise parts
// kb = b k e^gc, kg = k e^(gc_last - gc), qg = q e^gc, wv = w v
// (kernel_bwd_b3_wy_dqkg.py:53-58), per block element.
__global__ __launch_bounds__(256) void g256_b3_prep_k(Gdn2Dims d, In q, In k, In b, In w, In v,
                                                      const float* __restrict__ gc, float* __restrict__ kb,
                                                      float* __restrict__ kgo, float* __restrict__ qgo,
                                                      float* __restrict__ wv) {
  const int K = d.K;
  const size_t total = (size_t)d.B * d.H * d.NT * kStageBlock * K;
  for (size_t e = (size_t)blockIdx.x * 256 + threadIdx.x; e < total; e += (size_t)gridDim.x * 256) {
    const size_t blk = e / ((size_t)kStageBlock * K);
    const int col = (int)(e % K);
    const float g = gc[e], gl = gc[(blk * kStageBlock + kStageBlock - 1) * K + col];
    const float kv = ld(k, e), eg = __expf(g);
    kb[e] = ld(b, e) * kv * eg;
    kgo[e] = kv * __expf(gl - g);
    qgo[e] = ld(q, e) * eg;
    wv[e] = ld(w, e) * ld(v, e);
  }
}

// The gc_last row term per (block, column): sum over rows of dkg kg plus
// e^(gc_last) sum_v dh_next h_pre (kernel_bwd_b3_wy_dqkg.py:92-107).
__global__ __launch_bounds__(256) void g256_b3_row_k(Gdn2Dims d, const float* __restrict__ gc,
                                                     const float* __restrict__ dkg, const float* __restrict__ kgo,
                                                     const float* __restrict__ dh_next,
                                                     const float* __restrict__ h_pre, float* __restrict__ row) {
  const int K = d.K, V = d.V;
  const size_t total = (size_t)d.B * d.H * d.NT * K;
  const size_t e = (size_t)blockIdx.x * 256 + threadIdx.x;
  if (e >= total) return;
  const size_t blk = e / K;
  const int col = (int)(e % K);
  float sx = 0.f;
  for (int r = 0; r < kStageBlock; ++r) {
    const size_t o = (blk * kStageBlock + r) * K + col;
    sx += dkg[o] * kgo[o];
  }
  float sh = 0.f;
  for (int j = 0; j < V; ++j) {
    const size_t o = (blk * K + col) * V + j;
    sh += dh_next[o] * h_pre[o];
  }
  const float gl = gc[(blk * kStageBlock + kStageBlock - 1) * K + col];
  row[e] = sx + __expf(gl) * sh;
}

// dq, dk, db, dw, dv_raw, dgc (kernel_bwd_b3_wy_dqkg.py:88-119).
__global__ __launch_bounds__(256) void g256_b3_final_k(Gdn2Dims d, In k, In b, In w, In v,
                                                       const float* __restrict__ gc, const float* __restrict__ kb,
                                                       const float* __restrict__ kgo, const float* __restrict__ qgo,
                                                       const float* __restrict__ dqg, const float* __restrict__ dkg,
                                                       const float* __restrict__ dkb, const float* __restrict__ dwv,
                                                       const float* __restrict__ row, float* __restrict__ dq,
                                                       float* __restrict__ dk, float* __restrict__ db,
                                                       float* __restrict__ dw, float* __restrict__ dvr,
                                                       float* __restrict__ dgc) {
  const int K = d.K;
  const size_t total = (size_t)d.B * d.H * d.NT * kStageBlock * K;
  for (size_t e = (size_t)blockIdx.x * 256 + threadIdx.x; e < total; e += (size_t)gridDim.x * 256) {
    const size_t blk = e / ((size_t)kStageBlock * K);
    const int r = (int)((e / K) % kStageBlock), col = (int)(e % K);
    const float g = gc[e], gl = gc[(blk * kStageBlock + kStageBlock - 1) * K + col];
    const float eg = __expf(g), ekg = __expf(gl - g);
    const float vdkb = dkb[e], vdkg = dkg[e], vdqg = dqg[e];
    const float dkfkb = vdkb * eg * ld(b, e);                     // :88
    const float dbv = vdkb * eg * ld(k, e);                       // :89
    const float dgkb = vdkb * kb[e];                              // :90
    const float dx = vdkg * kgo[e];                               // :92
    const float dkfkg = vdkg * ekg;                               // :93
    const float dqv = vdqg * eg;                                  // :97
    const float dgqg = vdqg * qgo[e];                             // :98
    dq[e] = n2n_acc(dqv);
    dk[e] = n2n_acc(dkfkb + dkfkg);                               // :103
    db[e] = n2n_acc(dbv);
    dw[e] = n2n_acc(dwv[e] * ld(v, e));                           // :100
    dvr[e] = n2n_acc(dwv[e] * ld(w, e));                          // :101
    float dg = dgkb + dgqg + (-dx);                               // :104
    if (r == kStageBlock - 1) dg = dg + row[blk * K + col];       // :108-111
    dgc[e] = n2n_acc(dg);
  }
}

// ------------------------------------------------------------------ GDN2 B4
// One workgroup per (batch, head, block, 16-column slice); thread (row
// group, column): rows rg + 16 i.  Sub-blocks of 128 rows, pairs (si >= sj)
// in the reference's order, with a clip after every accumulation
// (kernel_bwd_b4_intra.py:77-121).
constexpr int B4_SUB = 128, B4_DS = 16, B4_L = B4_DS + 1;

__global__ __launch_bounds__(256) void g256_b4_k(Gdn2Dims d, const float* __restrict__ daqk,
                                                 const float* __restrict__ dakk, In q, In k, In b,
                                                 const float* __restrict__ g, float* __restrict__ dq,
                                                 float* __restrict__ dk, float* __restrict__ db,
                                                 float* __restrict__ dgc) {
  constexpr int BT = kStageBlock;
  __shared__ float sGc[BT][B4_L], sLq[BT][B4_L], sK[BT][B4_L], sBk[BT][B4_L];
  const int K = d.K, nds = K / B4_DS;
  const int blk = blockIdx.x / nds, d0 = (blockIdx.x % nds) * B4_DS;
  const int n = blk % d.NT, bh = blk / d.NT, h = bh % d.H, bb = bh / d.H;
  const int t = threadIdx.x, c = t % B4_DS, rg = t / B4_DS;
  const size_t row0 = (size_t)bb * d.T + (size_t)n * BT;
  const size_t hk = (size_t)h * K + d0 + c;
  for (int i = 0; i < BT / 16; ++i) {
    const int r = rg + 16 * i;
    const size_t rr = row0 + r;
    const float kv = ld(k, rr * d.rk + hk);
    sLq[r][c] = d.scale * ld(q, rr * d.rq + hk);
    sK[r][c] = kv;
    sBk[r][c] = ld(b, rr * d.rb + hk) * kv;
    sGc[r][c] = g[rr * d.rg + hk];
  }
  __syncthreads();
  if (rg == 0) {  // gc = tril @ g over the block's rows (:66-68)
    float s = 0.f;
    for (int r = 0; r < BT; ++r) {
      s += sGc[r][c];
      sGc[r][c] = s;
    }
  }
  __syncthreads();
  const float* mq = daqk + (size_t)blk * BT * BT;
  const float* mk = dakk + (size_t)blk * BT * BT;
  const size_t ob = (size_t)blk * BT * K + d0 + c;
  for (int i = 0; i < BT / 16; ++i) {
    const int r = rg + 16 * i, rb = r / B4_SUB;
    const float gr = sGc[r][c], lq = sLq[r][c], kr = sK[r][c], bkr = sBk[r][c];
    float aq = 0.f, abk = 0.f, ak = 0.f, ag = 0.f;
    for (int si = 0; si < BT / B4_SUB; ++si) {
      for (int sj = 0; sj <= si; ++sj) {
        if (si == rb) {  // r as a row i of the pair
          float sq = 0.f, sk = 0.f, gq = 0.f, gk = 0.f;
          for (int j = sj * B4_SUB; j < (sj + 1) * B4_SUB; ++j) {
            const bool diag = si == sj;
            const float mqv = (diag && j > r) ? 0.f : mq[(size_t)r * BT + j];   // causal (:95-99)
            const float mkv = (diag && j >= r) ? 0.f : mk[(size_t)r * BT + j];  // strict
            const float dd = gr - sGc[j][c];
            const float e = __expf(fminf(fmaxf(dd, -kClipDecay), kClipDecay));
            const float cm = (dd >= -kClipDecay && dd <= kClipDecay) ? 1.f : 0.f;
            const float kj = sK[j][c];
            sq += mqv * e * kj;                                   // _dL_pair_sum (:38-41)
            sk += mkv * e * kj;
            gq += mqv * lq * kj * e * cm;                         // _dgc_pair_sum (:50-54)
            gk += mkv * bkr * kj * e * cm;
          }
          aq = sanitize(aq + sq * d.scale);                       // :117
          abk = sanitize(abk + sk);                               // :118
          ag = sanitize(ag + gq + gk);                            // :120
        }
        if (sj == rb) {  // r as a column j of the pair
          float sq = 0.f, sk = 0.f, gq = 0.f, gk = 0.f;
          for (int i2 = si * B4_SUB; i2 < (si + 1) * B4_SUB; ++i2) {
            const bool diag = si == sj;
            const float mqv = (diag && r > i2) ? 0.f : mq[(size_t)i2 * BT + r];
            const float mkv = (diag && r >= i2) ? 0.f : mk[(size_t)i2 * BT + r];
            const float dd = sGc[i2][c] - gr;
            const float e = __expf(fminf(fmaxf(dd, -kClipDecay), kClipDecay));
            const float cm = (dd >= -kClipDecay && dd <= kClipDecay) ? 1.f : 0.f;
            const float li = sLq[i2][c], bki = sBk[i2][c];
            sq += mqv * e * li;                                   // _dR_pair_sum (:44-47)
            sk += mkv * e * bki;
            gq += mqv * li * kr * e * cm;
            gk += mkv * bki * kr * e * cm;
          }
          ak = sanitize(ak + sq + sk);                            // :119
          ag = sanitize(ag + (-gq) + (-gk));                      // :121
        }
      }
    }
    const size_t o = ob + (size_t)r * K;
    const float bv = ld(b, (row0 + r) * d.rb + hk);
    dq[o] = sanitize(aq);                                         // :128-132
    dk[o] = sanitize(ak + abk * bv);                              // :124
    db[o] = sanitize(abk * kr);                                   // :125
    dgc[o] = sanitize(ag);
  }
}

// ------------------------------------------------------------------ B5
// dg = sanitize(reverse cumsum over the block's rows) per (block, column)
// (kernel_bwd_b5_reverse_cumsum.py:17-24).
__global__ __launch_bounds__(256) void rev_cumsum_k(const float* __restrict__ x, float* __restrict__ y,
                                                    long long blocks, int rows, int cols) {
  const long long e = (long long)blockIdx.x * 256 + threadIdx.x;
  if (e >= blocks * cols) return;
  const long long blk = e / cols;
  const int col = (int)(e % cols);
  const float* xp = x + (size_t)blk * rows * cols + col;
  float* yp = y + (size_t)blk * rows * cols + col;
  float s = 0.f;
  for (int r = rows - 1; r >= 0; --r) {
    s += xp[(size_t)r * cols];
    yp[(size_t)r * cols] = sanitize(s);
  }
}

// ------------------------------------------------------------------ Mamba2 MB2
// Per (batch, head, chunk) item z = (b H + h) NT + n, chunk rows C, sub-blocks
// of bc = min(128, C) rows (kernel_mamba2_bwd_b2_intra.py:20-21,35), pairs
// (si >= sj) in the reference's order.  Work arrays [Z][C][P] fp32 unless
// noted.

// dBx, the decay to the chunk end and its derived per-element terms
// (kernel_mamba2_bwd_b2_intra.py:47-65): dbx = sanitize(dt x), write,
// d_dBx_1, and d_dte_diff (its negation and column sums enter dcum).
__global__ __launch_bounds__(256) void m2b_elem_k(Mamba2Dims d, In dt, In x, const float* __restrict__ cum,
                                                  const float* __restrict__ dwrite, float* __restrict__ dbx,
                                                  float* __restrict__ write, float* __restrict__ d1,
                                                  float* __restrict__ ddd) {
  const int C = d.C, P = d.P;
  const size_t total = (size_t)d.B * d.H * d.NT * C * P;
  for (size_t e = (size_t)blockIdx.x * 256 + threadIdx.x; e < total; e += (size_t)gridDim.x * 256) {
    const size_t z = e / ((size_t)C * P);
    const int i = (int)((e / P) % C), p = (int)(e % P);
    const int n = (int)(z % d.NT), h = (int)((z / d.NT) % d.H), b = (int)(z / ((size_t)d.NT * d.H));
    const size_t row = (size_t)b * d.T + (size_t)n * C + i;
    const float dtv = ld(dt, row * d.rdt + (size_t)h * P + p), xv = ld(x, row * d.rx + (size_t)h * P + p);
    const float bx = sanitize(dtv * xv);                                              // :47
    const float cl = cum[(z * C + C - 1) * P + p];
    const float raw = cl - cum[e];                                                    // :51
    const float dte = __expf(fminf(fmaxf(raw, -kClipDecay), kClipDecay));            // :52
    const float dw = dwrite[e];
    dbx[e] = bx;
    write[e] = sanitize(bx * dte);                                                    // :53
    d1[e] = sanitize(dw * dte);                                                       // :59
    const float dd = sanitize(dw * bx);                                               // :60
    const float m = (raw >= -kClipDecay && raw <= kClipDecay) ? 1.f : 0.f;
    ddd[e] = sanitize(dd * dte * m);                                                  // :61-63
  }
}

// dBC of each sub-block pair: sum_p dy_i dBx_j exp(clip(cum_i - cum_j)),
// causal on diagonal pairs (:94,98-100); one 16 x 16 tile of (i, j) per
// workgroup, lower pairs only.  dbc [Z][C][C].
__global__ __launch_bounds__(256) void m2b_dbc_k(Mamba2Dims d, In dy, const float* __restrict__ cum,
                                                 const float* __restrict__ dbx, float* __restrict__ dbc) {
  __shared__ float sDy[16][17], sCi[16][17], sBx[16][17], sCj[16][17];
  const int C = d.C, P = d.P, bc = C < 128 ? C : 128, nt16 = C / 16;
  const int z = blockIdx.y, ti = blockIdx.x / nt16, tj = blockIdx.x % nt16;
  const int i0 = 16 * ti, j0 = 16 * tj;
  const int t = threadIdx.x, il = t / 16, jl = t % 16, i = i0 + il, j = j0 + jl;
  const bool pair = i0 / bc >= j0 / bc;   // a lower sub-block pair (si >= sj)
  const int n = z % d.NT, h = (z / d.NT) % d.H, b = z / (d.NT * d.H);
  const size_t zr = (size_t)z * C;
  float s = 0.f;
  if (pair) {
    for (int p0 = 0; p0 < P; p0 += 16) {
      {
        const int r = t / 16, c = t % 16;
        const size_t row = (size_t)b * d.T + (size_t)n * C + i0 + r;
        sDy[r][c] = ld(dy, row * d.rdy + (size_t)h * P + p0 + c);
        sCi[r][c] = cum[(zr + i0 + r) * P + p0 + c];
        sBx[r][c] = dbx[(zr + j0 + r) * P + p0 + c];
        sCj[r][c] = cum[(zr + j0 + r) * P + p0 + c];
      }
      __syncthreads();
#pragma unroll 4
      for (int c = 0; c < 16; ++c) {
        const float e = __expf(fminf(fmaxf(sCi[il][c] - sCj[jl][c], -kClipDecay), kClipDecay));
        s += sDy[il][c] * sBx[jl][c] * e;
      }
      __syncthreads();
    }
    if (i / bc == j / bc && j > i) s = 0.f;   // causal on the diagonal pair
  }
  dbc[(zr + i) * C + j] = pair ? s : 0.f;
}

// d_dBx_2 and dcum over the sub-block pairs, then ddt, dx and dcum
// (:74-128).  One workgroup per (item, 64-row block R, 32 channels); thread
// (channel p = t % 32, rows 64 R + rg .. + 7, rg = 8 (t / 32)).  For each
// sub-block pair the partner rows are staged 64 at a time with the CB tile
// between them and block R; every row sums its partners in ascending order,
// masked pairs included (their zero weight multiplies in, as the reference's
// causal mask does).
__global__ __launch_bounds__(256) void m2b_pair_k(Mamba2Dims d, In dt, In x, In dy, const float* __restrict__ cum,
                                                  const float* __restrict__ bcin, const float* __restrict__ dbx,
                                                  const float* __restrict__ d1, const float* __restrict__ ddd,
                                                  float* __restrict__ ddt, float* __restrict__ dx,
                                                  float* __restrict__ dcum) {
  constexpr int NR = 8, PC = 32, LP = PC + 1, LB = 65;
  __shared__ float sCum[64 * LP], sVal[64 * LP], sCB[64 * LB];
  __shared__ float sLast[16][PC];
  const int C = d.C, P = d.P, bc = C < 128 ? C : 128, nrb = C / 64, npg = P / PC;
  const int z = blockIdx.x / (nrb * npg), rem = blockIdx.x % (nrb * npg);
  const int R = rem / npg, p0 = (rem % npg) * PC;
  const int n = z % d.NT, h = z / d.NT % d.H, b = z / (d.NT * d.H);
  const int t = threadIdx.x, p = t % PC, rg = NR * (t / PC);
  const size_t zr = (size_t)z * C, row0 = (size_t)b * d.T + (size_t)n * C;
  const size_t hp = (size_t)h * P + p0;
  const float* bcz = bcin + ((size_t)b * d.NT + n) * C * C;   // sanitize(C B^T) of (b, n)
  const int rb = 64 * R / bc, nsub = C / bc, bpb = bc / 64;  // R's sub-block; 64-row blocks per sub-block
  float cr[NR], dyr[NR], bxr[NR], a2[NR], ac[NR];
#pragma unroll
  for (int a = 0; a < NR; ++a) {
    const int r = 64 * R + rg + a;
    cr[a] = cum[(zr + r) * P + p0 + p];
    dyr[a] = ld(dy, (row0 + r) * d.rdy + hp + p);
    bxr[a] = dbx[(zr + r) * P + p0 + p];
    a2[a] = 0.f;
    ac[a] = 0.f;
  }
  for (int si = 0; si < nsub; ++si) {
    for (int sj = 0; sj <= si; ++sj) {
      const bool diag = si == sj;
      float sjs[NR];
#pragma unroll
      for (int a = 0; a < NR; ++a) sjs[a] = 0.f;
      if (sj == rb) {  // R's rows as the column j: d_dBx_2 (:95,109) and dcum_j (:107,113), one pass
        float s2[NR];
#pragma unroll
        for (int a = 0; a < NR; ++a) s2[a] = 0.f;
        for (int Q = si * bpb; Q < (si + 1) * bpb; ++Q) {
          __syncthreads();
          for (int e = t; e < 64 * PC; e += 256) {
            const int rr = e / PC, pp = e % PC;
            sCum[rr * LP + pp] = cum[(zr + 64 * Q + rr) * P + p0 + pp];
            sVal[rr * LP + pp] = ld(dy, (row0 + 64 * Q + rr) * d.rdy + hp + pp);
          }
          for (int e = t; e < 64 * 64; e += 256) {
            const int rr = e >> 6, cc = e & 63;
            sCB[rr * LB + cc] = bcz[(size_t)(64 * Q + rr) * C + 64 * R + cc];   // CB(i, j), i in Q, j in R
          }
          __syncthreads();
          for (int ii = 0; ii < 64; ++ii) {
            const int i = 64 * Q + ii;
            const float ci = sCum[ii * LP + p], dyi = sVal[ii * LP + p];
#pragma unroll
            for (int a = 0; a < NR; ++a) {
              const float bl = (diag && i < 64 * R + rg + a) ? 0.f : sCB[ii * LB + rg + a];
              const float dd = ci - cr[a];
              const float e = __expf(fminf(fmaxf(dd, -kClipDecay), kClipDecay));
              const float m = (dd >= -kClipDecay && dd <= kClipDecay) ? 1.f : 0.f;
              s2[a] += e * bl * dyi;
              sjs[a] += dyi * bxr[a] * bl * e * m;
            }
          }
        }
#pragma unroll
        for (int a = 0; a < NR; ++a) a2[a] = sanitize(a2[a] + s2[a]);
      }
      if (si == rb) {  // R's rows as the row i: dcum_i (:105-106,112)
        float sis[NR];
#pragma unroll
        for (int a = 0; a < NR; ++a) sis[a] = 0.f;
        for (int Q = sj * bpb; Q < (sj + 1) * bpb; ++Q) {
          __syncthreads();
          for (int e = t; e < 64 * PC; e += 256) {
            const int rr = e / PC, pp = e % PC;
            sCum[rr * LP + pp] = cum[(zr + 64 * Q + rr) * P + p0 + pp];
            sVal[rr * LP + pp] = dbx[(zr + 64 * Q + rr) * P + p0 + pp];
          }
          for (int e = t; e < 64 * 64; e += 256) {
            const int rr = e >> 6, cc = e & 63;
            sCB[rr * LB + cc] = bcz[(size_t)(64 * R + rr) * C + 64 * Q + cc];   // CB(i, j), i in R, j in Q
          }
          __syncthreads();
          for (int jj = 0; jj < 64; ++jj) {
            const int j = 64 * Q + jj;
            const float cj = sCum[jj * LP + p], bxj = sVal[jj * LP + p];
#pragma unroll
            for (int a = 0; a < NR; ++a) {
              const float bl = (diag && j > 64 * R + rg + a) ? 0.f : sCB[(rg + a) * LB + jj];
              const float dd = cr[a] - cj;
              const float e = __expf(fminf(fmaxf(dd, -kClipDecay), kClipDecay));
              const float m = (dd >= -kClipDecay && dd <= kClipDecay) ? 1.f : 0.f;
              sis[a] += dyr[a] * bxj * bl * e * m;
            }
          }
        }
#pragma unroll
        for (int a = 0; a < NR; ++a) ac[a] = sanitize(ac[a] + sis[a]);
      }
      if (sj == rb) {
#pragma unroll
        for (int a = 0; a < NR; ++a) ac[a] = sanitize(ac[a] + (-sjs[a]));   // dcum_j (:107,113)
      }
    }
  }
  // the last row's d_cum_last_b: ddd summed over the chunk's rows, per row
  // group g (rows g, g + 16, ..) and then over the groups (:64-65,122-123)
  const bool last = R == nrb - 1;
  if (last) {
#pragma unroll
    for (int u = 0; u < 2; ++u) {
      const int g = 2 * (t / PC) + u;
      float lp = 0.f;
      for (int r = g; r < C; r += 16) lp += ddd[(zr + r) * P + p0 + p];
      sLast[g][p] = lp;
    }
  }
  __syncthreads();
#pragma unroll
  for (int a = 0; a < NR; ++a) {
    const int r = 64 * R + rg + a;
    const size_t o = (zr + r) * P + p0 + p;
    const float dtot = sanitize(d1[o] + a2[a]);                                   // :116
    const size_t io = (row0 + r) * (size_t)d.H * P + hp + p;
    ddt[io] = sanitize(dtot * ld(x, (row0 + r) * d.rx + hp + p));                  // :118,126
    dx[io] = sanitize(dtot * ld(dt, (row0 + r) * d.rdt + hp + p));                 // :119,127
    float dc = ac[a] + (-ddd[o]);                                                 // :64,121
    if (r == C - 1) {                                                             // :65,122-123
      float lb = 0.f;
      for (int g2 = 0; g2 < 16; ++g2) lb += sLast[g2][p];
      dc = dc + lb;
    }
    dcum[o] = sanitize(dc);                                                       // :128
  }
}

// dB, dC summed over the heads (:176-178): [B][T][N] from [Z][C][N].
__global__ __launch_bounds__(256) void m2b_headsum_k(Mamba2Dims d, const float* __restrict__ wb,
                                                     const float* __restrict__ wc, float* __restrict__ dB,
                                                     float* __restrict__ dC) {
  const size_t total = (size_t)d.B * d.T * d.N;
  const size_t e = (size_t)blockIdx.x * 256 + threadIdx.x;
  if (e >= total) return;
  const int s = (int)(e % d.N);
  const size_t tok = e / d.N;
  const int b = (int)(tok / d.T), tt = (int)(tok % d.T), n = tt / d.C, i = tt % d.C;
  float sb = 0.f, sc = 0.f;
  for (int h = 0; h < d.H; ++h) {
    const size_t o = ((((size_t)b * d.H + h) * d.NT + n) * d.C + i) * d.N + s;
    sb += wb[o];
    sc += wc[o];
  }
  dB[e] = sb;
  dC[e] = sc;
}

__global__ __launch_bounds__(256) void fill0_k(float* __restrict__ p, size_t n) {
  for (size_t e = (size_t)blockIdx.x * 256 + threadIdx.x; e < n; e += (size_t)gridDim.x * 256) p[e] = 0.f;
}

// ------------------------------------------------------------------ Mamba2 MB1 + MB3, MB4
// The reference's trainable Mamba2 backward (kernel_mamba2_trainable_B6.py:
// 83-131): mamba2_bwd_scan (kernel_mamba2_bwd_b1_state.py:132-254) re-runs
// the reference chunk forward for the state entering each chunk, runs the
// state-only reverse scan (mamba2_bwd_state_reference.py:87-137), MB2 with the
// scan's carries, and sums the two halves; mamba2_dA_backward
// (mamba2_bwd_a_dA_reference.py:60-115) is M2's adjoint.  The scans take one
// workgroup per (batch, head, 32 channels); thread (channel dd, column group
// sg) owns state columns sg + 8 k.
constexpr int MS_PT = 32, MS_RB = 32;

// The reference chunk's state recurrence (mamba2_ssd_reference.py:125-146):
// state_end = sanitize(B^T (dBx sanitize(e^{clip(cl - cum, +-20)}, 1e6))),
// state = sanitize(state e^{clip(cl, -20, 0)} + state_end); the state entering
// each chunk goes to sprev [B][NT][H][P][N].  Every chunk's product at once
// (one workgroup per (batch, head, chunk, 32 channels); thread (channel dd,
// column group sg) owns state columns sg + 8 k and sums the chunk's rows in
// order), left unsanitised in sprev; m2s_fwd_pass_k then walks the chunks.
template <int N>
__global__ __launch_bounds__(256) void m2s_fwd_se_k(Mamba2Dims d, In dt, In x, In Bm, const float* __restrict__ cum,
                                                    float* __restrict__ sprev) {
  constexpr int NK = N / 8;
  __shared__ float sW[MS_RB][MS_PT + 1];
  __shared__ float sB[MS_RB][N + 1];
  const int C = d.C, P = d.P, npt = P / MS_PT;
  const size_t z = blockIdx.x / npt;   // (b H + h) NT + n
  const int p0 = (blockIdx.x % npt) * MS_PT;
  const int n = (int)(z % d.NT), bh = (int)(z / d.NT), h = bh % d.H, b = bh / d.H;
  const int t = threadIdx.x, dd = t % MS_PT, sg = t / MS_PT;
  const float* cz = cum + z * C * P;
  float acc[NK];
#pragma unroll
  for (int k = 0; k < NK; ++k) acc[k] = 0.f;
  for (int r0 = 0; r0 < C; r0 += MS_RB) {
    __syncthreads();
    for (int e = t; e < MS_RB * MS_PT; e += 256) {
      const int r = e / MS_PT, c = e % MS_PT;
      const size_t row = (size_t)b * d.T + (size_t)n * C + r0 + r, col = (size_t)h * P + p0 + c;
      const float bx = sanitize(ld(dt, row * d.rdt + col) * ld(x, row * d.rx + col));          // :125-126
      const float raw = cz[(size_t)(C - 1) * P + p0 + c] - cz[(size_t)(r0 + r) * P + p0 + c];
      const float dte = sanitize(__expf(fminf(fmaxf(raw, -kClipDecay), kClipDecay)), 1e6f);  // :133-134
      sW[r][c] = bx * dte;                                                                     // :135
    }
    for (int e = t; e < MS_RB * N; e += 256) {
      const int r = e / N, s = e % N;
      sB[r][s] = ld(Bm, ((size_t)b * d.T + (size_t)n * C + r0 + r) * d.rB + s);
    }
    __syncthreads();
    for (int r = 0; r < MS_RB; ++r) {
      const float w = sW[r][dd];
#pragma unroll
      for (int k = 0; k < NK; ++k) acc[k] = fmaf(w, sB[r][sg + 8 * k], acc[k]);
    }
  }
  float* sp = sprev + ((((size_t)b * d.NT + n) * d.H + h) * P + p0 + dd) * N;
#pragma unroll
  for (int k = 0; k < NK; ++k) sp[sg + 8 * k] = acc[k];
}

// The recurrence itself, one thread per (batch, head, channel, state column),
// in place: each chunk's product is replaced by the state entering the chunk
// (state0 sanitised, :168-170).
__global__ __launch_bounds__(256) void m2s_fwd_pass_k(Mamba2Dims d, const float* __restrict__ cum,
                                                      const float* __restrict__ state0, float* __restrict__ sprev) {
  const size_t e = (size_t)blockIdx.x * 256 + threadIdx.x;
  const size_t total = (size_t)d.B * d.H * d.P * d.N;
  if (e >= total) return;
  const int s = (int)(e % d.N), p = (int)((e / d.N) % d.P);
  const size_t bh = e / ((size_t)d.P * d.N);
  const int h = (int)(bh % d.H), b = (int)(bh / d.H);
  float st = state0 ? sanitize(state0[e]) : 0.f;
  for (int n = 0; n < d.NT; ++n) {
    const size_t o = ((((size_t)b * d.NT + n) * d.H + h) * d.P + p) * d.N + s;
    const float se = sprev[o];
    sprev[o] = st;
    const float cl = cum[((bh * d.NT + n) * d.C + d.C - 1) * d.P + p];
    const float dce = __expf(fminf(fmaxf(cl, -kClipDecay), 0.f));                                  // :144
    st = sanitize(st * dce + sanitize(se));                                                        // :136-137,145-146
  }
}

// The state-only reverse scan (kernel_mamba2_bwd_b1_state.py:205-219 over
// mamba2_bwd_state_reference.py:87-137): per chunk the sanitised carry (MB2's
// dstate_end_grad, dse [B][H][NT][P][N]), dcum_state [B][H][NT][C][P],
// dy_off_raw = dy e^{clip(cum, -20, 0)} ([B][T][H][P], for dC), and the next
// carry sanitize(carry e^{clip(cl, -20, 0)} + dy_off_raw^T C).  The parts that
// do not depend on the carry run for every chunk at once (this kernel: dy_off_raw,
// dcum_state but the last row's carry term, and dy_off_raw^T C unsanitised in
// dse); m2s_bwd_pass_k walks the chunks and m2s_bwd_last_k adds the last rows'
// carry term.
template <int N>
__global__ __launch_bounds__(256) void m2s_bwd_par_k(Mamba2Dims d, In Cm, In dy, const float* __restrict__ cum,
                                                     const float* __restrict__ sprev, float* __restrict__ dyoff,
                                                     float* __restrict__ dcum_s, float* __restrict__ dse) {
  constexpr int NK = N / 8;
  __shared__ float sSp[MS_PT][N + 1];
  __shared__ float sC[MS_RB][N + 1];
  __shared__ float sDo[MS_RB][MS_PT + 1];
  const int C = d.C, P = d.P, npt = P / MS_PT;
  const size_t z = blockIdx.x / npt;   // (b H + h) NT + n
  const int p0 = (blockIdx.x % npt) * MS_PT;
  const int n = (int)(z % d.NT), bh = (int)(z / d.NT), h = bh % d.H, b = bh / d.H;
  const int t = threadIdx.x, dd = t % MS_PT, sg = t / MS_PT;
  const float* cz = cum + z * C * P;
#pragma unroll
  for (int k = 0; k < NK; ++k) {
    const int s = sg + 8 * k;
    sSp[dd][s] = sprev[((((size_t)b * d.NT + n) * d.H + h) * P + p0 + dd) * N + s];
  }
  float acc[NK];
#pragma unroll
  for (int k = 0; k < NK; ++k) acc[k] = 0.f;
  for (int r0 = 0; r0 < C; r0 += MS_RB) {
    __syncthreads();
    for (int e = t; e < MS_RB * N; e += 256) {
      const int r = e / N, s = e % N;
      sC[r][s] = ld(Cm, ((size_t)b * d.T + (size_t)n * C + r0 + r) * d.rC + s);
    }
    for (int e = t; e < MS_RB * MS_PT; e += 256) {
      const int r = e / MS_PT, c = e % MS_PT;
      const size_t row = (size_t)b * d.T + (size_t)n * C + r0 + r, col = (size_t)h * P + p0 + c;
      const float dh = __expf(fminf(fmaxf(cz[(size_t)(r0 + r) * P + p0 + c], -kClipDecay), 0.f));   // :103-104
      const float v = ld(dy, row * d.rdy + col) * dh;                                   // :117
      sDo[r][c] = v;
      dyoff[row * (size_t)d.H * P + col] = v;
    }
    __syncthreads();
    for (int e = t; e < MS_RB * MS_PT; e += 256) {  // dcum_state of the piece (:118,123-127)
      const int r = e / MS_PT, c = e % MS_PT;
      float y = 0.f;
      for (int s = 0; s < N; ++s) y = fmaf(sC[r][s], sSp[c][s], y);                     // y_off_raw (:105)
      const size_t row = (size_t)b * d.T + (size_t)n * C + r0 + r, col = (size_t)h * P + p0 + c;
      const float cv = cz[(size_t)(r0 + r) * P + p0 + c];
      const float dhr = fminf(fmaxf(cv, -kClipDecay), 0.f);
      const float dh = __expf(dhr);
      // the reference masks on the clipped exponent (:123-124), not on cum
      // as MB0 does (mamba2_bwd_reference.py:131), so every cum passes
      const float m = (dhr >= -kClipDecay && dhr <= 0.f) ? 1.f : 0.f;
      const float v = ld(dy, row * d.rdy + col) * y * dh * m;
      // the last row waits for its carry term (m2s_bwd_last_k)
      dcum_s[(z * C + r0 + r) * P + p0 + c] = r0 + r == C - 1 ? v : sanitize(v);          // :131
    }
    for (int r = 0; r < MS_RB; ++r) {  // dy_off_raw^T C (:120)
      const float v = sDo[r][dd];
#pragma unroll
      for (int k = 0; k < NK; ++k) acc[k] = fmaf(v, sC[r][sg + 8 * k], acc[k]);
    }
  }
#pragma unroll
  for (int k = 0; k < NK; ++k) dse[(z * P + p0 + dd) * N + sg + 8 * k] = acc[k];
}

// The carries, one thread per (batch, head, channel, state column), reverse
// over the chunks and in place: each chunk's dy_off_raw^T C is replaced by the
// sanitised carry entering its backward (:208,216), and the carry becomes
// sanitize(carry e^{clip(cl, -20, 0)} + dy_off_raw^T C) (:112,120,130).
__global__ __launch_bounds__(256) void m2s_bwd_pass_k(Mamba2Dims d, const float* __restrict__ cum,
                                                      const float* __restrict__ dsf, float* __restrict__ dse,
                                                      float* __restrict__ ds0) {
  const size_t e = (size_t)blockIdx.x * 256 + threadIdx.x;
  const size_t total = (size_t)d.B * d.H * d.P * d.N;
  if (e >= total) return;
  const int s = (int)(e % d.N), p = (int)((e / d.N) % d.P);
  const size_t bh = e / ((size_t)d.P * d.N);
  float car = dsf ? dsf[e] : 0.f;
  for (int n = d.NT - 1; n >= 0; --n) {
    const size_t z = bh * d.NT + n;
    const size_t o = (z * d.P + p) * d.N + s;
    const float acc = dse[o];
    const float c = sanitize(car);
    dse[o] = c;
    const float dce = __expf(fminf(fmaxf(cum[(z * d.C + d.C - 1) * d.P + p], -kClipDecay), 0.f));
    car = sanitize(c * dce + acc);
  }
  ds0[e] = sanitize(car);                                                                 // :219
}

// The last row's carry term d_cumdecay_last_a = (carry . state_prev) e^{cl}
// masked on cl (:113-114), for 32 (batch, head, chunk, channel) rows per
// workgroup: their carry and state rows are staged through LDS (coalesced)
// and each row's dot product runs in state-column order.  The rows hold up to
// MAXN state columns; m_bwd_scan admits N = 64 or 128 only.
__global__ __launch_bounds__(256) void m2s_bwd_last_k(Mamba2Dims d, const float* __restrict__ cum,
                                                      const float* __restrict__ sprev, const float* __restrict__ dse,
                                                      float* __restrict__ dcum_s) {
  constexpr int RW = 32, MAXN = 128;
  __shared__ float sA[RW][MAXN + 1], sS[RW][MAXN + 1];
  const size_t total = (size_t)d.B * d.H * d.NT * d.P;
  const size_t e0 = (size_t)blockIdx.x * RW;
  const int N = d.N;
  for (int e = threadIdx.x; e < RW * N; e += 256) {
    const int rr = e / N, s = e % N;
    const size_t er = e0 + rr;
    if (er < total) {
      const int p = (int)(er % d.P);
      const size_t z = er / d.P;
      const int n = (int)(z % d.NT);
      const size_t bh = z / d.NT;
      const int h = (int)(bh % d.H), b = (int)(bh / d.H);
      sA[rr][s] = dse[(z * d.P + p) * N + s];
      sS[rr][s] = sprev[((((size_t)b * d.NT + n) * d.H + h) * d.P + p) * N + s];
    }
  }
  __syncthreads();
  const int rr = threadIdx.x;
  if (rr >= RW || e0 + rr >= total) return;
  const size_t er = e0 + rr;
  const int p = (int)(er % d.P);
  const size_t z = er / d.P;
  float a = 0.f;
  for (int s = 0; s < N; ++s) a = fmaf(sA[rr][s], sS[rr][s], a);
  const size_t o = (z * d.C + d.C - 1) * d.P + p;
  const float cl = cum[o];
  const float dce = __expf(fminf(fmaxf(cl, -kClipDecay), 0.f));
  dcum_s[o] = sanitize(dcum_s[o] + a * dce * ((cl >= -kClipDecay && cl <= 0.f) ? 1.f : 0.f));
}

// MB3's sums (kernel_mamba2_bwd_b1_state.py:249-256), in place on MB2's outputs.
__global__ __launch_bounds__(256) void m2s_comb_k(size_t nhp, size_t nn, size_t ncum, float* __restrict__ ddt,
                                                  float* __restrict__ dx, float* __restrict__ dB,
                                                  float* __restrict__ dC, const float* __restrict__ dC_s,
                                                  float* __restrict__ dcum, const float* __restrict__ dcum_s) {
  // the loop covers the longest of the three ranges (dB / dC is the longest
  // when the state size exceeds heads x channels)
  const size_t top = nhp > ncum ? (nhp > nn ? nhp : nn) : (ncum > nn ? ncum : nn);
  for (size_t e = (size_t)blockIdx.x * 256 + threadIdx.x; e < top; e += (size_t)gridDim.x * 256) {
    if (e < nhp) {
      ddt[e] = sanitize(ddt[e]);
      dx[e] = sanitize(dx[e]);
    }
    if (e < nn) {
      dB[e] = sanitize(dB[e]);
      dC[e] = sanitize(dC_s[e] + dC[e]);
    }
    if (e < ncum) dcum[e] = sanitize(dcum_s[e] + dcum[e]);
  }
}

// MB4 per (batch, head, chunk, 64 channels), one lane per channel: the step
// exponents' clipped cumsum (kept in LDS), then the masked cumdecay cotangent
// reverse-cumsummed and masked by the step clip: ddt's second part and the
// workgroup's part of dA (mamba2_bwd_a_dA_reference.py:89-113).
// tok: dt in the token layout [B][T][H][P] with row stride d.rdt instead of
// the per-chunk one.
__global__ __launch_bounds__(64) void m2s_da_k(Mamba2Dims d, In dtp, int tok, const float* __restrict__ A,
                                               const float* __restrict__ dcum, float* __restrict__ ddt2,
                                               float* __restrict__ part) {
  __shared__ float sCr[256][65];
  const int C = d.C, P = d.P, nps = (P + 63) / 64;
  const size_t z = blockIdx.x / nps;
  const int p0 = (blockIdx.x % nps) * 64, c = threadIdx.x, p = p0 + c;
  const int h = (int)((z / d.NT) % d.H);
  const size_t b_ = z / ((size_t)d.NT * d.H), n = z % d.NT;
  auto dt_at = [&](int i) {
    return tok ? ld(dtp, ((size_t)b_ * d.T + n * C + i) * d.rdt + (size_t)h * P + p) : ld(dtp, (z * C + i) * P + p);
  };
  const float a = A[h];
  float dsum = 0.f;
  if (p < P) {
    float s = 0.f;
    for (int i = 0; i < C; ++i) {                                        // :89-94
      s += fminf(fmaxf(dt_at(i) * a, -kClipDecay), kClipDecay);
      sCr[i][c] = s;
    }
    float acc = 0.f;
    for (int i = C - 1; i >= 0; --i) {
      const size_t o = (z * C + i) * P + p;
      const float cr = sCr[i][c];
      acc += dcum[o] * ((cr >= -kClipAcc && cr <= kClipAcc) ? 1.f : 0.f);   // :98,101-103
      const float dtv = dt_at(i), raw = dtv * a;
      const float dr = acc * ((raw >= -kClipDecay && raw <= kClipDecay) ? 1.f : 0.f);   // :106
      ddt2[o] = sanitize(dr * a);                                        // :109,112
      dsum = fmaf(dr, dtv, dsum);                                        // :110
    }
  }
#pragma unroll
  for (int sh = 1; sh < 64; sh <<= 1) dsum += __shfl_xor(dsum, sh);
  if (c == 0) part[blockIdx.x] = dsum;
}

// dA[h] = sanitize(sum of the head's workgroup parts), in a fixed order (:110,113).
__global__ __launch_bounds__(256) void m2s_da_sum_k(Mamba2Dims d, int nps, const float* __restrict__ part,
                                                    float* __restrict__ dA) {
  const int h = blockIdx.x * 256 + threadIdx.x;
  if (h >= d.H) return;
  float s = 0.f;
  for (int b = 0; b < d.B; ++b)
    for (int n = 0; n < d.NT; ++n)
      for (int q = 0; q < nps; ++q) s += part[(((size_t)b * d.H + h) * d.NT + n) * nps + q];
  dA[h] = sanitize(s);
}

// M2 for any chunk and operand type (kernel_mamba2_a_decay.py:53-66):
// cum = sanitize(cumsum over the chunk of sanitize(dt A, 20), 1e4), one thread
// per (batch, head, chunk, channel), the running sum kept unclipped.
__global__ __launch_bounds__(256) void m2s_cum_k(Mamba2Dims d, In dt, const float* __restrict__ A,
                                                 float* __restrict__ cum) {
  const size_t e = (size_t)blockIdx.x * 256 + threadIdx.x;
  const size_t total = (size_t)d.B * d.H * d.NT * d.P;
  if (e >= total) return;
  const int p = (int)(e % d.P);
  const size_t z = e / d.P;
  const int n = (int)(z % d.NT), h = (int)((z / d.NT) % d.H), b = (int)(z / ((size_t)d.NT * d.H));
  const float a = A[h];
  float s = 0.f;
  for (int i = 0; i < d.C; ++i) {
    const size_t row = (size_t)b * d.T + (size_t)n * d.C + i;
    s += sanitize(ld(dt, row * d.rdt + (size_t)h * d.P + p) * a, kClipDecay);
    cum[(z * d.C + i) * d.P + p] = sanitize(s);
  }
}

// ddt = sanitize(the dt x part + the dt A part), the latter in the per-chunk
// layout (kernel_mamba2_trainable_B6.py:100-106).
__global__ __launch_bounds__(256) void m2s_ddt_k(Mamba2Dims d, const float* __restrict__ ddt_p,
                                                 const float* __restrict__ ddt2, float* __restrict__ ddt) {
  const size_t e = (size_t)blockIdx.x * 256 + threadIdx.x;
  const size_t total = (size_t)d.B * d.T * d.H * d.P;
  if (e >= total) return;
  const int p = (int)(e % d.P), h = (int)((e / d.P) % d.H);
  const size_t tok = e / ((size_t)d.H * d.P);
  const int b = (int)(tok / d.T), t = (int)(tok % d.T), n = t / d.C, i = t % d.C;
  const size_t o = ((((size_t)b * d.H + h) * d.NT + n) * d.C + i) * d.P + p;
  ddt[e] = sanitize(ddt_p[e] + ddt2[o]);
}

}  // namespace

// ------------------------------------------------------------------ launchers
int g256_dav_bwd(const Gdn2Dims& d, int do_dtype, const float* aqk, const float* v_new, const void* dO,
                 float* daqk, float* dvn, Launch& L) {
  constexpr int BT = kStageBlock;
  const int Z = d.B * d.H * d.NT, V = d.V;
  const int dob = do_dtype == ATOMIC_BF16;
  // dAqk = nan_to_num((dO v_new^T) * causal)   (kernel_bwd_b2_dav.py:26,29)
  GemmOp g = gemm_op(BT, BT, V, Z);
  g.A = In{dO, dob}; g.lda = V; g.sa = dense(BT, V);
  g.B = In{v_new, 0}; g.ldb = V; g.sb = dense(BT, V); g.tb = 1;
  g.C = daqk; g.ldc = BT; g.sc = dense(BT, BT);
  g.mask = 1; g.post = 1;
  int rc = gemm(g, Z, "g256_dav_daqk", L);
  if (rc != ATOMIC_OK) return rc;
  // dv_new = nan_to_num(Aqk^T dO)   (:27,30)
  GemmOp h = gemm_op(BT, V, BT, Z);
  h.A = In{aqk, 0}; h.lda = BT; h.sa = dense(BT, BT); h.ta = 1;
  h.B = In{dO, dob}; h.ldb = V; h.sb = dense(BT, V);
  h.C = dvn; h.ldc = V; h.sc = dense(BT, V);
  h.post = 1;
  return gemm(h, Z, "g256_dav_dvnew", L);
}

int g256_dhu_bwd(const Gdn2Dims& d, int do_dtype, const void* dO, const float* dvp, const float* wp,
                 const float* qg, const float* kg, const float* gcl, const float* dht, float* dh_all, float* dh0,
                 float* dv_all, Launch& L) {
  const In o{dO, do_dtype == ATOMIC_BF16};
  const dim3 grid(d.B * d.H * (d.V / 32));
  if (d.K == 128)
    return L("g256_dhu", [&] {
      hipLaunchKernelGGL((g256_dhu_k<128>), grid, dim3(256), 0, L.st, d, o, dvp, wp, qg, kg, gcl, dht, dh_all,
                         dh0, dv_all);
    });
  return L("g256_dhu", [&] {
    hipLaunchKernelGGL((g256_dhu_k<64>), grid, dim3(256), 0, L.st, d, o, dvp, wp, qg, kg, gcl, dht, dh_all, dh0,
                       dv_all);
  });
}

size_t g256_b3_ws(const Gdn2Dims& d) {
  const size_t z = (size_t)d.B * d.H * d.NT, bk = (size_t)kStageBlock * d.K, bb = (size_t)kStageBlock * kStageBlock;
  // kb, kg, qg, wv, dqg, dw_pseudo, dkg, dkb, dwv ([BT][K] each), dA, tmp ([BT][BT]), row ([K])
  return (z * (9 * bk + 2 * bb + d.K)) * sizeof(float);
}

int g256_b3_bwd(const Gdn2Dims& d, int dtype, int do_dtype, const void* q, const void* k, const void* b,
                const void* w, const void* v, const float* gc, const float* A, const float* h_pre,
                const float* v_new, const void* dO, const float* dv, const float* dh_next, float* dq, float* dk,
                float* db, float* dw, float* dvr, float* dgc, float* dakk, float* ws, Launch& L) {
  constexpr int BT = kStageBlock;
  const int Z = d.B * d.H * d.NT, K = d.K, V = d.V;
  const int bf = dtype == ATOMIC_BF16;
  const size_t zk = (size_t)Z * BT * K, zb = (size_t)Z * BT * BT;
  float *kb = ws, *kgo = kb + zk, *qgo = kgo + zk, *wv = qgo + zk, *dqg = wv + zk, *dwp = dqg + zk,
        *dkg = dwp + zk, *dkb = dkg + zk, *dwv = dkb + zk, *dA = dwv + zk, *tmp = dA + zb, *row = tmp + zb;
  const In iq{q, bf}, ik{k, bf}, ib{b, bf}, iw{w, bf}, iv{v, bf}, ido{dO, do_dtype == ATOMIC_BF16};
  const int eb = (int)((zk + 255) / 256 < 65536 ? (zk + 255) / 256 : 65536);
  int rc = L("g256_b3_prep", [&] {
    hipLaunchKernelGGL(g256_b3_prep_k, dim3(eb), dim3(256), 0, L.st, d, iq, ik, ib, iw, iv, gc, kb, kgo, qgo, wv);
  });
  if (rc != ATOMIC_OK) return rc;
  auto mm = [&](int M, int N, int Kd, In a, long long lda, Bat sa, int ta, In bo, long long ldb, Bat sb, int tb,
                float* c, long long ldc, Bat sc, float alpha, int accum, int mask, int post, const char* name) {
    GemmOp g = gemm_op(M, N, Kd, Z);
    g.A = a; g.lda = lda; g.sa = sa; g.ta = ta;
    g.B = bo; g.ldb = ldb; g.sb = sb; g.tb = tb;
    g.C = c; g.ldc = ldc; g.sc = sc;
    g.alpha = alpha; g.accum = accum; g.mask = mask; g.post = post;
    return gemm(g, Z, name, L);
  };
  const Bat sBK = dense(BT, K), sBV = dense(BT, V), sKV = dense(K, V), sBB = dense(BT, BT);
  // dqg = (scale dO) h_pre^T; dw_pseudo = -dv h_pre^T; dkg = v_new dh_next^T   (:60-67)
  if ((rc = mm(BT, K, V, ido, V, sBV, 0, In{h_pre, 0}, V, sKV, 1, dqg, K, sBK, d.scale, 0, 0, 0, "g256_b3_dqg")))
    return rc;
  if ((rc = mm(BT, K, V, In{dv, 0}, V, sBV, 0, In{h_pre, 0}, V, sKV, 1, dwp, K, sBK, -1.f, 0, 0, 0, "g256_b3_dwp")))
    return rc;
  if ((rc = mm(BT, K, V, In{v_new, 0}, V, sBV, 0, In{dh_next, 0}, V, sKV, 1, dkg, K, sBK, 1.f, 0, 0, 0,
               "g256_b3_dkg")))
    return rc;
  // dA_total = sanitize(dw_pseudo kb^T + dv wv^T)   (:69,72,75,78)
  if ((rc = mm(BT, BT, K, In{dwp, 0}, K, sBK, 0, In{kb, 0}, K, sBK, 1, dA, BT, sBB, 1.f, 0, 0, 0, "g256_b3_daw")))
    return rc;
  if ((rc = mm(BT, BT, V, In{dv, 0}, V, sBV, 0, In{wv, 0}, V, sBV, 1, dA, BT, sBB, 1.f, 1, 0, 2, "g256_b3_dau")))
    return rc;
  // dkb = A^T dw_pseudo; dwv = A^T dv   (:70,73)
  if ((rc = mm(BT, K, BT, In{A, 0}, BT, sBB, 1, In{dwp, 0}, K, sBK, 0, dkb, K, sBK, 1.f, 0, 0, 0, "g256_b3_dkb")))
    return rc;
  if ((rc = mm(BT, V, BT, In{A, 0}, BT, sBB, 1, In{dv, 0}, V, sBV, 0, dwv, V, sBV, 1.f, 0, 0, 0, "g256_b3_dwv")))
    return rc;
  // tmp = sanitize(dA_total A^T); dAkk = nan_to_num(-(A^T tmp) * strict)   (:83-86,119)
  if ((rc = mm(BT, BT, BT, In{dA, 0}, BT, sBB, 0, In{A, 0}, BT, sBB, 1, tmp, BT, sBB, 1.f, 0, 0, 2, "g256_b3_tmp")))
    return rc;
  if ((rc = mm(BT, BT, BT, In{A, 0}, BT, sBB, 1, In{tmp, 0}, BT, sBB, 0, dakk, BT, sBB, -1.f, 0, 2, 1,
               "g256_b3_dakk")))
    return rc;
  const int rb = (int)(((size_t)Z * K + 255) / 256);
  rc = L("g256_b3_row", [&] {
    hipLaunchKernelGGL(g256_b3_row_k, dim3(rb), dim3(256), 0, L.st, d, gc, dkg, kgo, dh_next, h_pre, row);
  });
  if (rc != ATOMIC_OK) return rc;
  return L("g256_b3_final", [&] {
    hipLaunchKernelGGL(g256_b3_final_k, dim3(eb), dim3(256), 0, L.st, d, ik, ib, iw, iv, gc, kb, kgo, qgo, dqg,
                       dkg, dkb, dwv, row, dq, dk, db, dw, dvr, dgc);
  });
}

int g256_intra_bwd(const Gdn2Dims& d, int dtype, const float* daqk, const float* dakk, const void* q,
                   const void* k, const void* b, const float* g, float* dq, float* dk, float* db, float* dgc,
                   Launch& L) {
  const int bf = dtype == ATOMIC_BF16;
  const dim3 grid(d.B * d.H * d.NT * (d.K / B4_DS));
  return L("g256_intra_bwd", [&] {
    hipLaunchKernelGGL(g256_b4_k, grid, dim3(256), 0, L.st, d, daqk, dakk, In{q, bf}, In{k, bf}, In{b, bf}, g,
                       dq, dk, db, dgc);
  });
}

int rev_cumsum_bwd(const float* dgc, float* dg, long long blocks, int rows, int cols, Launch& L) {
  const long long n = blocks * cols;
  if (n <= 0) return ATOMIC_ERR_SHAPE;
  return L("reverse_cumsum_bwd", [&] {
    hipLaunchKernelGGL(rev_cumsum_k, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, L.st, dgc, dg, blocks, rows,
                       cols);
  });
}


size_t m_intra_bwd_ws(const Mamba2Dims& d) {
  const size_t Z = (size_t)d.B * d.H * d.NT, C = d.C;
  // CB ([B][NT][C][C]), dwrite, dbx, write, d_dBx_1, d_dte_diff ([Z][C][P]),
  // per-head dB, dC ([Z][C][N]), dBC ([Z][C][C])
  return ((size_t)d.B * d.NT * C * C + 5 * Z * C * d.P + 2 * Z * C * d.N + Z * C * C) * sizeof(float);
}

int m_intra_bwd(const Mamba2Dims& d, int dtype, int dy_dtype, const void* dt, const void* x, const void* Bm,
                const void* Cm, const float* cum, const void* dy, const float* dse, float* ddt, float* dx, float* dB,
                float* dC, float* dcum, float* ws, Launch& L) {
  const int C = d.C, P = d.P, N = d.N, H = d.H, NT = d.NT, bc = C < 128 ? C : 128;
  const int Z = d.B * H * NT;
  const size_t zcp = (size_t)Z * C * P, zcn = (size_t)Z * C * N;
  float *bcin = ws, *dwrite = bcin + (size_t)d.B * NT * C * C, *dbx = dwrite + zcp, *write = dbx + zcp,
        *d1 = write + zcp, *ddd = d1 + zcp, *wB = ddd + zcp, *wC = wB + zcn, *dbc = wC + zcn;
  const int bf = dtype == ATOMIC_BF16, es = bf ? 2 : 4;
  const In idt{dt, bf}, ix{x, bf}, idy{dy, dy_dtype == ATOMIC_BF16};
  const char* Bp = static_cast<const char*>(Bm);   // byte pointers: the rows of a sub-block start at an offset
  const char* Cp = static_cast<const char*>(Cm);
  // item z = (b H + h) NT + n: a dense per-item array of S elements, and the
  // chunk rows of a [B][T][.] input (shared by the heads)
  auto dense3 = [&](long long S) { return Bat{(long long)H * NT * S, (long long)NT * S, S}; };
  auto rows3 = [&](long long r) { return Bat{(long long)d.T * r, 0, (long long)C * r}; };
  // CB = sanitize(C B^T) per (batch, chunk)   (:48)
  int rc = m_cb(d, dtype, Bm, Cm, bcin, L);
  if (rc != ATOMIC_OK) return rc;
  GemmOp g;
  // dwrite = sanitize(B dstate_end^T)   (:56)
  g = gemm_op(C, P, N, Z);
  g.Z1 = H; g.Z0 = NT;
  g.A = In{Bp, bf}; g.lda = d.rB; g.sa = rows3(d.rB);
  g.B = In{dse, 0}; g.ldb = N; g.sb = dense3((long long)P * N); g.tb = 1;
  g.C = dwrite; g.ldc = P; g.sc = dense3((long long)C * P);
  g.post = 2;
  if ((rc = gemm(g, Z, "m2b_dwrite", L))) return rc;
  const int eb = (int)((zcp + 255) / 256 < 65536 ? (zcp + 255) / 256 : 65536);
  rc = L("m2b_elem", [&] {
    hipLaunchKernelGGL(m2b_elem_k, dim3(eb), dim3(256), 0, L.st, d, idt, ix, cum, dwrite, dbx, write, d1, ddd);
  });
  if (rc != ATOMIC_OK) return rc;
  // per-head dB = sanitize(write dstate_end)   (:57), dC = 0   (:70)
  g = gemm_op(C, N, P, Z);
  g.Z1 = H; g.Z0 = NT;
  g.A = In{write, 0}; g.lda = P; g.sa = dense3((long long)C * P);
  g.B = In{dse, 0}; g.ldb = N; g.sb = dense3((long long)P * N);
  g.C = wB; g.ldc = N; g.sc = dense3((long long)C * N);
  g.post = 2;
  if ((rc = gemm(g, Z, "m2b_db1", L))) return rc;
  const int fb = (int)((zcn + 255) / 256 < 65536 ? (zcn + 255) / 256 : 65536);
  rc = L("m2b_fill", [&] { hipLaunchKernelGGL(fill0_k, dim3(fb), dim3(256), 0, L.st, wC, zcn); });
  if (rc != ATOMIC_OK) return rc;
  const int nt16 = C / 16;
  rc = L("m2b_dbc", [&] {
    hipLaunchKernelGGL(m2b_dbc_k, dim3(nt16 * nt16, Z), dim3(256), 0, L.st, d, idy, cum, dbx, dbc);
  });
  if (rc != ATOMIC_OK) return rc;
  // the sub-block pairs in order: dB[J] += dBC[I,J]^T C[I], dC[I] += dBC[I,J] B[J],
  // each sanitised   (:102-103,110-111)
  for (int si = 0; si < C / bc; ++si) {
    for (int sj = 0; sj <= si; ++sj) {
      const int i0 = si * bc, j0 = sj * bc;
      g = gemm_op(bc, N, bc, Z);
      g.Z1 = H; g.Z0 = NT;
      g.A = In{dbc + (size_t)i0 * C + j0, 0};   // transposed: A(m = j, k = i) = dBC[i0 + i][j0 + j]
      g.lda = C; g.sa = dense3((long long)C * C); g.ta = 1;
      g.B = In{Cp + (size_t)i0 * d.rC * es, bf}; g.ldb = d.rC; g.sb = rows3(d.rC);
      g.C = wB + (size_t)j0 * N; g.ldc = N; g.sc = dense3((long long)C * N);
      g.accum = 1; g.post = 2;
      if ((rc = gemm(g, Z, "m2b_db_pair", L))) return rc;
      g = gemm_op(bc, N, bc, Z);
      g.Z1 = H; g.Z0 = NT;
      g.A = In{dbc + (size_t)i0 * C + j0, 0}; g.lda = C; g.sa = dense3((long long)C * C);
      g.B = In{Bp + (size_t)j0 * d.rB * es, bf}; g.ldb = d.rB; g.sb = rows3(d.rB);
      g.C = wC + (size_t)i0 * N; g.ldc = N; g.sc = dense3((long long)C * N);
      g.accum = 1; g.post = 2;
      if ((rc = gemm(g, Z, "m2b_dc_pair", L))) return rc;
    }
  }
  rc = L("m2b_pair", [&] {
    hipLaunchKernelGGL(m2b_pair_k, dim3(Z * (C / 64) * (P / 32)), dim3(256), 0, L.st, d, idt, ix, idy, cum, bcin, dbx, d1,
                       ddd, ddt, dx, dcum);
  });
  if (rc != ATOMIC_OK) return rc;
  const size_t tn = (size_t)d.B * d.T * N;
  return L("m2b_headsum", [&] {
    hipLaunchKernelGGL(m2b_headsum_k, dim3((unsigned)((tn + 255) / 256)), dim3(256), 0, L.st, d, wB, wC, dB, dC);
  });
}


size_t m_bwd_scan_ws(const Mamba2Dims& d) {
  const size_t Z = (size_t)d.B * d.H * d.NT, C = d.C;
  const size_t own = Z * C * d.P            // cumdecay
                     + (size_t)d.B * d.NT * d.H * d.P * d.N   // state entering each chunk
                     + (size_t)d.B * d.T * d.H * d.P          // dy_off_raw
                     + (size_t)d.B * d.T * d.N                // dC_state
                     + Z * C * d.P                            // dcum_state
                     + Z * d.P * d.N;                         // the carries (dstate_end_grad)
  return own * sizeof(float) + m_intra_bwd_ws(d);
}

int m_bwd_scan(const Mamba2Dims& d, int dtype, int dy_dtype, const void* dt, const void* x, const void* Bm,
               const void* Cm, const float* cum, const void* dy, const float* dsf, const float* state0, float* ddt,
               float* dB, float* dC, float* dx, float* ds0, float* dcum, float* ws, Launch& L) {
  const int C = d.C, P = d.P, N = d.N;
  const size_t Z = (size_t)d.B * d.H * d.NT;
  if (P % MS_PT != 0 || (N != 64 && N != 128)) return ATOMIC_ERR_SHAPE;
  float* sprev = ws + Z * C * P;   // ws starts with the cumdecay the caller wrote
  float* dyoff = sprev + (size_t)d.B * d.NT * d.H * P * N;
  float* dC_s = dyoff + (size_t)d.B * d.T * d.H * P;
  float* dcum_s = dC_s + (size_t)d.B * d.T * N;
  float* dse = dcum_s + Z * C * P;
  float* wmb2 = dse + Z * P * N;
  const int bf = dtype == ATOMIC_BF16;
  const In idt{dt, bf}, ix{x, bf}, iB{Bm, bf}, iC{Cm, bf}, idy{dy, dy_dtype == ATOMIC_BF16};
  const dim3 grid((unsigned)(Z * (P / MS_PT)));
  const size_t nst = (size_t)d.B * d.H * P * N, nlast = Z * P;
  const dim3 gst((unsigned)((nst + 255) / 256)), glast((unsigned)((nlast + 31) / 32));
  int rc = L("m2s_fwd", [&] {
    if (N == 128)
      hipLaunchKernelGGL((m2s_fwd_se_k<128>), grid, dim3(256), 0, L.st, d, idt, ix, iB, cum, sprev);
    else
      hipLaunchKernelGGL((m2s_fwd_se_k<64>), grid, dim3(256), 0, L.st, d, idt, ix, iB, cum, sprev);
  });
  if (rc != ATOMIC_OK) return rc;
  rc = L("m2s_fwd_pass", [&] {
    hipLaunchKernelGGL(m2s_fwd_pass_k, gst, dim3(256), 0, L.st, d, cum, state0, sprev);
  });
  if (rc != ATOMIC_OK) return rc;
  rc = L("m2s_bwd", [&] {
    if (N == 128)
      hipLaunchKernelGGL((m2s_bwd_par_k<128>), grid, dim3(256), 0, L.st, d, iC, idy, cum, sprev, dyoff, dcum_s, dse);
    else
      hipLaunchKernelGGL((m2s_bwd_par_k<64>), grid, dim3(256), 0, L.st, d, iC, idy, cum, sprev, dyoff, dcum_s, dse);
  });
  if (rc != ATOMIC_OK) return rc;
  rc = L("m2s_bwd_pass", [&] {
    hipLaunchKernelGGL(m2s_bwd_pass_k, gst, dim3(256), 0, L.st, d, cum, dsf, dse, ds0);
  });
  if (rc != ATOMIC_OK) return rc;
  rc = L("m2s_bwd_last", [&] {
    hipLaunchKernelGGL(m2s_bwd_last_k, glast, dim3(256), 0, L.st, d, cum, sprev, dse, dcum_s);
  });
  if (rc != ATOMIC_OK) return rc;
  // dC_state = sanitize(dy_off_raw C-rows x state_prev over (head, channel)) per (batch, chunk)   (:119,129)
  GemmOp g = gemm_op(C, N, d.H * P, d.B * d.NT);
  g.Z1 = 1; g.Z0 = d.NT;
  g.A = In{dyoff, 0}; g.lda = (long long)d.H * P;
  g.sa = Bat{(long long)d.T * d.H * P, 0, (long long)C * d.H * P};
  g.B = In{sprev, 0}; g.ldb = N; g.sb = Bat{(long long)d.NT * d.H * P * N, 0, (long long)d.H * P * N};
  g.C = dC_s; g.ldc = N; g.sc = Bat{(long long)d.T * N, 0, (long long)C * N};
  g.post = 2;
  if ((rc = gemm(g, d.B * d.NT, "m2s_dc_state", L))) return rc;
  // MB2 with the carries as dstate_end_grad (:240-243)
  if ((rc = m_intra_bwd(d, dtype, dy_dtype, dt, x, Bm, Cm, cum, dy, dse, ddt, dx, dB, dC, dcum, wmb2, L))) return rc;
  const size_t nhp = (size_t)d.B * d.T * d.H * P, nn = (size_t)d.B * d.T * N, ncum = Z * C * P;
  const size_t top = nhp > ncum ? (nhp > nn ? nhp : nn) : (ncum > nn ? ncum : nn);
  const int eb = (int)((top + 255) / 256 < 65536 ? (top + 255) / 256 : 65536);
  return L("m2s_comb", [&] {
    hipLaunchKernelGGL(m2s_comb_k, dim3(eb), dim3(256), 0, L.st, nhp, nn, ncum, ddt, dx, dB, dC, dC_s, dcum, dcum_s);
  });
}

size_t m_da_bwd_ws(const Mamba2Dims& d) {
  return (size_t)d.B * d.H * d.NT * ((d.P + 63) / 64) * sizeof(float);
}

int m_da_bwd(const Mamba2Dims& d, int dt_dtype, int tok, const void* dtp, const float* A, const float* dcum,
             float* ddt2, float* dA, float* ws, Launch& L) {
  if (d.C > 256) return ATOMIC_ERR_SHAPE;
  const int nps = (d.P + 63) / 64;
  const unsigned nb = (unsigned)((size_t)d.B * d.H * d.NT * nps);
  const In it{dtp, dt_dtype == ATOMIC_BF16};
  int rc = L("m2s_da", [&] {
    hipLaunchKernelGGL(m2s_da_k, dim3(nb), dim3(64), 0, L.st, d, it, tok, A, dcum, ddt2, ws);
  });
  if (rc != ATOMIC_OK) return rc;
  return L("m2s_da_sum", [&] {
    hipLaunchKernelGGL(m2s_da_sum_k, dim3((unsigned)((d.H + 255) / 256)), dim3(256), 0, L.st, d, nps, ws, dA);
  });
}


size_t m_cb_ws(const Mamba2Dims& d) { return (size_t)d.B * d.NT * d.C * d.C * sizeof(float); }

int m_cb(const Mamba2Dims& d, int dtype, const void* Bm, const void* Cm, float* cb, Launch& L) {
  const int C = d.C, N = d.N, NT = d.NT, bf = dtype == ATOMIC_BF16;
  GemmOp g = gemm_op(C, C, N, d.B * NT);
  g.Z1 = 1; g.Z0 = NT;
  g.A = In{Cm, bf}; g.lda = d.rC; g.sa = Bat{(long long)d.T * d.rC, 0, (long long)C * d.rC};
  g.B = In{Bm, bf}; g.ldb = d.rB; g.sb = Bat{(long long)d.T * d.rB, 0, (long long)C * d.rB}; g.tb = 1;
  g.C = cb; g.ldc = C; g.sc = Bat{(long long)NT * C * C, 0, (long long)C * C};
  g.post = 2;
  return gemm(g, d.B * NT, "mamba2_cb_f32", L);
}

int m_cumdecay(const Mamba2Dims& d, int dtype, const void* dt, const float* A, float* cum, Launch& L) {
  const size_t n = (size_t)d.B * d.H * d.NT * d.P;
  const In idt{dt, dtype == ATOMIC_BF16};
  return L("mamba2_cumdecay_f32", [&] {
    hipLaunchKernelGGL(m2s_cum_k, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, L.st, d, idt, A, cum);
  });
}

size_t m_f32_fwd_ws(const Mamba2Dims& d) {  // cum, y_diag, state_end, then M3's CB or M4's states
  const size_t Z = (size_t)d.B * d.H * d.NT;
  const size_t cb = m_cb_ws(d), st = m256_combine_ws(d);
  return (Z * d.C * d.P + (size_t)d.B * d.T * d.H * d.P + Z * d.P * d.N) * sizeof(float) + (cb > st ? cb : st);
}

int m_f32_fwd(const Mamba2Dims& d, const void* dt, const void* x, const void* Bm, const void* Cm, const float* A,
              const float* state0, float* y, float* state_final, float* ws, Launch& L) {
  const size_t Z = (size_t)d.B * d.H * d.NT;
  float* cum = ws;
  float* y_diag = cum + Z * d.C * d.P;
  float* state_end = y_diag + (size_t)d.B * d.T * d.H * d.P;
  float* pre = state_end + Z * d.P * d.N;
  int rc = m_cumdecay(d, ATOMIC_F32, dt, A, cum, L);
  if (rc) return rc;
  if ((rc = m256_intra(d, ATOMIC_F32, dt, x, Bm, Cm, cum, y_diag, state_end, pre, L))) return rc;
  return m256_combine(d, ATOMIC_F32, y_diag, state_end, cum, Cm, state0, y, state_final, pre, L);
}

size_t m_f32_bwd_ws(const Mamba2Dims& d) {
  const size_t Z = (size_t)d.B * d.H * d.NT;
  return m_bwd_scan_ws(d) + ((size_t)d.B * d.T * d.H * d.P + 2 * Z * d.C * d.P) * sizeof(float) + m_da_bwd_ws(d);
}

int m_f32_bwd(const Mamba2Dims& d, int dy_dtype, const void* dt, const void* x, const void* Bm, const void* Cm,
              const float* A, const float* state0, const void* dy, const float* dsf, float* ddt, float* dx,
              float* dB, float* dC, float* dA, float* ds0, float* ws, Launch& L) {
  const size_t Z = (size_t)d.B * d.H * d.NT;
  float* scan_ws = ws;                                  // cumdecay first
  float* ddt_p = ws + m_bwd_scan_ws(d) / sizeof(float);
  float* dcum = ddt_p + (size_t)d.B * d.T * d.H * d.P;
  float* ddt2 = dcum + Z * d.C * d.P;
  float* da_ws = ddt2 + Z * d.C * d.P;
  int rc = m_cumdecay(d, ATOMIC_F32, dt, A, scan_ws, L);
  if (rc) return rc;
  if ((rc = m_bwd_scan(d, ATOMIC_F32, dy_dtype, dt, x, Bm, Cm, scan_ws, dy, dsf, state0, ddt_p, dB, dC, dx, ds0,
                       dcum, scan_ws, L)))
    return rc;
  if ((rc = m_da_bwd(d, ATOMIC_F32, 1, dt, A, dcum, ddt2, dA, da_ws, L))) return rc;
  const size_t n = (size_t)d.B * d.T * d.H * d.P;
  return L("mamba2_ddt_f32", [&] {
    hipLaunchKernelGGL(m2s_ddt_k, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, L.st, d, ddt_p, ddt2, ddt);
  });
}

}  // namespace ah
