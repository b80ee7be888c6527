// GDN2 WY chunked forward for gfx950.
//
// gdn2_fwd_intra  (one workgroup per (batch, head, chunk); fully parallel)
//   Follows _build_chunk_wy (atomic_ops/gdn2_wy_reference.py:59-102):
//   gc = cumsum(g); Aqk / Akk intra-chunk scores; A = (I + Akk)^-1;
//   w_pseudo = A (b k e^gc); u = A (w v); kg, qg; gc_last.
//   The pairwise decay exp(gc_i - gc_j) is factorised as
//   (q e^{gc_i}) . (k e^{-gc_j}) so both score matrices are bf16 MFMA GEMMs.
//   The factorisation is exact while every g <= 0 in the chunk (then
//   gc_i - gc_j <= 0 on causal pairs, so the reference's +20 clip never
//   fires) and -gc_last <= kFactorLimit (so k e^{-gc} stays finite).  Pairs
//   whose decay falls below the reference's -20 floor then carry their true
//   (smaller) weight instead of e^-20, a difference below 2e-9 |q||k|.  Any
//   chunk outside those bounds takes an exact pairwise path that applies
//   exp(clip(gc_i - gc_j, -20, 20)) as the reference does.
//
// gdn2_fwd_state  (one workgroup per (batch, head, V tile); sequential over
//   chunks).  Follows the scan step of gdn2_chunked_wy_reference
//   (gdn2_wy_reference.py:125-144) / gdn2_inter_chunk_combine
//   (kernel_d_pipeline.py:94-124): v_new = u - w_pseudo h;
//   o = scale qg h + Aqk v_new; h = sanitize(h e^{gc_last} + kg^T v_new).
//   The fp32 state lives in MFMA accumulators for the whole sequence.
#include "gdn2.hpp"

namespace ah {

constexpr float kFactorLimit = 64.f;

// ------------------------------------------------------------------ cumsum
// Thread map for [C][K] fp32 element-wise passes: column group cg (8
// columns), segment seg (RS consecutive rows).
template <int C, int K>
struct ColMap {
  static constexpr int NCG = K / 8, NSEG = 256 / NCG, RS = C / NSEG;
  static_assert(RS >= 1, "chunk too small for the thread mapping");
};

// Exclusive scan over the row segments of a ColMap pass: t holds this
// thread's segment total for its 8 columns; out gets the sum over the lower
// segments (REV = false) or the higher ones (REV = true).  Within a wave by
// lane shuffles, across the 4 waves through sW (4 * K floats).
template <int NCG, bool REV>
__device__ __forceinline__ void seg_scan8(const float (&t)[8], float (&out)[8], float* sW) {
  constexpr int SPW = 64 / NCG;  // segments per wave
  static_assert(SPW * NCG == 64, "column groups must tile a wave");
  const int lane = lane_id(), w = wave_id(), sl = lane / NCG, cg = lane % NCG;
  float x[8];
#pragma unroll
  for (int j = 0; j < 8; ++j) x[j] = t[j];
#pragma unroll
  for (int d = 1; d < SPW; d <<= 1) {
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      const float y = REV ? __shfl_down(x[j], d * NCG) : __shfl_up(x[j], d * NCG);
      if (REV ? (sl + d < SPW) : (sl >= d)) x[j] += y;
    }
  }
  if (sl == (REV ? 0 : SPW - 1)) {
#pragma unroll
    for (int j = 0; j < 8; ++j) sW[w * NCG * 8 + cg * 8 + j] = x[j];
  }
  __syncthreads();
#pragma unroll
  for (int j = 0; j < 8; ++j) out[j] = x[j] - t[j];
#pragma unroll
  for (int w2 = 0; w2 < 4; ++w2)
    if (REV ? w2 > w : w2 < w) {
#pragma unroll
      for (int j = 0; j < 8; ++j) out[j] += sW[w2 * NCG * 8 + cg * 8 + j];
    }
}

// gc = cumsum(g) over one chunk (gdn2_wy_reference.py:63) for this thread's
// RS rows x 8 columns.  Writes gc_last to sGl[K] (sTot: NSEG*K floats of
// scratch).  Returns, uniformly over the workgroup, whether the factorised
// pairwise decay is unsafe for this chunk: some g > 0, or gc_last below
// -kFactorLimit in some column.
template <int C, int K>
__device__ __forceinline__ bool chunk_cumsum(const float* __restrict__ g, size_t rs,
                                             float (&gcr)[ColMap<C, K>::RS][8], float* sTot,
                                             float* sGl) {
  typedef ColMap<C, K> M;
  const int tid = threadIdx.x, cg = tid % M::NCG, seg = tid / M::NCG;
  bool positive = false;
#pragma unroll
  for (int rr = 0; rr < M::RS; ++rr) {
    load8(g + (size_t)(seg * M::RS + rr) * rs + cg * 8, gcr[rr]);
#pragma unroll
    for (int j = 0; j < 8; ++j) positive |= gcr[rr][j] > 0.f;
  }
#pragma unroll
  for (int rr = 1; rr < M::RS; ++rr)
#pragma unroll
    for (int j = 0; j < 8; ++j) gcr[rr][j] += gcr[rr - 1][j];
  float off[8];
  seg_scan8<M::NCG, false>(gcr[M::RS - 1], off, sTot);
#pragma unroll
  for (int rr = 0; rr < M::RS; ++rr)
#pragma unroll
    for (int j = 0; j < 8; ++j) gcr[rr][j] += off[j];
  bool too_deep = false;
  if (seg == M::NSEG - 1) {
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      sGl[cg * 8 + j] = gcr[M::RS - 1][j];
      too_deep |= gcr[M::RS - 1][j] < -kFactorLimit;
    }
  }
  return __syncthreads_or(positive || too_deep);
}

// ------------------------------------------------------------------ layout
template <typename T, int C, int K, int V>
struct IntraLds {
  static constexpr int PAD = Pad<T>::v;
  static constexpr int LK = K + PAD, LV = V + PAD;
  static constexpr int LA = C + 4;                 // fp32 score / inverse rows
  static constexpr int LAB = C + PAD;              // operand-type inverse rows
  static constexpr int NCG = K / 8, NSEG = 256 / NCG, RS = C / NSEG;
  static constexpr int NCGV = V / 8, NSEGV = 256 / NCGV, RSV = C / NSEGV;
  static constexpr int OPK = C * LK * (int)sizeof(T);
  static constexpr int OPV = C * LV * (int)sizeof(T);
  static constexpr int AF = C * LA * 4;
  static constexpr int off_q = 0, off_k = OPK, off_b = 2 * OPK, off_w = 3 * OPK;
  static constexpr int end_ops = 3 * OPK + OPV;
  static constexpr bool alias_a = 2 * OPK >= 2 * AF;
  static constexpr int off_af = alias_a ? 0 : end_ops;      // Akk (then operand-type A)
  static constexpr int off_x = off_af + AF;                 // fp32 inverse
  static constexpr int end_a = off_x + AF;
  static constexpr int off_tot = (end_ops > end_a ? end_ops : end_a);
  static constexpr int TOT = NSEG * K * 4;                  // cumsum segment totals; solve scratch
  static constexpr int off_gl = off_tot + (TOT > 4 * 16 * 17 * 4 ? TOT : 4 * 16 * 17 * 4);
  static constexpr int off_flag = off_gl + K * 4;
  static constexpr int total = off_flag + 16;
  // phase 4 (operand-type path): per-wave [16][LS] staging of one row block of
  // w_pseudo / u, placed over the operands that are dead by then (q, k, the
  // fp32 Akk / inverse), after the operand-type inverse
  static constexpr int LS = (K > V ? K : V) + PAD;
  static constexpr int off_stage =
      alias_a ? ((off_af + C * (C + PAD) * (int)sizeof(T) + 15) / 16) * 16 : 0;
  static constexpr int stage_end = off_stage + 4 * 16 * LS * (int)sizeof(T);
  static constexpr bool stage_fits = stage_end <= off_b && (alias_a || stage_end <= off_af);
  static_assert(RS >= 1 && RSV >= 1, "chunk too small for the thread mapping");
  static_assert(2 * OPK >= C * K * 4, "gc scratch of the exact path must fit in sQ+sK");
};

// Exact pairwise scores for one chunk (reference form, used when the
// factorised form could overflow or a positive gate breaks monotonicity).
template <typename T, int C, int K>
__device__ void intra_scores_exact(const float* sgc, const T* q, const T* k, const T* b, size_t sq,
                                   size_t sk, size_t sb, float scale, float* out_qk, float* out_kk) {
  // thread t computes entries e = t, t + 256, ... of the C x C matrices
  for (int e = threadIdx.x, s = 0; e < C * C; e += 256, ++s) {
    const int i = e / C, j = e % C;
    float aqk = 0.f, akk = 0.f;
    if (j <= i) {
      const T* qi = q + i * sq;
      const T* ki = k + i * sk;
      const T* bi = b + i * sb;
      const T* kj = k + j * sk;
      for (int d = 0; d < K; ++d) {
        const float dd = sgc[i * K + d] - sgc[j * K + d];
        const float ed = __expf(fminf(fmaxf(dd, -kClipDecay), kClipDecay));
        const float kjd = to_f(kj[d]);
        aqk += to_f(qi[d]) * ed * kjd;
        akk += to_f(bi[d]) * to_f(ki[d]) * ed * kjd;
      }
      aqk *= scale;
      if (j == i) akk = 0.f;
    }
    out_qk[s] = n2n(aqk);
    out_kk[s] = n2n(akk);
  }
}

// What one gdn2_fwd_intra launch builds: the whole per-chunk build (kernels
// A + B + C in one pass), or one of the reference's three kernels over
// caller-owned per-chunk arrays:
//   kIntraScores    A: Aqk and the strict Akk (kernel_a_scores.py:21-66)
//   kIntraSolve     B: A = (I + Akk)^-1 from a given Akk (kernel_b_solve.py)
//   kIntraRecompute C: w_pseudo = A kb, u = A (w v), kg, qg, gc_last from a
//                   given A, all clipped to +-1e4 (kernel_c_recompute.py:46-88)
enum { kIntraAll = 0, kIntraScores = 1, kIntraSolve = 2, kIntraRecompute = 3 };

template <typename T, int C, int K, int V, int ST = kIntraAll>
__global__ __launch_bounds__(256) void gdn2_fwd_intra(Gdn2Dims dm, const T* __restrict__ q,
                                                     const T* __restrict__ k, const T* __restrict__ v,
                                                     const T* __restrict__ w, const T* __restrict__ b,
                                                     const float* __restrict__ g, Gdn2Chunks<T> ck) {
  typedef IntraLds<T, C, K, V> L;
  __shared__ __attribute__((aligned(16))) unsigned char lds[L::total];
  T* sQ = reinterpret_cast<T*>(lds + L::off_q);
  T* sK = reinterpret_cast<T*>(lds + L::off_k);
  T* sB = reinterpret_cast<T*>(lds + L::off_b);
  T* sW = reinterpret_cast<T*>(lds + L::off_w);
  float* sAf = reinterpret_cast<float*>(lds + L::off_af);
  float* sX = reinterpret_cast<float*>(lds + L::off_x);
  float* sTot = reinterpret_cast<float*>(lds + L::off_tot);
  float* sGl = reinterpret_cast<float*>(lds + L::off_gl);
  float* sGcExact = reinterpret_cast<float*>(lds + L::off_q);  // exact path only

  const int tid = threadIdx.x;
  const int bhn = blockIdx.x;
  const int n = bhn % dm.NT;
  const int bh = bhn / dm.NT;
  const int h = bh % dm.H;
  const int bb = bh / dm.H;
  const size_t t0 = (size_t)bb * dm.T + (size_t)n * C;
  const T* qc = q + t0 * dm.rq + (size_t)h * K;
  const T* kc = k + t0 * dm.rk + (size_t)h * K;
  const T* bc = b + t0 * dm.rb + (size_t)h * K;
  const float* gc_in = g + t0 * dm.rg + (size_t)h * K;
  const T* vc = v + t0 * dm.rv + (size_t)h * V;
  const T* wc = w + t0 * dm.rw + (size_t)h * V;

  // q, k, b, v, w are requested before the cumsum of g, so their latency overlaps it
  const int cg = tid % L::NCG, seg = tid / L::NCG;
  const int cgv = tid % L::NCGV, segv = tid / L::NCGV;
  constexpr bool kRows = ST != kIntraSolve;                          // reads q, k, b, g
  constexpr bool kVals = ST == kIntraAll || ST == kIntraRecompute;   // reads v, w; writes qg, kg
  constexpr bool kScores = ST == kIntraAll || ST == kIntraScores;
  // the stage-level kernel C clips every output to +-1e4 (kernel_c_recompute.py:74-82)
  auto fin = [](float x) { return ST == kIntraRecompute ? sanitize(x) : n2n(x); };
  Raw8<T> rq[L::RS], rk[L::RS], rb[L::RS], rv[L::RSV], rw[L::RSV];
  if constexpr (kRows) {
#pragma unroll
    for (int rr = 0; rr < L::RS; ++rr) {
      const size_t r = (size_t)(seg * L::RS + rr);
      rq[rr].load(qc + r * dm.rq + cg * 8);
      rk[rr].load(kc + r * dm.rk + cg * 8);
      rb[rr].load(bc + r * dm.rb + cg * 8);
    }
  }
  if constexpr (kVals) {
#pragma unroll
    for (int rr = 0; rr < L::RSV; ++rr) {
      const size_t r = (size_t)(segv * L::RSV + rr);
      rv[rr].load(vc + r * dm.rv + cgv * 8);
      rw[rr].load(wc + r * dm.rw + cgv * 8);
    }
  }

  bool exact = false;
  if constexpr (kRows) {
  // ---- phase 0: gc = cumsum(g) over the chunk (gdn2_wy_reference.py:63)
  float gcr[L::RS][8];
  exact = chunk_cumsum<C, K>(gc_in, (size_t)dm.rg, gcr, sTot, sGl);
  if (kVals && tid < K) ck.gcl[(size_t)bhn * K + tid] = fin(sGl[tid]);

  // ---- phase 1: elementwise operands (gdn2_wy_reference.py:92-100)
  T* g_qg = ck.qg + (size_t)bhn * C * K;
  T* g_kg = ck.kg + (size_t)bhn * C * K;
#pragma unroll
  for (int rr = 0; rr < L::RS; ++rr) {
    const int r = seg * L::RS + rr;
    float qv[8], kv[8], bv[8], o_qg[8], o_kt[8], o_kb[8], o_kg[8];
#pragma unroll
    for (int j = 0; j < 8; ++j) { qv[j] = rq[rr][j]; kv[j] = rk[rr][j]; bv[j] = rb[rr][j]; }
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      const float gcv = gcr[rr][j];
      const float e = __expf(gcv);
      o_qg[j] = qv[j] * e;
      o_kt[j] = kv[j] * __expf(-gcv);
      o_kb[j] = (bv[j] * kv[j]) * e;
      o_kg[j] = kv[j] * __expf(sGl[cg * 8 + j] - gcv);
    }
    store8(sB + r * L::LK + cg * 8, o_kb);
    if constexpr (kScores) {
      if (!exact) {
        store8(sQ + r * L::LK + cg * 8, o_qg);
        store8(sK + r * L::LK + cg * 8, o_kt);
      } else {
#pragma unroll
        for (int j = 0; j < 8; ++j) sGcExact[r * K + cg * 8 + j] = gcr[rr][j];
      }
    }
    if constexpr (kVals) {
      if constexpr (ST == kIntraRecompute) {
#pragma unroll
        for (int j = 0; j < 8; ++j) { o_qg[j] = fin(o_qg[j]); o_kg[j] = fin(o_kg[j]); }
      }
      store8(g_qg + r * K + cg * 8, o_qg);
      store8(g_kg + r * K + cg * 8, o_kg);
    }
  }
  if constexpr (kVals) {
#pragma unroll
    for (int rr = 0; rr < L::RSV; ++rr) {
      const int r = segv * L::RSV + rr;
      float vv[8], wv[8];
#pragma unroll
      for (int j = 0; j < 8; ++j) { vv[j] = rv[rr][j]; wv[j] = rw[rr][j]; }
      // w * v is formed in the input dtype before the upcast (gdn2_wy_reference.py:94)
#pragma unroll
      for (int j = 0; j < 8; ++j) wv[j] = to_f(from_f<T>(wv[j] * vv[j]));
      store8(sW + r * L::LV + cgv * 8, wv);
    }
  }
  __syncthreads();
  }  // kRows

  // ---- phase 2: Aqk (causal, scaled) and Akk (strict) (gdn2_wy_reference.py:79-87)
  constexpr int NB = C / 16;
  constexpr int NTRI = NB * (NB + 1) / 2;
  T* g_aqk = ck.aqk + (size_t)bhn * C * C;
  T* g_akk = ck.akk + (size_t)bhn * C * C;  // kernel A alone: Akk leaves in the operand type
  const int wv_id = wave_id();
  if constexpr (kScores) {
  if (!exact) {
    constexpr int JPW = (2 * NTRI + 3) / 4;
    f32x4 res[JPW];
#pragma unroll
    for (int cnt = 0; cnt < JPW; ++cnt) {
      const int job = wv_id + 4 * cnt;
      if (job >= 2 * NTRI) break;
      const int which = job / NTRI;  // 0: Aqk, 1: Akk
      int t = job % NTRI, mi = 0;
      while (t > mi) { t -= mi + 1; ++mi; }
      const int ni = t;
      f32x4 acc = zero4();
      acc = tile_mma<T, false, false>(acc, which ? sB : sQ, L::LK, sK, L::LK, 16 * mi, 16 * ni, K);
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int r = 16 * mi + tile_row(i), c = 16 * ni + tile_col();
        float x = which ? acc[i] : dm.scale * acc[i];
        const bool keep = which ? (r > c) : (r >= c);
        acc[i] = keep ? n2n(x) : 0.f;
      }
      res[cnt] = acc;
    }
    __syncthreads();  // sQ / sK are dead from here on; sAf may alias them
#pragma unroll
    for (int cnt = 0; cnt < JPW; ++cnt) {
      const int job = wv_id + 4 * cnt;
      if (job >= 2 * NTRI) break;
      const int which = job / NTRI;
      int t = job % NTRI, mi = 0;
      while (t > mi) { t -= mi + 1; ++mi; }
      const int ni = t;
      if (which == 0) store_tile_n(g_aqk, C, 16 * mi, 16 * ni, res[cnt]);
      else if constexpr (ST == kIntraScores) store_tile_n(g_akk, C, 16 * mi, 16 * ni, res[cnt]);
      else store_tile_n(sAf, L::LA, 16 * mi, 16 * ni, res[cnt]);
    }
  } else {
    constexpr int PER = C * C / 256;
    float eqk[PER], ekk[PER];
    intra_scores_exact<T, C, K>(sGcExact, qc, kc, bc, dm.rq, dm.rk, dm.rb, dm.scale, eqk, ekk);
    __syncthreads();
#pragma unroll
    for (int s = 0; s < PER; ++s) {
      const int e = tid + 256 * s, i = e / C, j = e % C;
      g_aqk[i * C + j] = from_f<T>(eqk[s]);
      if constexpr (ST == kIntraScores) g_akk[i * C + j] = from_f<T>(ekk[s]);
      else sAf[i * L::LA + j] = ekk[s];
    }
  }
  // upper tiles of Aqk / Akk are zero
  for (int e = tid; e < C * C; e += 256) {
    const int i = e / C, j = e % C;
    if ((j >> 4) > (i >> 4)) {
      if (!exact) g_aqk[i * C + j] = from_f<T>(0.f);
      if constexpr (ST == kIntraScores) g_akk[i * C + j] = from_f<T>(0.f);
      else sAf[i * L::LA + j] = 0.f;
    }
    if constexpr (ST == kIntraAll) sX[i * L::LA + j] = 0.f;
  }
  if constexpr (ST == kIntraScores) return;
  __syncthreads();
  }  // kScores
  if constexpr (ST == kIntraSolve) {
    // Akk from the caller (only its strictly lower blocks are read below)
    for (int e = tid; e < C * C; e += 256) {
      const int i = e / C, j = e % C;
      sAf[i * L::LA + j] = to_f(g_akk[i * C + j]);
      sX[i * L::LA + j] = 0.f;
    }
    __syncthreads();
  }

  // ---- phase 3: A = (I + Akk)^-1 (gdn2_wy_reference.py:16-30,89-90)
  T* g_ainv = ck.ainv + (size_t)bhn * C * C;
  const T* opA;
  int ldA;
  if constexpr (ST != kIntraRecompute) {
  // Diagonal 16x16 blocks by forward substitution (wave w, lane = column).
  {
    const int lane = lane_id();
    if (wv_id < NB && lane < 16) {
      const int o = 16 * wv_id;
      float x[16];
#pragma unroll
      for (int i = 0; i < 16; ++i) {
        float s = (i == lane) ? 1.f : 0.f;
#pragma unroll
        for (int j = 0; j < 15; ++j)  // constant trip count: x stays in registers
          if (j < i) s -= sAf[(o + i) * L::LA + o + j] * x[j];
        x[i] = s;
      }
#pragma unroll
      for (int i = 0; i < 16; ++i) sX[(o + i) * L::LA + o + lane] = x[i];
    }
  }
  __syncthreads();
  // Off-diagonal blocks, one column block per wave:
  //   A_mn = -A_mm (sum_{k=n}^{m-1} T_mk A_kn)
  {
    float* scr = sTot + wv_id * 16 * 17;
    for (int nb = wv_id; nb < NB; nb += 4) {
      for (int mb = nb + 1; mb < NB; ++mb) {
        f32x4 acc = zero4();
        acc = tile_mma<float, false, true>(acc, sAf + 16 * nb, L::LA, sX + 16 * nb * L::LA, L::LA,
                                           16 * mb, 16 * nb, 16 * (mb - nb));
        store_tile_n(scr, 17, 0, 0, acc);
        wave_lds_sync();  // scr is private to this wave
        f32x4 a2 = zero4();
        a2 = tile_mma<float, false, true>(a2, sX + 16 * mb * L::LA + 16 * mb, L::LA, scr, 17, 0, 0, 16);
#pragma unroll
        for (int i = 0; i < 4; ++i) a2[i] = -a2[i];
        store_tile_n(sX, L::LA, 16 * mb, 16 * nb, a2);
      }
    }
  }
  __syncthreads();
  // n2n, operand-type copy, global A
  if constexpr (sizeof(T) == 2) {
    T* sAb = reinterpret_cast<T*>(lds + L::off_af);  // Akk is dead
    for (int e = tid; e < C * C / 8; e += 256) {  // 8 consecutive columns per item
      const int i = e / (C / 8), j = (e % (C / 8)) * 8;
      float x[8];
      load8(sX + i * L::LA + j, x);
#pragma unroll
      for (int t = 0; t < 8; ++t) x[t] = n2n(x[t]);
      store8(sAb + i * (C + Pad<T>::v) + j, x);
      store8(g_ainv + i * C + j, x);
    }
    opA = sAb;
    ldA = C + Pad<T>::v;
  } else {
    for (int e = tid; e < C * C; e += 256) {
      const int i = e / C, j = e % C;
      const float x = n2n(sX[i * L::LA + j]);
      sX[i * L::LA + j] = x;
      g_ainv[i * C + j] = from_f<T>(x);
    }
    opA = reinterpret_cast<const T*>(sX);
    ldA = L::LA;
  }
  if constexpr (ST == kIntraSolve) return;
  } else {
    // A from the caller, into the operand-type rows phase 4 reads
    if constexpr (sizeof(T) == 2) {
      T* sAb = reinterpret_cast<T*>(lds + L::off_af);
      for (int e = tid; e < C * C / 8; e += 256) {
        const int i = e / (C / 8), j = (e % (C / 8)) * 8;
        *reinterpret_cast<uint4*>(sAb + i * (C + Pad<T>::v) + j) =
            *reinterpret_cast<const uint4*>(g_ainv + i * C + j);
      }
      opA = sAb;
      ldA = C + Pad<T>::v;
    } else {
      for (int e = tid; e < C * C; e += 256) {
        const int i = e / C, j = e % C;
        sX[i * L::LA + j] = g_ainv[i * C + j];
      }
      opA = reinterpret_cast<const T*>(sX);
      ldA = L::LA;
    }
  }
  __syncthreads();

  // ---- phase 4: w_pseudo = A kb, u = A wv (gdn2_wy_reference.py:92-96)
  T* g_wt = ck.wt + (size_t)bhn * C * K;
  T* g_u = ck.u + (size_t)bhn * C * V;
  if constexpr (sizeof(T) == 2 && L::stage_fits) {
    // one row block per wave: its column tiles share the A reads, go through
    // the wave's LDS staging rows and leave as 16-byte row pieces
    T* stg = reinterpret_cast<T*>(lds + L::off_stage) + wv_id * 16 * L::LS;
    auto row_block = [&](int mi, int kr, const T* Bop, int ldb, auto ncol, T* gout) {
      constexpr int NC = decltype(ncol)::value;
      f32x4 acc[NC / 16];
#pragma unroll
      for (int t = 0; t < NC / 16; ++t) acc[t] = zero4();
      tile_mma_row<T, false, true, NC / 16>(acc, opA, ldA, Bop, ldb, 16 * mi, 0, kr);
#pragma unroll
      for (int t = 0; t < NC / 16; ++t) {
#pragma unroll
        for (int i = 0; i < 4; ++i) acc[t][i] = fin(acc[t][i]);
        store_tile_n(stg, L::LS, 0, 16 * t, acc[t]);
      }
      wave_lds_sync();
      constexpr int PR = NC / 8;  // 16-byte pieces per row
#pragma unroll
      for (int e = lane_id(); e < 16 * PR; e += 64) {
        const int r = e / PR, c = (e % PR) * 8;
        *reinterpret_cast<uint4*>(gout + (size_t)(16 * mi + r) * NC + c) =
            *reinterpret_cast<const uint4*>(stg + r * L::LS + c);
      }
      wave_lds_sync();  // the staging rows are rewritten next
    };
    for (int mi = wv_id; mi < NB; mi += 4) {
      // A is block lower triangular; a caller's A (kernel C alone) is read whole
      int kr = ST == kIntraRecompute ? C : 16 * (mi + 1);
      kr = ((kr + Mma<T>::KS - 1) / Mma<T>::KS) * Mma<T>::KS;
      if (kr > C) kr = C;
      row_block(mi, kr, sB, L::LK, std::integral_constant<int, K>(), g_wt);
      row_block(mi, kr, sW, L::LV, std::integral_constant<int, V>(), g_u);
    }
  } else {
    constexpr int TW = NB * (K / 16), TU = NB * (V / 16);
    for (int job = wv_id; job < TW + TU; job += 4) {
      const bool isu = job >= TW;
      const int jj = isu ? job - TW : job;
      const int nbk = isu ? V / 16 : K / 16;
      const int mi = jj / nbk, ni = jj % nbk;
      int kr = ST == kIntraRecompute ? C : 16 * (mi + 1);
      kr = ((kr + Mma<T>::KS - 1) / Mma<T>::KS) * Mma<T>::KS;
      if (kr > C) kr = C;
      f32x4 acc = zero4();
      if (isu) acc = tile_mma<T, false, true>(acc, opA, ldA, sW, L::LV, 16 * mi, 16 * ni, kr);
      else acc = tile_mma<T, false, true>(acc, opA, ldA, sB, L::LK, 16 * mi, 16 * ni, kr);
  #pragma unroll
      for (int i = 0; i < 4; ++i) acc[i] = fin(acc[i]);
      if (isu) store_tile_n(g_u, V, 16 * mi, 16 * ni, acc);
      else store_tile_n(g_wt, K, 16 * mi, 16 * ni, acc);
    }
  }
}

// ------------------------------------------------------------------ state
template <typename T, int C, int K, int V, int VT>
struct StateLds {
  static constexpr int PAD = Pad<T>::v;
  static constexpr int LK = K + PAD, LC = C + PAD, LU = VT + PAD;
  // one chunk's staged operands (offsets within a stage buffer)
  static constexpr int s_w = 0;
  static constexpr int s_q = s_w + C * LK * (int)sizeof(T);
  static constexpr int s_kg = s_q + C * LK * (int)sizeof(T);
  static constexpr int s_aqk = s_kg + C * LK * (int)sizeof(T);
  static constexpr int s_u = s_aqk + C * LC * (int)sizeof(T);
  static constexpr int s_gl = s_u + C * LU * (int)sizeof(T);
  static constexpr int SB = (s_gl + K * 4 + 15) / 16 * 16;
  static constexpr int REST = VT * LK * (int)sizeof(T) + VT * LC * (int)sizeof(T);
  // two stage buffers when they fit: chunk n + 1 is written while chunk n
  // computes, which also saves a barrier per chunk
  static constexpr int NBUF = 2 * SB + REST <= 160 * 1024 ? 2 : 1;
  static constexpr int off_ht = NBUF * SB;
  static constexpr int off_vn = off_ht + VT * LK * (int)sizeof(T);
  static constexpr int total = off_vn + VT * LC * (int)sizeof(T);
};

// gdn2_fwd_state mode bits: keep the per-chunk states and v_new for the
// backward; write o per chunk ([B][H][NT][C][V], the layout of
// gdn2_inter_chunk_combine's result, kernel_d_pipeline.py:94-124) instead of
// [B][T][H][V]; sanitise h0 (nan_to_num(clip(h0, +-1e4)), its _sanitize_h0).
enum { kStateSave = 1, kStateChunkO = 2, kStateSanitizeH0 = 4 };

// NW waves (NW / 4 per SIMD): the state tiles and the [w; q] h tiles of one
// V tile split over them by row blocks.  PD register sets of chunk operands
// are in flight (two at eight waves; one at sixteen, where the other waves
// hide the load latency and the VGPR budget is 128).  With DO, each step's o
// tiles stay in registers and are written by the next step between its
// commit and its prefetch (faster with 16-column tiles, slower with 32).
template <typename T, int C, int K, int V, int VT, int NW = 8, int PD = 2, bool DO = false>
__global__ __launch_bounds__(64 * NW) __attribute__((amdgpu_waves_per_eu(NW / 4, NW / 4))) void gdn2_fwd_state(Gdn2Dims dm, Gdn2Chunks<T> ck,
                                                     const float* __restrict__ h0, float* __restrict__ o,
                                                     float* __restrict__ h_final, int mode) {
  const int save = mode & kStateSave;
  typedef StateLds<T, C, K, V, VT> L;
  __shared__ __attribute__((aligned(16))) unsigned char lds[L::total];
  T* sHt = reinterpret_cast<T*>(lds + L::off_ht);
  T* sVn = reinterpret_cast<T*>(lds + L::off_vn);
  // the stage buffer the current chunk reads
  T *sW, *sQ, *sKg, *sAqk, *sU;
  float* sGl;
  auto use_buf = [&](int bsel) {
    unsigned char* bp = lds + bsel * L::SB;
    sW = reinterpret_cast<T*>(bp + L::s_w);
    sQ = reinterpret_cast<T*>(bp + L::s_q);
    sKg = reinterpret_cast<T*>(bp + L::s_kg);
    sAqk = reinterpret_cast<T*>(bp + L::s_aqk);
    sU = reinterpret_cast<T*>(bp + L::s_u);
    sGl = reinterpret_cast<float*>(bp + L::s_gl);
  };
  use_buf(0);

  constexpr int NVT = V / VT;
  int bh, vt;
  xcd_group_map(blockIdx.x, dm.B * dm.H, NVT, bh, vt);
  const int h = bh % dm.H, bb = bh / dm.H;
  const int v0 = vt * VT;
  const int wv_id = wave_id();

  // state tiles h[d][v]: (K/16) x (VT/16), TPW per wave
  constexpr int NTHR = 64 * NW;
  constexpr int NTI = VT / 16;
  constexpr int NTH = (K / 16) * NTI;
  constexpr int TPW = NTH / NW;
  static_assert(NTH % NW == 0 && TPW >= 1, "state tiles must split evenly over the waves");
  f32x4 hs[TPW];
#pragma unroll
  for (int t = 0; t < TPW; ++t) {
    const int tile = wv_id * TPW + t, mi = tile / NTI, ni = tile % NTI;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int d = 16 * mi + tile_row(i), vv = v0 + 16 * ni + tile_col();
      const float hv = h0 ? h0[((size_t)bh * K + d) * V + vv] : 0.f;
      hs[t][i] = (mode & kStateSanitizeH0) ? sanitize(hv) : hv;
    }
    store_tile_t(sHt, L::LK, 16 * mi, 16 * ni, hs[t]);
  }

  // X tiles: rows [0, C) = w_pseudo h, rows [C, 2C) = qg h; (2C/16) x NTI tiles
  constexpr int NTX = (2 * C / 16) * NTI;
  constexpr int XPW = NTX / NW;
  static_assert(NTX % NW == 0 && XPW >= 1, "output tiles must split evenly over the waves");
  // tiles of one row block computed together (sharing their A fragments)
  constexpr int GX = XPW < NTI ? XPW : NTI, GT = TPW < NTI ? TPW : NTI;
  static_assert(XPW % GX == 0 && NTI % GX == 0 && TPW % GT == 0 && NTI % GT == 0, "tile groups");

  // the chunk operands move global -> registers -> LDS; two register sets
  // keep the loads of chunk n + 2 in flight while chunk n computes
  struct Stage {
    RegStage<T, C, K, NTHR> w, q, k;
    RegStage<T, C, C, NTHR> a;
    RegStage<T, C, VT, NTHR> u;
    RegStage<float, 1, K, NTHR> g;
  };
  auto prefetch = [&](Stage& S, int n) {
    const size_t bhn = (size_t)bh * dm.NT + n;
    S.w.load(ck.wt + bhn * C * K, K);
    S.q.load(ck.qg + bhn * C * K, K);
    S.k.load(ck.kg + bhn * C * K, K);
    S.a.load(ck.aqk + bhn * C * C, C);
    S.u.load(ck.u + bhn * C * V + v0, V);
    S.g.load(ck.gcl + bhn * K, K);
  };
  auto commit = [&](const Stage& S, int bsel) {
    unsigned char* bp = lds + bsel * L::SB;
    S.w.store(reinterpret_cast<T*>(bp + L::s_w), L::LK);
    S.q.store(reinterpret_cast<T*>(bp + L::s_q), L::LK);
    S.k.store(reinterpret_cast<T*>(bp + L::s_kg), L::LK);
    S.a.store(reinterpret_cast<T*>(bp + L::s_aqk), L::LC);
    S.u.store(reinterpret_cast<T*>(bp + L::s_u), L::LU);
    S.g.store(reinterpret_cast<float*>(bp + L::s_gl), K);
  };
  // Every prefetch is issued on every path (past the last chunk it re-reads
  // chunk NT - 1, whose registers are never committed): the wait counter
  // before a commit then always has the other set's loads behind it, so the
  // commit waits for its own set only and the two-deep prefetch holds.
  const int last = dm.NT - 1;
  Stage s0, s1;
  prefetch(s0, 0);
  commit(s0, 0);
  __syncthreads();
  prefetch(s0, min(1, last));
  if constexpr (PD == 2) prefetch(s1, min(2, last));

  const bool chunk_o = (mode & kStateChunkO) != 0;
  const size_t ors = chunk_o ? (size_t)V : (size_t)dm.H * V;  // o's row stride
  static_assert(!DO || L::NBUF == 2, "deferred o stores follow the step-start commit");
  f32x4 po[XPW];
  float* pog = nullptr;
  // this wave's o tiles (rows of the qg half) at o's row base og
  auto store_o = [&](float* og, const f32x4 (&ov)[XPW]) {
#pragma unroll
    for (int gi = 0; gi < XPW / GX; ++gi) {
      const int tile0 = wv_id * XPW + gi * GX, mi = tile0 / NTI, ni0 = tile0 % NTI;
      if (mi >= C / 16) {
        const int mo = mi - C / 16;
#pragma unroll
        for (int u = 0; u < GX; ++u)
#pragma unroll
          for (int i = 0; i < 4; ++i) {
            const int r = 16 * mo + tile_row(i), c = 16 * (ni0 + u) + tile_col();
            og[(size_t)r * ors + c] = n2n(ov[gi * GX + u][i]);
          }
      }
    }
  };

  // One chunk step; S holds chunk n + 1 on entry and is refilled with chunk n + 3.
  // Two stage buffers: chunk n + 1 goes into the other buffer at the start (its
  // last readers finished before the previous step's final barrier), and only
  // two barriers are left per step (after v_new, after the new h).
  auto chunk_step = [&](int n, Stage& S) {
    const size_t bhn = (size_t)bh * dm.NT + n;
    use_buf(L::NBUF == 2 ? (n & 1) : 0);
    if constexpr (L::NBUF == 2) {
      if (n + 1 < dm.NT) commit(S, (n + 1) & 1);
      if constexpr (DO) {
        if (pog) store_o(pog, po);
        pog = nullptr;
      }
      prefetch(S, min(n + 1 + PD, last));
    }
      if (save) unstage_rows<T, VT, K, NTHR>(ck.hT + bhn * V * K + (size_t)v0 * K, K, sHt, L::LK);

      // v_new = u - w_pseudo h ; qh = qg h   (GX tiles of one row block share the A reads)
      f32x4 xo[XPW];
  #pragma unroll
      for (int gi = 0; gi < XPW / GX; ++gi) {
        const int tile0 = wv_id * XPW + gi * GX, mi = tile0 / NTI, ni0 = tile0 % NTI;
        const bool is_w = mi < C / 16;
        f32x4 acc[GX];
  #pragma unroll
        for (int u = 0; u < GX; ++u) acc[u] = zero4();
        tile_mma_row<T, false, false, GX>(acc, is_w ? sW : sQ, L::LK, sHt, L::LK,
                                          16 * (is_w ? mi : mi - C / 16), 16 * ni0, K);
  #pragma unroll
        for (int u = 0; u < GX; ++u) {
          const int ni = ni0 + u;
          if (is_w) {
  #pragma unroll
            for (int i = 0; i < 4; ++i) {
              const int j = 16 * mi + tile_row(i), vv = 16 * ni + tile_col();
              acc[u][i] = to_f(sU[j * L::LU + vv]) - acc[u][i];
            }
            store_tile_t(sVn, L::LC, 16 * mi, 16 * ni, acc[u]);
          } else {
  #pragma unroll
            for (int i = 0; i < 4; ++i) acc[u][i] *= dm.scale;
          }
          xo[gi * GX + u] = acc[u];
        }
      }
      __syncthreads();
      if (save) unstage_rows<T, VT, C, NTHR>(ck.vnT + bhn * V * C + (size_t)v0 * C, C, sVn, L::LC);

      // o = scale qg h + Aqk v_new   (rows of the qg half)
      float* og = !o ? nullptr
                     : chunk_o ? o + (size_t)bhn * C * V + v0
                               : o + (((size_t)bb * dm.T + (size_t)n * C) * dm.H + h) * V + v0;
  #pragma unroll
      for (int gi = 0; gi < XPW / GX; ++gi) {
        const int tile0 = wv_id * XPW + gi * GX, mi = tile0 / NTI, ni0 = tile0 % NTI;
        if (mi >= C / 16) {
          const int mo = mi - C / 16;
          int kr = 16 * (mo + 1);
          kr = ((kr + Mma<T>::KS - 1) / Mma<T>::KS) * Mma<T>::KS;
          if (kr > C) kr = C;
          f32x4 acc[GX];
  #pragma unroll
          for (int u = 0; u < GX; ++u) acc[u] = xo[gi * GX + u];
          tile_mma_row<T, false, false, GX>(acc, sAqk, L::LC, sVn, L::LC, 16 * mo, 16 * ni0, kr);
          if constexpr (DO) {
  #pragma unroll
            for (int u = 0; u < GX; ++u) po[gi * GX + u] = acc[u];
          } else if (og) {
  #pragma unroll
            for (int u = 0; u < GX; ++u)
  #pragma unroll
              for (int i = 0; i < 4; ++i) {
                const int r = 16 * mo + tile_row(i), c = 16 * (ni0 + u) + tile_col();
                og[(size_t)r * ors + c] = n2n(acc[u][i]);
              }
          }
        }
      }
      if constexpr (DO) pog = og;

      // h = sanitize(h e^{gc_last} + kg^T v_new)
  #pragma unroll
      for (int gi = 0; gi < TPW / GT; ++gi) {
        const int tile0 = wv_id * TPW + gi * GT, mi = tile0 / NTI, ni0 = tile0 % NTI;
        f32x4 acc[GT];
  #pragma unroll
        for (int u = 0; u < GT; ++u) {
          acc[u] = hs[gi * GT + u];
  #pragma unroll
          for (int i = 0; i < 4; ++i) acc[u][i] *= __expf(sGl[16 * mi + tile_row(i)]);
        }
        tile_mma_row<T, true, false, GT>(acc, sKg, L::LK, sVn, L::LC, 16 * mi, 16 * ni0, C);
  #pragma unroll
        for (int u = 0; u < GT; ++u) {
  #pragma unroll
          for (int i = 0; i < 4; ++i) acc[u][i] = sanitize(acc[u][i]);
          hs[gi * GT + u] = acc[u];
        }
      }
      // sHt was last read by this step's [w; q] h, before the v_new barrier;
      // with one stage buffer, the staged chunk is still being read here
      if constexpr (L::NBUF == 1) __syncthreads();
  #pragma unroll
      for (int t = 0; t < TPW; ++t) {
        const int tile = wv_id * TPW + t, mi = tile / NTI, ni = tile % NTI;
        store_tile_t(sHt, L::LK, 16 * mi, 16 * ni, hs[t]);
      }
    if constexpr (L::NBUF == 1) {
      if (n + 1 < dm.NT) commit(S, 0);
      prefetch(S, min(n + 1 + PD, last));
    }
    __syncthreads();
  };
  // both steps of a pair run on every trip (no path skips the second set's
  // loads); an odd last chunk runs after the loop
  int n = 0;
  if constexpr (PD == 2) {
    for (; n + 1 < dm.NT; n += 2) {
      chunk_step(n, s0);
      chunk_step(n + 1, s1);
    }
    if (n < dm.NT) chunk_step(n, s0);
  } else {
    for (; n < dm.NT; ++n) chunk_step(n, s0);
  }
  if constexpr (DO) {
    if (pog) store_o(pog, po);
  }
  if (h_final) {
#pragma unroll
    for (int t = 0; t < TPW; ++t) {
      const int tile = wv_id * TPW + t, mi = tile / NTI, ni = tile % NTI;
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int d = 16 * mi + tile_row(i), vv = v0 + 16 * ni + tile_col();
        h_final[((size_t)bh * K + d) * V + vv] = hs[t][i];
      }
    }
  }
}

}  // namespace ah
