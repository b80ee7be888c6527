// GDN2 WY chunked backward for gfx950: the B2 -> B1 -> B3 -> B4 -> B5 chain of
// _gdn2_core_bwd (atomic_ops/kernel_trainable_B6.py:97-181).
//
//   gdn2_bwd_dh     one workgroup per (batch, head, V tile), reverse over
//                   chunks: B2's dv_partial = Aqk^T dO, then B1
//                   (kernel_bwd_b1_dhu.py:22-39) with the fp32 dh carried in
//                   MFMA accumulators.  Saves dv_new and the carry entering
//                   each chunk (dh_next).
//   gdn2_bwd_hgrad  per chunk: the state contractions of B2/B3
//                   (kernel_bwd_b2_dav.py:69, kernel_bwd_b3_wy_dqkg.py:154-161,
//                   :200-201): dAqk, dqg, dw_pseudo, dkg and the gc_last row term.
//   gdn2_bwd_wy     per chunk: the WY part of B3 (kernel_bwd_b3_wy_dqkg.py:163-180):
//                   dA, dAkk = -A^T clip(clip(dA) A^T) (strict), dkb = A^T dw_pseudo,
//                   dwv = A^T dv and the final dw, dv (:164,167,194-195).
//   gdn2_bwd_intra  per chunk: B4 (kernel_bwd_b4_intra.py:57-132) in the
//                   factorised form (or exact pairwise, same criterion as the
//                   forward), the B3 element-wise terms, the combine of
//                   kernel_trainable_B6.py:139-147, and B5's reverse cumsum
//                   (kernel_bwd_b5_reverse_cumsum.py:17-24).  Writes dq, dk, db, dg.
#include "gdn2_fwd.hip"

namespace ah {

// First k (rounded down to the MFMA k step) of a lower-triangular operand
// whose nonzeros start at row 16 * tile.
template <typename T>
__device__ __forceinline__ int tri_k0(int tile) {
  return (16 * tile / Mma<T>::KS) * Mma<T>::KS;
}
template <typename T>
__device__ __forceinline__ int tri_k1(int tile, int C) {
  int k = 16 * (tile + 1);
  k = ((k + Mma<T>::KS - 1) / Mma<T>::KS) * Mma<T>::KS;
  return k > C ? C : k;
}

// ------------------------------------------------------------------ B2 + B1
template <typename T, int C, int K, int V, int VT>
struct DhLds {
  static constexpr int PAD = Pad<T>::v;
  static constexpr int LK = K + PAD, LC = C + PAD, LD = VT + PAD;
  // one chunk's staged operands (offsets within a stage buffer)
  static constexpr int s_w = 0;
  static constexpr int s_q = s_w + C * LK * (int)sizeof(T);
  static constexpr int s_kg = s_q + C * LK * (int)sizeof(T);
  static constexpr int s_aqk = s_kg + C * LK * (int)sizeof(T);
  static constexpr int s_do = s_aqk + C * LC * (int)sizeof(T);
  static constexpr int s_dos = s_do + C * LD * (int)sizeof(T);
  static constexpr int s_gl = s_dos + C * LD * (int)sizeof(T);
  static constexpr int SB = (s_gl + K * 4 + 15) / 16 * 16;
  static constexpr int REST = VT * LK * (int)sizeof(T) + VT * LC * (int)sizeof(T);
  // two stage buffers when they fit: chunk n - 1 is written while chunk n
  // computes, which also saves a barrier per chunk
  static constexpr int NBUF = 2 * SB + REST <= 160 * 1024 ? 2 : 1;
  static constexpr int off_dht = NBUF * SB;
  static constexpr int off_dvt = off_dht + VT * LK * (int)sizeof(T);
  static constexpr int total = off_dvt + VT * LC * (int)sizeof(T);
};

// Eight waves (two per SIMD): the dh tiles and the dv_new tiles of one V
// tile split over them by row blocks.  With DD, each step's dv_new tiles stay
// in registers and are written by the next step between its commit and its
// prefetch (bf16: 0.350 -> 0.332 ms with 32-column tiles, 0.78 -> 0.77 ms
// with 16; fp32 at K = 128 has one stage buffer and stores in place).
template <typename T, typename TD, int C, int K, int V, int VT, bool DD = false>
__global__ __launch_bounds__(512) __attribute__((amdgpu_waves_per_eu(2, 2))) void gdn2_bwd_dh(
    Gdn2Dims dm, Gdn2Chunks<T> ck, Gdn2Grads<T> gr, const TD* __restrict__ dO,
    const float* __restrict__ dh_final, float* __restrict__ dh0) {
  typedef DhLds<T, C, K, V, VT> L;
  __shared__ __attribute__((aligned(16))) unsigned char lds[L::total];
  T* sDht = reinterpret_cast<T*>(lds + L::off_dht);
  T* sDvT = reinterpret_cast<T*>(lds + L::off_dvt);
  // the stage buffer the current chunk reads
  T *sW, *sQ, *sKg, *sAqk, *sDO, *sDOs;
  float* sGl;
  auto use_buf = [&](int bsel) {
    unsigned char* bp = lds + bsel * L::SB;
    sW = reinterpret_cast<T*>(bp + L::s_w);
    sQ = reinterpret_cast<T*>(bp + L::s_q);
    sKg = reinterpret_cast<T*>(bp + L::s_kg);
    sAqk = reinterpret_cast<T*>(bp + L::s_aqk);
    sDO = reinterpret_cast<T*>(bp + L::s_do);
    sDOs = reinterpret_cast<T*>(bp + L::s_dos);
    sGl = reinterpret_cast<float*>(bp + L::s_gl);
  };

  constexpr int NVT = V / VT;
  int bh, vt;
  xcd_group_map(blockIdx.x, dm.B * dm.H, NVT, bh, vt);
  const int h = bh % dm.H, bb = bh / dm.H;
  const int v0 = vt * VT;
  const int wv_id = wave_id();
  const size_t ldo = (size_t)dm.rdo;

  constexpr int NW = 8, NTHR = 64 * NW;
  constexpr int NTI = VT / 16;
  constexpr int NTH = (K / 16) * NTI;  // dh tiles
  constexpr int TPW = NTH / NW;
  constexpr int NTV = (C / 16) * NTI;  // dv_new tiles
  // with fewer dv_new tiles than waves (16-column V tiles) the first NTV waves take one each
  constexpr int VPW = NTV >= NW ? NTV / NW : 1;
  static_assert(NTH % NW == 0 && (NTV % NW == 0 || NW % NTV == 0) && TPW >= 1,
                "tiles must split evenly over the waves");
  // tiles of one row block computed together (sharing their A fragments)
  constexpr int GV = VPW < NTI ? VPW : NTI, GT = TPW < NTI ? TPW : NTI;
  static_assert(VPW % GV == 0 && NTI % GV == 0 && TPW % GT == 0 && NTI % GT == 0, "tile groups");

  // dh carry = sanitize(dh_final) (kernel_bwd_b1_dhu.py:18)
  f32x4 hs[TPW];
#pragma unroll
  for (int t = 0; t < TPW; ++t) {
    const int tile = wv_id * TPW + t, mi = tile / NTI, ni = tile % NTI;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int d = 16 * mi + tile_row(i), vv = v0 + 16 * ni + tile_col();
      hs[t][i] = dh_final ? sanitize(dh_final[((size_t)bh * K + d) * V + vv]) : 0.f;
    }
    store_tile_t(sDht, L::LK, 16 * mi, 16 * ni, hs[t]);
  }

  // the chunk operands (and dO) move global -> registers -> LDS; two register
  // sets keep the loads of chunk n - 2 in flight while chunk n computes
  struct Stage {
    RegStage<T, C, K, NTHR> w, q, k;
    RegStage<T, C, C, NTHR> a;
    RegStage<float, 1, K, NTHR> g;
    RegStage<TD, C, VT, NTHR> o;
  };
  auto prefetch = [&](Stage& S, int n) {
    const size_t bhn = (size_t)bh * dm.NT + n;
    S.w.load(ck.wt + bhn * C * K, K);
    S.q.load(ck.qg + bhn * C * K, K);
    S.k.load(ck.kg + bhn * C * K, K);
    S.a.load(ck.aqk + bhn * C * C, C);
    S.g.load(ck.gcl + bhn * K, K);
    S.o.load(dO + ((size_t)bb * dm.T + (size_t)n * C) * ldo + (size_t)h * V + v0, ldo);
  };
  auto commit = [&](const Stage& S, int bsel) {
    unsigned char* bp = lds + bsel * L::SB;
    T* dW = reinterpret_cast<T*>(bp + L::s_w);
    T* dDO = reinterpret_cast<T*>(bp + L::s_do);
    T* dDOs = reinterpret_cast<T*>(bp + L::s_dos);
    S.w.store(dW, L::LK);
    S.q.store(reinterpret_cast<T*>(bp + L::s_q), L::LK);
    S.k.store(reinterpret_cast<T*>(bp + L::s_kg), L::LK);
    S.a.store(reinterpret_cast<T*>(bp + L::s_aqk), L::LC);
    S.g.store(reinterpret_cast<float*>(bp + L::s_gl), K);
    // dO and scale dO in the operand dtype
    typedef RegStage<TD, C, VT, NTHR> RO;
#pragma unroll
    for (int i = 0; i < RO::PT; ++i) {
      const int e = threadIdx.x + NTHR * i;
      if (RO::N % NTHR == 0 || e < RO::N) {
        const int r = e / RO::PER_ROW, c = (e % RO::PER_ROW) * RO::VEC;
        const uint4 raw = S.o.piece(i);
        const TD* v = reinterpret_cast<const TD*>(&raw);
#pragma unroll
        for (int j = 0; j < RO::VEC; ++j) {
          const float x = to_f(v[j]);
          dDO[r * L::LD + c + j] = from_f<T>(x);
          dDOs[r * L::LD + c + j] = from_f<T>(x * dm.scale);
        }
      }
    }
  };
  // Every prefetch is issued on every path (before chunk 0 it re-reads chunk
  // 0, whose registers are never committed): the wait counter before a
  // commit then always has the other set's loads behind it, so the commit
  // waits for its own set only and the two-deep prefetch holds.
  auto buf_of = [](int n) { return L::NBUF == 2 ? (n & 1) : 0; };
  static_assert(!DD || L::NBUF == 2, "deferred dv_new stores follow the step-start commit");
  f32x4 pdv[VPW];
  T* pdvn = nullptr;
  auto store_dv = [&](T* dvb) {
  #pragma unroll
    for (int gi = 0; gi < ((NTV >= NW || wv_id < NTV) ? VPW / GV : 0); ++gi) {
      const int tile0 = wv_id * VPW + gi * GV, mj = tile0 / NTI, ni0 = tile0 % NTI;
  #pragma unroll
      for (int u = 0; u < GV; ++u) store_tile_n(dvb, V, 16 * mj, 16 * (ni0 + u), pdv[gi * GV + u]);
    }
  };
  Stage s0, s1;
  prefetch(s0, dm.NT - 1);
  commit(s0, buf_of(dm.NT - 1));
  __syncthreads();
  prefetch(s0, max(dm.NT - 2, 0));
  prefetch(s1, max(dm.NT - 3, 0));

  // one chunk step (reverse); S holds chunk n - 1 on entry and is refilled with chunk n - 3.
  // Two stage buffers: chunk n - 1 goes into the other buffer at the start (its
  // last readers finished before the previous step's final barrier), and two
  // barriers are left per step (after dv_new, after the new dh).
  auto chunk_step = [&](int n, Stage& S) {
    const size_t bhn = (size_t)bh * dm.NT + n;
    use_buf(buf_of(n));
    if constexpr (L::NBUF == 2) {
      if (n > 0) commit(S, buf_of(n - 1));
      if constexpr (DD) {
        if (pdvn) store_dv(pdvn);
        pdvn = nullptr;
      }
      prefetch(S, max(n - 3, 0));
    }
      // dh_next of chunk n = the carry entering this step
      unstage_rows<T, VT, K, NTHR>(gr.dhT + bhn * V * K + (size_t)v0 * K, K, sDht, L::LK);

      // dv_new = sanitize(Aqk^T dO + kg dh)   (b2:70, b1:30-32)
  #pragma unroll
      for (int gi = 0; gi < ((NTV >= NW || wv_id < NTV) ? VPW / GV : 0); ++gi) {
        const int tile0 = wv_id * VPW + gi * GV, mj = tile0 / NTI, ni0 = tile0 % NTI;
        const int k0 = tri_k0<T>(mj);
        f32x4 acc[GV];
  #pragma unroll
        for (int u = 0; u < GV; ++u) acc[u] = zero4();
        tile_mma_row<T, true, true, GV>(acc, sAqk + k0 * L::LC, L::LC, sDO + k0 * L::LD, L::LD,
                                        16 * mj, 16 * ni0, C - k0);
        tile_mma_row<T, false, false, GV>(acc, sKg, L::LK, sDht, L::LK, 16 * mj, 16 * ni0, K);
  #pragma unroll
        for (int u = 0; u < GV; ++u) {
          const int ni = ni0 + u;
  #pragma unroll
          for (int i = 0; i < 4; ++i) acc[u][i] = sanitize(acc[u][i]);
          if constexpr (DD) pdv[gi * GV + u] = acc[u];
          else store_tile_n(gr.dvn + bhn * C * V + v0, V, 16 * mj, 16 * ni, acc[u]);
  #pragma unroll
          for (int i = 0; i < 4; ++i) acc[u][i] = -acc[u][i];
          store_tile_t(sDvT, L::LC, 16 * mj, 16 * ni, acc[u]);
        }
      }
      if constexpr (DD) pdvn = gr.dvn + bhn * C * V + v0;
      __syncthreads();

      // dh = sanitize(qg^T (scale dO) + dh e^{gc_last} - w_pseudo^T dv_new)   (b1:26-37)
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
        tile_mma_row<T, true, true, GT>(acc, sQ, L::LK, sDOs, L::LD, 16 * mi, 16 * ni0, C);
        tile_mma_row<T, true, false, GT>(acc, sW, L::LK, sDvT, L::LC, 16 * mi, 16 * ni0, C);
  #pragma unroll
        for (int u = 0; u < GT; ++u) {
  #pragma unroll
          for (int i = 0; i < 4; ++i) acc[u][i] = sanitize(acc[u][i]);
          hs[gi * GT + u] = acc[u];
        }
      }
      // sDht was last read by this step's dv_new, before the dv_new barrier;
      // with one stage buffer the commit below overwrites what dh just read
      if constexpr (L::NBUF == 1) __syncthreads();
  #pragma unroll
      for (int t = 0; t < TPW; ++t) {
        const int tile = wv_id * TPW + t, mi = tile / NTI, ni = tile % NTI;
        store_tile_t(sDht, L::LK, 16 * mi, 16 * ni, hs[t]);
      }
    if constexpr (L::NBUF == 1) {
      if (n > 0) commit(S, 0);
      prefetch(S, max(n - 3, 0));
    }
    __syncthreads();
  };
  // both steps of a pair run on every trip (no path skips the second set's
  // loads); an odd first chunk runs after the loop
  int n = dm.NT - 1;
  for (; n >= 1; n -= 2) {
    chunk_step(n, s0);
    chunk_step(n - 1, s1);
  }
  if (n == 0) chunk_step(0, s0);
  if constexpr (DD) {
    if (pdvn) store_dv(pdvn);
  }
  if (dh0) {
#pragma unroll
    for (int t = 0; t < TPW; ++t) {
      const int tile = wv_id * TPW + t, mi = tile / NTI, ni = tile % NTI;
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int d = 16 * mi + tile_row(i), vv = v0 + 16 * ni + tile_col();
        dh0[((size_t)bh * K + d) * V + vv] = hs[t][i];
      }
    }
  }
}

// ------------------------------------------------------------------ B2/B3 state terms
// One workgroup per (batch, head, chunk).  dO, dv_new and v_new stay in LDS;
// h_pre and dh_next ([V][K] per chunk) pass through in quarters of VQ whole
// rows (contiguous blocks, so every cache line is fetched once), the next
// quarter loaded into registers while the current one computes.  dqg, dw~ and
// dkg accumulate over the quarters in MFMA registers (wave w owns row blocks
// w, w + 4, ...) and are written once, whole rows at a time.
template <typename T, int C, int VQ, int K, int V>
struct HgLds {
  static constexpr int PAD = Pad<T>::v;
  // quarter rows padded by 16 elements: the transposed fragment reads of 16
  // lanes (4 rows, 32 bytes each at bf16) then land on distinct banks
  static constexpr int LK = K + 16, LV = V + PAD, LC = C + PAD;
  static constexpr int off_do = 0;
  static constexpr int off_dv = off_do + C * LV * (int)sizeof(T);
  static constexpr int off_vn = off_dv + C * LV * (int)sizeof(T);
  static constexpr int off_h = off_vn + V * LC * (int)sizeof(T);
  static constexpr int off_dh = off_h + VQ * LK * (int)sizeof(T);
  static constexpr int total = off_dh + VQ * LK * (int)sizeof(T);
  // row-term partials [16][K] over the quarter buffers, after the last quarter
  static constexpr int off_red = off_h;
  static_assert(16 * K * 4 <= 2 * VQ * LK * (int)sizeof(T), "row-term partials fit the quarter buffers");
};

template <typename T, typename TD, int C, int K, int V>
__global__ __launch_bounds__(256) void gdn2_bwd_hgrad(Gdn2Dims dm, Gdn2Chunks<T> ck, Gdn2Grads<T> gr,
                                                     const TD* __restrict__ dO) {
  constexpr int VQ = 32, NQ = V / VQ;
  static_assert(V % VQ == 0 && VQ % Mma<T>::KS == 0, "V splits into whole quarters");
  typedef HgLds<T, C, VQ, K, V> L;
  __shared__ __attribute__((aligned(16))) unsigned char lds[L::total];
  T* sDO = reinterpret_cast<T*>(lds + L::off_do);
  T* sDV = reinterpret_cast<T*>(lds + L::off_dv);
  T* sVn = reinterpret_cast<T*>(lds + L::off_vn);
  T* sH = reinterpret_cast<T*>(lds + L::off_h);
  T* sDh = reinterpret_cast<T*>(lds + L::off_dh);
  float* red = reinterpret_cast<float*>(lds + L::off_red);

  const int bhn = blockIdx.x;
  const int n = bhn % dm.NT;
  const int bh = bhn / dm.NT;
  const int h = bh % dm.H, bb = bh / dm.H;
  const int wv_id = wave_id();
  const size_t blk = (size_t)bhn;
  const T* hg = ck.hT + blk * V * K;
  const T* dhg = gr.dhT + blk * V * K;

  // every operand is requested before the first LDS store
  RegStage<T, VQ, K> ph, pdh;
  RegStage<TD, C, V> pdo;
  RegStage<T, C, V> pdv;
  RegStage<T, V, C> pvn;
  ph.load(hg, K);
  pdh.load(dhg, K);
  pdo.load(dO + ((size_t)bb * dm.T + (size_t)n * C) * dm.rdo + (size_t)h * V, (size_t)dm.rdo);
  pdv.load(gr.dvn + blk * C * V, V);
  pvn.load(ck.vnT + blk * V * C, C);
  store_convert(pdo, sDO, L::LV);
  pdv.store(sDV, L::LV);
  pvn.store(sVn, L::LC);
  ph.store(sH, L::LK);
  pdh.store(sDh, L::LK);
  __syncthreads();

  constexpr int MT = C / 16;
  // dAqk = n2n((dO v_new^T) * causal)   (kernel_bwd_b2_dav.py:69,72)
  T* g_daqk = gr.daqk + blk * C * C;
  for (int tile = wv_id; tile < MT * MT; tile += 4) {
    const int mi = tile / MT, nj = tile % MT;
    f32x4 acc = zero4();
    if (nj <= mi) acc = tile_mma<T, false, true>(acc, sDO, L::LV, sVn, L::LC, 16 * mi, 16 * nj, V);
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int r = 16 * mi + tile_row(i), c = 16 * nj + tile_col();
      acc[i] = r >= c ? n2n(acc[i]) * dm.scale : 0.f;  // the scale of Aqk folded in
    }
    store_tile_n(g_daqk, C, 16 * mi, 16 * nj, acc);
  }

  // dqg = scale dO h_pre^T ; dwt = -dv_new h_pre^T ; dkg = v_new dh_next^T:
  // each sum over v runs quarter by quarter in ascending v, as one sum would
  constexpr int RB = MT / 4, NT = K / 16;
  static_assert(MT % 4 == 0, "row blocks split evenly over 4 waves");
  f32x4 aq[RB][NT], aw[RB][NT], ak[RB][NT];
#pragma unroll
  for (int r = 0; r < RB; ++r)
#pragma unroll
    for (int t = 0; t < NT; ++t) aq[r][t] = aw[r][t] = ak[r][t] = zero4();
  // gc_last row term sum_v dh_next * h_pre: partial sums over the rows
  // v = j (mod 16), j = 0..15, each in ascending v, then summed over j.  A
  // thread takes a column pair and GPT of the residues j; consecutive lanes
  // take consecutive column pairs.
  constexpr int CP = K / 2, TG = 256 / CP, GPT = 16 / TG;
  static_assert(256 % CP == 0 && 16 % TG == 0 && VQ % 16 == 0, "row-term split");
  const int d = 2 * (threadIdx.x % CP), tg = threadIdx.x / CP;
  float rs[GPT][2];
#pragma unroll
  for (int j = 0; j < GPT; ++j) rs[j][0] = rs[j][1] = 0.f;
  for (int q = 0; q < NQ; ++q) {
    if (q + 1 < NQ) {
      ph.load(hg + (size_t)(q + 1) * VQ * K, K);
      pdh.load(dhg + (size_t)(q + 1) * VQ * K, K);
    }
#pragma unroll
    for (int r = 0; r < RB; ++r) {
      const int m0 = 16 * (wv_id + 4 * r);
#pragma unroll
      for (int k0 = 0; k0 < VQ; k0 += Mma<T>::KS) {
        const typename Mma<T>::frag fo = Mma<T>::ld_c(sDO, L::LV, m0, q * VQ + k0);
        const typename Mma<T>::frag fv = Mma<T>::ld_c(sDV, L::LV, m0, q * VQ + k0);
        const typename Mma<T>::frag fn = Mma<T>::ld_t(sVn, L::LC, m0, q * VQ + k0);
#pragma unroll
        for (int t = 0; t < NT; ++t) {
          const typename Mma<T>::frag bh_ = Mma<T>::ld_t(sH, L::LK, 16 * t, k0);
          const typename Mma<T>::frag bd = Mma<T>::ld_t(sDh, L::LK, 16 * t, k0);
          aq[r][t] = Mma<T>::mma(fo, bh_, aq[r][t]);
          aw[r][t] = Mma<T>::mma(fv, bh_, aw[r][t]);
          ak[r][t] = Mma<T>::mma(fn, bd, ak[r][t]);
        }
      }
    }
    {
      typedef T T2 __attribute__((ext_vector_type(2)));
#pragma unroll
      for (int jj = 0; jj < GPT; ++jj) {
#pragma unroll
        for (int u = 0; u < VQ / 16; ++u) {
          const int v = tg * GPT + jj + 16 * u;
          const T2 a = *reinterpret_cast<const T2*>(sDh + v * L::LK + d);
          const T2 c = *reinterpret_cast<const T2*>(sH + v * L::LK + d);
          rs[jj][0] += to_f(a[0]) * to_f(c[0]);
          rs[jj][1] += to_f(a[1]) * to_f(c[1]);
        }
      }
    }
    __syncthreads();  // the quarter's h / dh are read
    if (q + 1 < NQ) {
      ph.store(sH, L::LK);
      pdh.store(sDh, L::LK);
      __syncthreads();
    }
  }
  T* g_dqg = gr.dqg + blk * C * K;
  T* g_dwt = gr.dwt + blk * C * K;
  T* g_dkg = gr.dkg + blk * C * K;
#pragma unroll
  for (int r = 0; r < RB; ++r) {
    const int m0 = 16 * (wv_id + 4 * r);
#pragma unroll
    for (int t = 0; t < NT; ++t) {
      f32x4 a = aq[r][t], b = aw[r][t];
#pragma unroll
      for (int i = 0; i < 4; ++i) { a[i] *= dm.scale; b[i] = -b[i]; }
      store_tile_n(g_dqg, K, m0, 16 * t, a);
      store_tile_n(g_dwt, K, m0, 16 * t, b);
      store_tile_n(g_dkg, K, m0, 16 * t, ak[r][t]);
    }
  }
  // exp(gc_last) * sum_v dh_next * h_pre   (kernel_bwd_b3_wy_dqkg.py:200-201)
#pragma unroll
  for (int jj = 0; jj < GPT; ++jj) {
    red[(tg * GPT + jj) * K + d] = rs[jj][0];
    red[(tg * GPT + jj) * K + d + 1] = rs[jj][1];
  }
  __syncthreads();
  for (int c = threadIdx.x; c < K; c += 256) {
    float s = 0.f;
#pragma unroll
    for (int j = 0; j < 16; ++j) s += red[j * K + c];
    gr.rlast[blk * K + c] = __expf(ck.gcl[blk * K + c]) * s;
  }
}

// ------------------------------------------------------------------ B3 WY part
// gdn2_bwd_wy  per chunk, in 64-column halves of K / V:
//   dA = clip(dw_pseudo kb^T + dv_new wv^T)                     (b3:163-176)
//   dkb = n2n(A^T dw_pseudo), dwv = A^T dv_new,
//   dw = clip(n2n(dwv v)), dv = clip(n2n(dwv w))                (b3:164,167,194-195)
// and after the last half dAkk = n2n(-(A^T clip(dA A^T)) * strict) (b3:177-180,212).
// Each half's k, b, v, w, dw_pseudo and dv_new are read once for both parts.
template <typename T, int C, int KH>
struct WyLds {
  static constexpr int PAD = Pad<T>::v;
  static constexpr int LH = KH + PAD, LC = C + PAD;
  static constexpr int LW = KH + 4;  // fp32 dwv rows, 16-byte aligned
  static constexpr int OH = C * LH * (int)sizeof(T), OC = C * LC * (int)sizeof(T);
  static constexpr int off_a = 0;
  static constexpr int off_dw = off_a + OC;
  static constexpr int off_dv = off_dw + OH;
  static constexpr int off_kb = off_dv + OH;  // then clip(dA A^T)
  static constexpr int off_wv = off_kb + OH;
  static constexpr int off_da = off_wv + OH;  // during the halves: fp32 dwv over da and tot
  static constexpr int off_tot = off_da + OC;
  static constexpr int off_gl = off_tot + ColMap<C, KH>::NSEG * KH * 4;
  static constexpr int total = off_gl + KH * 4;
  static_assert(OC <= OH * 2, "dA A^T must fit in the kb / wv region");
  static_assert(C * LW * 4 <= off_gl - off_da, "fp32 dwv must fit in the da / tot region");
};

template <typename T, int C, int K, int V>
__global__ __launch_bounds__(256) void gdn2_bwd_wy(Gdn2Dims dm, Gdn2Chunks<T> ck, Gdn2Grads<T> gr,
                                                  const T* __restrict__ k, const T* __restrict__ v,
                                                  const T* __restrict__ w, const T* __restrict__ b,
                                                  const float* __restrict__ g, T* __restrict__ dw,
                                                  T* __restrict__ dv) {
  constexpr int KH = 64;
  static_assert(K == V && K % KH == 0, "K and V are staged in the same 64-column halves");
  typedef WyLds<T, C, KH> L;
  typedef ColMap<C, KH> M;
  __shared__ __attribute__((aligned(16))) unsigned char lds[L::total];
  T* sA = reinterpret_cast<T*>(lds + L::off_a);
  T* sDW = reinterpret_cast<T*>(lds + L::off_dw);
  T* sDV = reinterpret_cast<T*>(lds + L::off_dv);
  T* sKB = reinterpret_cast<T*>(lds + L::off_kb);
  T* sWV = reinterpret_cast<T*>(lds + L::off_wv);
  T* sDA = reinterpret_cast<T*>(lds + L::off_da);
  float* sDwv = reinterpret_cast<float*>(lds + L::off_da);
  T* sTmp = reinterpret_cast<T*>(lds + L::off_kb);
  float* sTot = reinterpret_cast<float*>(lds + L::off_tot);
  float* sGl = reinterpret_cast<float*>(lds + L::off_gl);

  const int tid = threadIdx.x;
  const int bhn = blockIdx.x;
  const int n = bhn % dm.NT;
  const int bh = bhn / dm.NT;
  const int h = bh % dm.H, bb = bh / dm.H;
  const int wv_id = wave_id();
  const size_t blk = (size_t)bhn;
  const size_t t0 = (size_t)bb * dm.T + (size_t)n * C;

  stage_rows<T, C, C>(sA, L::LC, ck.ainv + blk * C * C, C);
  constexpr int MT = C / 16;
  constexpr int TPW = MT * MT / 4;       // dA tiles per wave
  constexpr int TPH = MT * (KH / 16) / 4;  // dkb / dwv tiles per wave and half
  f32x4 da[TPW];
#pragma unroll
  for (int t = 0; t < TPW; ++t) da[t] = zero4();
  const int cg = tid % M::NCG, seg = tid / M::NCG;
  for (int c0 = 0; c0 < K; c0 += KH) {
    // kb = b k e^{gc} and wv = w v (rounded to the input dtype) for these
    // columns; k, b, v, w, dw~, dv_new are requested before the cumsum of g
    Raw8<T> rk[M::RS], rb[M::RS], rv[M::RS], rw[M::RS];
#pragma unroll
    for (int rr = 0; rr < M::RS; ++rr) {
      const size_t r = (size_t)(seg * M::RS + rr);
      rk[rr].load(k + (t0 + r) * dm.rk + (size_t)h * K + c0 + cg * 8);
      rb[rr].load(b + (t0 + r) * dm.rb + (size_t)h * K + c0 + cg * 8);
      rv[rr].load(v + (t0 + r) * dm.rv + (size_t)h * V + c0 + cg * 8);
      rw[rr].load(w + (t0 + r) * dm.rw + (size_t)h * V + c0 + cg * 8);
    }
    RegStage<T, C, KH> pdw, pdv;
    pdw.load(gr.dwt + blk * C * K + c0, K);
    pdv.load(gr.dvn + blk * C * V + c0, V);
    float gcr[M::RS][8];
    chunk_cumsum<C, KH>(g + t0 * dm.rg + (size_t)h * K + c0, (size_t)dm.rg, gcr, sTot, sGl);
#pragma unroll
    for (int rr = 0; rr < M::RS; ++rr) {
      const int r = seg * M::RS + rr;
      float kb[8], wv[8];
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        kb[j] = (rb[rr][j] * rk[rr][j]) * __expf(gcr[rr][j]);
        wv[j] = to_f(from_f<T>(rw[rr][j] * rv[rr][j]));
      }
      store8(sKB + r * L::LH + cg * 8, kb);
      store8(sWV + r * L::LH + cg * 8, wv);
    }
    pdw.store(sDW, L::LH);
    pdv.store(sDV, L::LH);
    __syncthreads();
#pragma unroll
    for (int t = 0; t < TPW; ++t) {
      const int tile = wv_id * TPW + t, mi = tile / MT, nj = tile % MT;
      da[t] = tile_mma<T, false, false>(da[t], sDW, L::LH, sKB, L::LH, 16 * mi, 16 * nj, KH);
      da[t] = tile_mma<T, false, false>(da[t], sDV, L::LH, sWV, L::LH, 16 * mi, 16 * nj, KH);
    }
    // dkb straight to memory; dwv (fp32) to LDS for the element-wise products
    T* g_dkb = gr.dkb + blk * C * K + c0;
#pragma unroll
    for (int t = 0; t < TPH; ++t) {
      const int tile = wv_id * TPH + t, mj = tile % MT, ni = tile / MT;
      const int k0 = tri_k0<T>(mj);  // A lower triangular: rows i >= j only
      f32x4 a = tile_mma<T, true, true>(zero4(), sA + k0 * L::LC, L::LC, sDW + k0 * L::LH, L::LH,
                                        16 * mj, 16 * ni, C - k0);
#pragma unroll
      for (int i = 0; i < 4; ++i) a[i] = n2n(a[i]);
      store_tile_n(g_dkb, K, 16 * mj, 16 * ni, a);
      const f32x4 d = tile_mma<T, true, true>(zero4(), sA + k0 * L::LC, L::LC, sDV + k0 * L::LH, L::LH,
                                              16 * mj, 16 * ni, C - k0);
#pragma unroll
      for (int i = 0; i < 4; ++i) sDwv[(16 * mj + tile_row(i)) * L::LW + 16 * ni + tile_col()] = d[i];
    }
    __syncthreads();
    // dw = dwv v, dv = dwv w with this thread's v / w rows still in registers
#pragma unroll
    for (int rr = 0; rr < M::RS; ++rr) {
      const int r = seg * M::RS + rr;
      float d8[8], gw[8], gv[8];
      load8(sDwv + r * L::LW + cg * 8, d8);
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        gw[j] = sanitize(n2n(d8[j] * rv[rr][j]));
        gv[j] = sanitize(n2n(d8[j] * rw[rr][j]));
      }
      const size_t o = ((t0 + r) * dm.H + h) * V + c0 + cg * 8;
      store8(dw + o, gw);
      store8(dv + o, gv);
    }
    __syncthreads();  // before the next half overwrites the operands
  }
#pragma unroll
  for (int t = 0; t < TPW; ++t) {
    const int tile = wv_id * TPW + t, mi = tile / MT, nj = tile % MT;
    f32x4 acc = da[t];
#pragma unroll
    for (int i = 0; i < 4; ++i) acc[i] = sanitize(acc[i]);
    store_tile_n(sDA, L::LC, 16 * mi, 16 * nj, acc);
  }
  __syncthreads();
  // tmp = clip(dA A^T)   (b3:177-178); A[j][l] = 0 for l > j
  for (int tile = wv_id; tile < MT * MT; tile += 4) {
    const int mi = tile / MT, nj = tile % MT;
    f32x4 acc = tile_mma<T, false, false>(zero4(), sDA, L::LC, sA, L::LC, 16 * mi, 16 * nj,
                                          tri_k1<T>(nj, C));
#pragma unroll
    for (int i = 0; i < 4; ++i) acc[i] = sanitize(acc[i]);
    store_tile_n(sTmp, L::LC, 16 * mi, 16 * nj, acc);
  }
  __syncthreads();
  // dAkk = n2n(-(A^T tmp) * strict)   (b3:179-180,212)
  T* g_dakk = gr.dakk + blk * C * C;
  for (int tile = wv_id; tile < MT * MT; tile += 4) {
    const int mj = tile / MT, nl = tile % MT;
    f32x4 acc = zero4();
    if (nl <= mj) {
      const int k0 = tri_k0<T>(mj);
      acc = tile_mma<T, true, true>(acc, sA + k0 * L::LC, L::LC, sTmp + k0 * L::LC, L::LC, 16 * mj,
                                    16 * nl, C - k0);
    }
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int r = 16 * mj + tile_row(i), c = 16 * nl + tile_col();
      acc[i] = r > c ? n2n(-acc[i]) : 0.f;
    }
    store_tile_n(g_dakk, C, 16 * mj, 16 * nl, acc);
  }
}

// ------------------------------------------------------------------ B4 + combine + B5
template <typename T, int C, int K>  // K here: the columns of one workgroup's slice
struct InLds {
  static constexpr int PAD = Pad<T>::v;
  static constexpr int LK = K + PAD, LC = C + PAD, LG = K + 4;
  static constexpr int OK_ = C * LK * (int)sizeof(T), OC = C * LC * (int)sizeof(T);
  static constexpr int off_gc = 0;           // fp32 gc, then fp32 dgc
  static constexpr int off_q = off_gc + C * LG * 4;  // q e^{gc}  (exact path: then raw q)
  static constexpr int off_kt = off_q + OK_; // k e^{-gc} (exact path: then raw k)
  static constexpr int off_kb = off_kt + OK_;// b k e^{gc} (exact path: then raw b)
  static constexpr int off_daqk = off_kb + OK_;
  static constexpr int off_dakk = off_daqk + OC;
  static constexpr int off_tot = off_dakk + OC;  // the cross-wave segment totals: 4 K floats
  // factorised path, after the MFMAs: dQ~, dK~, dKB as fp32 [C][LG] from off_q
  static constexpr int off_res = off_q;
  static constexpr int end_res = off_res + 3 * C * LG * 4;
  static constexpr int off_gl = end_res > off_tot + 4 * K * 4 ? end_res : off_tot + 4 * K * 4;
  static constexpr int off_part = off_gl + K * 4;  // [4 C / 16][K] column partial sums
  static constexpr int total = off_part + 4 * (C / 16) * K * 4;
};

// One workgroup per (batch, head, chunk, KH-column slice): every term of B4,
// B3's element-wise part and B5 is separable over the K columns (only the
// [C][C] dAqk / dAkk are shared by the slices).
template <typename T, int C, int K, int V, int KH>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(2, 2))) void gdn2_bwd_intra(Gdn2Dims dm, Gdn2Grads<T> gr,
                                                     const T* __restrict__ q, const T* __restrict__ k,
                                                     const T* __restrict__ b, const float* __restrict__ g,
                                                     T* __restrict__ dq, T* __restrict__ dk,
                                                     T* __restrict__ db, float* __restrict__ dg) {
  typedef InLds<T, C, KH> L;
  typedef ColMap<C, KH> M;
  __shared__ __attribute__((aligned(16))) unsigned char lds[L::total];
  T* sQ = reinterpret_cast<T*>(lds + L::off_q);
  T* sKt = reinterpret_cast<T*>(lds + L::off_kt);
  T* sKB = reinterpret_cast<T*>(lds + L::off_kb);
  T* sDAqk = reinterpret_cast<T*>(lds + L::off_daqk);
  T* sDAkk = reinterpret_cast<T*>(lds + L::off_dakk);
  float* sGc = reinterpret_cast<float*>(lds + L::off_gc);
  float* sTot = reinterpret_cast<float*>(lds + L::off_tot);
  float* sGl = reinterpret_cast<float*>(lds + L::off_gl);
  float* sPart = reinterpret_cast<float*>(lds + L::off_part);

  constexpr int NKS = K / KH;
  const int tid = threadIdx.x;
  // the NKS slices of one chunk share an XCD (dAqk / dAkk read once per L2)
  int bhn, ks;
  xcd_group_map(blockIdx.x, dm.B * dm.H * dm.NT, NKS, bhn, ks);
  const int d0 = ks * KH;
  const int n = bhn % dm.NT;
  const int bh = bhn / dm.NT;
  const int h = bh % dm.H, bb = bh / dm.H;
  const int wv_id = wave_id();
  const size_t blk = (size_t)bhn;
  const size_t rsK = (size_t)dm.H * K;  // the gradients' (dense) row stride
  const size_t t0 = (size_t)bb * dm.T + (size_t)n * C;
  const size_t base = (t0 * dm.H + h) * K + d0;  // this slice's column 0 in the gradients
  const size_t hk = (size_t)h * K + d0;           // ... and within an input row

  // q, k, b and dAqk / dAkk are requested before the cumsum of g, so their
  // latency overlaps it
  const int cg = tid % M::NCG, seg = tid / M::NCG;
  Raw8<T> rq[M::RS], rk[M::RS], rb[M::RS];
#pragma unroll
  for (int rr = 0; rr < M::RS; ++rr) {
    const size_t r = t0 + (size_t)(seg * M::RS + rr);
    rq[rr].load(q + r * dm.rq + hk + cg * 8);
    rk[rr].load(k + r * dm.rk + hk + cg * 8);
    rb[rr].load(b + r * dm.rb + hk + cg * 8);
  }
  RegStage<T, C, C> pqk, pkk;
  pqk.load(gr.daqk + blk * C * C, C);
  pkk.load(gr.dakk + blk * C * C, C);
  // the B3 intermediates of the element-wise stage (same thread map), likewise
  Raw8<T> rdqg[M::RS], rdkb[M::RS], rdkg[M::RS];
#pragma unroll
  for (int rr = 0; rr < M::RS; ++rr) {
    const size_t o = blk * C * K + d0 + (size_t)(seg * M::RS + rr) * K + cg * 8;
    rdqg[rr].load(gr.dqg + o);
    rdkb[rr].load(gr.dkb + o);
    rdkg[rr].load(gr.dkg + o);
  }
  float gcr[M::RS][8];
  const bool exact = chunk_cumsum<C, KH>(g + t0 * dm.rg + hk, (size_t)dm.rg, gcr, sTot, sGl);
#pragma unroll
  for (int rr = 0; rr < M::RS; ++rr) {
    const int r = seg * M::RS + rr;
    float qv[8], kv[8], bv[8], o1[8], o2[8], o3[8];
#pragma unroll
    for (int j = 0; j < 8; ++j) { qv[j] = rq[rr][j]; kv[j] = rk[rr][j]; bv[j] = rb[rr][j]; }
    if (!exact) {
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        const float e = __expf(gcr[rr][j]);
        o1[j] = qv[j] * e;
        o2[j] = kv[j] * __expf(-gcr[rr][j]);
        o3[j] = (bv[j] * kv[j]) * e;
      }
    } else {
#pragma unroll
      for (int j = 0; j < 8; ++j) { o1[j] = qv[j]; o2[j] = kv[j]; o3[j] = bv[j]; }
    }
    store8(sQ + r * L::LK + cg * 8, o1);
    store8(sKt + r * L::LK + cg * 8, o2);
    store8(sKB + r * L::LK + cg * 8, o3);
    // 16-byte row pieces: the eight threads of a row would put scalar
    // accesses of a wave on a handful of banks
    store8(sGc + r * L::LG + cg * 8, gcr[rr]);
  }
  // scale folded into the dAqk operand: Aqk = scale Q~ K~^T
  pqk.store(sDAqk, L::LC);
  pkk.store(sDAkk, L::LC);
  __syncthreads();

  // Tiles of [C][K], column-major over tiles so each wave owns whole columns.
  constexpr int MT = C / 16, NTK = KH / 16;
  constexpr int TPW = MT * NTK / 4;
  static_assert((MT * NTK) % 4 == 0 && (TPW % MT == 0 || MT % TPW == 0),
                "a wave's tiles must be whole tile columns or part of one");
  // waves sharing a tile column (exact path partial sums)
  constexpr int WPC = TPW < MT ? MT / TPW : 1;
  f32x4 dQt[TPW], dKt[TPW], dKB[TPW];
  if (!exact) {
    // dQ~ = (scale dAqk) K~ ; dK~ = (scale dAqk)^T Q~ + dAkk^T KB ; dKB = dAkk K~
#pragma unroll
    for (int t = 0; t < TPW; ++t) {
      const int tile = wv_id * TPW + t, mi = tile % MT, ni = tile / MT;
      const int k1 = tri_k1<T>(mi, C);   // dA* lower triangular: j <= i
      const int k0 = tri_k0<T>(mi);      // transposed use: i >= j
      dQt[t] = tile_mma<T, false, true>(zero4(), sDAqk, L::LC, sKt, L::LK, 16 * mi, 16 * ni, k1);
      dKB[t] = tile_mma<T, false, true>(zero4(), sDAkk, L::LC, sKt, L::LK, 16 * mi, 16 * ni, k1);
      f32x4 a = tile_mma<T, true, true>(zero4(), sDAqk + k0 * L::LC, L::LC, sQ + k0 * L::LK, L::LK,
                                        16 * mi, 16 * ni, C - k0);
      dKt[t] = tile_mma<T, true, true>(a, sDAkk + k0 * L::LC, L::LC, sKB + k0 * L::LK, L::LK,
                                       16 * mi, 16 * ni, C - k0);
    }
  }
  __syncthreads();
  const T* g_dqg = gr.dqg + blk * C * K + d0;
  const T* g_dkb = gr.dkb + blk * C * K + d0;
  const T* g_dkg = gr.dkg + blk * C * K + d0;
  if (!exact) {
    // ---- factorised path: the MFMA results go through LDS so the
    // element-wise stage runs in the row-contiguous layout (16-byte I/O)
    float* sRes = reinterpret_cast<float*>(lds + L::off_res);
    constexpr int RS3 = C * L::LG;
#pragma unroll
    for (int t = 0; t < TPW; ++t) {
      const int tile = wv_id * TPW + t, mi = tile % MT, ni = tile / MT;
      store_tile_n(sRes, L::LG, 16 * mi, 16 * ni, dQt[t]);
      store_tile_n(sRes + RS3, L::LG, 16 * mi, 16 * ni, dKt[t]);
      store_tile_n(sRes + 2 * RS3, L::LG, 16 * mi, 16 * ni, dKB[t]);
    }
    __syncthreads();
    float csum[8];
#pragma unroll
    for (int j = 0; j < 8; ++j) csum[j] = 0.f;
#pragma unroll
    for (int rr = 0; rr < M::RS; ++rr) {
      const int r = seg * M::RS + rr;
      const int c8 = cg * 8;
      float qv[8], kv[8], bv[8], dqg[8], dkb[8], dkg[8], oq[8], ok[8], ob[8];
#pragma unroll
      for (int j = 0; j < 8; ++j) { qv[j] = rq[rr][j]; kv[j] = rk[rr][j]; bv[j] = rb[rr][j]; }
#pragma unroll
      for (int j = 0; j < 8; ++j) { dqg[j] = rdqg[rr][j]; dkb[j] = rdkb[rr][j]; dkg[j] = rdkg[rr][j]; }
      // the row piece's gc, MFMA results and gc_last as 16-byte LDS reads
      float gc8[8], tq8[8], tk8[8], tb8[8], gl8[8], dgc8[8];
      load8(sGc + r * L::LG + c8, gc8);
      load8(sRes + r * L::LG + c8, tq8);
      load8(sRes + RS3 + r * L::LG + c8, tk8);
      load8(sRes + 2 * RS3 + r * L::LG + c8, tb8);
      load8(sGl + c8, gl8);
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        const float gcv = gc8[j];
        const float e = __expf(gcv), ei = __expf(-gcv), eg = __expf(gl8[j] - gcv);
        const float tq = tq8[j], tk = tk8[j], tb = tb8[j];
        // B4 (kernel_bwd_b4_intra.py:101-132)
        const float dq4 = sanitize(tq * e);
        const float dk4 = sanitize(tk * ei + tb * bv[j] * e);
        const float db4 = sanitize(tb * kv[j] * e);
        const float dgc4 = sanitize(tq * (qv[j] * e) - tk * (kv[j] * ei) + tb * (bv[j] * kv[j] * e));
        // B3 element-wise terms (kernel_bwd_b3_wy_dqkg.py:182-198)
        const float kgv = kv[j] * eg;
        const float dq3 = n2n(dqg[j] * e);
        const float dk3 = n2n(dkb[j] * e * bv[j] + dkg[j] * eg);
        const float db3 = n2n(dkb[j] * e * kv[j]);
        const float dx = dkg[j] * kgv;
        const float dgc3 = dkb[j] * (bv[j] * kv[j] * e) + dqg[j] * (qv[j] * e) - dx;
        csum[j] += dx;
        oq[j] = sanitize(dq3 + dq4);
        ok[j] = sanitize(dk3 + dk4);
        ob[j] = sanitize(db3 + db4);
        dgc8[j] = dgc3 + dgc4;
      }
      store8(sGc + r * L::LG + c8, dgc8);  // each element read (as gc) and written by this thread only
      const size_t go = base + (size_t)r * rsK + c8;
      store8(dq + go, oq);
      store8(dk + go, ok);
      store8(db + go, ob);
    }
    __syncthreads();  // the MFMA results are dead: column partial sums go to their space
    float* sCol = sRes;  // [NSEG][KH]
    store8(sCol + seg * KH + cg * 8, csum);
    __syncthreads();
    if (tid < KH) {
      float extra = gr.rlast[blk * K + d0 + tid];
      for (int sg = 0; sg < M::NSEG; ++sg) extra += sCol[sg * KH + tid];
      sGc[(C - 1) * L::LG + tid] += extra;
    }
    __syncthreads();
  } else {
    // ---- exact path: raw q, k, b for the element-wise stage (fp32 exact multipliers)
    stage_rows<T, C, KH>(sQ, L::LK, q + t0 * dm.rq + hk, (size_t)dm.rq);
    stage_rows<T, C, KH>(sKt, L::LK, k + t0 * dm.rk + hk, (size_t)dm.rk);
    stage_rows<T, C, KH>(sKB, L::LK, b + t0 * dm.rb + hk, (size_t)dm.rb);
    __syncthreads();
    // dgc is parked in this slice's dg rows (written by B5 below) until every
    // lane has read gc; the loop is kept rolled, this path is the rare one
    float* dgp = dg + base;
    float colsum = 0.f;
  #pragma unroll 1
    for (int t = 0; t < TPW; ++t) {
      const int tile = wv_id * TPW + t, mi = tile % MT, ni = tile / MT;
  #pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int r = 16 * mi + tile_row(i), d = 16 * ni + tile_col();
        const float gcv = sGc[r * L::LG + d];
        const float e = __expf(gcv), ei = __expf(-gcv), eg = __expf(sGl[d] - gcv);
        const float qv = to_f(sQ[r * L::LK + d]), kv = to_f(sKt[r * L::LK + d]),
                    bv = to_f(sKB[r * L::LK + d]);
        // B4 (kernel_bwd_b4_intra.py:101-132)
        float dq4, dk4, db4, dgc4;
        {
          // pairwise with exp(clip(gc_i - gc_j, -20, 20)) and the clip mask
          float sq = 0.f, sb = 0.f, sk = 0.f, sgi = 0.f, sgj = 0.f;
          for (int j = 0; j <= r; ++j) {
            const float dd = gcv - sGc[j * L::LG + d];
            const float E = __expf(fminf(fmaxf(dd, -kClipDecay), kClipDecay));
            const float msk = (dd >= -kClipDecay && dd <= kClipDecay) ? 1.f : 0.f;
            const float kj = to_f(sKt[j * L::LK + d]);
            const float aq = to_f(sDAqk[r * L::LC + j]);  // holds scale * dAqk
            const float ak = (j < r) ? to_f(sDAkk[r * L::LC + j]) : 0.f;
            sq += aq * E * kj;
            sb += ak * E * kj;
            sgi += (aq * qv + ak * bv * kv) * E * kj * msk;
          }
          for (int i2 = r; i2 < C; ++i2) {
            const float dd = sGc[i2 * L::LG + d] - gcv;
            const float E = __expf(fminf(fmaxf(dd, -kClipDecay), kClipDecay));
            const float msk = (dd >= -kClipDecay && dd <= kClipDecay) ? 1.f : 0.f;
            const float aq = to_f(sDAqk[i2 * L::LC + r]);
            const float ak = (i2 > r) ? to_f(sDAkk[i2 * L::LC + r]) : 0.f;
            const float li = aq * to_f(sQ[i2 * L::LK + d]) +
                             ak * to_f(sKB[i2 * L::LK + d]) * to_f(sKt[i2 * L::LK + d]);
            sk += li * E;
            sgj += li * E * kv * msk;
          }
          dq4 = sq;
          dk4 = sk + sb * bv;
          db4 = sb * kv;
          dgc4 = sgi - sgj;
        }
        dq4 = sanitize(dq4); dk4 = sanitize(dk4); db4 = sanitize(db4); dgc4 = sanitize(dgc4);
        // B3 element-wise terms (kernel_bwd_b3_wy_dqkg.py:182-198)
        const size_t o = (size_t)r * K + d;
        const float dqg = to_f(g_dqg[o]), dkb = to_f(g_dkb[o]), dkg = to_f(g_dkg[o]);
        const float kgv = kv * eg;
        const float dq3 = n2n(dqg * e);
        const float dk3 = n2n(dkb * e * bv + dkg * eg);
        const float db3 = n2n(dkb * e * kv);
        const float dx = dkg * kgv;
        const float dgc3 = dkb * (bv * kv * e) + dqg * (qv * e) - dx;
        colsum += dx;
        const size_t go = base + (size_t)r * rsK + d;
        dq[go] = from_f<T>(sanitize(dq3 + dq4));
        dk[go] = from_f<T>(sanitize(dk3 + dk4));
        db[go] = from_f<T>(sanitize(db3 + db4));
        dgp[(size_t)r * rsK + d] = dgc3 + dgc4;
      }
      if ((t + 1) % MT == 0 || t + 1 == TPW) {  // this wave's part of a tile column is done
        const int ni = tile / MT, pi = WPC > 1 ? (wv_id * TPW % MT) / TPW : 0;
        sPart[(4 * pi + (lane_id() >> 4)) * KH + 16 * ni + tile_col()] = colsum;
        colsum = 0.f;
      }
    }
    __syncthreads();  // every lane has read gc: the parked dgc replaces it
    for (int e = tid; e < C * KH; e += 256) {
      const int r = e / KH, d = e % KH;
      sGc[r * L::LG + d] = dgp[(size_t)r * rsK + d];
    }
    __syncthreads();
    if (tid < KH) {
      float extra = 0.f;
#pragma unroll
      for (int sl = 0; sl < 4 * WPC; ++sl) extra += sPart[sl * KH + tid];
      extra += gr.rlast[blk * K + d0 + tid];
      // dgc3 gets the row term before its n2n in the reference; dgc4 is already
      // sanitized, so the sum below matches dgc3 + dgc4 in unclipped regimes.
      sGc[(C - 1) * L::LG + tid] += extra;
    }
    __syncthreads();
  }
  // B5: dg = sanitize(reverse cumsum over the chunk)   (kernel_bwd_b5_reverse_cumsum.py:17-24)
  // thread (column group, row segment): suffix sums within the segment, then
  // the totals of the later segments
  {
    const int cg = tid % M::NCG, seg = tid / M::NCG;
    float v[M::RS][8];
#pragma unroll
    for (int rr = M::RS - 1; rr >= 0; --rr) {
      const int r = seg * M::RS + rr;
#pragma unroll
      for (int j = 0; j < 8; ++j) v[rr][j] = sGc[r * L::LG + cg * 8 + j] + (rr + 1 < M::RS ? v[rr + 1][j] : 0.f);
    }
    float off[8];
    seg_scan8<M::NCG, true>(v[0], off, sTot);
#pragma unroll
    for (int rr = 0; rr < M::RS; ++rr) {
      const int r = seg * M::RS + rr;
      float o8[8];
#pragma unroll
      for (int j = 0; j < 8; ++j) o8[j] = sanitize(v[rr][j] + off[j]);
      store8(dg + base + (size_t)r * rsK + cg * 8, o8);
    }
  }
}

}  // namespace ah
