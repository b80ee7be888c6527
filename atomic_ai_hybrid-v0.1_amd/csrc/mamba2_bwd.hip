// Mamba2 SSD chunk-scan backward for gfx950, with the semantics of the
// hand-derived MB0 backward (atomic_ops/mamba2_bwd_reference.py:55-266):
// every clip contributes a straight-through mask (:48-52) and the per-chunk
// sanitising of :166-195 is kept.
//
// mamba2_bwd_dstate  one workgroup per (batch, head, PT channels), reverse over
//                    chunks with the fp32 dstate carry in MFMA accumulators:
//                    dstate_prev = sanitize(dstate dce + (dy decay_h)^T C)   (:115,128,195)
//                    and the decay_chunk_end row term d_cum_last_a (:116,120).
// mamba2_bwd_chunk   one workgroup per (batch, chunk, head group): every other
//                    term of :123-190 for each head and 32-channel slice, with
//                    the cross-head sums dCB (:147-152), dC_1 (:127) and dB_1
//                    (:135) accumulated in registers.  The pairwise decay of the
//                    off-diagonal 16-row blocks is factorised exactly as in the
//                    forward scan; diagonal blocks are evaluated pairwise with
//                    the reference's clip masks.
// mamba2_bwd_bc      one workgroup per (batch, chunk): dB = dB_1 + dCB^T C and
//                    dC = dC_1 + dCB B (:154-156,191-192), final sanitize / cast.
// mamba2_bwd_da      dA = sum over chunks of sanitize(sum over batch) (:188,194,263).
#include "mamba2_fwd.hip"

namespace ah {

template <typename T>
struct Mamba2Grads {
  T* dstate;     // [B][H][NT][P][N]  dstate_new of each chunk (the carry its backward starts from)
  float* lasta;  // [B][H][NT][P]     d cum_last through decay_chunk_end
  float* part;   // [B][NT][G][C*C + 2*C*N] cross-head partial sums: dCB, dC_1, dB_1
  float* dap;    // [B][NT][H]        per (batch, chunk, head) dA contribution
};

// ------------------------------------------------------------------ dstate scan
template <typename T, int C, int N, int PT>
struct DsLds {
  static constexpr int PAD = Pad<T>::v;
  static constexpr int LN = N + PAD, LPT = PT + PAD;
  static constexpr int NSEG = 256 / PT;
  static constexpr int off_c = 0;
  static constexpr int off_ydh = off_c + C * LN * (int)sizeof(T);
  static constexpr int off_cum = off_ydh + C * LPT * (int)sizeof(T);
  static constexpr int off_tot = off_cum + C * PT * 4;
  static constexpr int off_red = off_tot + NSEG * PT * 4;
  static constexpr int total = off_red + 4 * PT * 4;
};

template <typename T, typename TD, int C, int P, int N, int PT>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(1, 1))) void mamba2_bwd_dstate(
    Mamba2Dims dm, const T* __restrict__ dt, const float* __restrict__ A, const T* __restrict__ Cm,
    const TD* __restrict__ dy, const float* __restrict__ dstate_final, Mamba2Chunks<T> ck,
    Mamba2Grads<T> gr, float* __restrict__ dstate0) {
  typedef DsLds<T, C, N, PT> L;
  __shared__ __attribute__((aligned(16))) unsigned char lds[L::total];
  T* sC = reinterpret_cast<T*>(lds + L::off_c);
  T* sYdh = reinterpret_cast<T*>(lds + L::off_ydh);
  float* sCum = reinterpret_cast<float*>(lds + L::off_cum);
  float* sTot = reinterpret_cast<float*>(lds + L::off_tot);
  float* sRed = reinterpret_cast<float*>(lds + L::off_red);

  constexpr int NPT = P / PT;
  const int pt = blockIdx.x % NPT;
  const int bh = blockIdx.x / NPT;
  const int h = bh % dm.H, bb = bh / dm.H;
  const int p0 = pt * PT;
  const int wv_id = wave_id();
  const float Ah = A[h];
  const size_t rsx = (size_t)dm.H * P;

  constexpr int SNI = N / 16;
  constexpr int NTS = (PT / 16) * SNI;
  constexpr int SPW = NTS / 4;
  static_assert(NTS % 4 == 0, "state tiles must split evenly over 4 waves");

  f32x4 ds[SPW];
#pragma unroll
  for (int t = 0; t < SPW; ++t) {
    const int tile = wv_id * SPW + t, mi = tile / SNI, ni = tile % SNI;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int p = 16 * mi + tile_row(i), s = 16 * ni + tile_col();
      ds[t][i] = dstate_final ? dstate_final[((size_t)bh * P + p0 + p) * N + s] : 0.f;
    }
  }

  RegStage<T, C, N> pC;
  RegStage<T, C, PT> pdt;
  RegStage<TD, C, PT> pdy;
  auto prefetch = [&](int n) {
    const size_t row0 = (size_t)bb * dm.T + (size_t)n * C;
    pC.load(Cm + row0 * N, N);
    pdt.load(dt + (row0 * dm.H + h) * P + p0, rsx);
    pdy.load(dy + (row0 * dm.H + h) * P + p0, rsx);
  };
  auto commit = [&]() {
    pC.store(sC, L::LN);
    constexpr int VEC = 16 / (int)sizeof(T), PER_ROW = PT / VEC;
#pragma unroll
    for (int i = 0; i < RegStage<T, C, PT>::PT; ++i) {
      const int e = threadIdx.x + 256 * i;
      if (e < C * PER_ROW) {
        const int r = e / PER_ROW, c = (e % PER_ROW) * VEC;
        const T* dv = reinterpret_cast<const T*>(&pdt.r[i]);
#pragma unroll
        for (int j = 0; j < VEC; ++j) sCum[r * PT + c + j] = sanitize(to_f(dv[j]) * Ah, kClipDecay);
      }
    }
  };
  prefetch(dm.NT - 1);
  commit();
  __syncthreads();

  for (int n = dm.NT - 1; n >= 0; --n) {
    column_cumsum<C, PT>(sCum, sTot);
    __syncthreads();
    // dy decay_h, decay_h = exp(clip(cum, -20, 0))   (:123)
    {
      constexpr int VEC = 16 / (int)sizeof(TD), PER_ROW = PT / VEC;
#pragma unroll
      for (int i = 0; i < RegStage<TD, C, PT>::PT; ++i) {
        const int e = threadIdx.x + 256 * i;
        if (e < C * PER_ROW) {
          const int r = e / PER_ROW, c = (e % PER_ROW) * VEC;
          const TD* dv = reinterpret_cast<const TD*>(&pdy.r[i]);
#pragma unroll
          for (int j = 0; j < VEC; ++j) {
            const float dh = __expf(fminf(fmaxf(sCum[r * PT + c + j], -kClipDecay), 0.f));
            sYdh[r * L::LPT + c + j] = from_f<T>(to_f(dv[j]) * dh);
          }
        }
      }
    }
    // the carry entering this chunk's backward, and
    // d_cum_last_a = sum_s dstate state_prev * dce * mask   (:116,120)
    const size_t bhn = (size_t)bh * dm.NT + n;
    T* dsg = gr.dstate + (bhn * P + p0) * N;
    const T* spg = ck.state_pre + (bhn * P + p0) * N;
    float part[4] = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int t = 0; t < SPW; ++t) {
      const int tile = wv_id * SPW + t, mi = tile / SNI, ni = tile % SNI;
      store_tile_n(dsg, N, 16 * mi, 16 * ni, ds[t]);
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int p = 16 * mi + tile_row(i), s = 16 * ni + tile_col();
        part[i] += ds[t][i] * to_f(spg[(size_t)p * N + s]);
      }
    }
    static_assert(PT == 16, "the d_cum_last_a reduction assumes one row tile of channels");
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      float v = part[i];
      v += __shfl_xor(v, 1); v += __shfl_xor(v, 2); v += __shfl_xor(v, 4); v += __shfl_xor(v, 8);
      if (tile_col() == 0) sRed[wv_id * PT + tile_row(i)] = v;
    }
    if (n > 0) prefetch(n - 1);
    __syncthreads();
    if (threadIdx.x < PT) {
      const int p = threadIdx.x;
      const float cl = sCum[(C - 1) * PT + p];
      const float m = (cl >= -kClipDecay && cl <= 0.f) ? 1.f : 0.f;
      const float s = sRed[p] + sRed[PT + p] + sRed[2 * PT + p] + sRed[3 * PT + p];
      gr.lasta[bhn * P + p0 + p] = s * __expf(fminf(fmaxf(cl, -kClipDecay), 0.f)) * m;
    }
    // dstate_prev = sanitize(dstate dce + (dy decay_h)^T C)
#pragma unroll
    for (int t = 0; t < SPW; ++t) {
      const int tile = wv_id * SPW + t, mi = tile / SNI, ni = tile % SNI;
      f32x4 acc = ds[t];
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int p = 16 * mi + tile_row(i);
        acc[i] *= __expf(fminf(fmaxf(sCum[(C - 1) * PT + p], -kClipDecay), 0.f));
      }
      acc = tile_mma<T, true, true>(acc, sYdh, L::LPT, sC, L::LN, 16 * mi, 16 * ni, C);
#pragma unroll
      for (int i = 0; i < 4; ++i) acc[i] = sanitize(acc[i]);
      ds[t] = acc;
    }
    __syncthreads();
    if (n > 0) commit();
    __syncthreads();
  }
  if (dstate0) {
#pragma unroll
    for (int t = 0; t < SPW; ++t) {
      const int tile = wv_id * SPW + t, mi = tile / SNI, ni = tile % SNI;
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int p = 16 * mi + tile_row(i), s = 16 * ni + tile_col();
        dstate0[((size_t)bh * P + p0 + p) * N + s] = sanitize(ds[t][i]);  // :264 + final clip
      }
    }
  }
}

// ------------------------------------------------------------------ per-chunk gradients
// Y^(I) rows start at the MFMA k step at or below 16 (I + 1).
template <typename T>
__host__ __device__ constexpr int ybase(int I) {
  return (16 * (I + 1) / Mma<T>::KS) * Mma<T>::KS;
}

template <typename T, int C, int N, int PT>
struct CkLds {
  static constexpr int PAD = Pad<T>::v;
  static constexpr int LCB = C + PAD, LN = N + PAD, LPT = PT + PAD;
  static constexpr int NSEG = 256 / PT;
  static constexpr int OPT = C * LPT * (int)sizeof(T);
  static constexpr int off_cb = 0;
  static constexpr int off_st = off_cb + C * LCB * (int)sizeof(T);
  static constexpr int off_dst = off_st + PT * LN * (int)sizeof(T);
  static constexpr int off_dy = off_dst + PT * LN * (int)sizeof(T);
  static constexpr int off_ydh = off_dy + OPT;   // then fp32 ddt_1 (with off_w)
  static constexpr int off_w = off_ydh + OPT;
  static constexpr int off_ydec = off_w + OPT;   // then fp32 d_cum (with off_z, off_y)
  static constexpr int off_z = off_ydec + OPT;
  static constexpr int off_y = off_z + OPT;
  static constexpr int off_cum = off_y + OPT;
  static constexpr int off_dbx = off_cum + C * PT * 4;
  static constexpr int off_tot = off_dbx + C * PT * 4;
  static constexpr int off_misc = off_tot + NSEG * PT * 4;   // lasta[PT], lastb[4][PT], dA[8]
  static constexpr int total = off_misc + (PT + 4 * PT + 8) * 4;
  static_assert(2 * OPT >= C * PT * 4 && 3 * OPT >= C * PT * 4, "fp32 aliases must fit");
};

template <typename T, typename TD, int C, int P, int N>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(1, 1))) void mamba2_bwd_chunk(
    Mamba2Dims dm, int G, const T* __restrict__ dt, const T* __restrict__ x,
    const float* __restrict__ A, const T* __restrict__ Bm, const T* __restrict__ Cm,
    const TD* __restrict__ dy, Mamba2Chunks<T> ck, Mamba2Grads<T> gr, T* __restrict__ ddt,
    T* __restrict__ dx) {
  constexpr int PT = 32;
  typedef CkLds<T, C, N, PT> L;
  __shared__ __attribute__((aligned(16))) unsigned char lds[L::total];
  T* sCB = reinterpret_cast<T*>(lds + L::off_cb);
  T* sSt = reinterpret_cast<T*>(lds + L::off_st);
  T* sDst = reinterpret_cast<T*>(lds + L::off_dst);
  T* sDy = reinterpret_cast<T*>(lds + L::off_dy);
  T* sYdh = reinterpret_cast<T*>(lds + L::off_ydh);
  T* sW = reinterpret_cast<T*>(lds + L::off_w);
  T* sYdec = reinterpret_cast<T*>(lds + L::off_ydec);
  T* sZ = reinterpret_cast<T*>(lds + L::off_z);
  T* sY = reinterpret_cast<T*>(lds + L::off_y);
  float* sCum = reinterpret_cast<float*>(lds + L::off_cum);
  float* sDbx = reinterpret_cast<float*>(lds + L::off_dbx);
  float* sTot = reinterpret_cast<float*>(lds + L::off_tot);
  float* sLastA = reinterpret_cast<float*>(lds + L::off_misc);
  float* sLastB = sLastA + PT;
  float* sDa = sLastB + 4 * PT;
  // Low halves of the split Z / Y operands: Ydh / W are dead once the block
  // loop starts.
  T* sZlo = reinterpret_cast<T*>(lds + L::off_ydh);
  T* sYlo = reinterpret_cast<T*>(lds + L::off_w);
  float* sDdt1 = reinterpret_cast<float*>(lds + L::off_ydh);   // aliases Ydh + W in the epilogue
  float* sRed = reinterpret_cast<float*>(lds + L::off_ydec);   // aliases Ydec + Z + Y in the epilogue

  const int tid = threadIdx.x;
  const int g = blockIdx.x % G;
  const int bn = blockIdx.x / G;
  const int bb = bn / dm.NT, n = bn % dm.NT;
  const int HG = dm.H / G;
  const int wv_id = wave_id();
  const size_t row0 = (size_t)bb * dm.T + (size_t)n * C;
  const size_t rsx = (size_t)dm.H * P;
  const T* Bg = Bm + row0 * N;
  const T* Cg = Cm + row0 * N;
  constexpr int NB = C / 16;
  constexpr int MTN = N / 16;

  stage_rows<T, C, C>(sCB, L::LCB, ck.cb + (size_t)bn * C * C, C);

  // cross-head accumulators: dCB lower tiles (I >= J), dC_1, dB_1 tiles of [C][N]
  constexpr int NBC = NB * (NB + 1) / 2;
  constexpr int BCPW = (NBC + 3) / 4;
  constexpr int CPW = NB * MTN / 4;
  f32x4 acc_bc[BCPW], acc_c1[CPW], acc_b1[CPW];
#pragma unroll
  for (int i = 0; i < BCPW; ++i) acc_bc[i] = zero4();
#pragma unroll
  for (int i = 0; i < CPW; ++i) { acc_c1[i] = zero4(); acc_b1[i] = zero4(); }
  auto bc_tile = [](int k, int& I, int& J) {  // k-th lower tile in row order
    I = 0;
    while (k > I) { k -= I + 1; ++I; }
    J = k;
  };

  // y-shaped tiles [C][PT]: wave w owns row blocks 2w, 2w+1 (NB = 8) or w (NB = 4)
  constexpr int BPW = NB / 4;          // row blocks per wave
  constexpr int YNI = PT / 16;         // column tiles
  static_assert(NB % 4 == 0, "row blocks must split evenly over 4 waves");

  for (int hh = 0; hh < HG; ++hh) {
    const int h = g * HG + hh;
    const float Ah = A[h];
    if (tid == 0) sDa[0] = 0.f;
    for (int p0 = 0; p0 < P; p0 += PT) {
      const size_t bhn = ((size_t)bb * dm.H + h) * dm.NT + n;
      // ---- A: slice inputs
      {
        constexpr int VEC = 8, PER_ROW = PT / VEC;
        for (int e = tid; e < C * PER_ROW; e += 256) {
          const int r = e / PER_ROW, c = (e % PER_ROW) * VEC;
          const size_t o = ((row0 + r) * dm.H + h) * P + p0 + c;
          float dv[8], xv[8], yv[8];
          load8(dt + o, dv);
          load8(x + o, xv);
          load8(dy + o, yv);
#pragma unroll
          for (int j = 0; j < 8; ++j) {
            sCum[r * PT + c + j] = sanitize(dv[j] * Ah, kClipDecay);
            sDbx[r * PT + c + j] = sanitize(dv[j] * xv[j]);
          }
          store8(sDy + r * L::LPT + c, yv);
        }
      }
      stage_rows<T, PT, N>(sSt, L::LN, ck.state_pre + (bhn * P + p0) * N, N);
      stage_rows<T, PT, N>(sDst, L::LN, gr.dstate + (bhn * P + p0) * N, N);
      if (tid < PT) sLastA[tid] = gr.lasta[bhn * P + p0 + tid];
      __syncthreads();
      column_cumsum<C, PT>(sCum, sTot);
      __syncthreads();
      // ---- B: dy decay_h, write, dy exp(cum - cum_{block start})
      for (int e = tid; e < C * PT; e += 256) {
        const int r = e / PT, p = e % PT;
        const float cum = sCum[r * PT + p];
        const float dyv = to_f(sDy[r * L::LPT + p]);
        sYdh[r * L::LPT + p] = from_f<T>(dyv * __expf(fminf(fmaxf(cum, -kClipDecay), 0.f)));
        const float dte = sanitize(__expf(fminf(fmaxf(sCum[(C - 1) * PT + p] - cum, -kClipDecay),
                                                kClipDecay)), 1e6f);
        sW[r * L::LPT + p] = from_f<T>(sanitize(sDbx[r * PT + p] * dte));
        sYdec[r * L::LPT + p] = from_f<T>(dyv * __expf(cum - sCum[(r & ~15) * PT + p]));
      }
      __syncthreads();
      // ---- C: y_off_raw = C state^T, dwrite = B dstate^T, dC_1 += Ydh^T-contractions, dB_1
      f32x4 yoff[BPW][YNI], dwr[BPW][YNI], ydo[BPW][YNI], dd2[BPW][YNI];
#pragma unroll
      for (int bi = 0; bi < BPW; ++bi)
#pragma unroll
        for (int ni = 0; ni < YNI; ++ni) {
          const int mi = wv_id * BPW + bi;
          yoff[bi][ni] = tile_mma<T, false, false>(zero4(), Cg, N, sSt, L::LN, 16 * mi, 16 * ni, N);
          dwr[bi][ni] = tile_mma<T, false, false>(zero4(), Bg, N, sDst, L::LN, 16 * mi, 16 * ni, N);
          ydo[bi][ni] = zero4();
          dd2[bi][ni] = zero4();
        }
#pragma unroll
      for (int t = 0; t < CPW; ++t) {
        const int tile = wv_id * CPW + t, mi = tile / MTN, ni = tile % MTN;
        acc_c1[t] = tile_mma<T, false, true>(acc_c1[t], sYdh, L::LPT, sSt, L::LN, 16 * mi, 16 * ni, PT);
        acc_b1[t] = tile_mma<T, false, true>(acc_b1[t], sW, L::LPT, sDst, L::LN, 16 * mi, 16 * ni, PT);
      }
      // ---- D: off-diagonal blocks, one output block I at a time.
      // d_cum receives every pairwise term dy_i W_ij dBx_j twice, with opposite
      // signs at i and at j (:159-163), and the reverse cumsum cancels the
      // pairs that do not straddle a row.  Both sides therefore use Z / Y
      // split into bf16 high + low parts (about 16 mantissa bits), so the two
      // copies of each term agree and the cancellation survives.
      __syncthreads();  // Ydh / W reads (dC_1, dB_1) done before Zlo / Ylo overwrite them
      for (int I = 0; I < NB; ++I) {
        const int zr = zrows<T>(I), yb = ybase<T>(I);
        for (int e = tid; e < zr * PT; e += 256) {
          const int j = e / PT, p = e % PT;
          float v = 0.f;
          if (j < 16 * I) v = __expf(sCum[16 * I * PT + p] - sCum[j * PT + p]) * sDbx[j * PT + p];
          const T hi = from_f<T>(v);
          sZ[j * L::LPT + p] = hi;
          sZlo[j * L::LPT + p] = from_f<T>(v - to_f(hi));
        }
        for (int e = tid; e < (C - yb) * PT; e += 256) {
          const int i = yb + e / PT, p = e % PT;
          float v = 0.f;
          if (i >= 16 * (I + 1))
            v = __expf(sCum[i * PT + p] - sCum[(16 * I + 15) * PT + p]) * to_f(sDy[i * L::LPT + p]);
          const T hi = from_f<T>(v);
          sY[(i - yb) * L::LPT + p] = hi;
          sYlo[(i - yb) * L::LPT + p] = from_f<T>(v - to_f(hi));
        }
        __syncthreads();
        if (I / BPW == wv_id) {
          const int bi = I % BPW;
#pragma unroll
          for (int ni = 0; ni < YNI; ++ni) {
            if (I > 0) {
              f32x4 a = tile_mma<T, false, true>(zero4(), sCB, L::LCB, sZ, L::LPT, 16 * I, 16 * ni, zr);
              ydo[bi][ni] = tile_mma<T, false, true>(a, sCB, L::LCB, sZlo, L::LPT, 16 * I, 16 * ni, zr);
            }
            if (yb < C) {
              f32x4 a = tile_mma<T, true, true>(zero4(), sCB + yb * L::LCB, L::LCB, sY, L::LPT,
                                                16 * I, 16 * ni, C - yb);
              dd2[bi][ni] = tile_mma<T, true, true>(a, sCB + yb * L::LCB, L::LCB, sYlo, L::LPT,
                                                    16 * I, 16 * ni, C - yb);
            }
          }
        }
        // dCB tiles (I, J < I): sum_p Ydec_i Z_j
#pragma unroll
        for (int s = 0; s < BCPW; ++s) {
          const int k = wv_id + 4 * s;
          if (k < NBC) {
            int TI, TJ;
            bc_tile(k, TI, TJ);
            if (TI == I && TJ < I)
              acc_bc[s] = tile_mma<T, false, false>(acc_bc[s], sYdec, L::LPT, sZ, L::LPT, 16 * TI,
                                                    16 * TJ, PT);
          }
        }
        __syncthreads();
      }
      // ---- E: diagonal blocks pairwise (reference clip masks)
#pragma unroll
      for (int s = 0; s < BCPW; ++s) {
        const int k = wv_id + 4 * s;
        if (k < NBC) {
          int TI, TJ;
          bc_tile(k, TI, TJ);
          if (TI == TJ) {
#pragma unroll
            for (int ii = 0; ii < 4; ++ii) {
              const int i = 16 * TI + tile_row(ii), j = 16 * TI + tile_col();
              if (j <= i) {
                float sum = 0.f;
                for (int p = 0; p < PT; ++p) {
                  const float dd = fminf(fmaxf(sCum[i * PT + p] - sCum[j * PT + p], -kClipDecay), kClipDecay);
                  sum += to_f(sDy[i * L::LPT + p]) * sDbx[j * PT + p] * __expf(dd);
                }
                acc_bc[s][ii] += sum;
              }
            }
          }
        }
      }
      // ---- F: per-element terms (tile layout of this wave's row blocks)
      float lastb[YNI][4];
#pragma unroll
      for (int ni = 0; ni < YNI; ++ni)
#pragma unroll
        for (int ii = 0; ii < 4; ++ii) lastb[ni][ii] = 0.f;
      float dcum_v[BPW][YNI][4], ddt1_v[BPW][YNI][4];
#pragma unroll
      for (int bi = 0; bi < BPW; ++bi) {
        const int I = wv_id * BPW + bi;
#pragma unroll
        for (int ni = 0; ni < YNI; ++ni) {
#pragma unroll
          for (int ii = 0; ii < 4; ++ii) {
            const int i = 16 * I + tile_row(ii), p = 16 * ni + tile_col();
            const float ci = sCum[i * PT + p];
            const float cl = sCum[(C - 1) * PT + p];
            const float dyi = to_f(sDy[i * L::LPT + p]);
            const float dbxi = sDbx[i * PT + p];
            // diagonal block: S1m (i as row), S2 / S2m (i as column)
            float s1m = 0.f, s2 = 0.f, s2m = 0.f;
            for (int j = 16 * I; j <= i; ++j) {
              const float dd = ci - sCum[j * PT + p];
              const float m = (dd >= -kClipDecay && dd <= kClipDecay) ? 1.f : 0.f;
              s1m += to_f(sCB[i * L::LCB + j]) * __expf(fminf(fmaxf(dd, -kClipDecay), kClipDecay)) *
                     sDbx[j * PT + p] * m;
            }
            for (int i2 = i; i2 < 16 * I + 16; ++i2) {
              const float dd = sCum[i2 * PT + p] - ci;
              const float m = (dd >= -kClipDecay && dd <= kClipDecay) ? 1.f : 0.f;
              const float v = to_f(sCB[i2 * L::LCB + i]) * __expf(fminf(fmaxf(dd, -kClipDecay), kClipDecay)) *
                              to_f(sDy[i2 * L::LPT + p]);
              s2 += v;
              s2m += v * m;
            }
            const float ydo_f = I > 0 ? ydo[bi][ni][ii] * __expf(ci - sCum[16 * I * PT + p]) : 0.f;
            const float dd2_f = ybase<T>(I) < C ? dd2[bi][ni][ii] * __expf(sCum[(16 * I + 15) * PT + p] - ci) : 0.f;
            const float dte_raw = cl - ci;
            const float dte = sanitize(__expf(fminf(fmaxf(dte_raw, -kClipDecay), kClipDecay)), 1e6f);
            const float m2 = (dte_raw >= -kClipDecay && dte_raw <= kClipDecay) ? 1.f : 0.f;
            const float dh = __expf(fminf(fmaxf(ci, -kClipDecay), 0.f));
            const float m1 = (ci >= -kClipDecay && ci <= 0.f) ? 1.f : 0.f;
            const float dw = dwr[bi][ni][ii];
            const float ddbx = sanitize(dw * dte + dd2_f + s2);          // :138,148,166
            const size_t o = ((row0 + i) * dm.H + h) * P + p0 + p;
            const float dtv = to_f(dt[o]), xv = to_f(x[o]);
            ddt1_v[bi][ni][ii] = ddbx * xv;                               // :167
            dx[o] = from_f<T>(sanitize(ddbx * dtv));                     // :168,193 + final
            const float dte_term = dw * dbxi * dte * m2;                  // d_decay_to_end_diff :142
            lastb[ni][ii] += dte_term;
            dcum_v[bi][ni][ii] = sanitize(dyi * (ydo_f + s1m) - dbxi * (dd2_f + s2m) +
                                          dyi * yoff[bi][ni][ii] * dh * m1 - dte_term);  // :162-173
          }
        }
      }
      __syncthreads();  // Ydh / W / Ydec / Z / Y are dead: reuse as fp32 scratch
#pragma unroll
      for (int bi = 0; bi < BPW; ++bi) {
        const int I = wv_id * BPW + bi;
#pragma unroll
        for (int ni = 0; ni < YNI; ++ni)
#pragma unroll
          for (int ii = 0; ii < 4; ++ii) {
            const int i = 16 * I + tile_row(ii), p = 16 * ni + tile_col();
            sRed[i * PT + p] = dcum_v[bi][ni][ii];
            sDdt1[i * PT + p] = ddt1_v[bi][ni][ii];
          }
      }
      // column sums of the decay_to_end term over this wave's rows
#pragma unroll
      for (int ni = 0; ni < YNI; ++ni) {
        float v = lastb[ni][0] + lastb[ni][1] + lastb[ni][2] + lastb[ni][3];
        v += __shfl_xor(v, 16);
        v += __shfl_xor(v, 32);
        if (lane_id() < 16) sLastB[wv_id * PT + 16 * ni + lane_id()] = v;
      }
      __syncthreads();
      if (tid < PT) {  // row C-1 extra terms (:176-177)
        const float lb = sLastB[tid] + sLastB[PT + tid] + sLastB[2 * PT + tid] + sLastB[3 * PT + tid];
        sRed[(C - 1) * PT + tid] += sLastA[tid] + lb;
      }
      __syncthreads();
      // ---- reverse cumsum over the chunk with the clip masks (:181-189)
      {
        constexpr int NSEG = 256 / PT, RS = C / NSEG;
        const int p = tid % PT, seg = tid / PT;
        float v[RS];
#pragma unroll
        for (int r = 0; r < RS; ++r) {
          const int row = seg * RS + r;
          const float cum = sCum[row * PT + p];
          v[r] = (fabsf(cum) < kClipAcc) ? sRed[row * PT + p] : 0.f;
        }
#pragma unroll
        for (int r = RS - 2; r >= 0; --r) v[r] += v[r + 1];
        sTot[seg * PT + p] = v[0];
        __syncthreads();
        float off = 0.f;
        for (int s = seg + 1; s < NSEG; ++s) off += sTot[s * PT + p];
        float da = 0.f;
#pragma unroll
        for (int r = 0; r < RS; ++r) {
          const int row = seg * RS + r;
          const size_t o = ((row0 + row) * dm.H + h) * P + p0 + p;
          const float dtv = to_f(dt[o]);
          const float araw = dtv * Ah;
          const float dA = (araw >= -kClipDecay && araw <= kClipDecay) ? (v[r] + off) : 0.f;
          ddt[o] = from_f<T>(sanitize(sDdt1[row * PT + p] + dA * Ah));   // :187,190 + final
          da += dA * dtv;
        }
        // workgroup sum of this slice's dA contribution
#pragma unroll
        for (int sh = 1; sh < 64; sh <<= 1) da += __shfl_xor(da, sh);
        __syncthreads();
        if (lane_id() == 0) sDa[1 + wv_id] = da;
        __syncthreads();
        if (tid == 0) sDa[0] += sDa[1] + sDa[2] + sDa[3] + sDa[4];
      }
      __syncthreads();
    }
    if (tid == 0) gr.dap[((size_t)bb * dm.NT + n) * dm.H + h] = sDa[0];
    __syncthreads();
  }
  // partial sums of this head group
  float* part = gr.part + ((size_t)bn * G + g) * (C * C + 2 * C * N);
#pragma unroll
  for (int s = 0; s < BCPW; ++s) {
    const int k = wv_id + 4 * s;
    if (k < NBC) {
      int TI, TJ;
      bc_tile(k, TI, TJ);
      f32x4 v = acc_bc[s];
#pragma unroll
      for (int ii = 0; ii < 4; ++ii) {
        const int i = 16 * TI + tile_row(ii), j = 16 * TJ + tile_col();
        if (j > i) v[ii] = 0.f;
      }
      store_tile_n(part, C, 16 * TI, 16 * TJ, v);
    }
  }
#pragma unroll
  for (int t = 0; t < CPW; ++t) {
    const int tile = wv_id * CPW + t, mi = tile / MTN, ni = tile % MTN;
    store_tile_n(part + C * C, N, 16 * mi, 16 * ni, acc_c1[t]);
    store_tile_n(part + C * C + C * N, N, 16 * mi, 16 * ni, acc_b1[t]);
  }
}

// ------------------------------------------------------------------ dB, dC
template <typename T, int C, int N>
__global__ __launch_bounds__(256) void mamba2_bwd_bc(Mamba2Dims dm, int G, const T* __restrict__ Bm,
                                                    const T* __restrict__ Cm, Mamba2Grads<T> gr,
                                                    T* __restrict__ dB, T* __restrict__ dC) {
  constexpr int PAD = Pad<T>::v, LN = N + PAD, LCB = C + PAD;
  __shared__ __attribute__((aligned(16))) T sB[C * LN];
  __shared__ __attribute__((aligned(16))) T sC[C * LN];
  __shared__ __attribute__((aligned(16))) T sD[C * LCB];
  const int bn = blockIdx.x;
  const size_t row0 = (size_t)bn * C;
  stage_rows<T, C, N>(sB, LN, Bm + row0 * N, N);
  stage_rows<T, C, N>(sC, LN, Cm + row0 * N, N);
  const size_t stride = (size_t)C * C + 2 * (size_t)C * N;
  const float* part = gr.part + (size_t)bn * G * stride;
  for (int e = threadIdx.x; e < C * C; e += 256) {
    const int i = e / C, j = e % C;
    float s = 0.f;
    if (j <= i)
      for (int gg = 0; gg < G; ++gg) s += part[gg * stride + e];
    sD[i * LCB + j] = from_f<T>(s);
  }
  __syncthreads();
  constexpr int MT = C / 16, NTN = N / 16;
  const int wv = wave_id();
  for (int tile = wv; tile < MT * NTN; tile += 4) {
    const int mi = tile / NTN, ni = tile % NTN;
    // dC = sanitize(dC_1 + dCB B)    dB = sanitize(dB_1 + dCB^T C)
    f32x4 c = tile_mma<T, false, true>(zero4(), sD, LCB, sB, LN, 16 * mi, 16 * ni, C);
    f32x4 b = tile_mma<T, true, true>(zero4(), sD, LCB, sC, LN, 16 * mi, 16 * ni, C);
#pragma unroll
    for (int ii = 0; ii < 4; ++ii) {
      const int r = 16 * mi + tile_row(ii), s = 16 * ni + tile_col();
      float c1 = 0.f, b1 = 0.f;
      for (int gg = 0; gg < G; ++gg) {
        c1 += part[gg * stride + C * C + r * N + s];
        b1 += part[gg * stride + C * C + C * N + r * N + s];
      }
      dC[(row0 + r) * N + s] = from_f<T>(sanitize(c1 + c[ii]));
      dB[(row0 + r) * N + s] = from_f<T>(sanitize(b1 + b[ii]));
    }
  }
}

// dA[h] = sanitize(sum_n sanitize(sum_b dap[b][n][h]))
__global__ __launch_bounds__(256) void mamba2_bwd_da(Mamba2Dims dm, const float* __restrict__ dap,
                                                    float* __restrict__ dA) {
  for (int h = threadIdx.x; h < dm.H; h += 256) {
    float tot = 0.f;
    for (int n = 0; n < dm.NT; ++n) {
      float s = 0.f;
      for (int b = 0; b < dm.B; ++b) s += dap[((size_t)b * dm.NT + n) * dm.H + h];
      tot += sanitize(s);
    }
    dA[h] = sanitize(tot);
  }
}

}  // namespace ah
