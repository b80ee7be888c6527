// Mamba2 SSD chunk-scan backward for gfx950, with the semantics of the
// hand-derived MB0 backward (atomic_ops/mamba2_bwd_reference.py:55-266):
// every clip contributes a straight-through mask (:48-52) and the per-chunk
// sanitising of :166-195 is kept.
//
// mamba2_chunk_outer<BWD>  (mamba2_fwd.hip) per (batch, chunk, head, slice):
//                    (dy decay_h)^T C, and the operands Ydh, W of dC_1, dB_1.
// mamba2_state_pass<BWD>   (mamba2_fwd.hip) reverse elementwise dstate carry
//                    and the decay_chunk_end row term d_cum_last_a.
// mamba2_bwd_chunk   one workgroup per (batch, chunk, head group): every
//                    per-head term of :123-190 for each head and 32-channel
//                    slice, with the cross-head sum dCB (:147-152) accumulated
//                    in registers.  The pairwise decay of the off-diagonal
//                    16-row blocks is factorised as in the forward; diagonal
//                    blocks are evaluated pairwise with the reference's clip
//                    masks.
// mamba2_bwd_bc      one workgroup per (batch, chunk, 32 state columns):
//                    dC = dC_1 + dCB B and dB = dB_1 + dCB^T C (:127,135,
//                    :154-156,191-192) with dC_1 = Ydh . state_prev and
//                    dB_1 = W . dstate contracted over (head, channel).
// mamba2_bwd_da      dA = sum over chunks of sanitize(sum over batch) (:188,194,263).
#include "mamba2_fwd.hip"

namespace ah {

template <typename T>
struct Mamba2Grads {
  T* dstate;     // [B][NT][H][P][N]  dstate_new of each chunk (the carry its backward starts from)
  float* lasta;  // [B][NT][H][P]     d cum_last through decay_chunk_end
  T* ydh;        // [B][T][H][P]      dy decay_h
  T* wr;         // [B][T][H][P]      sanitize(dBx decay_to_end)
  float* part;   // [B][NT][G][C*C]   dCB summed over the heads of each group
  float* dap;    // [B][NT][H]        per (batch, chunk, head) dA contribution
};

// ------------------------------------------------------------------ per-chunk gradients
// Rows of the block-I operand Z^(I) (source rows j < 16 I, padded to the MFMA k step).
template <typename T>
__host__ __device__ constexpr int zrows(int I) {
  return ((16 * I + Mma<T>::KS - 1) / Mma<T>::KS) * Mma<T>::KS;
}
// Y^(I) rows start at the MFMA k step at or below 16 (I + 1).
template <typename T>
__host__ __device__ constexpr int ybase(int I) {
  return (16 * (I + 1) / Mma<T>::KS) * Mma<T>::KS;
}

template <typename T, int C, int N, int PT>
struct CkLds {
  static constexpr int PAD = Pad<T>::v;
  static constexpr int LCB = C + PAD, LN = N + PAD, LPT = PT + PAD;
  static constexpr int LC = PT + 1;  // fp32 [C][PT] rows, padded against bank conflicts
  static constexpr int NSEG = 256 / PT;
  static constexpr int OPT = C * LPT * (int)sizeof(T);
  static constexpr int off_cb = 0;
  static constexpr int off_st = off_cb + C * LCB * (int)sizeof(T);
  static constexpr int off_dst = off_st + PT * LN * (int)sizeof(T);
  static constexpr int off_dy = off_dst + PT * LN * (int)sizeof(T);
  static constexpr int off_zlo = off_dy + OPT;   // then fp32 ddt_1 (with off_ylo)
  static constexpr int off_ylo = off_zlo + OPT;
  static constexpr int off_ydec = off_ylo + OPT;  // then fp32 d_cum (with off_z, off_y)
  static constexpr int off_z = off_ydec + OPT;
  static constexpr int off_y = off_z + OPT;
  static constexpr int off_cum = off_y + OPT;
  static constexpr int off_dbx = off_cum + C * LC * 4;
  static constexpr int off_tot = off_dbx + C * LC * 4;
  static constexpr int off_misc = off_tot + NSEG * PT * 4;   // lasta[PT], lastb[4][PT], dA[8]
  static constexpr int total = off_misc + (PT + 4 * PT + 8) * 4;
  static_assert(2 * OPT >= C * LC * 4 && 3 * OPT >= C * LC * 4, "fp32 aliases must fit");
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
  // LDS views; rebuilt from an opaque base at every (head, slice) iteration so
  // the compiler cannot hoist the hundreds of per-lane addresses of the
  // unrolled loop bodies out of the iteration loop (that hoisting spilled them).
  T *sCB, *sSt, *sDst, *sDy, *sYdec, *sZ, *sY, *sZlo, *sYlo;
  float *sCum, *sDbx, *sTot, *sLastA, *sLastB, *sDa, *sDdt1, *sRed;
  auto views = [&](int z) {
    unsigned char* lb = lds + z;
    sCB = reinterpret_cast<T*>(lb + L::off_cb);
    sSt = reinterpret_cast<T*>(lb + L::off_st);
    sDst = reinterpret_cast<T*>(lb + L::off_dst);
    sDy = reinterpret_cast<T*>(lb + L::off_dy);
    sYdec = reinterpret_cast<T*>(lb + L::off_ydec);
    sZ = reinterpret_cast<T*>(lb + L::off_z);
    sY = reinterpret_cast<T*>(lb + L::off_y);
    sCum = reinterpret_cast<float*>(lb + L::off_cum);
    sDbx = reinterpret_cast<float*>(lb + L::off_dbx);
    sTot = reinterpret_cast<float*>(lb + L::off_tot);
    sLastA = reinterpret_cast<float*>(lb + L::off_misc);
    sLastB = sLastA + PT;
    sDa = sLastB + 4 * PT;
    // low halves of the split Z / Y operands
    sZlo = reinterpret_cast<T*>(lb + L::off_zlo);
    sYlo = reinterpret_cast<T*>(lb + L::off_ylo);
    sDdt1 = reinterpret_cast<float*>(lb + L::off_zlo);  // aliases Zlo + Ylo in the epilogue
    sRed = reinterpret_cast<float*>(lb + L::off_ydec);  // aliases Ydec + Z + Y in the epilogue
  };
  views(0);

  const int tid = threadIdx.x;
  const int g = blockIdx.x % G;
  const int bn = blockIdx.x / G;
  const int bb = bn / dm.NT, n = bn % dm.NT;
  const int HG = dm.H / G;
  const int wv_id = wave_id();
  const size_t row0 = (size_t)bb * dm.T + (size_t)n * C;
  const size_t rsx = (size_t)dm.H * P;
  const T* Bg0 = Bm + row0 * N;
  const T* Cg0 = Cm + row0 * N;
  constexpr int NB = C / 16;

  stage_rows<T, C, C>(sCB, L::LCB, ck.cb + (size_t)bn * C * C, C);

  // cross-head accumulator: dCB lower tiles (I >= J)
  constexpr int NBC = NB * (NB + 1) / 2;
  constexpr int BCPW = (NBC + 3) / 4;
  f32x4 acc_bc[BCPW];
#pragma unroll
  for (int i = 0; i < BCPW; ++i) acc_bc[i] = zero4();
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
      const int z = opaque_zero();
      views(z);
      const T* Bg = Bg0 + z;
      const T* Cg = Cg0 + z;
      const size_t bnh = (size_t)bn * dm.H + h;
      // ---- A: slice inputs
      int pos = 0;
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
            pos |= dv[j] * Ah > 0.f;
            sCum[r * L::LC + c + j] = sanitize(dv[j] * Ah, kClipDecay);
            sDbx[r * L::LC + c + j] = sanitize(dv[j] * xv[j]);
          }
          store8(sDy + r * L::LPT + c, yv);
        }
      }
      stage_rows<T, PT, N>(sSt, L::LN, ck.state_pre + (bnh * P + p0) * N, N);
      stage_rows<T, PT, N>(sDst, L::LN, gr.dstate + (bnh * P + p0) * N, N);
      if (tid < PT) sLastA[tid] = gr.lasta[bnh * P + p0 + tid];
      // a slice with a positive step exponent is evaluated pairwise everywhere
      const bool exact = __syncthreads_or(pos);
      column_cumsum<C, PT, L::LC>(sCum, sTot);
      __syncthreads();
      // ---- B: dy exp(cum - cum_{block start})
      for (int e = tid; e < C * PT; e += 256) {
        const int r = e / PT, p = e % PT;
        const float cum = sCum[r * L::LC + p];
        const float dyv = to_f(sDy[r * L::LPT + p]);
        sYdec[r * L::LPT + p] = from_f<T>(dyv * __expf(cum - sCum[(r & ~15) * L::LC + p]));
      }
      __syncthreads();
      f32x4 ydo[BPW][YNI], dd2[BPW][YNI];
#pragma unroll
      for (int bi = 0; bi < BPW; ++bi)
#pragma unroll
        for (int ni = 0; ni < YNI; ++ni) {
          ydo[bi][ni] = zero4();
          dd2[bi][ni] = zero4();
        }
      // ---- D: off-diagonal blocks, one output block I at a time.
      // d_cum receives every pairwise term dy_i W_ij dBx_j twice, with opposite
      // signs at i and at j (:159-163), and the reverse cumsum cancels the
      // pairs that do not straddle a row.  Both sides therefore use Z / Y
      // split into bf16 high + low parts (about 16 mantissa bits), so the two
      // copies of each term agree and the cancellation survives.
      for (int I = 0; I < (exact ? 0 : NB); ++I) {
        const int zr = zrows<T>(I), yb = ybase<T>(I);
        for (int e = tid; e < zr * PT; e += 256) {
          const int j = e / PT, p = e % PT;
          float v = 0.f;
          if (j < 16 * I) v = __expf(sCum[16 * I * L::LC + p] - sCum[j * L::LC + p]) * sDbx[j * L::LC + p];
          const T hi = from_f<T>(v);
          sZ[j * L::LPT + p] = hi;
          sZlo[j * L::LPT + p] = from_f<T>(v - to_f(hi));
        }
        for (int e = tid; e < (C - yb) * PT; e += 256) {
          const int i = yb + e / PT, p = e % PT;
          float v = 0.f;
          if (i >= 16 * (I + 1))
            v = __expf(sCum[i * L::LC + p] - sCum[(16 * I + 15) * L::LC + p]) * to_f(sDy[i * L::LPT + p]);
          const T hi = from_f<T>(v);
          sY[(i - yb) * L::LPT + p] = hi;
          sYlo[(i - yb) * L::LPT + p] = from_f<T>(v - to_f(hi));
        }
        __syncthreads();
        if (I / BPW == wv_id) {
          const int bi = I % BPW;
#pragma unroll
          for (int ni = 0; ni < YNI; ++ni) {
            f32x4 r1 = zero4(), r2 = zero4();
            if (I > 0) {
              r1 = tile_mma<T, false, true>(r1, sCB, L::LCB, sZ, L::LPT, 16 * I, 16 * ni, zr);
              r1 = tile_mma<T, false, true>(r1, sCB, L::LCB, sZlo, L::LPT, 16 * I, 16 * ni, zr);
            }
            if (yb < C) {
              r2 = tile_mma<T, true, true>(r2, sCB + yb * L::LCB, L::LCB, sY, L::LPT, 16 * I, 16 * ni,
                                           C - yb);
              r2 = tile_mma<T, true, true>(r2, sCB + yb * L::LCB, L::LCB, sYlo, L::LPT, 16 * I,
                                           16 * ni, C - yb);
            }
            // static register indices (a runtime index would put the arrays in scratch)
#pragma unroll
            for (int b2 = 0; b2 < BPW; ++b2)
              if (b2 == bi) { ydo[b2][ni] = r1; dd2[b2][ni] = r2; }
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
      // ---- E: diagonal blocks (every lower block on the exact path) pairwise
#pragma unroll
      for (int s = 0; s < BCPW; ++s) {
        const int k = wv_id + 4 * s;
        if (k < NBC) {
          int TI, TJ;
          bc_tile(k, TI, TJ);
          if (TI == TJ || exact) {
#pragma unroll
            for (int ii = 0; ii < 4; ++ii) {
              const int i = 16 * TI + tile_row(ii), j = 16 * TJ + tile_col();
              if (j <= i) {
                float sum = 0.f;
#pragma unroll 4
                for (int p = 0; p < PT; ++p) {
                  const float dd = fminf(fmaxf(sCum[i * L::LC + p] - sCum[j * L::LC + p], -kClipDecay), kClipDecay);
                  sum += to_f(sDy[i * L::LPT + p]) * sDbx[j * L::LC + p] * fminf(__expf(dd), 1e6f);
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
          // y_off_raw = C state^T and dwrite = B dstate^T for this tile (:126,134)
          const f32x4 yoff = tile_mma<T, false, false>(zero4(), Cg, N, sSt, L::LN, 16 * I, 16 * ni, N);
          const f32x4 dwr = tile_mma<T, false, false>(zero4(), Bg, N, sDst, L::LN, 16 * I, 16 * ni, N);
#pragma unroll
          for (int ii = 0; ii < 4; ++ii) {
            const int i = 16 * I + tile_row(ii), p = 16 * ni + tile_col();
            const float ci = sCum[i * L::LC + p];
            const float cl = sCum[(C - 1) * L::LC + p];
            const float dyi = to_f(sDy[i * L::LPT + p]);
            const float dbxi = sDbx[i * L::LC + p];
            // pairwise part (the diagonal block, or every pair on the exact
            // path): S1m (i as row), S2 / S2m (i as column)
            float s1m = 0.f, s2 = 0.f, s2m = 0.f;
            for (int j = exact ? 0 : 16 * I; j <= i; ++j) {
              const float dd = ci - sCum[j * L::LC + p];
              const float m = (dd >= -kClipDecay && dd <= kClipDecay) ? 1.f : 0.f;
              s1m += to_f(sCB[i * L::LCB + j]) *
                     fminf(__expf(fminf(fmaxf(dd, -kClipDecay), kClipDecay)), 1e6f) * sDbx[j * L::LC + p] * m;
            }
            for (int i2 = i; i2 < (exact ? C : 16 * I + 16); ++i2) {
              const float dd = sCum[i2 * L::LC + p] - ci;
              const float m = (dd >= -kClipDecay && dd <= kClipDecay) ? 1.f : 0.f;
              const float v = to_f(sCB[i2 * L::LCB + i]) *
                              fminf(__expf(fminf(fmaxf(dd, -kClipDecay), kClipDecay)), 1e6f) *
                              to_f(sDy[i2 * L::LPT + p]);
              s2 += v;
              s2m += v * m;
            }
            const float ydo_f =
                (!exact && I > 0) ? ydo[bi][ni][ii] * __expf(ci - sCum[16 * I * L::LC + p]) : 0.f;
            const float dd2_f = (!exact && ybase<T>(I) < C)
                                    ? dd2[bi][ni][ii] * __expf(sCum[(16 * I + 15) * L::LC + p] - ci)
                                    : 0.f;
            const float dte_raw = cl - ci;
            const float dte = sanitize(__expf(fminf(fmaxf(dte_raw, -kClipDecay), kClipDecay)), 1e6f);
            const float m2 = (dte_raw >= -kClipDecay && dte_raw <= kClipDecay) ? 1.f : 0.f;
            const float dh = __expf(fminf(fmaxf(ci, -kClipDecay), 0.f));
            const float m1 = (ci >= -kClipDecay && ci <= 0.f) ? 1.f : 0.f;
            const float dw = dwr[ii];
            const float ddbx = sanitize(dw * dte + dd2_f + s2);          // :138,148,166
            const size_t o = ((row0 + i) * dm.H + h) * P + p0 + p;
            const float dtv = to_f(dt[o]), xv = to_f(x[o]);
            ddt1_v[bi][ni][ii] = ddbx * xv;                               // :167
            dx[o] = from_f<T>(sanitize(ddbx * dtv));                     // :168,193 + final
            const float dte_term = dw * dbxi * dte * m2;                  // d_decay_to_end_diff :142
            lastb[ni][ii] += dte_term;
            dcum_v[bi][ni][ii] = sanitize(dyi * (ydo_f + s1m) - dbxi * (dd2_f + s2m) +
                                          dyi * yoff[ii] * dh * m1 - dte_term);  // :162-173
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
            sRed[i * L::LC + p] = dcum_v[bi][ni][ii];
            sDdt1[i * L::LC + p] = ddt1_v[bi][ni][ii];
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
        sRed[(C - 1) * L::LC + tid] += sLastA[tid] + lb;
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
          const float cum = sCum[row * L::LC + p];
          v[r] = (fabsf(cum) < kClipAcc) ? sRed[row * L::LC + p] : 0.f;
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
          ddt[o] = from_f<T>(sanitize(sDdt1[row * L::LC + p] + dA * Ah));   // :187,190 + final
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
    if (tid == 0) gr.dap[(size_t)bn * dm.H + h] = sDa[0];
    __syncthreads();
  }
  // partial sums of this head group
  float* part = gr.part + ((size_t)bn * G + g) * C * C;
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
}

// ------------------------------------------------------------------ dB, dC
template <typename T, int C, int NTL, int KB>
struct BcLds {
  static constexpr int PAD = Pad<T>::v;
  static constexpr int LCB = C + PAD, LK = NTL + PAD;
  static constexpr int off_s = 0;                                   // state_prev rows [KB][NTL]
  static constexpr int off_d = off_s + KB * LK * (int)sizeof(T);    // dstate rows [KB][NTL]
  static constexpr int off_cb = off_d + KB * LK * (int)sizeof(T);   // dCB [C][C]
  static constexpr int off_b = off_cb + C * LCB * (int)sizeof(T);   // B [C][NTL]
  static constexpr int off_c = off_b + C * LK * (int)sizeof(T);     // C [C][NTL]
  static constexpr int total = off_c + C * LK * (int)sizeof(T);
};

// One workgroup per (batch, chunk, NTL state columns):
//   dC = sanitize(Ydh . state_prev + dCB B)     dB = sanitize(W . dstate + dCB^T C)
// the first terms contracted over k = (head, channel): Ydh / W rows are the
// [B][T][H][P] rows of the chunk, state_prev / dstate the [NT][H][P][N] block.
template <typename T, int C, int P, int N>
__global__ __launch_bounds__(256) void mamba2_bwd_bc(Mamba2Dims dm, int G, const T* __restrict__ Bm,
                                                    const T* __restrict__ Cm, Mamba2Chunks<T> ck,
                                                    Mamba2Grads<T> gr, T* __restrict__ dB,
                                                    T* __restrict__ dC) {
  constexpr int NTL = 32, KB = 64, NNT = N / NTL;
  typedef BcLds<T, C, NTL, KB> L;
  __shared__ __attribute__((aligned(16))) unsigned char lds[L::total];
  T* sS = reinterpret_cast<T*>(lds + L::off_s);
  T* sD = reinterpret_cast<T*>(lds + L::off_d);
  T* sCB = reinterpret_cast<T*>(lds + L::off_cb);
  T* sB = reinterpret_cast<T*>(lds + L::off_b);
  T* sC = reinterpret_cast<T*>(lds + L::off_c);

  int bn, nt;
  xcd_group_map(blockIdx.x, dm.B * dm.NT, NNT, bn, nt);
  const int n0 = nt * NTL;
  const size_t row0 = (size_t)bn * C;  // rows of [B*T][...]
  const int HP = dm.H * P;
  const T* yg = gr.ydh + row0 * HP;
  const T* wg = gr.wr + row0 * HP;
  const T* sg = ck.state_pre + (size_t)bn * HP * N + n0;
  const T* dg = gr.dstate + (size_t)bn * HP * N + n0;

  stage_rows<T, C, NTL>(sB, L::LK, Bm + row0 * N + n0, N);
  stage_rows<T, C, NTL>(sC, L::LK, Cm + row0 * N + n0, N);
  const float* part = gr.part + (size_t)bn * G * C * C;
  for (int e = threadIdx.x; e < C * C; e += 256) {
    const int i = e / C, j = e % C;
    float s = 0.f;
    if (j <= i)
      for (int gg = 0; gg < G; ++gg) s += part[(size_t)gg * C * C + e];
    sCB[i * L::LCB + j] = from_f<T>(s);
  }

  constexpr int RT = C / 64, CT = NTL / 16;  // row tiles per wave, column tiles
  const int wv_id = wave_id();
  f32x4 accC[RT][CT], accB[RT][CT];
#pragma unroll
  for (int rt = 0; rt < RT; ++rt)
#pragma unroll
    for (int ct = 0; ct < CT; ++ct) { accC[rt][ct] = zero4(); accB[rt][ct] = zero4(); }

  RegStage<T, KB, NTL> ps, pd;
  ps.load(sg, N);
  pd.load(dg, N);
  for (int kb = 0; kb < HP; kb += KB) {
    __syncthreads();  // previous block's reads done
    ps.store(sS, L::LK);
    pd.store(sD, L::LK);
    if (kb + KB < HP) {
      ps.load(sg + (size_t)(kb + KB) * N, N);
      pd.load(dg + (size_t)(kb + KB) * N, N);
    }
    __syncthreads();
#pragma unroll
    for (int kk = 0; kk < KB; kk += Mma<T>::KS) {
#pragma unroll
      for (int rt = 0; rt < RT; ++rt) {
        const int m0 = 16 * (RT * wv_id + rt);
        const typename Mma<T>::frag ay = Mma<T>::ld_c(yg, HP, m0, kb + kk);
        const typename Mma<T>::frag aw = Mma<T>::ld_c(wg, HP, m0, kb + kk);
#pragma unroll
        for (int ct = 0; ct < CT; ++ct) {
          accC[rt][ct] = Mma<T>::mma(ay, Mma<T>::ld_t(sS, L::LK, 16 * ct, kk), accC[rt][ct]);
          accB[rt][ct] = Mma<T>::mma(aw, Mma<T>::ld_t(sD, L::LK, 16 * ct, kk), accB[rt][ct]);
        }
      }
    }
  }
  T* dCo = dC + row0 * N + n0;
  T* dBo = dB + row0 * N + n0;
#pragma unroll
  for (int rt = 0; rt < RT; ++rt)
#pragma unroll
    for (int ct = 0; ct < CT; ++ct) {
      const int m0 = 16 * (RT * wv_id + rt);
      f32x4 c = tile_mma<T, false, true>(accC[rt][ct], sCB, L::LCB, sB, L::LK, m0, 16 * ct, C);
      f32x4 b = tile_mma<T, true, true>(accB[rt][ct], sCB, L::LCB, sC, L::LK, m0, 16 * ct, C);
#pragma unroll
      for (int k = 0; k < 4; ++k) { c[k] = sanitize(c[k]); b[k] = sanitize(b[k]); }
      store_tile_n(dCo, N, m0, 16 * ct, c);
      store_tile_n(dBo, N, m0, 16 * ct, b);
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
