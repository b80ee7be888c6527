// Mamba2 SSD chunk-scan backward for gfx950, with the semantics of the
// hand-derived MB0 backward (atomic_ops/mamba2_bwd_reference.py:55-266):
// every clip contributes a straight-through mask (:48-52) and the per-chunk
// sanitising of :166-195 is kept.
//
// mamba2_chunk_outer<BWD>  (mamba2_fwd.hip) per (batch, chunk, head, slice):
//                    Ydh = dy decay_h and W, the operands of the carry's
//                    (dy decay_h)^T C and of dC_1, dB_1.
// mamba2_state_chain<BWD>  (mamba2_seq.hpp) the reverse dstate carry, its
//                    (dy decay_h)^T C on MFMA, and the decay_chunk_end row
//                    term d_cum_last_a.
// mamba2_bwd_chunk   one workgroup (8 waves) per (batch, chunk, head group):
//                    every per-head term of :123-190 for each head and
//                    32-channel slice, with the cross-head sum dCB (:147-152)
//                    accumulated in registers.  The pairwise decay is
//                    factorised on 16-row blocks (below); slices outside the
//                    factorisation's bounds are evaluated pairwise with the
//                    reference's clip masks.
// mamba2_bwd_bc      one workgroup per (batch, chunk, 64 state columns):
//                    dC = dC_1 + dCB B and dB = dB_1 + dCB^T C (:127,135,
//                    :154-156,191-192) with dC_1 = Ydh . state_prev and
//                    dB_1 = W . dstate contracted over (head, channel).
//                    Its first H workgroups also reduce dA = sum over chunks
//                    of sanitize(sum over batch) (:188,194,263).
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
// The pair sums of the chunk, for channel p and rows i, j of the chunk:
//   R_i   = sum_{j<=i} CB_ij exp(cum_i - cum_j) dBx_j     (row side; d_cum_i, :162)
//   S_j   = sum_{i>=j} CB_ij exp(cum_i - cum_j) dy_i      (column side; d_dBx_2, :148; d_cum_j, :163)
//   dCB_ij += sum_p dy_i exp(cum_i - cum_j) dBx_j         (cross-head, :152)
// On 16-row blocks I (rows 16I..16I+15) the decay factorises into
//   U_i = exp(cum_i - cum_{16I}),  M_IJ = exp(cum_{16I} - cum_{16J+15}),
//   V_j = exp(cum_{16J+15} - cum_j),
// all <= 1 when dt A <= 0, and inside a diagonal block into U_i and
// exp(cum_{16I} - cum_j) <= exp(range_I), range_I = cum_{16I} - cum_{16I+15}.
// Every pair is then an MFMA on Yu = dy U or Vd = V dBx with per-channel
// scales; the two copies of each pair term in d_cum (row and column side)
// use Yu / Vd split into bf16 high + low parts so the reverse cumsum's
// cancellation survives.  Masks |cum_i - cum_j| <= 20 and the exp(-20) floor
// change only pairs whose weight is below exp(-20) (a relative 2e-9).
// A slice with a positive step exponent or a block range above kMaxRange is
// evaluated pairwise with the reference's clips and masks instead.

// The pair sums take one K = 32 MFMA per 16-row block: the A fragment holds
// the 16 x 16 CB block twice along K, the B fragment the block's 16 rows of
// the high part and then of the low part, so hi and lo are summed in the MFMA.
// The A fragments come from the chunk's CB staged in LDS (row pitch ld):
// CB(m0.., k0..) for the row side, CB^T(m0.., k0..) by a transposed read for
// the column side.  The staged CB has its strict upper triangle zeroed, so a
// diagonal block reads as its lower triangle (row side) and the transpose of
// it (column side) with no per-element masks.
template <typename T>
__device__ __forceinline__ typename Mma<T>::frag cb_lds_dup(const T* s, int ld, int m0, int k0, bool transposed) {
  typedef typename Mma<T>::frag frag;
  const int l = lane_id(), m = l & 15, g2 = l >> 5, kb = 8 * ((l >> 4) & 1);
  return transposed ? Mma<T>::ld_t(s, ld, m0, k0 - 16 * g2)
                    : *reinterpret_cast<const frag*>(s + (m0 + m) * ld + k0 + kb);
}
template <typename T>
__device__ __forceinline__ typename Mma<T>::frag ld_t_hilo(const T* hi, const T* lo, int ld, int i0, int k0) {
  const int g2 = lane_id() >> 5;  // lanes 32..63 hold K rows 16..31
  return Mma<T>::ld_t(g2 ? lo : hi, ld, i0, k0 - 16 * g2);
}

// Rows r0 + 4g .. r0 + 4g + 3 of column c0 + (lane % 16) of a row-major bf16
// LDS array (row pitch ld), g = lane / 16: the MFMA result-tile layout's four
// elements of a lane, in one transposed read (ds_read_b64_tr_b16: lane s of a
// 16-lane group points at row r0 + 4g + s / 4, columns c0 + 4 (s % 4) ..;
// lane j receives column c0 + j of the four rows).
__device__ __forceinline__ bf16x4 tile_rows4(const bf16* p, int ld, int r0, int c0) {
  const int l = lane_id(), s = l & 15, g = l >> 4;
  typedef __attribute__((address_space(3))) bf16x4* lds_p;
  return __builtin_amdgcn_ds_read_tr16_b64_v4bf16((lds_p)(p + (r0 + 4 * g + (s >> 2)) * ld + c0 + 4 * (s & 3)));
}

template <typename T, int C, int N, int PT, int NTH>
struct CkLds {
  static constexpr int PAD = Pad<T>::v;
  // state_pre / dstate rows and the CB rows padded by 32 bytes: the y_off /
  // dwrite and pair-sum fragment reads of 16 rows then spread over the banks
  // (SQ_LDS_BANK_CONFLICT 3.07e7 -> 1.99e7 per launch against 16-byte pads;
  // the [C][PT] operand rows keep 16 bytes, which the LDS budget needs)
  static constexpr int LN = N + 2 * PAD, LPT = PT + PAD;
  // fp32 [C][PT] rows: 16-byte aligned, and rows 4 apart land 16 banks apart
  // (the MFMA tile layout reads 4 row groups x 16 columns)
  static constexpr int LC = PT + 4;
  static constexpr int NW = NTH / 64;
  static constexpr int NSEG = NTH / PT;
  static constexpr int OPT = C * LPT * (int)sizeof(T);
  static constexpr int OPR = C * LPT * (int)sizeof(T);  // MFMA operand
  static constexpr int off_st = 0;
  static constexpr int off_dst = off_st + PT * LN * (int)sizeof(T);
  static constexpr int off_dy = off_dst + PT * LN * (int)sizeof(T);
  static constexpr int off_dt = off_dy + OPT;
  static constexpr int off_x = off_dt + OPT;
  static constexpr int off_yu = off_x + OPT;  // Yu hi, Yu lo, Vd hi, Vd lo
  static constexpr int off_yul = off_yu + OPR;
  static constexpr int off_vd = off_yul + OPR;
  static constexpr int off_vdl = off_vd + OPR;
  static constexpr int off_cum = off_vdl + OPR;
  static constexpr int off_tot = off_cum + C * LC * 4;  // column / block totals
  static_assert(NSEG >= C / 16, "the block totals reuse the column-scan totals");
  static constexpr int off_misc = off_tot + NSEG * PT * 4;   // lasta[PT], lastb[NW][PT], dA[1 + NW]
  static constexpr int LCB = C + 2 * PAD;
  static constexpr int off_cb = (off_misc + (PT + NW * PT + 1 + NW) * 4 + 15) / 16 * 16;  // CB [C][LCB]
  static constexpr int off_m = off_cb + C * LCB * (int)sizeof(T);
  static_assert(off_cb % 16 == 0 && off_m % 16 == 0, "16-byte LDS accesses");
  // M_IJ[p] = exp(cum_{16I} - cum_{16J+15}) for the 16-row block pairs I >= J
  static constexpr int total = off_m + (C / 16) * (C / 16 + 1) / 2 * PT * 4;
};

// 512 threads: eight waves, two per SIMD, so one wave's LDS / global / MFMA
// latency overlaps the other's work; wave w owns one 16-row block.
template <typename T, typename TD, int C, int P, int N>
__global__ __launch_bounds__(512) __attribute__((amdgpu_waves_per_eu(2, 2))) void mamba2_bwd_chunk(
    Mamba2Dims dm, int G, const T* __restrict__ dt, const T* __restrict__ x,
    const float* __restrict__ A, const T* __restrict__ Bm, const T* __restrict__ Cm,
    const TD* __restrict__ dy, Mamba2Chunks<T> ck, Mamba2Grads<T> gr, T* __restrict__ ddt,
    T* __restrict__ dx) {
  constexpr int PT = 32, NTH = 512, NW = NTH / 64;
  typedef CkLds<T, C, N, PT, NTH> L;
  typedef typename Mma<T>::frag frag;
  __shared__ __attribute__((aligned(16))) unsigned char lds[L::total];
  // LDS views; rebuilt from an opaque base at every (head, slice) iteration so
  // the compiler cannot hoist the hundreds of per-lane addresses of the
  // unrolled loop bodies out of the iteration loop (that hoisting spilled them).
  T *sSt, *sDst, *sDy, *sDt, *sX, *sYu, *sYul, *sVd, *sVdl;
  float *sCum, *sTot, *sLastA, *sLastB, *sDa, *sM;
  T* sCB;
  auto views = [&](int z) {
    unsigned char* lb = lds + z;
    sSt = reinterpret_cast<T*>(lb + L::off_st);
    sDst = reinterpret_cast<T*>(lb + L::off_dst);
    sDy = reinterpret_cast<T*>(lb + L::off_dy);
    sDt = reinterpret_cast<T*>(lb + L::off_dt);
    sX = reinterpret_cast<T*>(lb + L::off_x);
    sYu = reinterpret_cast<T*>(lb + L::off_yu);
    sYul = reinterpret_cast<T*>(lb + L::off_yul);
    sVd = reinterpret_cast<T*>(lb + L::off_vd);
    sVdl = reinterpret_cast<T*>(lb + L::off_vdl);
    sCum = reinterpret_cast<float*>(lb + L::off_cum);
    sTot = reinterpret_cast<float*>(lb + L::off_tot);
    sLastA = reinterpret_cast<float*>(lb + L::off_misc);
    sLastB = sLastA + PT;
    sDa = sLastB + NW * PT;
    sM = reinterpret_cast<float*>(lb + L::off_m);
    sCB = reinterpret_cast<T*>(lb + L::off_cb);
  };
  views(0);

  const int tid = threadIdx.x;
  // the G head groups of one (batch, chunk) share an XCD (and its L2) for CB, B, C
  int bn, g;
  xcd_group_map(blockIdx.x, dm.B * dm.NT, G, bn, g);
  const int bb = bn / dm.NT, n = bn % dm.NT;
  const int HG = dm.H / G;
  const int wv_id = wave_id();
  const size_t row0 = (size_t)bb * dm.T + (size_t)n * C;
  const T* Bg0 = Bm + row0 * dm.rB;
  const T* Cg0 = Cm + row0 * dm.rC;
  const int ldb = (int)dm.rB, ldc = (int)dm.rC;
  const T* cb0 = ck.cb + (size_t)bn * C * C;
  constexpr int NB = C / 16;

  // cross-head accumulator: dCB lower tiles (I >= J), tile k of wave w = w + NW s
  constexpr int NBC = NB * (NB + 1) / 2;
  constexpr int BCPW = (NBC + NW - 1) / NW;
  f32x4 acc_bc[BCPW];
#pragma unroll
  for (int i = 0; i < BCPW; ++i) acc_bc[i] = zero4();
  auto bc_tile = [](int k, int& I, int& J) {  // k-th lower tile in row order
    int i = 0;
#pragma unroll
    for (int t = 1; t < NB; ++t) i += k >= t * (t + 1) / 2;
    I = i;
    J = k - i * (i + 1) / 2;
  };

  // y-shaped tiles [C][PT] as (row block I, column tile ni) units: wave w owns
  // NIW consecutive units, all in one row block
  constexpr int YNI = PT / 16;
  constexpr int NIW = NB * YNI / NW;
  static_assert(NIW >= 1 && (NB * YNI) % NW == 0 && YNI % NIW == 0, "units must split evenly over the waves");
  const int I0 = (wv_id * NIW) / YNI, ni00 = (wv_id * NIW) % YNI;

  // slice inputs of the next (head, slice), loaded while the current one computes:
  // thread item = 8 channels of one row of dt / x / dy, one 16-byte piece of
  // each of the state_pre / dstate rows, one lasta value
  constexpr int PER_ROW = PT / 8, NE = C * PER_ROW, EPT = (NE + NTH - 1) / NTH;
  // item e -> (row, 8 channels): 16 consecutive items take 16 consecutive rows
  // at the same columns, so a 16-lane group's 16-byte LDS accesses start 16
  // rows apart in the bank map instead of four lanes sharing each row
  auto item_row = [](int e) { return (e % 16) + 16 * (e / (16 * PER_ROW)); };
  auto item_col = [](int e) { return ((e / 16) % PER_ROW) * 8; };
  constexpr int SPR = N * (int)sizeof(T) / 16, NS = PT * SPR, SPT = (NS + NTH - 1) / NTH;
  Raw8<T> ndt[EPT], nx[EPT];
  Raw8<TD> ndy[EPT];
  uint4 nst[SPT], ndst[SPT];
  float nla = 0.f;
  auto load_slice = [&](int hn, int pn, size_t rowb) {
    const size_t bnhn = (size_t)bn * dm.H + hn;
#pragma unroll
    for (int it = 0; it < EPT; ++it) {
      const int e = tid + NTH * it;
      if (NE % NTH == 0 || e < NE) {
        const int r = item_row(e), c = item_col(e);
        const size_t hp = (size_t)hn * P + pn + c;
        ndt[it].load(dt + (rowb + r) * dm.rdt + hp);
        nx[it].load(x + (rowb + r) * dm.rx + hp);
        ndy[it].load(dy + (rowb + r) * dm.rdy + hp);
      }
    }
#pragma unroll
    for (int it = 0; it < SPT; ++it) {
      const int e = tid + NTH * it;
      if (NS % NTH == 0 || e < NS) {
        const size_t o = (bnhn * P + pn + e / SPR) * N + (e % SPR) * (16 / sizeof(T));
        nst[it] = *reinterpret_cast<const uint4*>(ck.state_pre + o);
        ndst[it] = *reinterpret_cast<const uint4*>(gr.dstate + o);
      }
    }
    if (tid < PT) nla = gr.lasta[bnhn * P + pn + tid];
  };
  load_slice(g * HG, 0, row0);
  // the chunk's CB, shared by every head and slice of this workgroup, with its
  // strict upper triangle (j > i) zeroed: the pair sums read only the blocks
  // at and below the diagonal, and of a diagonal block its lower triangle, so
  // the zeros are the triangle masks of those blocks
  {
    static_assert(sizeof(T) == 2, "two elements per dword");
    constexpr int VEC = 8, PR = C / VEC, NP = C * PR, IT = (NP + NTH - 1) / NTH;
    u32x4 tmp[IT];
#pragma unroll
    for (int it = 0; it < IT; ++it) {
      const int e = tid + NTH * it;
      if (NP % NTH == 0 || e < NP) tmp[it] = *reinterpret_cast<const u32x4*>(cb0 + (size_t)(e / PR) * C + (e % PR) * VEC);
    }
#pragma unroll
    for (int it = 0; it < IT; ++it) {
      const int e = tid + NTH * it;
      if (NP % NTH == 0 || e < NP) {
        const int r = e / PR, c0 = (e % PR) * VEC;
        u32x4 v = tmp[it];
#pragma unroll
        for (int d = 0; d < 4; ++d)
          v[d] &= (c0 + 2 * d <= r ? 0xffffu : 0u) | (c0 + 2 * d + 1 <= r ? 0xffff0000u : 0u);
        *reinterpret_cast<u32x4*>(sCB + r * L::LCB + c0) = v;
      }
    }
  }
  for (int hh = 0; hh < HG; ++hh) {
    const int h = g * HG + hh;
    const float Ah = A[h];
    if (tid == 0) sDa[0] = 0.f;
    for (int p0 = 0; p0 < P; p0 += PT) {
      const int z = opaque_zero();
      views(z);
      const T* Bg = opaque_ptr(Bg0);
      const T* Cg = opaque_ptr(Cg0);
      const T* cbg = opaque_ptr(cb0);
      // this wave's block, also rebuilt per iteration (its addresses stay in the loop)
      const int I = I0 + z, ni0 = ni00 + z;
      const size_t rowz = row0 + z;
      // dx / ddt of this lane (rows 16 I + tile_row(ii), channels p0 + 16 (ni0 + q) + tile_col())
      // as a uniform base and 32-bit lane offsets
      const unsigned HP = (unsigned)(dm.H * P);
      const unsigned olane = (unsigned)tile_row(0) * HP + (unsigned)(16 * ni0 + tile_col());
      // the C / B rows of this wave's block for y_off / dwrite, requested now
      frag cfr[N / 32], bfr[N / 32];
#pragma unroll
      for (int kk = 0; kk < N / 32; ++kk) {
        cfr[kk] = Mma<T>::ld_c(Cg, ldc, 16 * I, 32 * kk);
        bfr[kk] = Mma<T>::ld_c(Bg, ldb, 16 * I, 32 * kk);
      }
      // ---- A: slice inputs (dt, x, dy kept exactly as bf16), a = sanitize(dt A, 20);
      // thread item = 8 channels of one row, kept in registers for B
      int flag = 0;
      Raw8<T> rdt[EPT], rx[EPT];
      Raw8<TD> rdy[EPT];
#pragma unroll
      for (int it = 0; it < EPT; ++it) {
        rdt[it] = ndt[it];
        rx[it] = nx[it];
        rdy[it] = ndy[it];
      }
#pragma unroll
      for (int it = 0; it < SPT; ++it) {
        const int e = tid + NTH * it;
        if (NS % NTH == 0 || e < NS) {
          const int r = e / SPR, c = (e % SPR) * (16 / (int)sizeof(T));
          *reinterpret_cast<uint4*>(sSt + r * L::LN + c) = nst[it];
          *reinterpret_cast<uint4*>(sDst + r * L::LN + c) = ndst[it];
        }
      }
      if (tid < PT) sLastA[tid] = nla;
#pragma unroll
      for (int it = 0; it < EPT; ++it) {
        const int e = tid + NTH * it;
        if (NE % NTH == 0 || e < NE) {
          const int r = item_row(e), c = item_col(e);
          *reinterpret_cast<uint4*>(sDt + r * L::LPT + c) = rdt[it].v;
          *reinterpret_cast<uint4*>(sX + r * L::LPT + c) = rx[it].v;
          float yv[8], av[8];
#pragma unroll
          for (int j = 0; j < 8; ++j) {
            const float a = rdt[it][j] * Ah;
            flag |= a > 0.f;
            av[j] = sanitize(a, kClipDecay);
            yv[j] = rdy[it][j];
          }
          store8(sCum + r * L::LC + c, av);
          store8(sDy + r * L::LPT + c, yv);
        }
      }
      __syncthreads();
      column_cumsum<C, PT, L::LC, NTH>(sCum, sTot);
      __syncthreads();
      // block-pair decays (one exp per pair and channel, shared by phases C and D)
      // and the range check on the diagonal pairs
#pragma unroll
      for (int e = tid; e < NBC * PT; e += NTH) {
        const int k = e / PT, p = e % PT;
        int TI, TJ;
        bc_tile(k, TI, TJ);
        const float d = sCum[16 * TI * L::LC + p] - sCum[(16 * TJ + 15) * L::LC + p];
        sM[e] = __expf(d);
        if (TI == TJ) flag |= d > kMaxRange;
      }
      // positive step exponent or too steep a block: pairwise evaluation
      const bool exact = __builtin_amdgcn_readfirstlane(__syncthreads_or(flag)) != 0;

      // ---- B: operands Yu = dy U, Vd = V dBx (bf16 high + low parts), from the
      // registers of A
      if (!exact) {
#pragma unroll
        for (int it = 0; it < EPT; ++it) {
          const int e = tid + NTH * it;
          if (NE % NTH == 0 || e < NE) {
            const int r = item_row(e), c = item_col(e);
            float cr[8], cs[8], ce[8];
            load8(sCum + r * L::LC + c, cr);
            load8(sCum + (r & ~15) * L::LC + c, cs);
            load8(sCum + (r | 15) * L::LC + c, ce);
            float yh[8], yl[8], vh[8], vl[8];
#pragma unroll
            for (int j = 0; j < 8; ++j) {
              const float cj = cr[j];
              const float dbx = sanitize(rdt[it][j] * rx[it][j]);
              const float yu = rdy[it][j] * __expf(cj - cs[j]);
              const float vd = dbx * __expf(ce[j] - cj);
              yh[j] = to_f(from_f<T>(yu));
              yl[j] = yu - yh[j];
              vh[j] = to_f(from_f<T>(vd));
              vl[j] = vd - vh[j];
            }
            store8(sYu + r * L::LPT + c, yh);
            store8(sYul + r * L::LPT + c, yl);
            store8(sVd + r * L::LPT + c, vh);
            store8(sVdl + r * L::LPT + c, vl);
          }
        }
        __syncthreads();
      }

      // the next slice's loads (the registers of A are free again)
      {
        const bool last_p = p0 + PT >= P;
        if (!(last_p && hh + 1 == HG)) load_slice(last_p ? h + 1 : h, last_p ? 0 : p0 + PT, rowz);
      }

      // ---- C: dCB tiles
      if (!exact) {
        // sum_p Yu_i M_IJ[p] Vd_j (M_II = exp(range_I)); the upper half of
        // diagonal tiles is dropped when the partials are written
#pragma unroll
        for (int s = 0; s < BCPW; ++s) {
          const int k = wv_id + NW * s;
          if (k < NBC) {
            int TI, TJ;
            bc_tile(k, TI, TJ);
            frag a = Mma<T>::ld_c(sYu, L::LPT, 16 * TI, 0);
            const float* mk = sM + k * PT + 8 * (lane_id() >> 4);
#pragma unroll
            for (int e = 0; e < 8; ++e) a[e] = from_f<T>(to_f(a[e]) * mk[e]);
            acc_bc[s] = Mma<T>::mma(a, Mma<T>::ld_c(sVd, L::LPT, 16 * TJ, 0), acc_bc[s]);
          }
        }
      } else {
        // exact path: pairwise with the reference's clips
#pragma unroll
        for (int s = 0; s < BCPW; ++s) {
          const int k = wv_id + NW * s;
          if (k < NBC) {
            int TI, TJ;
            bc_tile(k, TI, TJ);
#pragma unroll
            for (int ii = 0; ii < 4; ++ii) {
              const int i = 16 * TI + tile_row(ii), j = 16 * TJ + tile_col();
              if (j <= i) {
                float sum = 0.f;
                for (int p = 0; p < PT; ++p) {
                  const float dd = fminf(fmaxf(sCum[i * L::LC + p] - sCum[j * L::LC + p], -kClipDecay), kClipDecay);
                  const float dbx = sanitize(to_f(sDt[j * L::LPT + p]) * to_f(sX[j * L::LPT + p]));
                  sum += to_f(sDy[i * L::LPT + p]) * dbx * fminf(__expf(dd), 1e6f);
                }
                acc_bc[s][ii] += sum;
              }
            }
          }
        }
      }

      // ---- D: per row block of this wave: R, S and the per-element terms
      float lastb[NIW][4], redv[NIW][4], ddt1v[NIW][4];
#pragma unroll
      for (int q = 0; q < NIW; ++q)
#pragma unroll
        for (int ii = 0; ii < 4; ++ii) lastb[q][ii] = 0.f;
      {
        f32x4 ra[NIW], sa[NIW];
        if (!exact) {
          // ra = sum_{J <= I} M_IJ (CB_IJ Vd_J) and sa = sum_{J >= I} M_JI (CB_JI^T Yu_J),
          // the diagonal block masked to its lower / upper triangle.  With
          // M_II = exp(cum_{16I} - cum_{16I+15}) the row scales U_i, V_i below turn
          // the diagonal terms into exp(ci - ce) (CB_II Vd_I) and exp(cs - ci) (CB_II^T Yu_I).
          // Compiled per block index, so every operand read is issued up front.
#pragma unroll
          for (int q = 0; q < NIW; ++q) { ra[q] = zero4(); sa[q] = zero4(); }
          static_switch<NB>(I - z, [&](auto Ic) {
            constexpr int IS = decltype(Ic)::value;
#pragma unroll
            for (int J = 0; J <= IS; ++J) {  // sources at or below the block (row side)
              const frag fa = cb_lds_dup<T>(sCB, L::LCB, 16 * IS, 16 * J, false);
              const float* mr = sM + (IS * (IS + 1) / 2 + J) * PT;
#pragma unroll
              for (int q = 0; q < NIW; ++q) {
                const int ni = ni0 + q;
                const f32x4 m = Mma<T>::mma(fa, ld_t_hilo<T>(sVd, sVdl, L::LPT, 16 * ni, 16 * J), zero4());
                const float mf = mr[16 * ni + tile_col()];
#pragma unroll
                for (int k = 0; k < 4; ++k) ra[q][k] += mf * m[k];
              }
            }
#pragma unroll
            for (int J = IS; J < NB; ++J) {  // targets at or above the block (column side)
              const frag fa = cb_lds_dup<T>(sCB, L::LCB, 16 * IS, 16 * J, true);
              const float* mc = sM + (J * (J + 1) / 2 + IS) * PT;
#pragma unroll
              for (int q = 0; q < NIW; ++q) {
                const int ni = ni0 + q;
                const f32x4 m = Mma<T>::mma(fa, ld_t_hilo<T>(sYu, sYul, L::LPT, 16 * ni, 16 * J), zero4());
                const float mf = mc[16 * ni + tile_col()];
#pragma unroll
                for (int k = 0; k < 4; ++k) sa[q][k] += mf * m[k];
              }
            }
          });
        }
        // exp(-20): the floor of the decay to the chunk end
        const float dte_floor = __expf(-kClipDecay);
#pragma unroll
        for (int q = 0; q < NIW; ++q) {
          const int ni = ni0 + q;
          const int pc = 16 * ni + tile_col();
          // the lane's four rows of dy, dt, x (one transposed read each)
          const bf16x4 dy4 = tile_rows4(sDy, L::LPT, 16 * I, 16 * ni);
          const bf16x4 dt4 = tile_rows4(sDt, L::LPT, 16 * I, 16 * ni);
          const bf16x4 x4 = tile_rows4(sX, L::LPT, 16 * I, 16 * ni);
          const float cl = sCum[(C - 1) * L::LC + pc];
          const float cs = sCum[16 * I * L::LC + pc], ce = sCum[(16 * I + 15) * L::LC + pc];
          // factorised path: exp(cl - ci) = E V_i and exp(ci) = D U_i with the
          // row scales U_i = exp(ci - cs), V_i = exp(ce - ci) of the pair sums
          // and the block factors E = exp(cl - ce), D = exp(cs)
          const float Eb = __expf(cl - ce), Db = __expf(cs);
          // y_off_raw = C state^T and dwrite = B dstate^T for this tile (:126,134)
          f32x4 yoff = zero4(), dwr = zero4();
#pragma unroll
          for (int kk = 0; kk < N / 32; ++kk) {
            yoff = Mma<T>::mma(cfr[kk], Mma<T>::ld_c(sSt, L::LN, 16 * ni, 32 * kk), yoff);
            dwr = Mma<T>::mma(bfr[kk], Mma<T>::ld_c(sDst, L::LN, 16 * ni, 32 * kk), dwr);
          }
#pragma unroll
          for (int ii = 0; ii < 4; ++ii) {
            const int i = 16 * I + tile_row(ii), p = pc;
            const float ci = sCum[i * L::LC + p];
            const float dyi = (float)dy4[ii];
            const float dtv = (float)dt4[ii], xv = (float)x4[ii];
            const float dbxi = sanitize(dtv * xv);
            const float dte_raw = cl - ci;
            float rsum, ssum, ssum_m, dte, dh;
            if (!exact) {
              // every step exponent <= 0 here, so cl <= ci <= 0: the clip of
              // the decay to the chunk end is its exp(-20) floor alone, and
              // exp(ci) is only used where ci >= -20
              const float U = __expf(ci - cs), V = __expf(ce - ci);
              rsum = U * ra[q][ii];
              ssum = ssum_m = V * sa[q][ii];
              dte = fmaxf(Eb * V, dte_floor);
              dh = Db * U;
            } else {
              // every pair with the reference's clip, 1e6 cap and masks:
              // R (i as row, masked), S / S_m (i as column)
              rsum = 0.f; ssum = 0.f; ssum_m = 0.f;
              for (int j = 0; j <= i; ++j) {
                const float dd = ci - sCum[j * L::LC + p];
                const float m = (dd >= -kClipDecay && dd <= kClipDecay) ? 1.f : 0.f;
                const float dbx = sanitize(to_f(sDt[j * L::LPT + p]) * to_f(sX[j * L::LPT + p]));
                rsum += to_f(cbg[(size_t)i * C + j]) *
                        fminf(__expf(fminf(fmaxf(dd, -kClipDecay), kClipDecay)), 1e6f) * dbx * m;
              }
              for (int i2 = i; i2 < C; ++i2) {
                const float dd = sCum[i2 * L::LC + p] - ci;
                const float m = (dd >= -kClipDecay && dd <= kClipDecay) ? 1.f : 0.f;
                const float v = to_f(cbg[(size_t)i2 * C + i]) *
                                fminf(__expf(fminf(fmaxf(dd, -kClipDecay), kClipDecay)), 1e6f) *
                                to_f(sDy[i2 * L::LPT + p]);
                ssum += v;
                ssum_m += v * m;
              }
              dte = sanitize(__expf(fminf(fmaxf(dte_raw, -kClipDecay), kClipDecay)), 1e6f);
              dh = __expf(fminf(fmaxf(ci, -kClipDecay), 0.f));
            }
            const float m2 = (dte_raw >= -kClipDecay && dte_raw <= kClipDecay) ? 1.f : 0.f;
            const float m1 = (ci >= -kClipDecay && ci <= 0.f) ? 1.f : 0.f;
            const float dw = dwr[ii];
            const float ddbx = sanitize(dw * dte + ssum);                 // :138,148,166
            ddt1v[q][ii] = ddbx * xv;                                     // :167
            dx[((rowz + 16 * I) * dm.H + h) * P + p0 + (olane + ii * HP + 16 * q)] =
                from_f<T>(sanitize(ddbx * dtv));                          // :168,193 + final
            const float dte_term = dw * dbxi * dte * m2;                  // d_decay_to_end_diff :142
            lastb[q][ii] += dte_term;
            // d_cum of this element (:162-173), masked for the reverse cumsum (:181-186)
            redv[q][ii] = (fabsf(ci) < kClipAcc)
                              ? sanitize(dyi * rsum - dbxi * ssum_m + dyi * yoff[ii] * dh * m1 - dte_term)
                              : 0.f;
          }
        }
      }
      // ---- reverse cumsum over the chunk with the clip masks (:181-189), in the
      // tile layout: the lane's 4 rows, the lane groups below it in the block,
      // then the blocks below (block totals through LDS), then the row C-1 terms
      const int g4 = lane_id() >> 4;
      float gsuf[NIW];
#pragma unroll
      for (int q = 0; q < NIW; ++q) {
#pragma unroll
        for (int ii = 2; ii >= 0; --ii) redv[q][ii] += redv[q][ii + 1];
        const float tg = redv[q][0];
        const float t1 = __shfl_down(tg, 16), t2 = __shfl_down(tg, 32), t3 = __shfl_down(tg, 48);
        gsuf[q] = (g4 < 3 ? t1 : 0.f) + (g4 < 2 ? t2 : 0.f) + (g4 < 1 ? t3 : 0.f);
        if (g4 == 0) sTot[I * PT + 16 * (ni0 + q) + tile_col()] = tg + gsuf[q];
      }
      // column sums of the decay_to_end term over this wave's rows
#pragma unroll
      for (int ni = 0; ni < YNI; ++ni) {  // columns outside this wave's units get 0
        float v = 0.f;
#pragma unroll
        for (int q = 0; q < NIW; ++q)
          if (ni == ni0 + q) v = lastb[q][0] + lastb[q][1] + lastb[q][2] + lastb[q][3];
        v += __shfl_xor(v, 16);
        v += __shfl_xor(v, 32);
        if (lane_id() < 16) sLastB[wv_id * PT + 16 * ni + lane_id()] = v;
      }
      __syncthreads();
      float da = 0.f;
#pragma unroll
      for (int q = 0; q < NIW; ++q) {
        const int p = 16 * (ni0 + q) + tile_col();
        float off = gsuf[q];
#pragma unroll
        for (int J = 1; J < NB; ++J) off += J > I ? sTot[J * PT + p] : 0.f;
        // row C-1 extra terms (:176-177), under row C-1's clip mask
        float extra = sLastA[p];
#pragma unroll
        for (int w = 0; w < NW; ++w) extra += sLastB[w * PT + p];
        if (fabsf(sCum[(C - 1) * L::LC + p]) < kClipAcc) off += extra;
        const bf16x4 dt4 = tile_rows4(sDt, L::LPT, 16 * I, 16 * (ni0 + q));
#pragma unroll
        for (int ii = 0; ii < 4; ++ii) {
          const float dtv = (float)dt4[ii];
          const float araw = dtv * Ah;
          const float dA = (araw >= -kClipDecay && araw <= kClipDecay) ? (redv[q][ii] + off) : 0.f;
          ddt[((rowz + 16 * I) * dm.H + h) * P + p0 + (olane + ii * HP + 16 * q)] =
              from_f<T>(sanitize(ddt1v[q][ii] + dA * Ah));                // :187,190 + final
          da += dA * dtv;
        }
      }
      // workgroup sum of this slice's dA contribution
#pragma unroll
      for (int sh = 1; sh < 64; sh <<= 1) da += __shfl_xor(da, sh);
      if (lane_id() == 0) sDa[1 + wv_id] = da;
      // every read of this slice's LDS is done when the barrier below is passed
      __syncthreads();
      if (tid == 0) {
        float t = 0.f;
#pragma unroll
        for (int w = 0; w < NW; ++w) t += sDa[1 + w];
        sDa[0] += t;
      }
    }
    if (tid == 0) gr.dap[(size_t)bn * dm.H + h] = sDa[0];
    __syncthreads();
  }
  // partial sums of this head group
  float* part = gr.part + ((size_t)bn * G + g) * C * C;
#pragma unroll
  for (int s = 0; s < BCPW; ++s) {
    const int k = wv_id + NW * s;
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

// dA[h] = sanitize(sum_n sanitize(sum_b dap[b][n][h])) (:188,194,263), by the
// whole workgroup of NTH threads; red holds NTH / 64 floats of LDS.
template <int NTH>
__device__ __forceinline__ void mamba2_da_head(const Mamba2Dims& dm, const float* __restrict__ dap,
                                               float* __restrict__ dA, int h, float* red) {
  float tot = 0.f;
  for (int n = threadIdx.x; n < dm.NT; n += NTH) {
    float s = 0.f;
    for (int b = 0; b < dm.B; ++b) s += dap[((size_t)b * dm.NT + n) * dm.H + h];
    tot += sanitize(s);
  }
#pragma unroll
  for (int sh = 1; sh < 64; sh <<= 1) tot += __shfl_xor(tot, sh);
  if (lane_id() == 0) red[wave_id()] = tot;
  __syncthreads();
  if (threadIdx.x == 0) {
    float t = 0.f;
#pragma unroll
    for (int w = 0; w < NTH / 64; ++w) t += red[w];
    dA[h] = sanitize(t);
  }
  __syncthreads();
}

// ------------------------------------------------------------------ dB, dC
template <typename T, int C, int NTL, int KB>
struct BcLds {
  static constexpr int PAD = Pad<T>::v;
  static constexpr int LCB = C + PAD, LK = NTL + PAD;
  // the k loop's blocks, then (the same bytes) the epilogue's operands
  static constexpr int off_s = 0;                                   // state_prev rows [KB][NTL]
  static constexpr int off_d = off_s + KB * LK * (int)sizeof(T);    // dstate rows [KB][NTL]
  static constexpr int end_loop = off_d + KB * LK * (int)sizeof(T);
  static constexpr int off_cb = 0;                                  // dCB [C][C]
  static constexpr int off_b = off_cb + C * LCB * (int)sizeof(T);   // B [C][NTL]
  static constexpr int off_c = off_b + C * LK * (int)sizeof(T);     // C [C][NTL]
  static constexpr int end_epi = off_c + C * LK * (int)sizeof(T);
  static constexpr int total = end_loop > end_epi ? end_loop : end_epi;
};

// One workgroup per (batch, chunk, NTL state columns):
//   dC = sanitize(Ydh . state_prev + dCB B)     dB = sanitize(W . dstate + dCB^T C)
// the first terms contracted over k = (head, channel): Ydh / W rows are the
// [B][T][H][P] rows of the chunk, state_prev / dstate the [NT][H][P][N] block.
// The first H workgroups also reduce dA (the dA partials of the chunk
// backward are complete when this kernel starts).  Eight waves, four per SIMD
// with two workgroups on a CU, so many k blocks' loads are in flight at once;
// PD k blocks are staged ahead in registers.  The dCB / B / C operands of the
// epilogue are staged after the k loop into the same LDS bytes, which keeps
// two 64-column workgroups per CU (64 columns read each chunk's Ydh / W rows
// half as often as 32).
template <typename T, int C, int P, int N, int NTL = 64, int PD = 1>
__global__ __launch_bounds__(512) __attribute__((amdgpu_waves_per_eu(4, 4))) void mamba2_bwd_bc(
    Mamba2Dims dm, int G, const T* __restrict__ Bm, const T* __restrict__ Cm, Mamba2Chunks<T> ck,
    Mamba2Grads<T> gr, T* __restrict__ dB, T* __restrict__ dC, float* __restrict__ dA) {
  constexpr int NTH = 512, NW = NTH / 64;
  constexpr int KB = 64, NNT = N / NTL;
  static_assert(P % KB == 0, "whole k blocks per head");
  static_assert(N % NTL == 0, "whole column blocks");
  typedef BcLds<T, C, NTL, KB> L;
  __shared__ __attribute__((aligned(16))) unsigned char lds[L::total];
  T* sS = reinterpret_cast<T*>(lds + L::off_s);
  T* sD = reinterpret_cast<T*>(lds + L::off_d);
  T* sCB = reinterpret_cast<T*>(lds + L::off_cb);
  T* sB = reinterpret_cast<T*>(lds + L::off_b);
  T* sC = reinterpret_cast<T*>(lds + L::off_c);

  {
    __shared__ float red[NW];
    for (int hh = blockIdx.x; hh < dm.H; hh += gridDim.x) mamba2_da_head<NTH>(dm, gr.dap, dA, hh, red);
  }
  int bn, nt;
  xcd_group_map(blockIdx.x, dm.B * dm.NT, NNT, bn, nt);
  const int n0 = nt * NTL;
  const size_t row0 = (size_t)bn * C;  // rows of [B*T][...]
  const int HP = dm.H * P;
  const T* yg = gr.ydh + row0 * HP;
  const T* wg = gr.wr + row0 * HP;
  const T* sg = ck.state_pre + (size_t)bn * HP * N + n0;
  const T* dg = gr.dstate + (size_t)bn * HP * N + n0;

  // output tiles [C / 16][NTL / 16]: wave w owns TPW consecutive column tiles of one row tile
  constexpr int CT = NTL / 16, NTILE = (C / 16) * CT, TPW = NTILE / NW;
  static_assert(TPW >= 1 && NTILE % NW == 0 && CT % TPW == 0, "a wave's tiles share one row tile");
  const int wv_id = wave_id();
  const int m0 = 16 * ((wv_id * TPW) / CT), ct0 = (wv_id * TPW) % CT;
  f32x4 accC[TPW], accB[TPW];
#pragma unroll
  for (int u = 0; u < TPW; ++u) { accC[u] = zero4(); accB[u] = zero4(); }

  // k blocks in flight two ahead: the state_prev / dstate block staged in
  // registers and the Ydh / W fragments of this wave's rows
  constexpr int KK = KB / Mma<T>::KS;
  typedef typename Mma<T>::frag frag;
  struct Stage {
    RegStage<T, KB, NTL, NTH> ps, pd;
    frag ay[KK], aw[KK];
  };
  auto load = [&](Stage& st, int kb) {
    st.ps.load(sg + (size_t)kb * N, N);
    st.pd.load(dg + (size_t)kb * N, N);
#pragma unroll
    for (int q = 0; q < KK; ++q) {
      st.ay[q] = Mma<T>::ld_c(yg, HP, m0, kb + q * Mma<T>::KS);
      st.aw[q] = Mma<T>::ld_c(wg, HP, m0, kb + q * Mma<T>::KS);
    }
  };
  Stage s0, s1;
  load(s0, 0);
  if (PD == 2 && KB < HP) load(s1, KB);

  // one k block: its staged rows to LDS, the stage refilled two blocks ahead,
  // then the MFMAs on the fragments kept from the stage
  auto step = [&](Stage& st, int kb) {
    frag ay[KK], aw[KK];
#pragma unroll
    for (int q = 0; q < KK; ++q) { ay[q] = st.ay[q]; aw[q] = st.aw[q]; }
    __syncthreads();  // previous block's reads done
    st.ps.store(sS, L::LK);
    st.pd.store(sD, L::LK);
    if (kb + PD * KB < HP) load(st, kb + PD * KB);
    __syncthreads();
#pragma unroll
    for (int q = 0; q < KK; ++q) {
      const int kk = q * Mma<T>::KS;
#pragma unroll
      for (int u = 0; u < TPW; ++u) {
        const int ct = ct0 + u;
        accC[u] = Mma<T>::mma(ay[q], Mma<T>::ld_t(sS, L::LK, 16 * ct, kk), accC[u]);
        accB[u] = Mma<T>::mma(aw[q], Mma<T>::ld_t(sD, L::LK, 16 * ct, kk), accB[u]);
      }
    }
  };
  if constexpr (PD == 2) {
    for (int kb = 0; kb < HP; kb += 2 * KB) {
      step(s0, kb);
      if (kb + KB < HP) step(s1, kb + KB);
    }
  } else {
    for (int kb = 0; kb < HP; kb += KB) step(s0, kb);
  }

  // the epilogue's operands, into the bytes of the k loop's blocks:
  // dCB = the sum of the head-group partials (lower triangle), 4 columns per
  // item (requested before the barrier), and the chunk's B / C rows
  const float* part = gr.part + (size_t)bn * G * C * C;
  constexpr int E4 = C * C / 4 / NTH;
  static_assert(E4 * NTH * 4 == C * C, "whole items per thread");
  f32x4 cbs[E4];
#pragma unroll
  for (int t = 0; t < E4; ++t) cbs[t] = zero4();
  for (int gg = 0; gg < G; ++gg) {
    f32x4 v[E4];
#pragma unroll
    for (int t = 0; t < E4; ++t)
      v[t] = *reinterpret_cast<const f32x4*>(part + (size_t)gg * C * C + 4 * (threadIdx.x + NTH * t));
#pragma unroll
    for (int t = 0; t < E4; ++t) cbs[t] += v[t];
  }
  __syncthreads();  // the last k block's reads are done
#pragma unroll
  for (int t = 0; t < E4; ++t) {
    const int e4 = threadIdx.x + NTH * t, i = (4 * e4) / C, j = (4 * e4) % C;
    f32x4 sv;
#pragma unroll
    for (int c = 0; c < 4; ++c) sv[c] = j + c <= i ? cbs[t][c] : 0.f;
    store4(sCB + i * L::LCB + j, sv);
  }
  stage_rows<T, C, NTL, NTH>(sB, L::LK, Bm + row0 * dm.rB + n0, dm.rB);
  stage_rows<T, C, NTL, NTH>(sC, L::LK, Cm + row0 * dm.rC + n0, dm.rC);
  __syncthreads();
  T* dCo = dC + row0 * N + n0;
  T* dBo = dB + row0 * N + n0;
#pragma unroll
  for (int u = 0; u < TPW; ++u) {
    const int ct = ct0 + u;
    f32x4 c = tile_mma<T, false, true>(accC[u], sCB, L::LCB, sB, L::LK, m0, 16 * ct, C);
    f32x4 b = tile_mma<T, true, true>(accB[u], sCB, L::LCB, sC, L::LK, m0, 16 * ct, C);
#pragma unroll
    for (int k = 0; k < 4; ++k) { c[k] = sanitize(c[k]); b[k] = sanitize(b[k]); }
    store_tile_n(dCo, N, m0, 16 * ct, c);
    store_tile_n(dBo, N, m0, 16 * ct, b);
  }
}

}  // namespace ah
