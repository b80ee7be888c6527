// Mamba2 SSD chunk-scan forward for gfx950.
//
// The state transition of a chunk is diagonal (state[p][s] decays by
// exp(cum_last[p]) independently of s), so the only sequential part of the
// scan is an elementwise recurrence; the scans and everything but the
// state's own contraction run chunk-parallel.  Per chunk the arithmetic
// follows _chunk_ssd
// (mamba2_ssd_reference.py:70-149):
//   a      = sanitize(dt A, 20)                 cum = sanitize(cumsum(a), 1e4)
//   y_diag = sum_{j<=i} min(exp(clip(cum_i - cum_j, +-20)), 1e6) CB_ij dBx_j
//   s_end  = sanitize(B^T (dBx sanitize(exp(clip(cum_last - cum, +-20)), 1e6)))
//   y_off  = sanitize((C state^T) exp(clip(cum, -20, 0)))
//   state  = sanitize(state exp(clip(cum_last, -20, 0)) + s_end)
//
// mamba2_cb           one workgroup per (batch, chunk): CB = sanitize(C B^T),
//                     shared by every head (the reference's M3 broadcasts B/C
//                     to every head instead, kernel_mamba2_b_intra.py:136-142).
// mamba2_chunk_outer  one workgroup per (batch, chunk, head, channel slice):
//                     the chunk's cum and its S rows, dBx dte (forward) or
//                     the backward's Ydh = dy decay_h and W (BWD = true), and
//                     in the two-pass form the per-chunk S^T B (S^T C).
// mamba2_state_chain  (mamba2_seq.hpp) one workgroup per (batch, head, 32
//                     channels), sequential over chunks: s_end = S^T B on
//                     MFMA and the recurrence, the state entering every chunk
//                     (forward), or the dstate carry and the decay_chunk_end
//                     term (backward).
// mamba2_state_pass   one workgroup per (batch, head, 8 or 16 channels),
//                     sequential over chunks, elementwise: the two-pass form
//                     of the state loop over the per-chunk state_end (or the
//                     backward's (dy decay_h)^T C) that mamba2_chunk_outer
//                     formed, for grids too small for mamba2_state_chain; and
//                     the stage-level kernel M4.
// mamba2_chunk_y      one workgroup per (batch, chunk, head, 32 channels):
//                     y = y_diag + y_off.
// mamba2_cumdecay     one workgroup per (batch, chunk, head, 64 channels):
//                     the stage-level kernel M2 alone (cumdecay to HBM).
//
// The stage-level entries (the reference's M2, M3 and M4 over caller-owned
// arrays) run the same kernels in a stage mode: the cum comes from the
// caller's cumdecay, the per-chunk arrays are in the reference's [B][H][NT]
// order, and the arithmetic is that of the stage kernels, which drop the
// 1e6 caps (kernel_mamba2_b_intra.py:96-112) and sanitise the chunk's write
// and the initial state (kernel_mamba2_c_interchunk.py:58).
//
// y_diag on 16-row blocks: for output block I and source block J < I the
// decay factorises as
//   exp(cum_i - cum_j) = exp(cum_i - cum_{16I}) exp(cum_{16I} - cum_{16J+15})
//                        exp(cum_{16J+15} - cum_j),
// each factor <= 1 whenever dt A <= 0 (the model's A < 0, dt > 0), so the
// pair (I, J) is one MFMA on V_j = exp(cum_{16J+15} - cum_j) dBx_j with a
// per-channel scale, and nothing overflows.  Inside the diagonal block the
// same V_j carries a factor exp(cum_i - cum_{16I+15}) <= exp(range_I), used
// while every block's range stays below kMaxRange.  Pairs whose decay is
// below -20 carry their true weight instead of the reference's exp(-20)
// floor (a difference below 2e-9 |CB dBx|).  A slice with any dt A > 0, or a
// steeper block, evaluates every pair with the reference's clip and cap.
#include "mamba2.hpp"
#include "mamba2_seq.hpp"

namespace ah {

// One workgroup per (batch, chunk, RB-row block of CB): with RB < C a small
// batch still spreads over the CUs.
template <typename T, int C, int N, int RB = C>
__global__ __launch_bounds__(256) void mamba2_cb(Mamba2Dims dm, const T* __restrict__ Bm,
                                                const T* __restrict__ Cm, Mamba2Chunks<T> ck) {
  constexpr int PAD = Pad<T>::v, LN = N + PAD, NRB = C / RB;
  static_assert(C % RB == 0, "whole row blocks");
  __shared__ __attribute__((aligned(16))) T sB[C * LN];
  __shared__ __attribute__((aligned(16))) T sC[RB * LN];
  const int bn = blockIdx.x / NRB, rb = blockIdx.x % NRB;  // b * NT + n, row block
  const size_t row0 = (size_t)bn * C;  // rows of [B*T][N]
  stage_rows<T, C, N>(sB, LN, Bm + row0 * dm.rB, dm.rB);
  stage_rows<T, RB, N>(sC, LN, Cm + (row0 + (size_t)rb * RB) * dm.rC, dm.rC);
  __syncthreads();
  constexpr int MT = RB / 16, NTT = C / 16;
  T* out = ck.cb + (size_t)bn * C * C + (size_t)rb * RB * C;
  for (int tile = wave_id(); tile < MT * NTT; tile += 4) {
    const int mi = tile / NTT, nj = tile % NTT;
    f32x4 acc = tile_mma<T, false, false>(zero4(), sC, LN, sB, LN, 16 * mi, 16 * nj, N);
#pragma unroll
    for (int i = 0; i < 4; ++i) acc[i] = sanitize(acc[i]);
    store_tile_n(out, C, 16 * mi, 16 * nj, acc);
  }
}

// Inclusive column scan of sCum ([C][PT] fp32 with row stride LD, holding
// sanitize(dt A, 20) on entry) into sanitize(cumsum, 1e4).  Thread map:
// column tid % PT, RS rows (NTH threads in the workgroup).
template <int C, int PT, int LD = PT, int NTH = 256>
__device__ __forceinline__ void column_cumsum(float* sCum, float* sTot) {
  constexpr int NSEG = NTH / PT, RS = C / NSEG;
  const int p = threadIdx.x % PT, seg = threadIdx.x / PT;
  float v[RS];
#pragma unroll
  for (int r = 0; r < RS; ++r) v[r] = sCum[(seg * RS + r) * LD + p];
#pragma unroll
  for (int r = 1; r < RS; ++r) v[r] += v[r - 1];
  sTot[seg * PT + p] = v[RS - 1];
  __syncthreads();
  float off = 0.f;  // all lower segment totals requested at once
#pragma unroll
  for (int s = 0; s < NSEG - 1; ++s) off += s < seg ? sTot[s * PT + p] : 0.f;
#pragma unroll
  for (int r = 0; r < RS; ++r) sCum[(seg * RS + r) * LD + p] = sanitize(v[r] + off, kClipAcc);
}

// ------------------------------------------------------------------ cumdecay (M2 alone)
// build_chunk_cumdecay_pallas (kernel_mamba2_a_decay.py:53-66):
// sanitize(cumsum(sanitize(dt A, 20)), 1e4), out[B][H][NT][C][P] fp32 (the
// same cum the chunk kernels build in LDS).
template <typename T, int C, int P, int PT>
__global__ __launch_bounds__(256) void mamba2_cumdecay(Mamba2Dims dm, const T* __restrict__ dt,
                                                      const float* __restrict__ A, float* __restrict__ out) {
  constexpr int LC = PT + 4, NSEG = 256 / PT, NPT = P / PT;
  __shared__ __attribute__((aligned(16))) float sCum[C * LC];
  __shared__ __attribute__((aligned(16))) float sTot[NSEG * PT];
  const int m = blockIdx.x % (dm.H * NPT), bn = blockIdx.x / (dm.H * NPT);
  const int h = m / NPT, p0 = (m % NPT) * PT;
  const int bb = bn / dm.NT, n = bn % dm.NT;
  const size_t row0 = (size_t)bb * dm.T + (size_t)n * C;
  const size_t hp = (size_t)h * P + p0;
  const float Ah = A[h];
  constexpr int PER_ROW = PT / 8, NE = C * PER_ROW, EPT = NE / 256;
  static_assert(NE % 256 == 0, "slice must split evenly over the workgroup");
#pragma unroll
  for (int i = 0; i < EPT; ++i) {
    const int e = threadIdx.x + 256 * i, r = e / PER_ROW, c = (e % PER_ROW) * 8;
    Raw8<T> rdt;
    rdt.load(dt + (row0 + r) * dm.rdt + hp + c);
    float av[8];
#pragma unroll
    for (int j = 0; j < 8; ++j) av[j] = sanitize(rdt[j] * Ah, kClipDecay);
    store8(sCum + r * LC + c, av);
  }
  __syncthreads();
  column_cumsum<C, PT, LC>(sCum, sTot);
  __syncthreads();
  float* o = out + (((size_t)bb * dm.H + h) * dm.NT + n) * C * P + p0;
#pragma unroll
  for (int i = 0; i < EPT; ++i) {
    const int e = threadIdx.x + 256 * i, r = e / PER_ROW, c = (e % PER_ROW) * 8;
    *reinterpret_cast<float4*>(o + (size_t)r * P + c) = *reinterpret_cast<const float4*>(sCum + r * LC + c);
    *reinterpret_cast<float4*>(o + (size_t)r * P + c + 4) =
        *reinterpret_cast<const float4*>(sCum + r * LC + c + 4);
  }
}

// Rows [0, C) of one (batch, head, chunk)'s cumdecay slice into sCum.
template <int C, int PT, int LC>
__device__ __forceinline__ void load_cum_rows(float* sCum, const float* __restrict__ g, int P) {
  constexpr int PER_ROW = PT / 4;  // float4 pieces per row
  for (int e = threadIdx.x; e < C * PER_ROW; e += 256) {
    const int r = e / PER_ROW, c = (e % PER_ROW) * 4;
    *reinterpret_cast<float4*>(sCum + r * LC + c) = *reinterpret_cast<const float4*>(g + (size_t)r * P + c);
  }
}

// ------------------------------------------------------------------ chunk outer products
template <typename T, int C, int N, int PT, bool ROWS>
struct OuterLds {
  static constexpr int PAD = Pad<T>::v;
  static constexpr int LS = PT + PAD, LN = N + PAD;
  static constexpr int LC = PT + 4;  // fp32 cum rows: 16-byte aligned, 4 banks apart
  static constexpr int NSEG = 256 / PT;
  static constexpr int off_cum = 0;  // fp32 cum [C][LC]; then the bf16 operand S [C][LS]
  static constexpr int off_tot = off_cum + C * LC * 4;
  static constexpr int off_r = off_tot + NSEG * PT * 4;   // the rows R (stage mode only)
  static constexpr int total = off_r + (ROWS ? C * LN * (int)sizeof(T) : 0);
  static_assert(C * LS * (int)sizeof(T) <= C * LC * 4, "S must fit in the cum buffer");
};

// The chunk's cum and S for (batch, chunk, head, PT channels), SL
// consecutive (head, slice) pairs per workgroup; (dm.H * P / PT) % SL == 0:
//   forward  (BWD = false): S = dBx dte (the chunk's write, :133-135) and
//            cum_last; with PROD the chunk's state_end = sanitize(S^T B)
//            (:136-137) into ck.src, without it S into srows ([B][T][H][P],
//            bf16) for the state loop that forms S^T B on chip
//            (mamba2_seq.hpp).
//   backward (BWD = true):  S = Ydh = dy decay_h (:123 of mamba2_bwd_reference.py)
//            into srows and W = sanitize(dBx dte) (:135) into wr, the
//            operands of dC_1 and dB_1; with PROD also (dy decay_h)^T C
//            (:128) into ck.src, else the state loop forms it.
//   stage M3 (STG = true, forward): cum from ck.cum, S = sanitize(dBx
//            exp(clip(cum_last - cum, +-20))) and state_end in
//            [B][H][NT][P][N] (kernel_mamba2_b_intra.py:110-116).
// With PROD the SL pairs share the staged rows R (B forward, C backward) and
// out[p][s] = sum_i S[i][p] R[i][s] runs on MFMA.
template <typename T, typename TD, int C, int P, int N, int PT, bool BWD, int SL, bool STG = false,
          bool PROD = STG>
__global__ __launch_bounds__(256) void mamba2_chunk_outer(
    Mamba2Dims dm, const T* __restrict__ dt, const T* __restrict__ x, const float* __restrict__ A,
    const T* __restrict__ R, const TD* __restrict__ dy, Mamba2Chunks<T> ck, T* __restrict__ srows,
    T* __restrict__ wr) {
  typedef OuterLds<T, C, N, PT, PROD> L;
  __shared__ __attribute__((aligned(16))) unsigned char lds[L::total];
  float* sCum = reinterpret_cast<float*>(lds + L::off_cum);
  T* sS = reinterpret_cast<T*>(lds + L::off_cum);
  float* sTot = reinterpret_cast<float*>(lds + L::off_tot);
  T* sR = reinterpret_cast<T*>(lds + L::off_r);

  constexpr int NPT = P / PT;
  int bn, m2;
  xcd_group_map(blockIdx.x, dm.B * dm.NT, dm.H * NPT / SL, bn, m2);
  const int bb = bn / dm.NT, n = bn % dm.NT;
  const size_t row0 = (size_t)bb * dm.T + (size_t)n * C;
  const size_t rsx = (size_t)dm.H * P;  // the workspace rows (Ydh, W)
  // R (B or C of the chunk) is shared by the workgroup's SL (head, slice) pairs
  // R (B or C of the chunk) is shared by the workgroup's SL (head, slice) pairs
  const size_t rR = BWD ? (size_t)dm.rC : (size_t)dm.rB;
  if constexpr (PROD) stage_rows<T, C, N>(sR, L::LN, R + row0 * rR, rR);
  for (int sl = 0; sl < SL; ++sl) {
  const int m = m2 * SL + sl;
  const int h = m / NPT, p0 = (m % NPT) * PT;
  const size_t base = (row0 * dm.H + h) * P + p0;  // element (r, c) at base + r * rsx + c
  const size_t bhn_ref = ((size_t)bb * dm.H + h) * dm.NT + n;  // [B][H][NT] order (stage mode)

  constexpr int PER_ROW = PT / 8, NE = C * PER_ROW, EPT = NE / 256;
  static_assert(NE % 256 == 0, "slice must split evenly over the workgroup");
  Raw8<T> rdt[EPT], rx[EPT];
  Raw8<TD> rdy[BWD ? EPT : 1];
#pragma unroll
  for (int i = 0; i < EPT; ++i) {
    const int e = threadIdx.x + 256 * i, r = e / PER_ROW, c = (e % PER_ROW) * 8;
    const size_t hp = (size_t)h * P + p0 + c, rr = row0 + r;
    rdt[i].load(dt + rr * dm.rdt + hp);
    rx[i].load(x + rr * dm.rx + hp);
    if constexpr (BWD) rdy[i].load(dy + rr * dm.rdy + hp);
  }
  if constexpr (STG) {
    load_cum_rows<C, PT, L::LC>(sCum, ck.cum + bhn_ref * C * P + p0, P);
    __syncthreads();
  } else {
    const float Ah = A[h];
#pragma unroll
    for (int i = 0; i < EPT; ++i) {
      const int e = threadIdx.x + 256 * i, r = e / PER_ROW, c = (e % PER_ROW) * 8;
      float av[8];
#pragma unroll
      for (int j = 0; j < 8; ++j) av[j] = sanitize(rdt[i][j] * Ah, kClipDecay);
      store8(sCum + r * L::LC + c, av);
    }
    __syncthreads();
    column_cumsum<C, PT, L::LC>(sCum, sTot);
    __syncthreads();
  }

  float sv[EPT][8];
#pragma unroll
  for (int i = 0; i < EPT; ++i) {
    const int e = threadIdx.x + 256 * i, r = e / PER_ROW, c = (e % PER_ROW) * 8;
    float wv[8], cr[8], clr[8];
    load8(sCum + r * L::LC + c, cr);
    load8(sCum + (C - 1) * L::LC + c, clr);
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      const float ci = cr[j];
      const float cl = clr[j];
      const float dbx = sanitize(rdt[i][j] * rx[i][j]);
      const float ed = __expf(fminf(fmaxf(cl - ci, -kClipDecay), kClipDecay));
      const float dte = sanitize(ed, 1e6f);
      if constexpr (BWD) {
        sv[i][j] = rdy[i][j] * __expf(fminf(fmaxf(ci, -kClipDecay), 0.f));
        wv[j] = sanitize(dbx * dte);
      } else if constexpr (STG) {
        sv[i][j] = sanitize(dbx * ed);
      } else {
        sv[i][j] = dbx * dte;
      }
    }
    if constexpr (BWD || !PROD) store8(srows + base + r * rsx + c, sv[i]);
    if constexpr (BWD) store8(wr + base + r * rsx + c, wv);
  }
  const size_t bnh = (size_t)bn * dm.H + h;
  if (!BWD && !STG && threadIdx.x < PT) ck.cl[bnh * P + p0 + threadIdx.x] = sCum[(C - 1) * L::LC + threadIdx.x];
  __syncthreads();  // every cum read is done: S overwrites the cum buffer
  if constexpr (PROD) {
#pragma unroll
    for (int i = 0; i < EPT; ++i) {
      const int e = threadIdx.x + 256 * i, r = e / PER_ROW, c = (e % PER_ROW) * 8;
      store8(sS + r * L::LS + c, sv[i]);
    }
    __syncthreads();

    constexpr int NI = N / 16, TILES = (PT / 16) * NI, TPW = TILES / 4;
    static_assert(TILES % 4 == 0, "tiles must split evenly over 4 waves");
    float* out = ck.src + ((STG ? bhn_ref : bnh) * P + p0) * N;
    const int wv_id = wave_id();
#pragma unroll
    for (int t = 0; t < TPW; ++t) {
      const int tile = wv_id * TPW + t, mi = tile / NI, ni = tile % NI;
      f32x4 acc = tile_mma<T, true, true>(zero4(), sS, L::LS, sR, L::LN, 16 * mi, 16 * ni, C);
      if constexpr (!BWD) {
#pragma unroll
        for (int k = 0; k < 4; ++k) acc[k] = sanitize(acc[k]);
      }
      store_tile_n(out, N, 16 * mi, 16 * ni, acc);
    }
    __syncthreads();  // the next pair rewrites the cum / S buffer
  }
  }
}

// ------------------------------------------------------------------ sequential pass
// Forward: state entering chunk n -> state_pre (bf16), then
//   state = sanitize(state exp(clip(cum_last, -20, 0)) + s_end)      (:144-146)
// Backward (MB0, mamba2_bwd_reference.py:236-247), reverse over chunks:
//   dstate carry entering chunk n's backward -> dstate (bf16);
//   d_cum_last_a = sum_s dstate state_prev * decay_chunk_end * mask  (:116,120)
//   dstate = sanitize(dstate decay_chunk_end + (dy decay_h)^T C)      (:115,128,195)
// Thread map: one float4 of one channel row; RP channel rows per workgroup.
// Stage M4 (STG = true, forward): src = the caller's state_end in
// [B][H][NT][P][N], cum_last from the caller's cumdecay, and the initial
// state sanitised (kernel_mamba2_c_interchunk.py:58,68-78).  The whole-path
// forward sanitises it too when dm.sanitize_state0 is set.
template <typename T, int P, int N, bool BWD, bool STG = false>
__global__ __launch_bounds__(256) void mamba2_state_pass(Mamba2Dims dm, Mamba2Chunks<T> ck,
                                                        T* __restrict__ dstate, float* __restrict__ lasta,
                                                        const float* __restrict__ init,
                                                        float* __restrict__ fin) {
  constexpr int TPR = N / 4, RP = 256 / TPR, NRP = P / RP;
  const int bh = blockIdx.x / NRP, rp = blockIdx.x % NRP;
  const int bb = bh / dm.H, h = bh % dm.H;
  const int r = threadIdx.x / TPR, c4 = threadIdx.x % TPR;
  const int p = rp * RP + r, s0 = 4 * c4;
  const int NT = dm.NT;
  auto rowi = [&](int n) { return (((size_t)bb * NT + n) * dm.H + h) * P + p; };
  // src and cum_last rows: the workspace's [B][NT][H] order, or the caller's
  // [B][H][NT] arrays in stage mode
  auto rows = [&](int n) { return STG ? ((size_t)bh * NT + n) * P + p : rowi(n); };
  auto cl_at = [&](int n) {
    return STG ? ck.cum[(((size_t)bh * NT + n) * dm.C + dm.C - 1) * P + p] : ck.cl[rowi(n)];
  };

  float4 st = make_float4(0.f, 0.f, 0.f, 0.f);
  if (init) st = *reinterpret_cast<const float4*>(init + ((size_t)bh * P + p) * N + s0);
  if (STG || (!BWD && dm.sanitize_state0)) {
    st.x = sanitize(st.x); st.y = sanitize(st.y); st.z = sanitize(st.z); st.w = sanitize(st.w);
  }

  constexpr int D = 4;  // chunks in flight
  float4 src[D];
  float cl[D];
  uint2 sp[D];
  auto load = [&](int k, int it) {
    const int n = BWD ? NT - 1 - it : it;
    const size_t ri = rowi(n);
    src[k] = *reinterpret_cast<const float4*>(ck.src + rows(n) * N + s0);
    cl[k] = cl_at(n);
    if (BWD) sp[k] = *reinterpret_cast<const uint2*>(ck.state_pre + ri * N + s0);
  };
  // Every load is issued on every path (past the last chunk it re-reads that
  // chunk, whose registers are never used), and the loop body runs whole
  // groups of D chunks: the wait before a chunk's use then leaves the other
  // D - 1 chunks' loads in flight.
  auto step = [&](int k, int it) {
    const int n = BWD ? NT - 1 - it : it;
    const size_t ri = rowi(n);
    const float c = cl[k];
    const float dce = __expf(fminf(fmaxf(c, -kClipDecay), 0.f));
    f32x4 sv = {st.x, st.y, st.z, st.w};
    store4((BWD ? dstate : ck.state_pre) + ri * N + s0, sv);
    if (BWD) {
      const bf16* spv = reinterpret_cast<const bf16*>(&sp[k]);
      float part = st.x * (float)spv[0] + st.y * (float)spv[1] + st.z * (float)spv[2] +
                   st.w * (float)spv[3];
#pragma unroll
      for (int o = 1; o < TPR; o <<= 1) part += __shfl_xor(part, o);
      const float msk = (c >= -kClipDecay && c <= 0.f) ? 1.f : 0.f;
      if (c4 == 0) lasta[ri] = part * dce * msk;
    }
    st.x = sanitize(st.x * dce + src[k].x);
    st.y = sanitize(st.y * dce + src[k].y);
    st.z = sanitize(st.z * dce + src[k].z);
    st.w = sanitize(st.w * dce + src[k].w);
    load(k, min(it + D, NT - 1));
  };
#pragma unroll
  for (int k = 0; k < D; ++k) load(k, min(k, NT - 1));
  int it0 = 0;
  for (; it0 + D <= NT; it0 += D) {
#pragma unroll
    for (int k = 0; k < D; ++k) step(k, it0 + k);
  }
#pragma unroll
  for (int k = 0; k < D; ++k)
    if (it0 + k < NT) step(k, it0 + k);
  if (fin) {
    if (BWD) {  // :264 and the final clip
      st.x = sanitize(st.x); st.y = sanitize(st.y); st.z = sanitize(st.z); st.w = sanitize(st.w);
    }
    *reinterpret_cast<float4*>(fin + ((size_t)bh * P + p) * N + s0) = st;
  }
}

// ------------------------------------------------------------------ outputs
// Blocks whose decay range cum_{16I} - cum_{16I+15} exceeds this are not
// factorised (the factor exp(cum_{16I} - cum_j) >= 1 must stay finite).
constexpr float kMaxRange = 60.f;

// A fragment of a 16x16 (k = 16) block of a row-major [C][C] matrix in global
// memory: lanes of groups 0, 1 hold k = 0..15; groups 2, 3 hold zeros (and
// read nothing).  mask: 0 none, 1 keep k <= m (lower), 2 keep k >= m (upper).
template <typename T>
__device__ __forceinline__ typename Mma<T>::frag cb_frag(const T* g, int ld, int m0, int k0, int mask) {
  typename Mma<T>::frag a;
  const int l = lane_id();
  if (l < 32) {
    a = Mma<T>::ld_c(g, ld, m0, k0);
    if (mask) {
      const int m = l & 15, kb = 8 * (l >> 4);
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        const bool keep = mask == 1 ? (kb + e <= m) : (kb + e >= m);
        if (!keep) a[e] = (T)0.f;
      }
    }
  } else {
#pragma unroll
    for (int e = 0; e < 8; ++e) a[e] = (T)0.f;
  }
  return a;
}

template <typename T, int C, int N, int PT>
struct YLds {
  static constexpr int PAD = Pad<T>::v;
  static constexpr int LPT = PT + PAD, LN = N + PAD;
  // fp32 rows: 16-byte aligned, rows 4 apart 16 banks apart (tile-layout reads)
  static constexpr int LC = PT + 4;
  static constexpr int NSEG = 256 / PT;
  static constexpr int off_cum = 0;
  static constexpr int off_dbx = off_cum + C * LC * 4;
  static constexpr int off_v = off_dbx + C * LC * 4;                 // V dBx, + 16 zero rows
  static constexpr int off_st = off_v + (C + 16) * LPT * (int)sizeof(T);
  static constexpr int off_tot = off_st + PT * LN * (int)sizeof(T);
  static constexpr int total = off_tot + NSEG * PT * 4;
};

// Output block of wave w's b-th assignment: blocks {w, NB-1-w} balance the
// number of off-diagonal source blocks over the four waves.
template <int NB>
__device__ __forceinline__ constexpr int y_block(int w, int b) {
  return b == 0 ? w : NB - 1 - w;
}

// y_diag on 16-row blocks, Vd_j = exp(cum_{16J+15} - cum_j) dBx_j:
//   off the diagonal  U_i sum_{J<I} M_IJ (CB_IJ Vd_J)_i
//   diagonal block    exp(cum_i - cum_{16I+15}) (tril(CB_II) Vd_I)_i
// with U_i = exp(cum_i - cum_{16I}), M_IJ = exp(cum_{16I} - cum_{16J+15}).
// SL consecutive (head, channel slice) pairs of one chunk per workgroup (the
// CB / C fragments are loaded once for them); (dm.H * P / PT) % SL == 0.
// YM: 0 the whole path's y; 1 stage M3's y_diag alone, cum from ck.cum and
// no 1e6 cap on the pair weight (kernel_mamba2_b_intra.py:96-108); 2 stage
// M4's combine, y = sanitize(y_diag + y_off) with y_diag from ck.ydiag and
// cum from ck.cum (kernel_mamba2_c_interchunk.py:68-78).
template <typename T, int C, int P, int N, int PT, int SL, int YM = 0>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(2, 2))) void mamba2_chunk_y(Mamba2Dims dm, const T* __restrict__ dt,
                                                     const T* __restrict__ x, const float* __restrict__ A,
                                                     const T* __restrict__ Cm, Mamba2Chunks<T> ck,
                                                     float* __restrict__ y) {
  typedef YLds<T, C, N, PT> L;
  __shared__ __attribute__((aligned(16))) unsigned char lds[L::total];
  float* sCum = reinterpret_cast<float*>(lds + L::off_cum);
  float* sDbx = reinterpret_cast<float*>(lds + L::off_dbx);
  T* sV = reinterpret_cast<T*>(lds + L::off_v);
  T* sSt = reinterpret_cast<T*>(lds + L::off_st);
  float* sTot = reinterpret_cast<float*>(lds + L::off_tot);

  constexpr int NPT = P / PT;
  int bn, m2;
  xcd_group_map(blockIdx.x, dm.B * dm.NT, dm.H * NPT / SL, bn, m2);
  const int bb = bn / dm.NT, n = bn % dm.NT;
  const size_t row0 = (size_t)bb * dm.T + (size_t)n * C;
  const size_t rsx = (size_t)dm.H * P;
  const T* cbg = ck.cb + (size_t)bn * C * C;
  const T* cg = Cm + row0 * dm.rC;
  const int ldc = (int)dm.rC;
  constexpr int NB = C / 16, BPW = NB / 4, YNI = PT / 16, KN = N / Mma<T>::KS;
  static_assert(NB % 4 == 0, "row blocks must split evenly over 4 waves");
  // compiled per wave (its output blocks are constants): the fragment arrays
  // hold exactly the blocks used and no branch depends on the block index
  static_switch<4>(wave_id(), [&](auto Wc) {
  constexpr int W = decltype(Wc)::value;

  // the global operands of the output blocks (CB fragments, C rows), shared by
  // the workgroup's slices, requested before the first slice's cumsum
  typedef typename Mma<T>::frag frag;
  frag fa[BPW][NB], fd[BPW], fc[BPW][KN];
  static_for<BPW>([&](auto Bc) {
    constexpr int bi = decltype(Bc)::value, I = y_block<NB>(W, bi);
    if constexpr (YM != 2) {
#pragma unroll
      for (int J = 0; J < I; ++J) fa[bi][J] = cb_frag<T>(cbg, C, 16 * I, 16 * J, 0);
      fd[bi] = cb_frag<T>(cbg, C, 16 * I, 16 * I, 1);
    }
    if constexpr (YM != 1) {
#pragma unroll
      for (int kk = 0; kk < KN; ++kk) fc[bi][kk] = Mma<T>::ld_c(cg, ldc, 16 * I, kk * Mma<T>::KS);
    }
  });
  // thread item = 8 channels of one row; 16 consecutive items take 16
  // consecutive rows (conflict-free 16-byte LDS accesses)
  constexpr int PER_ROW = PT / 8, NE = C * PER_ROW, EPT = NE / 256;
  static_assert(NE % 256 == 0, "slice must split evenly over the workgroup");
  auto item_row = [](int e) { return (e % 16) + 16 * (e / (16 * PER_ROW)); };
  auto item_col = [](int e) { return ((e / 16) % PER_ROW) * 8; };
  auto slice_base = [&](int sl) {
    const int m = m2 * SL + sl;
    return (row0 * dm.H + m / NPT) * P + (m % NPT) * PT;
  };
  auto slice_hp = [&](int sl) {  // the slice's column within an input row
    const int m = m2 * SL + sl;
    return (size_t)(m / NPT) * P + (m % NPT) * PT;
  };
  // dt, x of a slice: the next slice's are requested once the current one's
  // registers are free, so their latency overlaps its MFMA phase
  Raw8<T> rdt[EPT], rx[EPT];
  auto load_dtx = [&](int sl) {
    const size_t hp = slice_hp(sl);
#pragma unroll
    for (int i = 0; i < EPT; ++i) {
      const int e = threadIdx.x + 256 * i, r = item_row(e), c = item_col(e);
      rdt[i].load(dt + (row0 + r) * dm.rdt + hp + c);
      rx[i].load(x + (row0 + r) * dm.rx + hp + c);
    }
  };
  if constexpr (YM != 2) load_dtx(0);
  for (int sl = 0; sl < SL; ++sl) {
  const int m = m2 * SL + sl;
  const int h = m / NPT, p0 = (m % NPT) * PT;
  const size_t base = slice_base(sl);
  const float Ah = YM == 0 ? A[h] : 0.f;
  if constexpr (YM != 1)
    stage_rows<T, PT, N>(sSt, L::LN, ck.state_pre + (((size_t)bn * dm.H + h) * P + p0) * N, N);
  if constexpr (YM != 0)
    load_cum_rows<C, PT, L::LC>(sCum, ck.cum + (((size_t)bb * dm.H + h) * dm.NT + n) * C * P + p0, P);
  int flag = 0;
  if constexpr (YM != 2) {
#pragma unroll
    for (int i = 0; i < EPT; ++i) {
      const int e = threadIdx.x + 256 * i, r = item_row(e), c = item_col(e);
      float av[8], dbx[8];
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        const float a = rdt[i][j] * Ah;
        flag |= YM == 0 && a > 0.f;
        av[j] = sanitize(a, kClipDecay);
        dbx[j] = sanitize(rdt[i][j] * rx[i][j]);
      }
      if constexpr (YM == 0) store8(sCum + r * L::LC + c, av);
      store8(sDbx + r * L::LC + c, dbx);
    }
    // the 16 zero rows below the chunk (read by the K = 32 steps of the last block)
    if (threadIdx.x < 16 * PER_ROW) {
      const int r = C + threadIdx.x / PER_ROW, c = (threadIdx.x % PER_ROW) * 8;
      *reinterpret_cast<uint4*>(sV + r * L::LPT + c) = make_uint4(0u, 0u, 0u, 0u);
    }
  }
  __syncthreads();
  if constexpr (YM == 0) {
    column_cumsum<C, PT, L::LC>(sCum, sTot);
    __syncthreads();
  }
  bool exact = false;
  if constexpr (YM != 2) {
  for (int e = threadIdx.x; e < NB * PT; e += 256) {
    const int I = e / PT, p = e % PT;
    flag |= sCum[16 * I * L::LC + p] - sCum[(16 * I + 15) * L::LC + p] > kMaxRange;
  }
  if constexpr (YM == 1) {
    // the caller's cum: a rise between consecutive rows is a positive step
    for (int e = threadIdx.x; e < (C - 1) * PT; e += 256) {
      const int r = 1 + e / PT, p = e % PT;
      flag |= sCum[r * L::LC + p] > sCum[(r - 1) * L::LC + p];
    }
  }
  // a positive step exponent (or too steep a block) is evaluated pairwise
  exact = __builtin_amdgcn_readfirstlane(__syncthreads_or(flag)) != 0;
  if (!exact) {
#pragma unroll
    for (int i = 0; i < EPT; ++i) {
      const int e = threadIdx.x + 256 * i, r = item_row(e), c = item_col(e);
      float cr[8], ce[8], v[8];
      load8(sCum + r * L::LC + c, cr);
      load8(sCum + (r | 15) * L::LC + c, ce);
#pragma unroll
      for (int j = 0; j < 8; ++j) v[j] = __expf(ce[j] - cr[j]) * sanitize(rdt[i][j] * rx[i][j]);
      store8(sV + r * L::LPT + c, v);
    }
  }
  if (sl + 1 < SL) load_dtx(sl + 1);
  }  // YM != 2
  __syncthreads();

  // this lane's y elements: a uniform base and 32-bit lane offsets
  float* const yb = y + base;
  const unsigned ylane = (unsigned)tile_row(0) * (unsigned)rsx + (unsigned)tile_col();
  static_for<BPW>([&](auto Bc) {
    constexpr int bi = decltype(Bc)::value, I = y_block<NB>(W, bi);
    f32x4 off[YNI], yo[YNI];
#pragma unroll
    for (int ni = 0; ni < YNI; ++ni) { off[ni] = zero4(); yo[ni] = zero4(); }
    if (YM != 2 && !exact) {
      // off = sum_{J < I} M_IJ (CB_IJ Vd_J) + M_II (tril(CB_II) Vd_I): with the row
      // scale U_i below, the diagonal term becomes exp(cum_i - cum_{16I+15}) (.)
      static_for<I + 1>([&](auto Jc) {
        constexpr int J = decltype(Jc)::value;
        frag a;
        if constexpr (J < I) a = fa[bi][J];
        else a = fd[bi];
#pragma unroll
        for (int ni = 0; ni < YNI; ++ni) {
          const f32x4 q = Mma<T>::mma(a, Mma<T>::ld_t(sV, L::LPT, 16 * ni, 16 * J), zero4());
          const int pc = 16 * ni + tile_col();
          const float mf = __expf(sCum[16 * I * L::LC + pc] - sCum[(16 * J + 15) * L::LC + pc]);
#pragma unroll
          for (int k = 0; k < 4; ++k) off[ni][k] += mf * q[k];
        }
      });
    }
    if constexpr (YM != 1) {
#pragma unroll
      for (int kk = 0; kk < KN; ++kk) {
#pragma unroll
        for (int ni = 0; ni < YNI; ++ni)
          yo[ni] = Mma<T>::mma(fc[bi][kk], Mma<T>::ld_c(sSt, L::LN, 16 * ni, kk * Mma<T>::KS), yo[ni]);
      }
    }
#pragma unroll
    for (int ni = 0; ni < YNI; ++ni) {
#pragma unroll
      for (int k = 0; k < 4; ++k) {
        const int i = 16 * I + tile_row(k), p = 16 * ni + tile_col();
        const float ci = sCum[i * L::LC + p];
        const unsigned yi = ylane + (unsigned)(16 * I + k) * (unsigned)rsx + 16 * ni;
        float ydiag = 0.f;
        if constexpr (YM != 2) {
          if (!exact) {
            ydiag = off[ni][k] * __expf(ci - sCum[16 * I * L::LC + p]);
          } else {
            for (int j = 0; j <= i; ++j) {
              const float dd = fminf(fmaxf(ci - sCum[j * L::LC + p], -kClipDecay), kClipDecay);
              const float wgt = YM == 1 ? __expf(dd) : fminf(__expf(dd), 1e6f);
              ydiag += wgt * to_f(cbg[(size_t)i * C + j]) * sDbx[j * L::LC + p];
            }
          }
        }
        const float yoff = YM == 1 ? 0.f : sanitize(yo[ni][k] * __expf(fminf(fmaxf(ci, -kClipDecay), 0.f)));
        float yv;
        if constexpr (YM == 0) yv = sanitize(sanitize(ydiag) + yoff);
        else if constexpr (YM == 1) yv = sanitize(ydiag);
        else yv = sanitize(ck.ydiag[base + yi] + yoff);
        yb[yi] = yv;
      }
    }
  });
  __syncthreads();  // the next slice rewrites the LDS
  }
  });
}

}  // namespace ah
