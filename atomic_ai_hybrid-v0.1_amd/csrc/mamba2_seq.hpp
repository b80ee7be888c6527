// Mamba2 sequential state passes that take each chunk's contribution on chip.
//
// mamba2_chunk_outer leaves each chunk's S in HBM (bf16 [B][T][H][P]: the
// forward's dBx dte, the backward's Ydh = dy decay_h) and its cum_last;
// these loops form the per-chunk contribution S^T R (R = B forward, C
// backward) on MFMA as they go, so its fp32 [P][N] copy never reaches HBM:
//   forward   state_pre[n] = state (bf16);
//             state = sanitize(state exp(clip(cum_last, -20, 0)) + sanitize(S^T B))
//                                                    (mamba2_ssd_reference.py:133-146)
//   backward  dstate[n] = carry (bf16); d_cum_last_a = sum_s carry state_prev
//             decay_chunk_end mask; carry = sanitize(carry decay_chunk_end + S^T C)
//                                                    (mamba2_bwd_reference.py:115-128,195)
// One workgroup of NW waves carries one (batch, head, 32 channels) state,
// each wave N / NW of its state columns (NW = 8: two waves per SIMD, so one
// wave's LDS and MFMA latencies overlap the other's work).  A step stages the
// next chunk's S and rows in the other LDS buffer (their loads were issued
// two steps earlier), runs this chunk's product and the recurrence, and ends
// in the step's one barrier.
//
// The product is the MFMA of the stage-mode state_end in mamba2_chunk_outer
// over the same bf16 operands, so where the two forms' clips agree the
// states equal those of the staged forward (M3 state_end, then M4) bit for
// bit.
#pragma once
#include "mamba2.hpp"

namespace ah {

template <typename T, int C, int N>
struct ChainLds {
  static constexpr int PW = 32;                     // channels per workgroup
  static constexpr int LN = N + Pad<T>::v;          // B / C rows
  static constexpr int LS = PW + Pad<T>::v;         // S rows
  static constexpr int R_BYTES = C * LN * (int)sizeof(T);
  static constexpr int S_BYTES = C * LS * (int)sizeof(T);
  static constexpr int off_r = 0;                        // rows, two buffers
  static constexpr int off_s = off_r + 2 * R_BYTES;      // S, two buffers
  static constexpr int off_cl = off_s + 2 * S_BYTES;     // cum_last, two buffers of PW
  static constexpr int off_red = off_cl + 2 * PW * 4;    // backward: [2][8][PW] row-term partials
  static constexpr int total = off_red + 2 * 8 * PW * 4;
  static_assert(off_s % 16 == 0, "16-byte LDS rows");
};

// Grid: B H P / 32 workgroups of 64 NW threads; H P / 32 workgroups per batch
// row, dealt so that each XCD holds consecutive ones (the rows of one batch
// stay in one L2).
template <typename T, int C, int P, int N, bool BWD, int NW>
__global__ __launch_bounds__(64 * NW) void mamba2_state_chain(Mamba2Dims dm, const T* __restrict__ S,
                                                         const T* __restrict__ R, Mamba2Chunks<T> ck,
                                                         T* __restrict__ dstate, float* __restrict__ lasta,
                                                         const float* __restrict__ init, float* __restrict__ fin) {
  typedef ChainLds<T, C, N> L;
  constexpr int PW = L::PW;
  static_assert(P % PW == 0 && (NW == 4 || NW == 8) && N % (16 * NW) == 0, "whole 16-column tiles per wave");
  constexpr int NTH = 64 * NW;
  constexpr int NWV = N / NW;          // state columns per wave
  constexpr int NTI = NWV / 16;        // state tiles per wave
  constexpr int PTI = PW / 16;         // channel tiles
  constexpr int GPH = P / PW;          // workgroups per head
  __shared__ __attribute__((aligned(16))) unsigned char lds[L::total];
  const int wv = wave_id(), lane = lane_id();
  float* sCl = reinterpret_cast<float*>(lds + L::off_cl);
  float* sRed = reinterpret_cast<float*>(lds + L::off_red);

  int wg = blockIdx.x;
  if (gridDim.x % 8 == 0) wg = (blockIdx.x % 8) * (gridDim.x / 8) + blockIdx.x / 8;
  const int bh = wg / GPH, p0 = (wg % GPH) * PW;
  const int bb = bh / dm.H, h = bh % dm.H;
  const int NT = dm.NT;
  const size_t rR = BWD ? (size_t)dm.rC : (size_t)dm.rB;
  const size_t rS = (size_t)dm.H * P;
  const int pl = lane & 15, g4 = lane >> 4;    // tile column, row group

  auto chunk_of = [&](int it) { return BWD ? NT - 1 - it : it; };
  auto rows0 = [&](int n) { return (size_t)bb * dm.T + (size_t)n * C; };
  auto srow = [&](int n) { return ((((size_t)bb * NT + n) * dm.H + h) * P) * N; };   // [B][NT][H][P][N]
  auto clrow = [&](int n) { return (((size_t)bb * NT + n) * dm.H + h) * P + p0; };   // [B][NT][H][P]
  // state element (tile i, j; k) of this lane: channel p0 + 16 j + pl, column
  // NWV wv + 16 i + 4 g4 + k of a [P][N] state
  auto soff = [&](int i, int j) { return (size_t)(p0 + 16 * j + pl) * N + NWV * wv + 16 * i + 4 * g4; };

  f32x4 st[NTI][PTI];
#pragma unroll
  for (int i = 0; i < NTI; ++i)
#pragma unroll
    for (int j = 0; j < PTI; ++j) {
      st[i][j] = zero4();
      if (init) {
        const float4 v = *reinterpret_cast<const float4*>(init + (size_t)bh * P * N + soff(i, j));
        st[i][j][0] = v.x; st[i][j][1] = v.y; st[i][j][2] = v.z; st[i][j][3] = v.w;
        if (!BWD && dm.sanitize_state0)
#pragma unroll
          for (int k = 0; k < 4; ++k) st[i][j][k] = sanitize(st[i][j][k]);
      }
    }

  // one chunk's S [C][PW], rows [C][N] and (wave 0) cum_last; two sets, so
  // a chunk's loads are issued two steps before it is staged
  struct In {
    RegStage<T, C, PW, NTH> s;
    RegStage<T, C, N, NTH> r;
    float cl;
  };
  In inA, inB;
  uint2 isp[NTI][PTI];   // backward: this lane's state_pre elements of the next chunk
  auto load = [&](In& in, int it) {
    const int n = chunk_of(it < NT ? it : NT - 1);   // past the last chunk: that chunk again
    const size_t r0 = rows0(n);
    in.s.load(S + r0 * rS + (size_t)h * P + p0, rS);
    in.r.load(R + r0 * rR, rR);
    if (wv == 0 && lane < PW) in.cl = ck.cl[clrow(n) + lane];
  };
  auto stage = [&](const In& in, int it) {
    in.s.store(reinterpret_cast<T*>(lds + L::off_s + (it & 1) * L::S_BYTES), L::LS);
    in.r.store(reinterpret_cast<T*>(lds + L::off_r + (it & 1) * L::R_BYTES), L::LN);
    if (wv == 0 && lane < PW) sCl[(it & 1) * PW + lane] = in.cl;
  };
  auto load_sp = [&](int it) {
    const int n = chunk_of(it < NT ? it : NT - 1);
#pragma unroll
    for (int i = 0; i < NTI; ++i)
#pragma unroll
      for (int j = 0; j < PTI; ++j)
        isp[i][j] = *reinterpret_cast<const uint2*>(ck.state_pre + srow(n) + soff(i, j));
  };

  // one step: `in` holds chunk it + 1 on entry and chunk it + 3 on exit
  auto step = [&](In& in, int it) {
    const int n = chunk_of(it);
    // the next chunk into the other buffers (read two steps ago, before the
    // previous step's barrier); past the last chunk, the last one again
    stage(in, it + 1);
    load(in, it + 3);
    // out^T[s][p] = sum_t R[t][s] S[t][p] over this wave's state columns
    const T* sS = reinterpret_cast<const T*>(lds + L::off_s + (it & 1) * L::S_BYTES);
    const T* sR = reinterpret_cast<const T*>(lds + L::off_r + (it & 1) * L::R_BYTES);
    f32x4 acc[NTI][PTI];
#pragma unroll
    for (int i = 0; i < NTI; ++i) {
#pragma unroll
      for (int j = 0; j < PTI; ++j) acc[i][j] = zero4();
      tile_mma_row<T, true, true, PTI>(acc[i], sR, L::LN, sS, L::LS, NWV * wv + 16 * i, 0, C);
    }
    uint2 sp[NTI][PTI];
    if constexpr (BWD) {
#pragma unroll
      for (int i = 0; i < NTI; ++i)
#pragma unroll
        for (int j = 0; j < PTI; ++j) sp[i][j] = isp[i][j];
    }
    T* sout = (BWD ? dstate : ck.state_pre) + srow(n);
#pragma unroll
    for (int j = 0; j < PTI; ++j) {
      const float cl = sCl[(it & 1) * PW + 16 * j + pl];
      const float dce = __expf(fminf(fmaxf(cl, -kClipDecay), 0.f));
      float part = 0.f;
#pragma unroll
      for (int i = 0; i < NTI; ++i) {
        store4(sout + soff(i, j), st[i][j]);
        if constexpr (BWD) {
          const T* spv = reinterpret_cast<const T*>(&sp[i][j]);
#pragma unroll
          for (int k = 0; k < 4; ++k) part += st[i][j][k] * to_f(spv[k]);
#pragma unroll
          for (int k = 0; k < 4; ++k) st[i][j][k] = sanitize(st[i][j][k] * dce + acc[i][j][k]);
        } else {
#pragma unroll
          for (int k = 0; k < 4; ++k) st[i][j][k] = sanitize(st[i][j][k] * dce + sanitize(acc[i][j][k]));
        }
      }
      if constexpr (BWD) {
        part += __shfl_xor(part, 16);
        part += __shfl_xor(part, 32);
        if (g4 == 0) sRed[((it & 1) * NW + wv) * PW + 16 * j + pl] = part;
      }
    }
    if constexpr (BWD) load_sp(it + 1);
    __syncthreads();
    if constexpr (BWD) {
      // wave 0 alone writes cum_last buffer it & 1 again, two steps on
      if (wv == 0 && lane < PW) {
        const float* rd = sRed + (it & 1) * NW * PW + lane;
        float tot = rd[0];
#pragma unroll
        for (int w = 1; w < NW; ++w) tot += rd[w * PW];
        const float cl = sCl[(it & 1) * PW + lane];
        const float dce = __expf(fminf(fmaxf(cl, -kClipDecay), 0.f));
        const float msk = (cl >= -kClipDecay && cl <= 0.f) ? 1.f : 0.f;
        lasta[clrow(n) + lane] = tot * dce * msk;
      }
    }
  };

  load(inA, 0);
  if constexpr (BWD) load_sp(0);
  stage(inA, 0);
  load(inA, 1);
  load(inB, 2);
  __syncthreads();
  int it = 0;
  for (; it + 2 <= NT; it += 2) {
    step(inA, it);
    step(inB, it + 1);
  }
  if (it < NT) step(inA, it);
  if (fin) {
#pragma unroll
    for (int i = 0; i < NTI; ++i)
#pragma unroll
      for (int j = 0; j < PTI; ++j) {
        float4 v;
        v.x = st[i][j][0]; v.y = st[i][j][1]; v.z = st[i][j][2]; v.w = st[i][j][3];
        if (BWD) { v.x = sanitize(v.x); v.y = sanitize(v.y); v.z = sanitize(v.z); v.w = sanitize(v.w); }
        *reinterpret_cast<float4*>(fin + (size_t)bh * P * N + soff(i, j)) = v;
      }
  }
}

}  // namespace ah
