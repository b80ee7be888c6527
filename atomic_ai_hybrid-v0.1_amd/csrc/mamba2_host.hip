// Host side of the Mamba2 SSD chunk scan: argument checks, workspace layout,
// template dispatch and the extern "C" entry points of include/atomic_hybrid.h.
#include "../../include/atomic_hybrid.h"
#include "diag.hpp"
#include "mamba2_bwd.hip"
#include "launch.hpp"
#include "stage256.hpp"
#include "ws_tag.hpp"

namespace ah {

static size_t m2_align(size_t x) { return (x + 255) & ~size_t(255); }

struct Mamba2Plan {
  Mamba2Dims dm;
  size_t o_cb, o_state, o_cl, o_rows, o_src;
  size_t o_dstate, o_lasta, o_wr, o_part, o_dap, total;
  int G;       // head groups of the cross-head dCB reduction
  bool chain;  // state loops with the per-chunk product on chip (else two passes)
  bool f32;    // fp32 operands: the float32 staged kernels, at the caller's chunk (f32dm)
  Mamba2Dims f32dm;
};

static int mamba2_plan(const atomic_mamba2_args* a, Mamba2Plan* p) {
  if (!a) return ATOMIC_ERR_NULL;
  if (a->dtype != ATOMIC_BF16 && a->dtype != ATOMIC_F32) return ATOMIC_ERR_DTYPE;
  if (a->dy_dtype != ATOMIC_F32 && a->dy_dtype != ATOMIC_BF16) return ATOMIC_ERR_DTYPE;
  if (a->batch <= 0 || a->heads <= 0 || a->seqlen <= 0) return ATOMIC_ERR_SHAPE;
  if (a->chunk != 64 && a->chunk != 128 && a->chunk != 256) return ATOMIC_ERR_SHAPE;
  if (a->seqlen % a->chunk != 0) return ATOMIC_ERR_SHAPE;
  if (a->headdim != 64 && a->headdim != 128 && a->headdim != 192) return ATOMIC_ERR_SHAPE;
  if (a->dstate != 64 && a->dstate != 128) return ATOMIC_ERR_SHAPE;
  if (a->headdim == 192 && a->dstate != 128) return ATOMIC_ERR_SHAPE;
  Mamba2Dims d;
  d.B = a->batch; d.T = a->seqlen; d.H = a->heads; d.P = a->headdim; d.N = a->dstate;
  d.sanitize_state0 = (a->flags & ATOMIC_MAMBA2_SANITIZE_STATE0) != 0;
  // Chunk 256 (the model's chunk_size = min(256, L), model.py:436) runs as
  // 128-row chunks.  With every step exponent dt A <= 0 (the model's A < 0,
  // dt > 0) the two differ only in the reference's exp(-20) floors on pairs
  // 128..255 rows apart and on the old state's decay, below 1e-7 of y; with a
  // positive exponent the reference's per-chunk caps (1e6 on the pair weight,
  // exp(20) on the decay to the chunk end) apply over 256 rows instead.
  d.C = a->chunk == 256 ? 128 : a->chunk;
  d.NT = a->seqlen / d.C;
  {
    const long long dP = (long long)a->heads * a->headdim, dN = a->dstate;
    const long long dense[5] = {dP, dP, dN, dN, dP};
    long long* out[5] = {&d.rdt, &d.rx, &d.rB, &d.rC, &d.rdy};
    for (int i = 0; i < 5; ++i) {
      const long long s = a->row_stride[i];
      if (s != 0 && (s < dense[i] || s % 8 != 0)) return ATOMIC_ERR_SHAPE;
      *out[i] = s ? s : dense[i];
    }
  }
  p->dm = d;
  p->f32 = a->dtype == ATOMIC_F32;
  p->f32dm = d;
  p->f32dm.C = a->chunk;
  p->f32dm.NT = a->seqlen / a->chunk;
  const size_t es = 2, B = d.B, H = d.H, NT = d.NT, C = d.C, P = d.P, N = d.N, T = d.T;
  // enough (batch, chunk, head group) workgroups for two rounds of the chip's
  // 256 CUs (one 8-wave workgroup each); more groups (1024 workgroups) cost
  // 2-3 % in the chunk backward and its dB / dC reduction at the benchmark shape
  int G = 1;
  while ((size_t)G * B * NT < 512 && (size_t)(2 * G) <= H && H % (size_t)(2 * G) == 0) G *= 2;
  p->G = G;
  // The state loops walk the chunks with one 32-channel workgroup per
  // (batch, head, slice) and form each chunk's product on chip; their step is
  // latency-bound, so they pay only when the workgroups fill the 256 CUs.
  // Smaller grids (long sequences over few heads) run the two-pass form: the
  // chunk kernel writes each chunk's fp32 product and an element-wise pass
  // with four chunks in flight carries the state (configuration 4, B1 H64
  // P64 over 256 chunks: 3.15 against 3.37 ms for its Mamba2 fwd + bwd).
  p->chain = B * H * (P / 32) >= 256;
  size_t off = 0;
  auto take = [&](size_t bytes) { size_t o = off; off += m2_align(bytes); return o; };
  p->o_cb = take(B * NT * C * C * es);
  p->o_state = take(B * NT * H * P * N * es);        // state entering each chunk
  p->o_cl = take(B * NT * H * P * 4);                // cum at each chunk's last row
  // S rows: the state loops' forward dBx dte, then the backward's Ydh =
  // dy decay_h (a REUSE backward needs only the states and cum_last)
  p->o_rows = take(B * T * H * P * es);
  // the two-pass form's per-chunk product (forward state_end, backward (dy decay_h)^T C)
  p->o_src = p->chain ? 0 : take(B * NT * H * P * N * 4);
  p->o_dstate = take(B * NT * H * P * N * es);       // dstate entering each chunk's backward
  p->o_lasta = take(B * NT * H * P * 4);             // d cum_last from decay_chunk_end
  p->o_wr = take(B * T * H * P * es);                // sanitize(dBx decay_to_end)
  p->o_part = take(B * NT * (size_t)p->G * C * C * 4);  // dCB per head group
  p->o_dap = take(B * NT * H * 4);                   // per-chunk dA
  p->total = off;
  return ATOMIC_OK;
}

template <typename T>
static Mamba2Chunks<T> mamba2_chunks(const Mamba2Plan& p, void* ws) {
  char* base = static_cast<char*>(ws);
  Mamba2Chunks<T> c;
  c.cb = reinterpret_cast<T*>(base + p.o_cb);
  c.state_pre = reinterpret_cast<T*>(base + p.o_state);
  c.cl = reinterpret_cast<float*>(base + p.o_cl);
  c.src = p.chain ? nullptr : reinterpret_cast<float*>(base + p.o_src);
  c.cum = nullptr;
  c.ydiag = nullptr;
  return c;
}

template <typename T>
static Mamba2Grads<T> mamba2_grads(const Mamba2Plan& p, void* ws) {
  char* base = static_cast<char*>(ws);
  Mamba2Grads<T> g;
  g.dstate = reinterpret_cast<T*>(base + p.o_dstate);
  g.lasta = reinterpret_cast<float*>(base + p.o_lasta);
  g.ydh = reinterpret_cast<T*>(base + p.o_rows);
  g.wr = reinterpret_cast<T*>(base + p.o_wr);
  g.part = reinterpret_cast<float*>(base + p.o_part);
  g.dap = reinterpret_cast<float*>(base + p.o_dap);
  return g;
}

// channels per workgroup of the chunk-parallel kernels
constexpr int kOuterPT = 64, kYPT = 32;
// the workgroups of two per CU on the 256 CUs: chunk-parallel kernels take
// fewer pairs per workgroup on grids smaller than this
constexpr size_t kFullGrid = 512;

template <int P, int N>
static unsigned pass_grid(const Mamba2Dims& d) {
  constexpr int RP = 256 / (N / 4);
  return (unsigned)(d.B * d.H * (P / RP));
}

// The state loops: one workgroup per (batch, head, 32 channels), eight waves
// (four at N = 64, whose 64 columns make four 16-column tiles).
template <typename T, int C, int P, int N, bool BWD>
static void launch_state_chain(const Mamba2Dims& d, hipStream_t st, const T* S, const T* R,
                               const Mamba2Chunks<T>& ck, T* dstate, float* lasta, const float* init,
                               float* fin) {
  constexpr int NW = N == 128 ? 8 : 4;
  hipLaunchKernelGGL((mamba2_state_chain<T, C, P, N, BWD, NW>), dim3((unsigned)(d.B * d.H * (P / 32))),
                     dim3(64 * NW), 0, st, d, S, R, ck, dstate, lasta, init, fin);
}

// Forward: CB, the chunks' S rows and cum_last, the state loop and (when y
// is wanted) the outputs.  The state entering every chunk always lands in
// the workspace.
template <int C, int P, int N>
static int mamba2_forward_impl(const Mamba2Plan& p, const void* dt, const void* x, const void* Bm,
                               const void* Cm, const float* A, const float* state0, float* y,
                               float* state_final, void* ws, Launch& L) {
  typedef bf16 T;
  const Mamba2Dims& d = p.dm;
  Mamba2Chunks<T> ck = mamba2_chunks<T>(p, ws);
  hipStream_t st = L.st;
  int rc = L("mamba2_cb", [&] {
    // one workgroup per chunk, or per 32-row block when the chunks are fewer
    // than the CUs (B2 T4096: 0.011 -> 0.007 ms)
    if (d.B * d.NT >= 256)
      hipLaunchKernelGGL((mamba2_cb<T, C, N>), dim3((unsigned)(d.B * d.NT)), dim3(256), 0, st, d,
                         (const T*)Bm, (const T*)Cm, ck);
    else
      hipLaunchKernelGGL((mamba2_cb<T, C, N, 32>), dim3((unsigned)(d.B * d.NT * (C / 32))), dim3(256), 0, st,
                         d, (const T*)Bm, (const T*)Cm, ck);
  });
  if (rc) return rc;
  constexpr int NPO = P / kOuterPT;
  if (p.chain) {
    // the chunk's S rows and cum_last, one workgroup per (batch, chunk, head,
    // 64 channels) (eight pairs per workgroup: 0.094 against 0.086 ms at the
    // benchmark shape), then the state loop with S^T B on chip
    T* srows = reinterpret_cast<T*>(static_cast<char*>(ws) + p.o_rows);
    rc = L("mamba2_chunk_rows", [&] {
      hipLaunchKernelGGL((mamba2_chunk_outer<T, T, C, P, N, kOuterPT, false, 1>),
                         dim3((unsigned)(d.B * d.NT * d.H * NPO)), dim3(256), 0, st, d, (const T*)dt,
                         (const T*)x, A, (const T*)nullptr, (const T*)nullptr, ck, srows, (T*)nullptr);
    });
    if (rc) return rc;
    rc = L("mamba2_state_chain", [&] {
      launch_state_chain<T, C, P, N, false>(d, st, srows, (const T*)Bm, ck, (T*)nullptr, (float*)nullptr,
                                            state0, state_final);
    });
  } else {
    // chunk_outer workgroups take 8 (head, channel slice) pairs of one chunk,
    // 4 when 8 would leave fewer than two workgroups per CU (0.045 -> 0.039 ms
    // at B2 T4096 H32 P64), else one head's slices; the backward likewise
    rc = L("mamba2_chunk_state", [&] {
      const size_t pairs = (size_t)d.H * NPO;
      if (pairs % 8 == 0 && d.B * d.NT * pairs / 8 >= kFullGrid)
        hipLaunchKernelGGL((mamba2_chunk_outer<T, T, C, P, N, kOuterPT, false, 8, false, true>),
                           dim3((unsigned)(d.B * d.NT * pairs / 8)), dim3(256), 0, st, d, (const T*)dt,
                           (const T*)x, A, (const T*)Bm, (const T*)nullptr, ck, (T*)nullptr, (T*)nullptr);
      else if (pairs % 4 == 0 && d.B * d.NT * pairs / 4 >= kFullGrid)
        hipLaunchKernelGGL((mamba2_chunk_outer<T, T, C, P, N, kOuterPT, false, 4, false, true>),
                           dim3((unsigned)(d.B * d.NT * pairs / 4)), dim3(256), 0, st, d, (const T*)dt,
                           (const T*)x, A, (const T*)Bm, (const T*)nullptr, ck, (T*)nullptr, (T*)nullptr);
      else
        hipLaunchKernelGGL((mamba2_chunk_outer<T, T, C, P, N, kOuterPT, false, NPO, false, true>),
                           dim3((unsigned)(d.B * d.NT * d.H)), dim3(256), 0, st, d, (const T*)dt,
                           (const T*)x, A, (const T*)Bm, (const T*)nullptr, ck, (T*)nullptr, (T*)nullptr);
    });
    if (rc) return rc;
    rc = L("mamba2_state_pass", [&] {
      hipLaunchKernelGGL((mamba2_state_pass<T, P, N, false>), dim3(pass_grid<P, N>(d)), dim3(256), 0, st,
                         d, ck, (T*)nullptr, (float*)nullptr, state0, state_final);
    });
  }
  if (rc || !y) return rc;
  // chunk_y workgroups take SL (head, channel slice) pairs of one chunk: 16
  // when they divide the pairs and the grid still holds two workgroups per
  // CU, else 8 under the same condition, else 4 (small batches: 0.093 ->
  // 0.066 ms at B2 T4096 H32 P64), else the channel slices of one head
  constexpr int NPT = P / kYPT;
  const size_t pairs = (size_t)d.H * NPT;
  return L("mamba2_chunk_y", [&] {
    if (pairs % 16 == 0 && d.B * d.NT * pairs / 16 >= kFullGrid)
      hipLaunchKernelGGL((mamba2_chunk_y<T, C, P, N, kYPT, 16>), dim3((unsigned)(d.B * d.NT * pairs / 16)),
                         dim3(256), 0, st, d, (const T*)dt, (const T*)x, A, (const T*)Cm, ck, y);
    else if (pairs % 8 == 0 && d.B * d.NT * pairs / 8 >= kFullGrid)
      hipLaunchKernelGGL((mamba2_chunk_y<T, C, P, N, kYPT, 8>), dim3((unsigned)(d.B * d.NT * pairs / 8)),
                         dim3(256), 0, st, d, (const T*)dt, (const T*)x, A, (const T*)Cm, ck, y);
    else if (pairs % 4 == 0)
      hipLaunchKernelGGL((mamba2_chunk_y<T, C, P, N, kYPT, 4>), dim3((unsigned)(d.B * d.NT * pairs / 4)),
                         dim3(256), 0, st, d, (const T*)dt, (const T*)x, A, (const T*)Cm, ck, y);
    else
      hipLaunchKernelGGL((mamba2_chunk_y<T, C, P, N, kYPT, NPT>), dim3((unsigned)(d.B * d.NT * d.H)),
                         dim3(256), 0, st, d, (const T*)dt, (const T*)x, A, (const T*)Cm, ck, y);
  });
}

template <int C, int P, int N, typename TD>
static int mamba2_backward_t(const Mamba2Plan& p, const void* dt, const void* x, const void* Bm,
                             const void* Cm, const float* A, const float* state0, const void* dy,
                             const float* dstate_final, void* ddt, void* dx, void* dB, void* dC,
                             float* dA, float* dstate0, void* ws, bool reuse, Launch& L);

#define AH_M2_DISPATCH(FN, ...)                                                         \
  do {                                                                                  \
    const int c_ = p.dm.C, p_ = p.dm.P, n_ = p.dm.N;                                    \
    if (c_ == 128 && p_ == 64 && n_ == 128) return FN<128, 64, 128>(__VA_ARGS__);       \
    if (c_ == 128 && p_ == 128 && n_ == 128) return FN<128, 128, 128>(__VA_ARGS__);     \
    if (c_ == 64 && p_ == 64 && n_ == 128) return FN<64, 64, 128>(__VA_ARGS__);         \
    if (c_ == 64 && p_ == 128 && n_ == 128) return FN<64, 128, 128>(__VA_ARGS__);       \
    if (c_ == 128 && p_ == 64 && n_ == 64) return FN<128, 64, 64>(__VA_ARGS__);         \
    if (c_ == 128 && p_ == 128 && n_ == 64) return FN<128, 128, 64>(__VA_ARGS__);       \
    if (c_ == 64 && p_ == 64 && n_ == 64) return FN<64, 64, 64>(__VA_ARGS__);           \
    if (c_ == 64 && p_ == 128 && n_ == 64) return FN<64, 128, 64>(__VA_ARGS__);         \
    if (c_ == 128 && p_ == 192 && n_ == 128) return FN<128, 192, 128>(__VA_ARGS__);     \
    if (c_ == 64 && p_ == 192 && n_ == 128) return FN<64, 192, 128>(__VA_ARGS__);       \
    return ATOMIC_ERR_SHAPE;                                                            \
  } while (0)

int mamba2_forward(const Mamba2Plan& p, const void* dt, const void* x, const void* Bm, const void* Cm,
                   const float* A, const float* state0, float* y, float* state_final, void* ws,
                   Launch& L) {
  AH_M2_DISPATCH(mamba2_forward_impl, p, dt, x, Bm, Cm, A, state0, y, state_final, ws, L);
}

template <int C, int P, int N, typename TD>
static int mamba2_backward_t(const Mamba2Plan& p, const void* dt, const void* x, const void* Bm,
                             const void* Cm, const float* A, const float* state0, const void* dy,
                             const float* dstate_final, void* ddt, void* dx, void* dB, void* dC,
                             float* dA, float* dstate0, void* ws, bool reuse, Launch& L) {
  typedef bf16 T;
  const Mamba2Dims& d = p.dm;
  int rc;
  if (!reuse) {
    // recompute the forward's per-chunk states (the reference re-runs the
    // forward scan, mamba2_bwd_reference.py:229-234)
    rc = mamba2_forward_impl<C, P, N>(p, dt, x, Bm, Cm, A, state0, nullptr, nullptr, ws, L);
    if (rc) return rc;
  }
  Mamba2Chunks<T> ck = mamba2_chunks<T>(p, ws);
  Mamba2Grads<T> gr = mamba2_grads<T>(p, ws);
  hipStream_t st = L.st;
  constexpr int NPO = P / kOuterPT;
  if (p.chain) {
    rc = L("mamba2_bwd_rows", [&] {
      hipLaunchKernelGGL((mamba2_chunk_outer<T, TD, C, P, N, kOuterPT, true, 1>),
                         dim3((unsigned)(d.B * d.NT * d.H * NPO)), dim3(256), 0, st, d, (const T*)dt,
                         (const T*)x, A, (const T*)nullptr, (const TD*)dy, ck, gr.ydh, gr.wr);
    });
    if (rc) return rc;
    rc = L("mamba2_bwd_state_chain", [&] {
      launch_state_chain<T, C, P, N, true>(d, st, gr.ydh, (const T*)Cm, ck, gr.dstate, gr.lasta,
                                           dstate_final, dstate0);
    });
  } else {
    rc = L("mamba2_bwd_source", [&] {
      const size_t pairs = (size_t)d.H * NPO;
      if (pairs % 8 == 0 && d.B * d.NT * pairs / 8 >= kFullGrid)
        hipLaunchKernelGGL((mamba2_chunk_outer<T, TD, C, P, N, kOuterPT, true, 8, false, true>),
                           dim3((unsigned)(d.B * d.NT * pairs / 8)), dim3(256), 0, st, d, (const T*)dt,
                           (const T*)x, A, (const T*)Cm, (const TD*)dy, ck, gr.ydh, gr.wr);
      else if (pairs % 4 == 0 && d.B * d.NT * pairs / 4 >= kFullGrid)
        hipLaunchKernelGGL((mamba2_chunk_outer<T, TD, C, P, N, kOuterPT, true, 4, false, true>),
                           dim3((unsigned)(d.B * d.NT * pairs / 4)), dim3(256), 0, st, d, (const T*)dt,
                           (const T*)x, A, (const T*)Cm, (const TD*)dy, ck, gr.ydh, gr.wr);
      else
        hipLaunchKernelGGL((mamba2_chunk_outer<T, TD, C, P, N, kOuterPT, true, NPO, false, true>),
                           dim3((unsigned)(d.B * d.NT * d.H)), dim3(256), 0, st, d, (const T*)dt,
                           (const T*)x, A, (const T*)Cm, (const TD*)dy, ck, gr.ydh, gr.wr);
    });
    if (rc) return rc;
    rc = L("mamba2_bwd_state_pass", [&] {
      hipLaunchKernelGGL((mamba2_state_pass<T, P, N, true>), dim3(pass_grid<P, N>(d)), dim3(256), 0, st,
                         d, ck, gr.dstate, gr.lasta, dstate_final, dstate0);
    });
  }
  if (rc) return rc;
  rc = L("mamba2_bwd_chunk", [&] {
    hipLaunchKernelGGL((mamba2_bwd_chunk<T, TD, C, P, N>), dim3((unsigned)(d.B * d.NT * p.G)),
                       dim3(512), 0, st, d, p.G, (const T*)dt, (const T*)x, A, (const T*)Bm,
                       (const T*)Cm, (const TD*)dy, ck, gr, (T*)ddt, (T*)dx);
  });
  if (rc) return rc;
  rc = L("mamba2_bwd_bc", [&] {
    // 64 state columns per workgroup: each chunk's Ydh / W rows are read half
    // as often as at 32 (32 on small grids measured no faster)
    constexpr int NTL = 64;
    hipLaunchKernelGGL((mamba2_bwd_bc<T, C, P, N, NTL>), dim3((unsigned)(d.B * d.NT * (N / NTL))), dim3(512),
                       0, st, d, p.G, (const T*)Bm, (const T*)Cm, ck, gr, (T*)dB, (T*)dC, dA);
  });
  return rc;
}

template <int C, int P, int N>
static int mamba2_backward_impl(const Mamba2Plan& p, int dy_dtype, const void* dt, const void* x,
                                const void* Bm, const void* Cm, const float* A, const float* state0,
                                const void* dy, const float* dstate_final, void* ddt, void* dx,
                                void* dB, void* dC, float* dA, float* dstate0, void* ws, bool reuse,
                                Launch& L) {
  if (dy_dtype == ATOMIC_BF16)
    return mamba2_backward_t<C, P, N, bf16>(p, dt, x, Bm, Cm, A, state0, dy, dstate_final, ddt, dx, dB,
                                            dC, dA, dstate0, ws, reuse, L);
  return mamba2_backward_t<C, P, N, float>(p, dt, x, Bm, Cm, A, state0, dy, dstate_final, ddt, dx, dB,
                                           dC, dA, dstate0, ws, reuse, L);
}

int mamba2_backward(const Mamba2Plan& p, int dy_dtype, const void* dt, const void* x, const void* Bm,
                    const void* Cm, const float* A, const float* state0, const void* dy,
                    const float* dstate_final, void* ddt, void* dx, void* dB, void* dC, float* dA,
                    float* dstate0, void* ws, bool reuse, Launch& L) {
  AH_M2_DISPATCH(mamba2_backward_impl, p, dy_dtype, dt, x, Bm, Cm, A, state0, dy, dstate_final, ddt, dx,
                 dB, dC, dA, dstate0, ws, reuse, L);
}

// Stage reports of the forward (CB, the states entering each chunk, y,
// state_final) and of the backward (the dstate entering each chunk's
// backward, then every gradient).
static int mamba2_forward_diag(const Mamba2Plan& p, StageDiag& D, const float* y, const float* state_final,
                               void* ws) {
  const Mamba2Dims& d = p.dm;
  const Mamba2Chunks<bf16> ck = mamba2_chunks<bf16>(p, ws);
  const size_t B = d.B, NT = d.NT, H = d.H, P = d.P, N = d.N, C = d.C, T = d.T;
  int rc;
  if ((rc = D.clear(0, ATOMIC_MAMBA2_DIAG_DSTATES))) return rc;
  if ((rc = D.reduce(ATOMIC_MAMBA2_DIAG_CB, ck.cb, B * NT * C * C))) return rc;
  if ((rc = D.reduce(ATOMIC_MAMBA2_DIAG_STATES, ck.state_pre, B * NT * H * P * N))) return rc;
  if ((rc = D.reduce(ATOMIC_MAMBA2_DIAG_Y, y, B * T * H * P))) return rc;
  return D.reduce(ATOMIC_MAMBA2_DIAG_STATE_FINAL, state_final, B * H * P * N);
}

static int mamba2_backward_diag(const Mamba2Plan& p, StageDiag& D, const void* ddt, const void* dx,
                                const void* dB, const void* dC, const float* dA, const float* dstate0,
                                void* ws) {
  const Mamba2Dims& d = p.dm;
  const Mamba2Grads<bf16> gr = mamba2_grads<bf16>(p, ws);
  const size_t B = d.B, NT = d.NT, H = d.H, P = d.P, N = d.N, T = d.T;
  int rc;
  if ((rc = D.clear(ATOMIC_MAMBA2_DIAG_DSTATES, ATOMIC_MAMBA2_DIAG_COUNT - ATOMIC_MAMBA2_DIAG_DSTATES)))
    return rc;
  if ((rc = D.reduce(ATOMIC_MAMBA2_DIAG_DSTATES, gr.dstate, B * NT * H * P * N))) return rc;
  if ((rc = D.reduce(ATOMIC_MAMBA2_DIAG_DDT, (const bf16*)ddt, B * T * H * P))) return rc;
  if ((rc = D.reduce(ATOMIC_MAMBA2_DIAG_DX, (const bf16*)dx, B * T * H * P))) return rc;
  if ((rc = D.reduce(ATOMIC_MAMBA2_DIAG_DB, (const bf16*)dB, B * T * N))) return rc;
  if ((rc = D.reduce(ATOMIC_MAMBA2_DIAG_DC, (const bf16*)dC, B * T * N))) return rc;
  if ((rc = D.reduce(ATOMIC_MAMBA2_DIAG_DA, dA, H))) return rc;
  return D.reduce(ATOMIC_MAMBA2_DIAG_DSTATE0, dstate0, B * H * P * N);
}

// ------------------------------------------------ stage-level forward
// The reference's M2, M3 and M4 (kernel_mamba2_a_decay.py:71,
// kernel_mamba2_b_intra.py:119, kernel_mamba2_c_interchunk.py:38) over
// caller-owned arrays in its layout: cumdecay [B][H][NT][C][P] fp32,
// state_end [B][H][NT][P][N] fp32, y_diag and y [B][T][H][P] fp32.  The
// arrays are per chunk of the requested size: chunks of 64 and 128 run the
// whole path's kernels in their stage modes; chunk 256 (which the whole path
// runs as 128-row chunks) runs the kernels of stage256.hip, with M3's two
// 128-row sub-blocks (kernel_mamba2_b_intra.py:61-62,86-108).
static int mamba2_stage_plan(const atomic_mamba2_args* a, Mamba2Plan* p) {
  const int rc = mamba2_plan(a, p);
  if (rc != ATOMIC_OK) return rc;
  if (a->chunk == kStageBlock) {
    p->dm.C = kStageBlock;
    p->dm.NT = a->seqlen / kStageBlock;
  }
  return ATOMIC_OK;
}

// M3 keeps CB ([B][NT][C][C] bf16) and M4 the states entering each chunk
// ([B][NT][H][P][N] bf16) in the caller's workspace.
static size_t m256_stage_ws(const Mamba2Dims& d) {  // M3's CB, or M4's fp32 states entering each chunk
  const size_t cb = m_cb_ws(d), st = m256_combine_ws(d);
  return m2_align(cb > st ? cb : st);
}
static size_t mamba2_stage_ws(const Mamba2Plan& p) {
  const Mamba2Dims& d = p.dm;
  if (d.C == kStageBlock) return m256_stage_ws(d);
  const size_t cb = (size_t)d.B * d.NT * d.C * d.C * 2;
  const size_t st = (size_t)d.B * d.NT * d.H * d.P * d.N * 2;
  return m2_align(cb > st ? cb : st);
}

template <int C, int P, int N>
static int mamba2_cumdecay_impl(const Mamba2Plan& p, const void* dt, const float* A, float* cum, Launch& L) {
  const Mamba2Dims& d = p.dm;
  hipStream_t st = L.st;
  return L("mamba2_cumdecay", [&] {
    hipLaunchKernelGGL((mamba2_cumdecay<bf16, C, P, kOuterPT>), dim3((unsigned)(d.B * d.NT * d.H * (P / kOuterPT))),
                       dim3(256), 0, st, d, (const bf16*)dt, A, cum);
  });
}

template <int C, int P, int N>
static int mamba2_intra_stage_impl(const Mamba2Plan& p, const void* dt, const void* x, const void* Bm,
                                   const void* Cm, const float* cum, float* y_diag, float* state_end, void* ws,
                                   Launch& L) {
  typedef bf16 T;
  const Mamba2Dims& d = p.dm;
  Mamba2Chunks<T> ck{};
  ck.cb = static_cast<T*>(ws);
  ck.src = state_end;
  ck.cum = cum;
  hipStream_t st = L.st;
  int rc = L("mamba2_cb", [&] {
    // one workgroup per chunk, or per 32-row block when the chunks are fewer
    // than the CUs (B2 T4096: 0.011 -> 0.007 ms)
    if (d.B * d.NT >= 256)
      hipLaunchKernelGGL((mamba2_cb<T, C, N>), dim3((unsigned)(d.B * d.NT)), dim3(256), 0, st, d,
                         (const T*)Bm, (const T*)Cm, ck);
    else
      hipLaunchKernelGGL((mamba2_cb<T, C, N, 32>), dim3((unsigned)(d.B * d.NT * (C / 32))), dim3(256), 0, st,
                         d, (const T*)Bm, (const T*)Cm, ck);
  });
  if (rc) return rc;
  // 8 pairs per workgroup, or one head's slices on grids under two per CU
  rc = L("mamba2_chunk_state", [&] {
    constexpr int NPO = P / kOuterPT;
    const size_t pairs = (size_t)d.H * NPO;
    if (pairs % 8 == 0 && d.B * d.NT * pairs / 8 >= kFullGrid)
      hipLaunchKernelGGL((mamba2_chunk_outer<T, T, C, P, N, kOuterPT, false, 8, true>),
                         dim3((unsigned)(d.B * d.NT * pairs / 8)), dim3(256), 0, st, d, (const T*)dt,
                         (const T*)x, (const float*)nullptr, (const T*)Bm, (const T*)nullptr, ck, (T*)nullptr,
                         (T*)nullptr);
    else
      hipLaunchKernelGGL((mamba2_chunk_outer<T, T, C, P, N, kOuterPT, false, NPO, true>),
                         dim3((unsigned)(d.B * d.NT * d.H)), dim3(256), 0, st, d, (const T*)dt, (const T*)x,
                         (const float*)nullptr, (const T*)Bm, (const T*)nullptr, ck, (T*)nullptr, (T*)nullptr);
  });
  if (rc) return rc;
  constexpr int NPT = P / kYPT;
  const size_t pairs = (size_t)d.H * NPT;
  return L("mamba2_chunk_y_diag", [&] {
    if (pairs % 16 == 0)
      hipLaunchKernelGGL((mamba2_chunk_y<T, C, P, N, kYPT, 16, 1>), dim3((unsigned)(d.B * d.NT * pairs / 16)),
                         dim3(256), 0, st, d, (const T*)dt, (const T*)x, (const float*)nullptr, (const T*)Cm,
                         ck, y_diag);
    else
      hipLaunchKernelGGL((mamba2_chunk_y<T, C, P, N, kYPT, NPT, 1>), dim3((unsigned)(d.B * d.NT * d.H)),
                         dim3(256), 0, st, d, (const T*)dt, (const T*)x, (const float*)nullptr, (const T*)Cm,
                         ck, y_diag);
  });
}

template <int C, int P, int N>
static int mamba2_combine_stage_impl(const Mamba2Plan& p, const float* y_diag, const float* state_end,
                                     const float* cum, const void* Cm, const float* state0, float* y,
                                     float* state_final, void* ws, Launch& L) {
  typedef bf16 T;
  const Mamba2Dims& d = p.dm;
  Mamba2Chunks<T> ck{};
  ck.state_pre = static_cast<T*>(ws);
  ck.src = const_cast<float*>(state_end);
  ck.cum = cum;
  ck.ydiag = y_diag;
  hipStream_t st = L.st;
  int rc = L("mamba2_state_pass", [&] {
    hipLaunchKernelGGL((mamba2_state_pass<T, P, N, false, true>), dim3(pass_grid<P, N>(d)), dim3(256), 0, st,
                       d, ck, (T*)nullptr, (float*)nullptr, state0, state_final);
  });
  if (rc) return rc;
  constexpr int NPT = P / kYPT;
  const size_t pairs = (size_t)d.H * NPT;
  return L("mamba2_chunk_y_combine", [&] {
    if (pairs % 16 == 0)
      hipLaunchKernelGGL((mamba2_chunk_y<T, C, P, N, kYPT, 16, 2>), dim3((unsigned)(d.B * d.NT * pairs / 16)),
                         dim3(256), 0, st, d, (const T*)nullptr, (const T*)nullptr, (const float*)nullptr,
                         (const T*)Cm, ck, y);
    else
      hipLaunchKernelGGL((mamba2_chunk_y<T, C, P, N, kYPT, NPT, 2>), dim3((unsigned)(d.B * d.NT * d.H)),
                         dim3(256), 0, st, d, (const T*)nullptr, (const T*)nullptr, (const float*)nullptr,
                         (const T*)Cm, ck, y);
  });
}

static int mamba2_cumdecay_stage(const Mamba2Plan& p, const void* dt, const float* A, float* cum, Launch& L) {
  if (p.dm.C == kStageBlock) {   // the cumsum kernel over 256 rows (N does not enter)
    if (p.dm.P == 64) return mamba2_cumdecay_impl<kStageBlock, 64, 128>(p, dt, A, cum, L);
    if (p.dm.P == 128) return mamba2_cumdecay_impl<kStageBlock, 128, 128>(p, dt, A, cum, L);
    return mamba2_cumdecay_impl<kStageBlock, 192, 128>(p, dt, A, cum, L);
  }
  AH_M2_DISPATCH(mamba2_cumdecay_impl, p, dt, A, cum, L);
}

static int mamba2_intra_stage(const Mamba2Plan& p, const void* dt, const void* x, const void* Bm, const void* Cm,
                              const float* cum, float* y_diag, float* state_end, void* ws, Launch& L) {
  if (p.dm.C == kStageBlock)
    return m256_intra(p.dm, ATOMIC_BF16, dt, x, Bm, Cm, cum, y_diag, state_end, static_cast<float*>(ws), L);
  AH_M2_DISPATCH(mamba2_intra_stage_impl, p, dt, x, Bm, Cm, cum, y_diag, state_end, ws, L);
}

static int mamba2_combine_stage(const Mamba2Plan& p, const float* y_diag, const float* state_end, const float* cum,
                                const void* Cm, const float* state0, float* y, float* state_final, void* ws,
                                Launch& L) {
  if (p.dm.C == kStageBlock)
    return m256_combine(p.dm, ATOMIC_BF16, y_diag, state_end, cum, Cm, state0, y, state_final,
                        static_cast<float*>(ws), L);
  AH_M2_DISPATCH(mamba2_combine_stage_impl, p, y_diag, state_end, cum, Cm, state0, y, state_final, ws, L);
}

}  // namespace ah

using namespace ah;

// fp32 operands run the float32 staged chain (csrc/stage256_bwd.hip) at the
// caller's chunk: the reference's trainable op composes the same stages
// (kernel_mamba2_trainable_B6.py:72-131).  Its workspace holds the larger of
// the forward's and the backward's arrays; the backward's are followed by
// room for dstate0 when the caller passes none.
static size_t mamba2_f32_ws(const Mamba2Plan& p) {
  const Mamba2Dims& d = p.f32dm;
  const size_t f = m_f32_fwd_ws(d);
  const size_t b = m2_align(m_f32_bwd_ws(d)) + (size_t)d.B * d.H * d.P * d.N * sizeof(float);
  return m2_align(f > b ? f : b);
}

extern "C" size_t atomic_mamba2_workspace_size(const atomic_mamba2_args* a) {
  Mamba2Plan p;
  if (mamba2_plan(a, &p) != ATOMIC_OK) return 0;
  return p.f32 ? mamba2_f32_ws(p) : p.total;
}

// the forward a Mamba2 workspace holds: shapes, dtype and the input pointers
static WsTag mamba2_tag(const atomic_mamba2_args* a, const void* dt, const void* x, const void* B, const void* C,
                        const void* A, const void* state0) {
  WsTag t{};
  t.kind = (a->flags & ATOMIC_MAMBA2_SANITIZE_STATE0) ? 0x102 : 2;  // the saved states depend on it
  const int32_t d[8] = {a->batch, a->seqlen, a->heads, a->headdim, a->dstate, a->chunk, a->dtype, 0};
  const void* ptr[8] = {dt, x, B, C, A, state0, nullptr, nullptr};
  for (int i = 0; i < 8; ++i) { t.dims[i] = d[i]; t.ptrs[i] = ptr[i]; }
  const int64_t dP = (int64_t)a->heads * a->headdim, dN = a->dstate;
  const int64_t dense[4] = {dP, dP, dN, dN};
  for (int i = 0; i < 4; ++i) t.strides[i] = a->row_stride[i] ? a->row_stride[i] : dense[i];  // dt, x, B, C
  return t;
}

extern "C" int atomic_mamba2_fwd(const atomic_mamba2_args* a, const void* dt, const void* x,
                                 const void* B, const void* C, const float* A, const float* state0,
                                 float* y, float* state_final, void* workspace,
                                 size_t workspace_bytes, void* stream) {
  Mamba2Plan p;
  const int rc = mamba2_plan(a, &p);
  if (rc != ATOMIC_OK) return rc;
  if (!dt || !x || !B || !C || !A || !y || !state_final) return ATOMIC_ERR_NULL;
  if (p.f32) {  // the float32 staged forward; no stage reports, nothing kept for a REUSE backward
    if (a->diag) return ATOMIC_ERR_DTYPE;
    if (!workspace || workspace_bytes < mamba2_f32_ws(p)) return ATOMIC_ERR_WORKSPACE;
    ws_tag_clobber(workspace, workspace_bytes);
    Launch L{a->profile, (hipStream_t)stream};
    return m_f32_fwd(p.f32dm, dt, x, B, C, A, state0, y, state_final, static_cast<float*>(workspace), L);
  }
  if (!workspace || workspace_bytes < p.total) return ATOMIC_ERR_WORKSPACE;
  Launch L{a->profile, (hipStream_t)stream};
  int r2 = mamba2_forward(p, dt, x, B, C, A, state0, y, state_final, workspace, L);
  // the forward always leaves its per-chunk states in the workspace
  if (r2 == ATOMIC_OK) ws_tag_set(workspace, p.total, mamba2_tag(a, dt, x, B, C, A, state0));
  else ws_tag_clobber(workspace, p.total);
  if (r2 || !a->diag) return r2;
  StageDiag D{a->diag, L};
  return mamba2_forward_diag(p, D, y, state_final, workspace);
}

extern "C" int atomic_mamba2_bwd(const atomic_mamba2_args* a, const void* dt, const void* x,
                                 const void* B, const void* C, const float* A, const float* state0,
                                 const void* dy, const float* dstate_final, void* ddt, void* dx,
                                 void* dB, void* dC, float* dA, float* dstate0, void* workspace,
                                 size_t workspace_bytes, void* stream) {
  Mamba2Plan p;
  const int rc = mamba2_plan(a, &p);
  if (rc != ATOMIC_OK) return rc;
  if (!dt || !x || !B || !C || !A || !dy || !ddt || !dx || !dB || !dC || !dA) return ATOMIC_ERR_NULL;
  if (p.f32) {  // the float32 staged backward, which always re-runs the forward (REUSE is not checked)
    if (a->diag) return ATOMIC_ERR_DTYPE;
    if (!workspace || workspace_bytes < mamba2_f32_ws(p)) return ATOMIC_ERR_WORKSPACE;
    ws_tag_clobber(workspace, workspace_bytes);
    Launch L{a->profile, (hipStream_t)stream};
    float* ws = static_cast<float*>(workspace);
    // the scan always writes dstate0: into the workspace's tail when the caller wants none
    float* ds0 = dstate0 ? dstate0 : ws + m2_align(m_f32_bwd_ws(p.f32dm)) / sizeof(float);
    return m_f32_bwd(p.f32dm, a->dy_dtype, dt, x, B, C, A, state0, dy, dstate_final, (float*)ddt, (float*)dx,
                     (float*)dB, (float*)dC, dA, ds0, ws, L);
  }
  if (!workspace || workspace_bytes < p.total) return ATOMIC_ERR_WORKSPACE;
  const bool reuse = (a->flags & ATOMIC_MAMBA2_REUSE) != 0;
  const WsTag tag = mamba2_tag(a, dt, x, B, C, A, state0);
  if (reuse && !ws_tag_matches(workspace, tag)) return ATOMIC_ERR_REUSE;
  Launch L{a->profile, (hipStream_t)stream};
  int r2 = mamba2_backward(p, a->dy_dtype, dt, x, B, C, A, state0, dy, dstate_final, ddt, dx, dB, dC, dA,
                           dstate0, workspace, reuse, L);
  // the per-chunk states (kept or recomputed) outlive the backward's own scratch
  if (r2 == ATOMIC_OK) ws_tag_set(workspace, p.total, tag);
  else ws_tag_clobber(workspace, p.total);
  if (r2 || !a->diag) return r2;
  StageDiag D{a->diag, L};
  return mamba2_backward_diag(p, D, ddt, dx, dB, dC, dA, dstate0, workspace);
}

extern "C" size_t atomic_mamba2_stage_workspace_size(const atomic_mamba2_args* a) {
  Mamba2Plan p;
  if (mamba2_stage_plan(a, &p) != ATOMIC_OK) return 0;
  return p.f32 ? m256_stage_ws(p.f32dm) : mamba2_stage_ws(p);
}

extern "C" int atomic_mamba2_chunk_cumdecay(const atomic_mamba2_args* a, const void* dt, const float* A,
                                            float* cumdecay, void* stream) {
  Mamba2Plan p;
  const int rc = mamba2_stage_plan(a, &p);
  if (rc != ATOMIC_OK) return rc;
  if (!dt || !A || !cumdecay) return ATOMIC_ERR_NULL;
  Launch L{a->profile, (hipStream_t)stream};
  if (p.f32) return m_cumdecay(p.f32dm, ATOMIC_F32, dt, A, cumdecay, L);
  return mamba2_cumdecay_stage(p, dt, A, cumdecay, L);
}

extern "C" int atomic_mamba2_intra_chunk_ssd(const atomic_mamba2_args* a, const void* dt, const void* x,
                                             const void* B, const void* C, const float* cumdecay, float* y_diag,
                                             float* state_end, void* workspace, size_t workspace_bytes,
                                             void* stream) {
  Mamba2Plan p;
  const int rc = mamba2_stage_plan(a, &p);
  if (rc != ATOMIC_OK) return rc;
  if (!dt || !x || !B || !C || !cumdecay || !y_diag || !state_end) return ATOMIC_ERR_NULL;
  if (p.f32) {
    if (!workspace || workspace_bytes < m256_stage_ws(p.f32dm)) return ATOMIC_ERR_WORKSPACE;
    ws_tag_clobber(workspace, workspace_bytes);
    Launch L{a->profile, (hipStream_t)stream};
    return m256_intra(p.f32dm, ATOMIC_F32, dt, x, B, C, cumdecay, y_diag, state_end, static_cast<float*>(workspace),
                      L);
  }
  if (!workspace || workspace_bytes < mamba2_stage_ws(p)) return ATOMIC_ERR_WORKSPACE;
  ws_tag_clobber(workspace, workspace_bytes);
  Launch L{a->profile, (hipStream_t)stream};
  return mamba2_intra_stage(p, dt, x, B, C, cumdecay, y_diag, state_end, workspace, L);
}

extern "C" int atomic_mamba2_inter_chunk_combine(const atomic_mamba2_args* a, const float* y_diag,
                                                 const float* state_end, const float* cumdecay, const void* C,
                                                 const float* state0, float* y, float* state_final,
                                                 void* workspace, size_t workspace_bytes, void* stream) {
  Mamba2Plan p;
  const int rc = mamba2_stage_plan(a, &p);
  if (rc != ATOMIC_OK) return rc;
  if (!y_diag || !state_end || !cumdecay || !C || !y || !state_final) return ATOMIC_ERR_NULL;
  if (p.f32) {
    if (!workspace || workspace_bytes < m256_combine_ws(p.f32dm)) return ATOMIC_ERR_WORKSPACE;
    ws_tag_clobber(workspace, workspace_bytes);
    Launch L{a->profile, (hipStream_t)stream};
    return m256_combine(p.f32dm, ATOMIC_F32, y_diag, state_end, cumdecay, C, state0, y, state_final,
                        static_cast<float*>(workspace), L);
  }
  if (!workspace || workspace_bytes < mamba2_stage_ws(p)) return ATOMIC_ERR_WORKSPACE;
  ws_tag_clobber(workspace, workspace_bytes);
  Launch L{a->profile, (hipStream_t)stream};
  return mamba2_combine_stage(p, y_diag, state_end, cumdecay, C, state0, y, state_final, workspace, L);
}

// ------------------------------------------------------------------ MB2 stage entry
extern "C" size_t atomic_mamba2_intra_chunk_ssd_bwd_workspace_size(const atomic_mamba2_args* a) {
  Mamba2Plan p;
  if (mamba2_plan(a, &p) != ATOMIC_OK) return 0;
  Mamba2Dims d = p.dm;
  d.C = a->chunk;
  d.NT = a->seqlen / a->chunk;
  return m2_align(m_intra_bwd_ws(d));
}

extern "C" int atomic_mamba2_intra_chunk_ssd_bwd(const atomic_mamba2_args* a, const void* dt, const void* x,
                                                 const void* B, const void* C, const float* cumdecay,
                                                 const void* dy, const float* dstate_end_grad, float* ddt,
                                                 float* dx, float* dB, float* dC, float* dcum, void* workspace,
                                                 size_t workspace_bytes, void* stream) {
  Mamba2Plan p;
  const int rc = mamba2_plan(a, &p);
  if (rc != ATOMIC_OK) return rc;
  if (!dt || !x || !B || !C || !cumdecay || !dy || !dstate_end_grad || !ddt || !dx || !dB || !dC || !dcum)
    return ATOMIC_ERR_NULL;
  Mamba2Dims d = p.dm;  // the caller's chunk, whatever the whole path runs
  d.C = a->chunk;
  d.NT = a->seqlen / a->chunk;
  if (!workspace || workspace_bytes < m_intra_bwd_ws(d)) return ATOMIC_ERR_WORKSPACE;
  ws_tag_clobber(workspace, workspace_bytes);
  Launch L{a->profile, (hipStream_t)stream};
  return m_intra_bwd(d, a->dtype, a->dy_dtype, dt, x, B, C, cumdecay, dy, dstate_end_grad, ddt, dx, dB, dC, dcum,
                     static_cast<float*>(workspace), L);
}

// ------------------------------------------------------------------ MB1 + MB3 and MB4 stage entries
static int mamba2_bwd_stage_dims(const atomic_mamba2_args* a, Mamba2Plan* p) {
  const int rc = mamba2_stage_plan(a, p);
  if (rc != ATOMIC_OK) return rc;
  return p->dm.P % 32 == 0 ? ATOMIC_OK : ATOMIC_ERR_SHAPE;
}

extern "C" size_t atomic_mamba2_bwd_scan_workspace_size(const atomic_mamba2_args* a) {
  Mamba2Plan p;
  if (mamba2_bwd_stage_dims(a, &p) != ATOMIC_OK) return 0;
  return m2_align(m_bwd_scan_ws(p.dm));
}

extern "C" int atomic_mamba2_bwd_scan(const atomic_mamba2_args* a, const void* dt, const float* A, const void* B,
                                      const void* C, const void* x, const void* dy, const float* dstate_final,
                                      const float* state0, float* ddt, float* dB, float* dC, float* dx,
                                      float* dstate0, float* dcumdecay, void* workspace, size_t workspace_bytes,
                                      void* stream) {
  Mamba2Plan p;
  const int rc = mamba2_bwd_stage_dims(a, &p);
  if (rc != ATOMIC_OK) return rc;
  if (!dt || !A || !B || !C || !x || !dy || !ddt || !dB || !dC || !dx || !dstate0 || !dcumdecay)
    return ATOMIC_ERR_NULL;
  if (!workspace || workspace_bytes < m_bwd_scan_ws(p.dm)) return ATOMIC_ERR_WORKSPACE;
  ws_tag_clobber(workspace, workspace_bytes);
  Launch L{a->profile, (hipStream_t)stream};
  // M2's cumdecay into the workspace's first array (kernel_mamba2_bwd_b1_state.py:184)
  float* cum = static_cast<float*>(workspace);
  const int r2 = p.f32 ? m_cumdecay(p.dm, ATOMIC_F32, dt, A, cum, L) : mamba2_cumdecay_stage(p, dt, A, cum, L);
  if (r2 != ATOMIC_OK) return r2;
  return m_bwd_scan(p.dm, a->dtype, a->dy_dtype, dt, x, B, C, cum, dy, dstate_final, state0, ddt, dB, dC, dx, dstate0,
                    dcumdecay, cum, L);
}

// MB4 takes dt in the per-chunk layout, bf16 or fp32 (args.dtype); dstate
// does not enter.
static int mamba2_da_dims(const atomic_mamba2_args* a, Mamba2Dims* d) {
  if (!a) return ATOMIC_ERR_NULL;
  if (a->dtype != ATOMIC_BF16 && a->dtype != ATOMIC_F32) return ATOMIC_ERR_DTYPE;
  if (a->batch <= 0 || a->heads <= 0 || a->seqlen <= 0) return ATOMIC_ERR_SHAPE;
  if (a->chunk != 64 && a->chunk != 128 && a->chunk != 256) return ATOMIC_ERR_SHAPE;
  if (a->seqlen % a->chunk != 0) return ATOMIC_ERR_SHAPE;
  if (a->headdim != 64 && a->headdim != 128 && a->headdim != 192) return ATOMIC_ERR_SHAPE;
  Mamba2Dims m{};
  m.B = a->batch; m.T = a->seqlen; m.H = a->heads; m.P = a->headdim; m.N = a->dstate;
  m.C = a->chunk; m.NT = a->seqlen / a->chunk;
  *d = m;
  return ATOMIC_OK;
}

extern "C" size_t atomic_mamba2_da_backward_workspace_size(const atomic_mamba2_args* a) {
  Mamba2Dims d;
  if (mamba2_da_dims(a, &d) != ATOMIC_OK) return 0;
  return m2_align(m_da_bwd_ws(d));
}

extern "C" int atomic_mamba2_da_backward(const atomic_mamba2_args* a, const void* dt_chunks, const float* A,
                                         const float* dcumdecay, float* ddt_contrib, float* dA, void* workspace,
                                         size_t workspace_bytes, void* stream) {
  Mamba2Dims d;
  const int rc = mamba2_da_dims(a, &d);
  if (rc != ATOMIC_OK) return rc;
  if (!dt_chunks || !A || !dcumdecay || !ddt_contrib || !dA) return ATOMIC_ERR_NULL;
  if (!workspace || workspace_bytes < m_da_bwd_ws(d)) return ATOMIC_ERR_WORKSPACE;
  ws_tag_clobber(workspace, workspace_bytes);
  Launch L{a->profile, (hipStream_t)stream};
  return m_da_bwd(d, a->dtype, 0, dt_chunks, A, dcumdecay, ddt_contrib, dA, static_cast<float*>(workspace), L);
}
