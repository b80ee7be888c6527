// Shared device helpers for the CDNA4 (gfx950) chunk kernels.
//
// Operand fetches for the 16x16 MFMA tiles:
//   * bf16: v_mfma_f32_16x16x32_bf16.  Lane l (r = l % 16, g = l / 16) holds
//     eight consecutive k values (k0 + 8g .. k0 + 8g + 7) of row r of A and of
//     column r of B; the result tile gives lane l rows 4g..4g+3 of column r.
//   * fp32: v_mfma_f32_16x16x4_f32.  Lane l holds one k value (k0 + g).
// Two fetch kinds cover every layout:
//   ld_c  "contiguous":  element (i, k) at p[i * ld + k]   (k runs along a row)
//   ld_t  "transposed":  element (i, k) at p[k * ld + i]   (i runs along a row)
// ld_t on bf16 uses ds_read_tr16_b64: within each 16-lane group, lane s points
// at four consecutive u16 of row (k0 + 8g + s/4) starting at column
// (i0 + 4 (s % 4)); lane j then receives column i0 + j of those four rows.
// Two such reads (rows +0..3 and +4..7) give the eight k values of a lane.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

namespace ah {

typedef __bf16 bf16;
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x4 __attribute__((ext_vector_type(4)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

constexpr float kClipAcc = 1e4f;
constexpr float kClipDecay = 20.0f;

__device__ __forceinline__ int lane_id() { return threadIdx.x & 63; }
// wave index of a 1-D workgroup, as a wave-uniform (scalar) value so that
// branches and addresses derived from it stay scalar
__device__ __forceinline__ int wave_id() { return __builtin_amdgcn_readfirstlane(threadIdx.x >> 6); }

__device__ __forceinline__ float to_f(float x) { return x; }
__device__ __forceinline__ float to_f(bf16 x) { return (float)x; }
template <typename T> __device__ __forceinline__ T from_f(float x);
template <> __device__ __forceinline__ float from_f<float>(float x) { return x; }
template <> __device__ __forceinline__ bf16 from_f<bf16>(float x) { return (bf16)x; }

// jnp.nan_to_num(x, nan=0, posinf=c, neginf=-c): finite values pass unchanged.
__device__ __forceinline__ float n2n(float x, float c = kClipAcc) {
  if (__builtin_isnan(x)) return 0.f;
  if (__builtin_isinf(x)) return x > 0.f ? c : -c;
  return x;
}
// clip to [-c, c] then nan_to_num.
__device__ __forceinline__ float sanitize(float x, float c = kClipAcc) {
  if (__builtin_isnan(x)) return 0.f;
  return fminf(fmaxf(x, -c), c);
}

// ---------------------------------------------------------------- vector I/O
// Eight consecutive elements as floats.
__device__ __forceinline__ void load8(const bf16* p, float* out) {
  bf16x8 v = *reinterpret_cast<const bf16x8*>(p);
#pragma unroll
  for (int i = 0; i < 8; ++i) out[i] = (float)v[i];
}
__device__ __forceinline__ void load8(const float* p, float* out) {
  float4 a = *reinterpret_cast<const float4*>(p);
  float4 b = *reinterpret_cast<const float4*>(p + 4);
  out[0] = a.x; out[1] = a.y; out[2] = a.z; out[3] = a.w;
  out[4] = b.x; out[5] = b.y; out[6] = b.z; out[7] = b.w;
}
__device__ __forceinline__ void store8(bf16* p, const float* v) {
  bf16x8 o;
#pragma unroll
  for (int i = 0; i < 8; ++i) o[i] = (bf16)v[i];
  *reinterpret_cast<bf16x8*>(p) = o;
}
__device__ __forceinline__ void store8(float* p, const float* v) {
  *reinterpret_cast<float4*>(p) = make_float4(v[0], v[1], v[2], v[3]);
  *reinterpret_cast<float4*>(p + 4) = make_float4(v[4], v[5], v[6], v[7]);
}
// Four consecutive elements (an MFMA result column written "transposed").
__device__ __forceinline__ void store4(bf16* p, f32x4 v) {
  bf16x4 o;
  o[0] = (bf16)v[0]; o[1] = (bf16)v[1]; o[2] = (bf16)v[2]; o[3] = (bf16)v[3];
  *reinterpret_cast<bf16x4*>(p) = o;
}
__device__ __forceinline__ void store4(float* p, f32x4 v) {
  *reinterpret_cast<float4*>(p) = make_float4(v[0], v[1], v[2], v[3]);
}

// --------------------------------------------------------------------- MFMA
template <typename T> struct Mma;

template <> struct Mma<bf16> {
  static constexpr int KS = 32;  // k per instruction
  typedef bf16x8 frag;
  static __device__ __forceinline__ frag ld_c(const bf16* p, int ld, int i0, int k0) {
    const int l = lane_id();
    return *reinterpret_cast<const bf16x8*>(p + (i0 + (l & 15)) * ld + k0 + 8 * (l >> 4));
  }
  static __device__ __forceinline__ frag ld_t(const bf16* p, int ld, int i0, int k0) {
    const int l = lane_id();
    const int s = l & 15, g = l >> 4;
    const bf16* q = p + (k0 + 8 * g + (s >> 2)) * ld + i0 + 4 * (s & 3);
    typedef __attribute__((address_space(3))) bf16x4* lds_p;
    bf16x4 lo = __builtin_amdgcn_ds_read_tr16_b64_v4bf16((lds_p)(q));
    bf16x4 hi = __builtin_amdgcn_ds_read_tr16_b64_v4bf16((lds_p)(q + 4 * ld));
    frag f = __builtin_shufflevector(lo, hi, 0, 1, 2, 3, 4, 5, 6, 7);
    return f;
  }
  static __device__ __forceinline__ f32x4 mma(frag a, frag b, f32x4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, c, 0, 0, 0);
  }
};

template <> struct Mma<float> {
  static constexpr int KS = 4;
  typedef float frag;
  static __device__ __forceinline__ frag ld_c(const float* p, int ld, int i0, int k0) {
    const int l = lane_id();
    return p[(i0 + (l & 15)) * ld + k0 + (l >> 4)];
  }
  static __device__ __forceinline__ frag ld_t(const float* p, int ld, int i0, int k0) {
    const int l = lane_id();
    return p[(k0 + (l >> 4)) * ld + i0 + (l & 15)];
  }
  static __device__ __forceinline__ f32x4 mma(frag a, frag b, f32x4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x4f32(a, b, c, 0, 0, 0);
  }
};

// acc(16x16 tile at rows m0.., cols n0..) += sum_{k < K} A(m, k) B(k, n)
//   A_T == false: A(m, k) = A[m * lda + k]      A_T == true: A(m, k) = A[k * lda + m]
//   B_T == false: B(k, n) = B[n * ldb + k]      B_T == true: B(k, n) = B[k * ldb + n]
template <typename T, bool A_T, bool B_T>
__device__ __forceinline__ f32x4 tile_mma(f32x4 acc, const T* A, int lda, const T* B, int ldb,
                                          int m0, int n0, int K) {
#pragma unroll 4
  for (int k0 = 0; k0 < K; k0 += Mma<T>::KS) {
    typename Mma<T>::frag a = A_T ? Mma<T>::ld_t(A, lda, m0, k0) : Mma<T>::ld_c(A, lda, m0, k0);
    typename Mma<T>::frag b = B_T ? Mma<T>::ld_t(B, ldb, n0, k0) : Mma<T>::ld_c(B, ldb, n0, k0);
    acc = Mma<T>::mma(a, b, acc);
  }
  return acc;
}

// NT adjacent column tiles (n0, n0 + 16, ...) of one row block: each A
// fragment is read once for all of them.
template <typename T, bool A_T, bool B_T, int NT>
__device__ __forceinline__ void tile_mma_row(f32x4 (&acc)[NT], const T* A, int lda, const T* B, int ldb,
                                             int m0, int n0, int K) {
#pragma unroll 4
  for (int k0 = 0; k0 < K; k0 += Mma<T>::KS) {
    typename Mma<T>::frag a = A_T ? Mma<T>::ld_t(A, lda, m0, k0) : Mma<T>::ld_c(A, lda, m0, k0);
#pragma unroll
    for (int t = 0; t < NT; ++t) {
      typename Mma<T>::frag b =
          B_T ? Mma<T>::ld_t(B, ldb, n0 + 16 * t, k0) : Mma<T>::ld_c(B, ldb, n0 + 16 * t, k0);
      acc[t] = Mma<T>::mma(a, b, acc[t]);
    }
  }
}

// Make this wave's LDS writes visible to its own later LDS reads (no
// workgroup barrier: only valid for data private to one wave).
__device__ __forceinline__ void wave_lds_sync() {
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}

// A zero the compiler cannot see through: offsets built from it are recomputed
// where they are used instead of being hoisted out of enclosing loops.
__device__ __forceinline__ int opaque_zero() {
  int z = 0;
  asm volatile("" : "+s"(z));
  return z;
}

// The same global-memory pointer, opaque to the compiler: per-lane addresses
// built from it stay inside the loop that calls this instead of being hoisted
// (and kept live).  The barrier is placed on the address-space-1 form, so the
// loads through the result stay global loads: through a generic pointer they
// would be flat loads, which also count in lgkmcnt, and every later wait for an
// LDS or scalar load would then wait for them as well.
template <typename P>
__device__ __forceinline__ P* opaque_ptr(P* p) {
  typedef __attribute__((address_space(1))) P* GP;
  GP q = (GP)p;
  asm volatile("" : "+s"(q));
  return (P*)q;
}

// f(IntC<i>{}) for a runtime i in [0, N): the body is compiled once per value
// with i a constant (for wave-uniform i, a chain of scalar compares).
template <int V> struct IntC { static constexpr int value = V; };
template <int N, int I = 0, typename F>
__device__ __forceinline__ void static_switch(int i, F&& f) {
  if constexpr (I + 1 >= N) {
    f(IntC<I>{});
  } else {
    if (i == I) f(IntC<I>{});
    else static_switch<N, I + 1>(i, f);
  }
}

// f(IntC<0>{}), ..., f(IntC<N - 1>{}): a loop whose index is a constant in the body.
template <int N, int I = 0, typename F>
__device__ __forceinline__ void static_for(F&& f) {
  if constexpr (I < N) {
    f(IntC<I>{});
    static_for<N, I + 1>(f);
  }
}

__device__ __forceinline__ f32x4 zero4() { f32x4 z = {0.f, 0.f, 0.f, 0.f}; return z; }

// Tile element coordinates held by this lane: rows m0 + 4g + i, column n0 + r.
__device__ __forceinline__ int tile_row(int i) { return 4 * (lane_id() >> 4) + i; }
__device__ __forceinline__ int tile_col() { return lane_id() & 15; }

// Write a result tile transposed: dst[(n0 + c) * ld + m0 + 4g .. +3] (one vector store).
template <typename T>
__device__ __forceinline__ void store_tile_t(T* dst, int ld, int m0, int n0, f32x4 v) {
  store4(dst + (n0 + tile_col()) * ld + m0 + tile_row(0), v);
}
// Write a result tile in natural layout: dst[(m0 + r) * ld + n0 + c].
template <typename T>
__device__ __forceinline__ void store_tile_n(T* dst, int ld, int m0, int n0, f32x4 v) {
#pragma unroll
  for (int i = 0; i < 4; ++i) dst[(m0 + tile_row(i)) * ld + n0 + tile_col()] = from_f<T>(v[i]);
}

// Eight consecutive elements held raw (loads stay in flight until first use).
template <typename T> struct Raw8;
template <> struct Raw8<bf16> {
  uint4 v;
  __device__ __forceinline__ void load(const bf16* p) { v = *reinterpret_cast<const uint4*>(p); }
  __device__ __forceinline__ float operator[](int j) const {
    return (float)reinterpret_cast<const bf16*>(&v)[j];
  }
};
template <> struct Raw8<float> {
  float4 a, b;
  __device__ __forceinline__ void load(const float* p) {
    a = *reinterpret_cast<const float4*>(p);
    b = *reinterpret_cast<const float4*>(p + 4);
  }
  __device__ __forceinline__ float operator[](int j) const {
    return j < 4 ? (&a.x)[j] : (&b.x)[j - 4];
  }
};

// Row padding (elements) that keeps rows 16-byte aligned.
template <typename T> struct Pad { static constexpr int v = 16 / sizeof(T); };

// ------------------------------------------------------------- staging
// A [R][D] block moved global -> registers -> LDS in 16-byte pieces, so the
// next chunk's loads can be in flight while the current chunk computes
// (NTH threads in the workgroup).
template <typename T, int R, int D, int NTH = 256>
struct RegStage {
  static constexpr int VEC = 16 / (int)sizeof(T);
  static constexpr int PER_ROW = D / VEC;
  static constexpr int N = R * PER_ROW;
  static constexpr int PT = (N + NTH - 1) / NTH;
  // one SSA vector (not an array) so the staging stays in registers
  typedef uint32_t vec_t __attribute__((ext_vector_type(4 * PT)));
  vec_t r;
  __device__ __forceinline__ void load(const T* src, size_t ld) {
#pragma unroll
    for (int i = 0; i < PT; ++i) {
      const int e = threadIdx.x + NTH * i;
      if (N % NTH == 0 || e < N) {
        const uint4 x = *reinterpret_cast<const uint4*>(src + (size_t)(e / PER_ROW) * ld + (e % PER_ROW) * VEC);
        r[4 * i] = x.x; r[4 * i + 1] = x.y; r[4 * i + 2] = x.z; r[4 * i + 3] = x.w;
      }
    }
  }
  __device__ __forceinline__ void store(T* dst, int ld) const {
#pragma unroll
    for (int i = 0; i < PT; ++i) {
      const int e = threadIdx.x + NTH * i;
      if (N % NTH == 0 || e < N)
        *reinterpret_cast<uint4*>(dst + (e / PER_ROW) * ld + (e % PER_ROW) * VEC) =
            make_uint4(r[4 * i], r[4 * i + 1], r[4 * i + 2], r[4 * i + 3]);
    }
  }
  // the i-th 16-byte piece, as loaded
  __device__ __forceinline__ uint4 piece(int i) const {
    return make_uint4(r[4 * i], r[4 * i + 1], r[4 * i + 2], r[4 * i + 3]);
  }
};

// Store a RegStage block of source type TS into LDS as type T (times mul).
template <typename T, typename TS, int R, int D, int NTH>
__device__ __forceinline__ void store_convert(const RegStage<TS, R, D, NTH>& S, T* dst, int ld,
                                              float mul = 1.f) {
  typedef RegStage<TS, R, D, NTH> RS;
#pragma unroll
  for (int i = 0; i < RS::PT; ++i) {
    const int e = threadIdx.x + NTH * i;
    if (RS::N % NTH == 0 || e < RS::N) {
      const int r = e / RS::PER_ROW, c = (e % RS::PER_ROW) * RS::VEC;
      const uint4 raw = S.piece(i);
      const TS* v = reinterpret_cast<const TS*>(&raw);
#pragma unroll
      for (int j = 0; j < RS::VEC; ++j) dst[r * ld + c + j] = from_f<T>(to_f(v[j]) * mul);
    }
  }
}

// Copy a [R][D] block (row stride `src_ld`) into LDS rows of length `dst_ld`
// (NTH threads in the workgroup).
// All of a thread's loads are issued before its stores (the pieces are held in
// registers), so the loads of one call are in flight together.
template <typename T, int R, int D, int NTH = 256>
__device__ __forceinline__ void stage_rows(T* dst, int dst_ld, const T* src, size_t src_ld) {
  constexpr int VEC = 16 / sizeof(T);
  constexpr int PER_ROW = D / VEC;
  constexpr int NP = R * PER_ROW, IT = (NP + NTH - 1) / NTH;
  u32x4 tmp[IT];  // native vectors: the array stays in registers
#pragma unroll
  for (int i = 0; i < IT; ++i) {
    const int e = threadIdx.x + NTH * i;
    if (NP % NTH == 0 || e < NP)
      tmp[i] = *reinterpret_cast<const u32x4*>(src + (size_t)(e / PER_ROW) * src_ld + (e % PER_ROW) * VEC);
  }
#pragma unroll
  for (int i = 0; i < IT; ++i) {
    const int e = threadIdx.x + NTH * i;
    if (NP % NTH == 0 || e < NP)
      *reinterpret_cast<u32x4*>(dst + (e / PER_ROW) * dst_ld + (e % PER_ROW) * VEC) = tmp[i];
  }
}
template <typename T, int R, int D, int NTH = 256>
__device__ __forceinline__ void unstage_rows(T* dst, size_t dst_ld, const T* src, int src_ld) {
  constexpr int VEC = 16 / sizeof(T);
  constexpr int PER_ROW = D / VEC;
  constexpr int NP = R * PER_ROW, IT = (NP + NTH - 1) / NTH;
  u32x4 tmp[IT];  // native vectors: the array stays in registers
#pragma unroll
  for (int i = 0; i < IT; ++i) {
    const int e = threadIdx.x + NTH * i;
    if (NP % NTH == 0 || e < NP)
      tmp[i] = *reinterpret_cast<const u32x4*>(src + (e / PER_ROW) * src_ld + (e % PER_ROW) * VEC);
  }
#pragma unroll
  for (int i = 0; i < IT; ++i) {
    const int e = threadIdx.x + NTH * i;
    if (NP % NTH == 0 || e < NP)
      *reinterpret_cast<u32x4*>(dst + (size_t)(e / PER_ROW) * dst_ld + (e % PER_ROW) * VEC) = tmp[i];
  }
}

// Workgroup -> (bh, vt) so that the V tiles of one head share an XCD (and
// its L2): consecutive workgroup ids are dealt round-robin over 8 XCDs.
__device__ __forceinline__ void xcd_group_map(int x, int groups, int per_group, int& grp, int& mem) {
  const int total = groups * per_group;
  if (per_group > 1 && total % (8 * per_group) == 0) {
    const int xcd = x % 8, slot = x / 8;
    grp = xcd * (total / (8 * per_group)) + slot / per_group;
    mem = slot % per_group;
  } else {
    grp = x / per_group;
    mem = x % per_group;
  }
}

// Elementwise copy of a [R][D] block into LDS converting to the operand type
// (optionally scaled).
template <typename TS, typename T, int R, int D, int NTH = 256>
__device__ __forceinline__ void stage_convert(T* dst, int ld, const TS* src, size_t src_ld,
                                              float mul = 1.f) {
  constexpr int PER_ROW = D / 8;
  constexpr int NP = R * PER_ROW, IT = (NP + NTH - 1) / NTH;
  Raw8<TS> tmp[IT];
#pragma unroll
  for (int i = 0; i < IT; ++i) {
    const int e = threadIdx.x + NTH * i;
    if (NP % NTH == 0 || e < NP) tmp[i].load(src + (size_t)(e / PER_ROW) * src_ld + (e % PER_ROW) * 8);
  }
#pragma unroll
  for (int i = 0; i < IT; ++i) {
    const int e = threadIdx.x + NTH * i;
    if (NP % NTH == 0 || e < NP) {
      float x[8];
#pragma unroll
      for (int j = 0; j < 8; ++j) x[j] = tmp[i][j] * mul;
      store8(dst + (e / PER_ROW) * ld + (e % PER_ROW) * 8, x);
    }
  }
}

}  // namespace ah
