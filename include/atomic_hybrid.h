/*
 * atomic_hybrid.h -- C ABI of the MI355X (gfx950) GDN2 WY chunk pipeline and
 * Mamba2 SSD chunk scan.
 *
 * Plain pointers and sizes only.  Every tensor is a device pointer to a dense
 * row-major array; every call is stream-ordered on `stream` (a hipStream_t,
 * or NULL for the default stream), allocates nothing and never synchronises
 * the host.  Scratch memory is a caller-owned `workspace` of at least the
 * size the matching *_workspace_size call returns.
 *
 * Host state: the library keeps one piece of mutable host state, the REUSE
 * table (a mutex-guarded list of at most 1024 records of which saving
 * forward each workspace address range holds; see ATOMIC_GDN2_REUSE).  The
 * entry points may be called from several host threads at once; the table's
 * only effect is the ATOMIC_ERR_REUSE refusal.  The no-allocation forward
 * also keeps a per-device scratch address (atomic_gdn2_fwd_noalloc).
 *
 * REUSE is safe only while the caller owns the workspace between the saving
 * forward and the reusing backward: the table is keyed by addresses, so a
 * workspace freed, reallocated at the same address and rewritten by other
 * code (not this library), or an input rewritten in place, passes the check
 * with stale intermediates.  A caller that cannot guarantee that passes no
 * REUSE flag (the backward then recomputes the forward).
 *
 * Return value: ATOMIC_OK (0) or a negative ATOMIC_ERR_* code.  The reference
 * raises shape errors at trace time and has no runtime error channel
 * (kernel_a_scores.py:71-72, gdn2_wy_reference.py:109-112); here the same
 * checks return ATOMIC_ERR_SHAPE before anything is launched.  Numerical
 * faults are absorbed by the same clip / nan_to_num placement as the
 * reference, never reported.
 */
#ifndef ATOMIC_HYBRID_H
#define ATOMIC_HYBRID_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

enum {
  ATOMIC_OK = 0,
  ATOMIC_ERR_SHAPE = -1,      /* unsupported or inconsistent dimensions       */
  ATOMIC_ERR_DTYPE = -2,      /* unsupported dtype code                       */
  ATOMIC_ERR_WORKSPACE = -3,  /* workspace NULL or smaller than required      */
  ATOMIC_ERR_LAUNCH = -4,     /* a kernel launch failed                       */
  ATOMIC_ERR_NULL = -5,       /* a required pointer is NULL                   */
  ATOMIC_ERR_SCRATCH = -6,    /* a no-allocation entry point: the shape does not
                                 fit its fixed scratch, or the flags ask for
                                 intermediates to outlive the call            */
  ATOMIC_ERR_REUSE = -7       /* a backward with the REUSE flag on a workspace
                                 that does not hold the matching forward (no
                                 saving forward on it, a forward of other
                                 shapes or input pointers, or written since by
                                 another call of this library)                */
};

enum { ATOMIC_F32 = 0, ATOMIC_BF16 = 1 };

/* Optional per-kernel timing: when an args struct's `profile` is non-NULL the
   call records start[k] / stop[k] (hipEvent_t created by the caller) on its
   stream around the k-th kernel it launches, for k < capacity, and reports
   how many kernels it launched in `count` with their names in `names`.  No
   host synchronisation; the caller reads the events after the stream. */
#define ATOMIC_PROFILE_MAX 16
typedef struct atomic_profile {
  void* start[ATOMIC_PROFILE_MAX];
  void* stop[ATOMIC_PROFILE_MAX];
  int32_t capacity;
  int32_t count;
  const char* names[ATOMIC_PROFILE_MAX];
} atomic_profile;

/* Optional per-stage report, the counterpart of the reference's opt-in
   GDN2_FWD_DIAG stage check (atomic_ops/kernel_d_pipeline.py:50-91, applied
   to each kernel's output at :177-187,121-123; model.py:107-124 for the
   Mamba2 output): for every stage a call covers, the number of non-finite
   entries of the stage's output and the largest |x| over its finite entries.
   When an args struct's `diag` is a device pointer to ATOMIC_*_DIAG_COUNT
   reports, the call clears the entries of the stages it covers and fills
   them with extra reductions launched on its stream after the path's own
   kernels (reading each stage's buffer; Akk, which no kernel stores, is
   recomputed from the inputs).  With `diag` NULL nothing extra runs.  The
   reference prints when a stage is non-finite or above 1e6; the caller reads
   the reports after the stream and decides. */
typedef struct atomic_stage_report {
  uint32_t n_nonfinite;  /* entries that are NaN or +-inf                     */
  float max_abs;         /* max |x| over the finite entries (0 if none)       */
} atomic_stage_report;

/* ------------------------------------------------------------------ GDN2 */

/* Stages of atomic_gdn2_args.diag: the forward fills [AQK, H_FINAL] (o and
   h_final when passed), the backward fills [DV_NEW, DH0]. */
enum {
  ATOMIC_GDN2_DIAG_AQK = 0,       /* kernel A: scale q k^T under the decay    */
  ATOMIC_GDN2_DIAG_AKK = 1,       /* kernel A: (b k) k^T under the decay      */
  ATOMIC_GDN2_DIAG_AINV = 2,      /* kernel B: (I + Akk)^-1                   */
  ATOMIC_GDN2_DIAG_W_PSEUDO = 3,  /* kernel C                                 */
  ATOMIC_GDN2_DIAG_U = 4,
  ATOMIC_GDN2_DIAG_KG = 5,
  ATOMIC_GDN2_DIAG_QG = 6,
  ATOMIC_GDN2_DIAG_O = 7,         /* kernel D                                 */
  ATOMIC_GDN2_DIAG_H_FINAL = 8,
  ATOMIC_GDN2_DIAG_DV_NEW = 9,    /* B2 + B1: dv_new per chunk                */
  ATOMIC_GDN2_DIAG_DH = 10,       /* B1: dh entering each chunk               */
  ATOMIC_GDN2_DIAG_DAQK = 11,     /* B2 dAqk times the query scale            */
  ATOMIC_GDN2_DIAG_DAKK = 12,     /* B3                                       */
  ATOMIC_GDN2_DIAG_DQ = 13,
  ATOMIC_GDN2_DIAG_DK = 14,
  ATOMIC_GDN2_DIAG_DV = 15,
  ATOMIC_GDN2_DIAG_DW = 16,
  ATOMIC_GDN2_DIAG_DB = 17,
  ATOMIC_GDN2_DIAG_DG = 18,
  ATOMIC_GDN2_DIAG_DH0 = 19,
  ATOMIC_GDN2_DIAG_COUNT = 20
};

/* Flags for atomic_gdn2_args.flags */
enum {
  /* forward: keep the per-chunk intermediates (state entering each chunk,
     v_new) in the workspace so a following atomic_gdn2_bwd on the same
     inputs and workspace can skip the forward recompute */
  ATOMIC_GDN2_SAVE = 1,
  /* backward: the workspace holds the intermediates of an
     atomic_gdn2_fwd(..., ATOMIC_GDN2_SAVE) call on identical inputs.  The
     library records (host side) which forward each workspace holds and
     returns ATOMIC_ERR_REUSE before launching anything when it is not this
     call's (same shapes, dtype and input pointers); contents rewritten in
     place between the calls are not detected */
  ATOMIC_GDN2_REUSE = 2,
  /* forward, and the backward's recompute of it: clip h0 to +-1e4 and
     nan_to_num it before the first chunk, as the reference's staged forward
     does (_sanitize_h0, kernel_d_pipeline.py:54-55,101), which the trainable
     op runs (kernel_trainable_B6.py:87-88).  Without the flag h0 enters as
     given, as in gdn2_chunked_wy_reference (gdn2_wy_reference.py:122-123).
     dh0 is the gradient at the sanitised h0, unmasked, as B1 returns it
     (kernel_bwd_b1_dhu.py:14-44).  The REUSE record includes the flag. */
  ATOMIC_GDN2_SANITIZE_H0 = 4
};

typedef struct atomic_gdn2_args {
  int32_t batch;     /* B                                                       */
  int32_t seqlen;    /* T, a multiple of chunk                                  */
  int32_t heads;     /* H                                                       */
  int32_t dk;        /* K: 64 or 128                                            */
  int32_t dv;        /* V: equal to dk                                          */
  int32_t chunk;     /* C: 64, 128 or 256 (all run as 64-row chunks: equal while
                        every gate g <= 0, up to exp(-20) floor terms)        */
  int32_t dtype;     /* q, k, v, w, b and their gradients: ATOMIC_F32 / _BF16  */
  int32_t do_dtype;  /* upstream gradient dO: ATOMIC_F32 / ATOMIC_BF16          */
  float scale;       /* query scale (the model passes 1.0, model.py:631)        */
  int32_t flags;     /* ATOMIC_GDN2_*                                           */
  atomic_profile* profile;  /* optional per-kernel event timing, or NULL      */
  atomic_stage_report* diag;  /* optional stage reports (device memory,
                                 ATOMIC_GDN2_DIAG_COUNT entries), or NULL    */
  /* Row strides of the [B, T, H, D] inputs q, k, v, w, b, g, dO, in elements:
     token t of batch row b starts at (b T + t) * row_stride[i] (a slice of a
     wider [B, T, F] tensor, e.g. one part of a fused projection).  0 = dense
     (H K or H V).  Otherwise at least the dense value and a multiple of 8;
     every input pointer 16-byte aligned.  Outputs and gradients are dense. */
  int64_t row_stride[7];
} atomic_gdn2_args;

/* Bytes of workspace atomic_gdn2_fwd / atomic_gdn2_bwd need for these args. */
size_t atomic_gdn2_workspace_size(const atomic_gdn2_args* a);

/* Byte offsets of the per-chunk intermediates inside the workspace, for
   stage-level inspection.  Each block is [B][H][NT][rows][cols] (NT = T / 64:
   the kernels' chunk length is 64 whatever `chunk` says) in the
   operand dtype (bf16 for bf16 inputs, fp32 for fp32 inputs) except gc_last
   (fp32).  Returns ATOMIC_OK or ATOMIC_ERR_SHAPE. */
typedef struct atomic_gdn2_layout {
  size_t qg, kg, w_pseudo, u, aqk, ainv, gc_last, h_pre_t, v_new_t;
  size_t total;
} atomic_gdn2_layout;
int atomic_gdn2_workspace_layout(const atomic_gdn2_args* a, atomic_gdn2_layout* out);

/*
 * GDN2 WY chunked forward.  Replaces gdn2_pallas_forward / the forward of
 * gdn2_pallas_forward_trainable(q, k, v, w, b, g, scale, h0)
 * (reference atomic_ops/kernel_trainable_B6.py:187-194,
 *  atomic_ops/kernel_d_pipeline.py:161-196); numerics follow
 * gdn2_chunked_wy_reference (atomic_ops/gdn2_wy_reference.py:105-152).
 *   q, k, b : [B, T, H, K]  dtype        v, w : [B, T, H, V]  dtype
 *   g       : [B, T, H, K]  fp32 log-decay
 *   h0      : [B, H, K, V]  fp32, NULL means zeros
 *   o       : [B, T, H, V]  fp32 (the reference returns fp32, :151)
 *   h_final : [B, H, K, V]  fp32
 */
int atomic_gdn2_fwd(const atomic_gdn2_args* a, const void* q, const void* k, const void* v,
                    const void* w, const void* b, const float* g, const float* h0, float* o,
                    float* h_final, void* workspace, size_t workspace_bytes, void* stream);

/*
 * GDN2 chunked backward: the B2 -> B1 -> B3 -> B4 -> B5 chain of
 * _gdn2_core_bwd (reference atomic_ops/kernel_trainable_B6.py:97-181), whose
 * result is the gradient of gdn2_chunked_wy_reference (kernel_trainable.py:38-55).
 *   dO       : [B, T, H, V]  do_dtype
 *   dh_final : [B, H, K, V]  fp32, NULL means zeros
 *   dq, dk, db : [B, T, H, K] dtype     dv, dw : [B, T, H, V] dtype
 *   dg       : [B, T, H, K]  fp32       dh0 : [B, H, K, V] fp32 (may be NULL)
 * Every gradient passes the final clip(+-1e4) / nan_to_num of
 * kernel_trainable_B6.py:64-66,173-179 and is cast to its primal's dtype.
 */
int atomic_gdn2_bwd(const atomic_gdn2_args* a, const void* q, const void* k, const void* v,
                    const void* w, const void* b, const float* g, const float* h0,
                    const void* dO, const float* dh_final, void* dq, void* dk, void* dv,
                    void* dw, void* db, float* dg, float* dh0, void* workspace,
                    size_t workspace_bytes, void* stream);

/*
 * GDN2 forward that allocates nothing and takes no workspace.  It has no
 * counterpart in the reference: it is for callers that cannot allocate
 * device memory (code under HIP graph capture, tight serving loops,
 * harnesses that forbid hipMalloc).  Arguments and results are those of
 * atomic_gdn2_fwd without the workspace; `a->flags` must be 0.
 * Scratch: a 64 MiB device array inside the library, one per device, held
 * from the library's first use on that device until the process ends.  The
 * call runs one batch row and a window of chunks at a time out of it, so any
 * batch and sequence length fit; it returns ATOMIC_ERR_SCRATCH when a single
 * chunk of all heads, with two fp32 states of all heads, does not fit (about
 * 310 heads at K = V = 128 in bf16).
 * Every call on a device shares that device's array: calls that overlap on
 * one device (concurrent streams or host threads) race and must be
 * serialised by the caller.  Nothing in it needs clearing: each call writes
 * what it reads.  The current device must be the one `stream` belongs to.
 */
int atomic_gdn2_fwd_noalloc(const atomic_gdn2_args* a, const void* q, const void* k, const void* v,
                            const void* w, const void* b, const float* g, const float* h0, float* o,
                            float* h_final, void* stream);

/* ------------------------------------------------------------------------
 * GDN2 stage-level forward: the staged pipeline's kernels A, B, C, D over
 * caller-owned per-block arrays in the reference's layout.  args.chunk picks
 * the block BT:
 *   256  the reference's Pallas block (kernel_a_scores.py:15-17): every
 *        array is float32 whatever args.dtype (the inputs' type), as the
 *        reference's are; the kernels follow kernel A's 128-row sub-blocks
 *        with pairwise exp(clip(gc_i - gc_j, +-20)), kernel B's 16-row block
 *        recursion over two 128-row halves and its A10 = -A11 T10 A00 step
 *        with a sanitise at every block product (kernel_b_solve.py:66-148),
 *        kernel C's float32 w v (kernel_c_recompute.py:49-82);
 *   64   this library's own chunk: the arrays are in args.dtype (gc_last,
 *        o, h_final fp32), from the whole path's kernels.
 * NT = T / BT.
 *   Aqk, A : [B][H][NT][BT][BT]   w_pseudo, kg, qg : [B][H][NT][BT][K]
 *   u : [B][H][NT][BT][V]         gc_last : [B][H][NT][K]
 *
 * Kernels A + B + C in one pass: build_chunk_scores_pallas (Aqk, scaled;
 * kernel_a_scores.py:69), wy_solve_pallas (A = (I + Akk)^-1;
 * kernel_b_solve.py:151) and recompute_wy_pallas (w_pseudo, u, kg, qg,
 * gc_last; kernel_c_recompute.py:91).  Akk itself stays on chip.
 */
/* (64-row chunks only: at 256 it returns ATOMIC_ERR_SHAPE, since Akk would
 * need caller memory; chain the three entries below instead.) */
int atomic_gdn2_chunk_wy(const atomic_gdn2_args* a, const void* q, const void* k, const void* v,
                         const void* w, const void* b, const float* g, void* Aqk, void* A, void* w_pseudo,
                         void* u, void* kg, void* qg, float* gc_last, void* stream);

/* Kernel A alone: build_chunk_scores_pallas(q, k, b, g, scale)
 * (kernel_a_scores.py:69-99): Aqk (causal, scaled) and the strict Akk,
 * [B][H][NT][BT][BT], nan_to_num'd (kernel_a_scores.py:65-66). */
int atomic_gdn2_chunk_scores(const atomic_gdn2_args* a, const void* q, const void* k, const void* b,
                             const float* g, void* Aqk, void* Akk, void* stream);

/* Kernel B alone: wy_solve_pallas(Akk) (kernel_b_solve.py:151-169),
 * A = (I + Akk)^-1 by 16-row block forward substitution; like the
 * reference, only the strictly lower part of Akk is read.  At BT = 256 Akk
 * and A are float32 and args.dtype is not read. */
int atomic_gdn2_wy_solve(const atomic_gdn2_args* a, const void* Akk, void* A, void* stream);

/* Kernel C alone: recompute_wy_pallas(q, k, v, w, b, g, A)
 * (kernel_c_recompute.py:91-123): w_pseudo = A (b k e^gc), u = A (w v),
 * kg, qg, gc_last, each clipped to +-1e4 (kernel_c_recompute.py:74-82);
 * the whole A is read. */
int atomic_gdn2_recompute_wy(const atomic_gdn2_args* a, const void* q, const void* k, const void* v,
                             const void* w, const void* b, const float* g, const void* A, void* w_pseudo,
                             void* u, void* kg, void* qg, float* gc_last, void* stream);

/* Kernel D: gdn2_inter_chunk_combine (kernel_d_pipeline.py:94-124), the
 * sequential state loop over those arrays.  h0 [B][H][K][V] (NULL: zeros) is
 * sanitised first like the reference's _sanitize_h0 (:54-55); o is written per
 * block, [B][H][NT][BT][V] fp32, and h_final [B][H][K][V] fp32. */
int atomic_gdn2_inter_chunk_combine(const atomic_gdn2_args* a, const void* Aqk, const void* w_pseudo,
                                    const void* u, const void* kg, const void* qg, const float* gc_last,
                                    const float* h0, float* o, float* h_final, void* stream);

/* Kernel D keeping its per-chunk states: gdn2_inter_chunk_combine_with_state
 * (kernel_d_pipeline.py:127-158), the residuals of the reference's backward.
 * Besides o and h_final it writes the state entering each block and v_new:
 * at BT = 64 in args.dtype and transposed (the layout this library's
 * backward reads), h_pre_t [B][H][NT][V][K] and v_new_t [B][H][NT][V][64];
 * at BT = 256 in float32, h_pre [B][H][NT][K][V] and v_new [B][H][NT][256][V]. */
int atomic_gdn2_inter_chunk_combine_with_state(const atomic_gdn2_args* a, const void* Aqk, const void* w_pseudo,
                                               const void* u, const void* kg, const void* qg,
                                               const float* gc_last, const float* h0, float* o, float* h_final,
                                               void* h_pre_t, void* v_new_t, void* stream);

/* ---- Backward stages at the reference's 256-row block
 * The staged backward of the reference's trainable op
 * (atomic_ops/kernel_trainable_B6.py:97-181): args.chunk must be 256
 * (ATOMIC_ERR_SHAPE otherwise).  Every per-block array is float32, in the
 * reference's layout: [B][H][NT][256][D] (D = K = V), scores [B][H][NT][256][256],
 * states [B][H][NT][K][V].  dO is of args.do_dtype; q, k, b, w, v of
 * args.dtype.  Block products accumulate in float32 in an order of their own;
 * the clip / nan_to_num placement is the reference kernels'. */

/* Kernel B2, dav_backward_pallas(Aqk, v_new, do) (kernel_bwd_b2_dav.py:17-51):
 * dAqk = nan_to_num((do v_new^T) * causal), dv_new = nan_to_num(Aqk^T do);
 * dO per block [B][H][NT][256][V]. */
int atomic_gdn2_dav_backward(const atomic_gdn2_args* a, const float* Aqk, const float* v_new, const void* dO,
                             float* dAqk, float* dv_new, void* stream);

/* Kernel B1, gdn2_dhu_backward(do, dv_partial, w_pseudo, qg, kg, gc_last,
 * scale, dht) (kernel_bwd_b1_dhu.py:14-44): the reverse scan.  dht
 * [B][H][K][V] (NULL: zeros) is sanitised first; dh_all[n] is the carry after
 * block n, dh0 the carry after block 0, dv_all the sanitised dv_new. */
int atomic_gdn2_dhu_backward(const atomic_gdn2_args* a, const void* dO, const float* dv_partial,
                             const float* w_pseudo, const float* qg, const float* kg, const float* gc_last,
                             const float* dht, float* dh_all, float* dh0, float* dv_all, void* stream);

/* Bytes of workspace atomic_gdn2_wy_dqkg_backward needs (0 for unsupported args). */
size_t atomic_gdn2_wy_dqkg_workspace_size(const atomic_gdn2_args* a);

/* Kernel B3, wy_dqkg_backward_pallas(q, k, b, w, v, gc, A, Akk, h_pre_all,
 * v_new_all, do, dv, dh_next_all, scale) (kernel_bwd_b3_wy_dqkg.py:33-148):
 * dq, dk, db, dw, dv_raw, dgc and dAkk, with dA_total and tmp clipped before
 * the products through A^T (:75-86).  q, k, b, w, v, gc, dO, dv per block;
 * Akk, which the reference reads for its shape only, is not an argument. */
int atomic_gdn2_wy_dqkg_backward(const atomic_gdn2_args* a, const void* q, const void* k, const void* b,
                                 const void* w, const void* v, const float* gc, const float* A, const float* h_pre,
                                 const float* v_new, const void* dO, const float* dv, const float* dh_next,
                                 float* dq, float* dk, float* db, float* dw, float* dv_raw, float* dgc,
                                 float* dAkk, void* workspace, size_t workspace_bytes, void* stream);

/* Kernel B4, intra_backward_pallas(dAqk, dAkk, q, k, b, g, scale)
 * (kernel_bwd_b4_intra.py:57-165): kernel A's backward over its 128-row
 * sub-block pairs with a clip after every accumulation.  q, k, b, g are the
 * [B][T][H][K] inputs (args.row_stride applies); dq, dk, db, dgc per block. */
int atomic_gdn2_intra_backward(const atomic_gdn2_args* a, const float* dAqk, const float* dAkk, const void* q,
                               const void* k, const void* b, const float* g, float* dq, float* dk, float* db,
                               float* dgc, void* stream);

/* Kernel B5, reverse_cumsum_bwd(dgc, chunk_size)
 * (kernel_bwd_b5_reverse_cumsum.py:17-24): dg = sanitize(suffix sum over
 * each block's rows) of a [B][H][T / chunk][chunk][K] float32 array, for any
 * args.chunk. */
int atomic_gdn2_reverse_cumsum_bwd(const atomic_gdn2_args* a, const float* dgc, float* dg, void* stream);

/* ---------------------------------------------------------------- Mamba2 */

enum {
  /* forward: the per-chunk states a following atomic_mamba2_bwd on the same
     inputs and workspace can reuse (the forward always leaves them in the
     workspace; the flag is accepted for symmetry with GDN2) */
  ATOMIC_MAMBA2_SAVE = 1,
  /* backward: the workspace holds the intermediates of an
     atomic_mamba2_fwd call on identical inputs (checked as for
     ATOMIC_GDN2_REUSE: ATOMIC_ERR_REUSE otherwise) */
  ATOMIC_MAMBA2_REUSE = 2,
  /* forward, and the backward's recompute of it: clip state0 to +-1e4 and
     nan_to_num it first, as the reference's staged combine does
     (kernel_mamba2_c_interchunk.py:56-58), which the trainable op runs
     (kernel_mamba2_trainable_B6.py:72-80).  Without the flag state0 enters
     as given, as in mamba2_ssd_reference.  dstate0 is unmasked. */
  ATOMIC_MAMBA2_SANITIZE_STATE0 = 4
};

/* Stages of atomic_mamba2_args.diag: the forward fills [CB, STATE_FINAL],
   the backward fills [DSTATES, DSTATE0]. */
enum {
  ATOMIC_MAMBA2_DIAG_CB = 0,           /* C B^T per chunk (shared by heads)   */
  ATOMIC_MAMBA2_DIAG_STATES = 1,       /* state entering each chunk           */
  ATOMIC_MAMBA2_DIAG_Y = 2,            /* the SSD output (model.py:519)       */
  ATOMIC_MAMBA2_DIAG_STATE_FINAL = 3,
  ATOMIC_MAMBA2_DIAG_DSTATES = 4,      /* dstate entering each chunk's bwd    */
  ATOMIC_MAMBA2_DIAG_DDT = 5,
  ATOMIC_MAMBA2_DIAG_DX = 6,
  ATOMIC_MAMBA2_DIAG_DB = 7,
  ATOMIC_MAMBA2_DIAG_DC = 8,
  ATOMIC_MAMBA2_DIAG_DA = 9,
  ATOMIC_MAMBA2_DIAG_DSTATE0 = 10,
  ATOMIC_MAMBA2_DIAG_COUNT = 11
};

typedef struct atomic_mamba2_args {
  int32_t batch;     /* B                                                  */
  int32_t seqlen;    /* T, a multiple of chunk                             */
  int32_t heads;     /* H                                                  */
  int32_t headdim;   /* P: 64, 128, or 192 (the model's d_inner / heads) with N = 128 */
  int32_t dstate;    /* N: 64 or 128 (ngroups = 1: B and C shared by heads) */
  int32_t chunk;     /* C: 64, 128 or 256 (256 runs as 128-row chunks: equal
                        while every dt A <= 0, up to exp(-20) floor terms)   */
  int32_t dtype;     /* dt, x, B, C and their gradients: ATOMIC_BF16, or
                        ATOMIC_F32: then atomic_mamba2_fwd / _bwd run the
                        float32 staged chain at the given chunk (M2 -> M3 ->
                        M4, MB1 + MB3 -> MB4; the stage entries' arithmetic,
                        state0 always sanitised), REUSE is not checked (the
                        backward re-runs the forward) and diag must be NULL */
  int32_t dy_dtype;  /* upstream gradient dy: ATOMIC_F32 / ATOMIC_BF16     */
  int32_t flags;     /* ATOMIC_MAMBA2_*                                    */
  atomic_profile* profile;  /* optional per-kernel event timing, or NULL */
  atomic_stage_report* diag;  /* optional stage reports (device memory,
                                 ATOMIC_MAMBA2_DIAG_COUNT entries), or NULL */
  /* Row strides of the inputs dt, x ([B, T, H, P]), B, C ([B, T, N]) and dy,
     in elements: token t of batch row b starts at (b T + t) * row_stride[i].
     0 = dense (H P, or N).  Otherwise at least the dense value and a multiple
     of 8; every input pointer 16-byte aligned.  Outputs and gradients are
     dense, and so are the stage entries' per-chunk arrays. */
  int64_t row_stride[5];
} atomic_mamba2_args;

/* Bytes of workspace atomic_mamba2_fwd / atomic_mamba2_bwd need. */
size_t atomic_mamba2_workspace_size(const atomic_mamba2_args* a);

/*
 * Mamba2 SSD chunk-scan forward.  Replaces mamba2_pallas_forward / the forward
 * of mamba2_pallas_forward_trainable_B6(dt, x, B, C, A, chunk_size, state0)
 * (reference atomic_ops/kernel_mamba2_trainable_B6.py:137-155,
 *  atomic_ops/kernel_mamba2_c_interchunk.py:90-100); numerics follow
 * mamba2_ssd_reference (atomic_ops/mamba2_ssd_reference.py:152-179).
 *   dt, x  : [B, T, H, P]  dtype       B, C : [B, T, N]  dtype
 *   A      : [H]           fp32 (negative log-decay rate per unit dt)
 *   state0 : [B, H, P, N]  fp32, NULL means zeros
 *   y      : [B, T, H, P]  fp32 (the reference returns fp32, :148,178)
 *   state_final : [B, H, P, N] fp32
 * There is no D * x skip term (the reference has none, :152).
 */
int atomic_mamba2_fwd(const atomic_mamba2_args* a, const void* dt, const void* x, const void* B,
                      const void* C, const float* A, const float* state0, float* y,
                      float* state_final, void* workspace, size_t workspace_bytes, void* stream);

/*
 * Mamba2 SSD chunk-scan backward with the semantics of the hand-derived MB0
 * backward chunk_ssd_bwd_scan (reference atomic_ops/mamba2_bwd_reference.py:55-266):
 * straight-through clip masks, per-chunk sanitising, dA summed over batch,
 * chunks, time and channels; then the final clip(+-1e4) / nan_to_num and
 * cast of kernel_mamba2_trainable_B6.py:108-129.
 *   dy : [B, T, H, P] dy_dtype          dstate_final : [B, H, P, N] fp32 or NULL
 *   ddt, dx : [B, T, H, P] dtype        dB, dC : [B, T, N] dtype
 *   dA : [H] fp32                       dstate0 : [B, H, P, N] fp32 (may be NULL)
 */
int atomic_mamba2_bwd(const atomic_mamba2_args* a, const void* dt, const void* x, const void* B,
                      const void* C, const float* A, const float* state0, const void* dy,
                      const float* dstate_final, void* ddt, void* dx, void* dB, void* dC, float* dA,
                      float* dstate0, void* workspace, size_t workspace_bytes, void* stream);

/* ------------------------------------------------------------------------
 * Mamba2 stage-level forward: the reference's staged pipeline M2 -> M3 -> M4
 * (mamba2_pallas_forward, kernel_mamba2_c_interchunk.py:90-100) over
 * caller-owned arrays in its layout.  args.chunk is 64, 128 or 256 (the
 * model's chunk, model.py:436), the arrays per chunk of that size; at 256,
 * M3 sums over the reference's two 128-row sub-blocks, sanitising each
 * sub-block's part before the next is added (kernel_mamba2_b_intra.py:61-62,
 * 86-108), and M4 keeps the states entering each chunk in float32.  dt, x,
 * B, C bf16 or fp32 (args.dtype; the backward stage entries too); the arrays
 * fp32:
 *   cumdecay : [B][H][NT][C][P]     state_end : [B][H][NT][P][N]
 *   y_diag, y : [B][T][H][P]        state0, state_final : [B][H][P][N]
 * The arithmetic is that of the stage kernels, which differ from the whole
 * path only where a step exponent dt A is positive: no 1e6 caps on the pair
 * weight and the decay to the chunk end (kernel_mamba2_b_intra.py:96-112).
 */

/* bytes of workspace atomic_mamba2_intra_chunk_ssd and
   atomic_mamba2_inter_chunk_combine need (0 for unsupported args) */
size_t atomic_mamba2_stage_workspace_size(const atomic_mamba2_args* a);

/* M2: build_chunk_cumdecay_pallas(dt, A, chunk_size)
 * (kernel_mamba2_a_decay.py:71-105): sanitize(cumsum(sanitize(dt A, 20)), 1e4). */
int atomic_mamba2_chunk_cumdecay(const atomic_mamba2_args* a, const void* dt, const float* A, float* cumdecay,
                                 void* stream);

/* M3: intra_chunk_ssd_pallas(dt, x, B, C, cumdecay, chunk_size)
 * (kernel_mamba2_b_intra.py:119-163): y_diag and each chunk's state_end
 * from the given cumdecay. */
int atomic_mamba2_intra_chunk_ssd(const atomic_mamba2_args* a, const void* dt, const void* x, const void* B,
                                  const void* C, const float* cumdecay, float* y_diag, float* state_end,
                                  void* workspace, size_t workspace_bytes, void* stream);

/* M4: mamba2_inter_chunk_combine(y_diag, state_end, cumdecay, C, chunk_size,
 * state0) (kernel_mamba2_c_interchunk.py:38-87): the sequential state pass
 * (state0 sanitised, NULL = zeros) and y = sanitize(y_diag + y_off). */
int atomic_mamba2_inter_chunk_combine(const atomic_mamba2_args* a, const float* y_diag, const float* state_end,
                                      const float* cumdecay, const void* C, const float* state0, float* y,
                                      float* state_final, void* workspace, size_t workspace_bytes,
                                      void* stream);

/* Bytes of workspace atomic_mamba2_intra_chunk_ssd_bwd needs (0 for unsupported args). */
size_t atomic_mamba2_intra_chunk_ssd_bwd_workspace_size(const atomic_mamba2_args* a);

/* MB2: intra_chunk_ssd_bwd_pallas(dt, x, B, C, cumdecay, dy, dstate_end_grad,
 * chunk_size) (kernel_mamba2_bwd_b2_intra.py:32-180): the backward of M3 at
 * args.chunk (64, 128 or 256, run as that chunk): the state-end part as
 * whole-chunk products, the y_diag part over min(128, chunk)-row sub-block
 * pairs with a sanitise after every accumulation, in float32.  cumdecay
 * [B][H][NT][C][P] and dstate_end_grad [B][H][NT][P][N] float32, dy of
 * args.dy_dtype; outputs float32: ddt, dx [B][T][H][P], dB, dC [B][T][N]
 * (the per-head values summed over the heads, :168-178) and dcum
 * [B][H][NT][C][P]. */
int atomic_mamba2_intra_chunk_ssd_bwd(const atomic_mamba2_args* a, const void* dt, const void* x, const void* B,
                                      const void* C, const float* cumdecay, const void* dy,
                                      const float* dstate_end_grad, float* ddt, float* dx, float* dB, float* dC,
                                      float* dcum, void* workspace, size_t workspace_bytes, void* stream);

/* Bytes of workspace atomic_mamba2_bwd_scan needs (0 for unsupported args). */
size_t atomic_mamba2_bwd_scan_workspace_size(const atomic_mamba2_args* a);

/* MB1 + MB3: mamba2_bwd_scan(dt, A, B, C, x, chunk_size, do, dstate_final,
 * state0) (kernel_mamba2_bwd_b1_state.py:132-254) at args.chunk (64, 128 or
 * 256; P a multiple of 32): M2's cumdecay, the reference chunk's forward
 * re-run for the state entering each chunk (state0 sanitised, NULL = zeros),
 * the state-only reverse scan (mamba2_bwd_state_reference.py:87-137; its
 * y_off decay term is masked on the clipped exponent as there, :123-124, so
 * every cum passes, where MB0 masks on cum) whose
 * sanitised carries are MB2's dstate_end_grad, MB2, and the sanitised sums
 * of the two halves.  dstate_final [B][H][P][N] or NULL.  Outputs float32:
 * ddt (the dt x part only, as the reference's), dx [B][T][H][P], dB, dC
 * [B][T][N], dstate0 [B][H][P][N] and dcumdecay [B][H][NT][C][P]. */
int atomic_mamba2_bwd_scan(const atomic_mamba2_args* a, const void* dt, const float* A, const void* B, const void* C,
                           const void* x, const void* dy, const float* dstate_final, const float* state0, float* ddt,
                           float* dB, float* dC, float* dx, float* dstate0, float* dcumdecay, void* workspace,
                           size_t workspace_bytes, void* stream);

/* Bytes of workspace atomic_mamba2_da_backward needs (0 for unsupported args). */
size_t atomic_mamba2_da_backward_workspace_size(const atomic_mamba2_args* a);

/* MB4: mamba2_dA_backward(dt_pallas, A, dcumdecay_combined, chunk_size)
 * (mamba2_bwd_a_dA_reference.py:60-115): M2's adjoint.  dt per chunk
 * [B][H][NT][C][P] in args.dtype (bf16 or fp32), A [H], dcumdecay
 * [B][H][NT][C][P] float32; ddt_contrib (float32, dt's layout) and dA [H],
 * each sanitised.  args.dstate is not read. */
int atomic_mamba2_da_backward(const atomic_mamba2_args* a, const void* dt_chunks, const float* A,
                              const float* dcumdecay, float* ddt_contrib, float* dA, void* workspace,
                              size_t workspace_bytes, void* stream);

/* ------------------------------------------- output epilogue (downstream) */

/* The two mixer blocks' output epilogue: RMSNorm over the model dimension
   and the SiLU gate, fused.
     ATOMIC_NORM_GATE_GDN2:   out = bf16(bf16(RMSNorm(x)) * silu(clip(gate, +-1e2)))
                              (reference model.py:612-613,650-653; x is the
                              GDN2 output o, gate the out_gate projection)
     ATOMIC_NORM_GATE_MAMBA2: out = clip(bf16(bf16(RMSNorm(bf16(x))) * silu(gate)), +-3e2)
                              (reference model.py:516-525; x is the SSD
                              output y, gate the `res` half of in_proj)
   RMSNorm(x) = x * rsqrt(mean(x^2) + eps) * weight, statistics in fp32 (flax
   linen RMSNorm).  The result feeds the block's out_proj GEMM. */
enum { ATOMIC_NORM_GATE_GDN2 = 0, ATOMIC_NORM_GATE_MAMBA2 = 1 };

typedef struct atomic_norm_gate_args {
  int32_t rows;      /* B * T                                                   */
  int32_t dim;       /* d (H * V, or H * P): 512 x {1,2,3,4,6,8,12,16}          */
  int32_t variant;   /* ATOMIC_NORM_GATE_*                                      */
  float eps;         /* 1e-6 in both blocks                                     */
  atomic_profile* profile;  /* optional per-kernel event timing, or NULL      */
} atomic_norm_gate_args;

/* Bytes of workspace atomic_norm_gate_bwd needs (0 for unsupported args). */
size_t atomic_norm_gate_workspace_size(const atomic_norm_gate_args* a);

/*
 * Forward.  Replaces the inline epilogue of GatedDeltaNet2J.__call__
 * (model.py:650-653) / the Mamba2 block (model.py:516-525).
 *   x      : [rows, dim] fp32 (o / y as the path returns them, [B, T, H, V])
 *   gate   : [rows, dim] bf16 (out_gate, or res)
 *   weight : [dim]       fp32 RMSNorm scale
 *   out    : [rows, dim] bf16
 */
int atomic_norm_gate_fwd(const atomic_norm_gate_args* a, const float* x, const void* gate,
                         const float* weight, void* out, void* stream);

/*
 * Backward of the same function for dout = d loss / d out (bf16):
 *   dx : [rows, dim] fp32    dgate : [rows, dim] bf16    dweight : [dim] fp32
 */
int atomic_norm_gate_bwd(const atomic_norm_gate_args* a, const float* x, const void* gate,
                         const float* weight, const void* dout, float* dx, void* dgate,
                         float* dweight, void* workspace, size_t workspace_bytes, void* stream);

/* ------------------------------------------- GDN2 prologue (upstream) */

/* The GDN2 block's prologue, fused: from the projection outputs to the
   chunk pipeline's inputs (reference model.py:574-619):
     q, k = normalize(silu(conv(q_lin / k_lin) + bias))   per head of dh channels
     v    = clip(silu(conv(v_lin) + bias), +-50)
     b, w = sigmoid(b_pre / w_pre)
     g    = nan_to_num(-exp(clip(a, +-20))[h] softplus(f_pre), nan 0, +inf 0, -inf -20)
     each = nan_to_num(clip(., +-1e3))
   conv is the causal depthwise convolution of short_causal_conv (d_conv taps,
   padding d_conv - 1 on the left) with the fp32 parameters cast to bf16;
   normalize(t) = t * rsqrt(sum t^2 + eps^2). */
typedef struct atomic_gdn2_prologue_args {
  int32_t batch;     /* B                                                     */
  int32_t seqlen;    /* L: a multiple of 128                                  */
  int32_t heads;     /* H                                                     */
  int32_t dhead;     /* dh: 64 or 128; d = H * dh a multiple of 512           */
  int32_t dconv;     /* d_conv: 4 (the model's)                               */
  float eps;         /* 1e-6 (the normalisation adds eps^2)                   */
  atomic_profile* profile;  /* optional per-kernel event timing, or NULL    */
} atomic_gdn2_prologue_args;

/* Bytes of workspace atomic_gdn2_prologue_bwd needs (0 for unsupported args). */
size_t atomic_gdn2_prologue_workspace_size(const atomic_gdn2_prologue_args* a);

/*
 * Forward.  Replaces GatedDeltaNet2J.__call__ between the projections and
 * the gdn2_pallas_forward_trainable call (model.py:574-619).
 *   q_lin, k_lin, v_lin, b_pre, w_pre, f_pre : [B, L, d] bf16 (projection outputs)
 *   conv_w : [3][d][dconv] fp32 (q, k, v)     conv_b : [3][d] fp32     a_param : [H] fp32
 *   q, k, v, w, b : [B, L, H, dh] bf16        g : [B, L, H, dh] fp32
 */
int atomic_gdn2_prologue_fwd(const atomic_gdn2_prologue_args* a, const void* q_lin, const void* k_lin,
                             const void* v_lin, const float* conv_w, const float* conv_b,
                             const void* b_pre, const void* w_pre, const void* f_pre,
                             const float* a_param, void* q, void* k, void* v, void* w, void* b,
                             float* g, void* stream);

/*
 * Backward for the cotangents dq, dk, dv, dw, db (bf16) and dg (fp32) of the
 * forward's outputs (the gradients atomic_gdn2_bwd returns):
 *   dq_lin, dk_lin, dv_lin, db_pre, dw_pre, df_pre : [B, L, d] bf16
 *   dconv_w : [3][d][dconv] fp32   dconv_b : [3][d] fp32   da_param : [H] fp32
 * q and k's cotangents pass the gradient sanitiser of model.py:192-217
 * (nan_to_num(clip(., +-1e3))) before the normalisation's VJP.
 */
int atomic_gdn2_prologue_bwd(const atomic_gdn2_prologue_args* a, const void* q_lin, const void* k_lin,
                             const void* v_lin, const float* conv_w, const float* conv_b,
                             const void* b_pre, const void* w_pre, const void* f_pre,
                             const float* a_param, const void* dq, const void* dk, const void* dv,
                             const void* dw, const void* db, const float* dg, void* dq_lin,
                             void* dk_lin, void* dv_lin, float* dconv_w, float* dconv_b,
                             void* db_pre, void* dw_pre, void* df_pre, float* da_param,
                             void* workspace, size_t workspace_bytes, void* stream);

/* ----------------------------------------- Mamba2 prologue (upstream) */

/* The Mamba2 block's element-wise prologue, fused (reference model.py:405-433),
   between in_proj / B_proj / C_proj / dt_proj (GEMMs, in the model) and the
   SSD call:
     x  = silu(conv(x_bc) + bias)                  (causal depthwise, dconv taps)
     dt = clip(softplus(dt_pre), bf16(1e-2), 1)
     x, dt, B, C = nan_to_num(clip(., +-1e3))
     A  = -exp(clip(A_log, +-20))                  (per head, fp32) */
typedef struct atomic_mamba2_prologue_args {
  int32_t batch;     /* B                                                   */
  int32_t seqlen;    /* L: a multiple of 128                                */
  int32_t heads;     /* H                                                   */
  int32_t headdim;   /* P; d_inner = H * P a multiple of 512                */
  int32_t dstate;    /* N: a multiple of 8                                  */
  int32_t dconv;     /* 4 (the model's)                                     */
  atomic_profile* profile;  /* optional per-kernel event timing, or NULL  */
} atomic_mamba2_prologue_args;

/* Bytes of workspace atomic_mamba2_prologue_bwd needs (0 for unsupported args). */
size_t atomic_mamba2_prologue_workspace_size(const atomic_mamba2_prologue_args* a);

/*
 * Forward.
 *   x_bc, dt_pre : [B, L, d_inner] bf16 (the in_proj half, the dt_proj output)
 *   conv_w : [d_inner][dconv] fp32   conv_b : [d_inner] fp32   a_log : [H] fp32
 *   b_pre, c_pre : [B, L, N] bf16 (B_proj, C_proj outputs)
 *   x, dt : [B, L, H, P] bf16   B, C : [B, L, N] bf16   A : [H] fp32
 */
int atomic_mamba2_prologue_fwd(const atomic_mamba2_prologue_args* a, const void* x_bc,
                               const float* conv_w, const float* conv_b, const void* dt_pre,
                               const void* b_pre, const void* c_pre, const float* a_log, void* x,
                               void* dt, void* B, void* C, float* A, void* stream);

/*
 * Backward for the cotangents dx, ddt (bf16), dB, dC (bf16) and dA (fp32) of
 * the forward's outputs (the gradients atomic_mamba2_bwd returns).  dx_bc is
 * the convolution path's part of x_bc's gradient (the B / C / dt projections'
 * parts come from their GEMMs in the model).
 *   dx_bc, ddt_pre : [B, L, d_inner] bf16   db_pre, dc_pre : [B, L, N] bf16
 *   dconv_w : [d_inner][dconv] fp32   dconv_b : [d_inner] fp32   da_log : [H] fp32
 */
int atomic_mamba2_prologue_bwd(const atomic_mamba2_prologue_args* a, const void* x_bc,
                               const float* conv_w, const float* conv_b, const void* dt_pre,
                               const void* b_pre, const void* c_pre, const float* a_log,
                               const void* dx, const void* ddt, const void* dB, const void* dC,
                               const float* dA, void* dx_bc, float* dconv_w, float* dconv_b,
                               void* ddt_pre, void* db_pre, void* dc_pre, float* da_log,
                               void* workspace, size_t workspace_bytes, void* stream);

/* ------------------------------------------------------------------------
 * Mamba2 prologue with its projections (Mamba2J.__call__, reference
 * model.py:405-433): from the in_proj output, read in place (its x_bc half,
 * the first d_inner columns of each [2 d_inner] row after jnp.split, :405-406)
 *   dt_pre = bf16(x_bc W_dt) + bf16(b_dt)      (dt_proj, :427)
 *   b_pre  = bf16(x_bc W_B)   c_pre = bf16(x_bc W_C)   (B_proj / C_proj, :425-426)
 * (bf16 products accumulated in fp32, as Dense(dtype=bfloat16)), then the
 * element-wise prologue of atomic_mamba2_prologue_fwd.  The three
 * projections are one MFMA GEMM of x_bc against [W_dt | W_B | W_C] whose
 * epilogue applies softplus / clip / sanitise; x_bc is read with its row
 * stride (no copy of the split).  Weights are the model's fp32 parameters in
 * the Dense layout ([in][out]): W_dt [d_inner][d_inner], b_dt [d_inner],
 * W_B and W_C [d_inner][N].  This pair has no single-function counterpart in
 * the reference (the block is inline in Mamba2J.__call__).
 */
typedef struct atomic_mamba2_proj_args {
  int32_t batch;      /* B                                                  */
  int32_t seqlen;     /* L: a multiple of 128                               */
  int32_t heads;      /* H                                                  */
  int32_t headdim;    /* P; d_inner = H * P a multiple of 512               */
  int32_t dstate;     /* N: a multiple of 64                                */
  int32_t dconv;      /* 4 (the model's)                                    */
  int64_t in_stride;  /* elements between consecutive tokens of x_bc and of
                         dx_bc (2 d_inner for the in_proj output); >= d_inner,
                         a multiple of 8                                    */
  atomic_profile* profile;  /* optional per-kernel event timing, or NULL  */
} atomic_mamba2_proj_args;

/* Bytes of workspace the forward (backward = 0) or backward (1) needs; 0 for
 * unsupported args. */
size_t atomic_mamba2_proj_workspace_size(const atomic_mamba2_proj_args* a, int backward);

/*
 * Forward.
 *   x_bc : [B * L] rows of in_stride bf16 (d_inner used)
 *   x, dt : [B, L, H, P] bf16   B, C : [B, L, N] bf16   A : [H] fp32
 *   dt_pre : [B, L, d_inner] bf16, b_pre / c_pre : [B, L, N] bf16 -- the
 *   projection outputs, written when non-NULL (the backward takes them)
 */
int atomic_mamba2_proj_fwd(const atomic_mamba2_proj_args* a, const void* x_bc, const float* conv_w,
                           const float* conv_b, const float* w_dt, const float* b_dt, const float* w_b,
                           const float* w_c, const float* a_log, void* x, void* dt, void* B, void* C,
                           float* A, void* dt_pre, void* b_pre, void* c_pre, void* workspace,
                           size_t workspace_bytes, void* stream);

/*
 * Backward for the cotangents dx, ddt, dB, dC (bf16) and dA (fp32) of the
 * forward's outputs.  dx_bc (rows of in_stride, d_inner columns written) is
 * x_bc's whole gradient: the convolution path's plus the three projections'.
 * Parameter gradients in fp32: dconv_w [d_inner][dconv], dconv_b [d_inner],
 * dw_dt [d_inner][d_inner], db_dt [d_inner], dw_b / dw_c [d_inner][N],
 * da_log [H]; the projection gradients are bf16-rounded like the reference's
 * bf16 dot / bias VJPs before the cast to the fp32 parameters.
 */
int atomic_mamba2_proj_bwd(const atomic_mamba2_proj_args* a, const void* x_bc, const float* conv_w,
                           const float* conv_b, const float* w_dt, const float* b_dt, const float* w_b,
                           const float* w_c, const float* a_log, const void* dt_pre, const void* b_pre,
                           const void* c_pre, const void* dx, const void* ddt, const void* dB, const void* dC,
                           const float* dA, void* dx_bc, float* dconv_w, float* dconv_b, float* dw_dt,
                           float* db_dt, float* dw_b, float* dw_c, float* da_log, void* workspace,
                           size_t workspace_bytes, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* ATOMIC_HYBRID_H */
