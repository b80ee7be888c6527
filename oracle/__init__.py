"""CPU oracle for the GDN2 WY chunk pipeline and the Mamba2 SSD chunk scan.

TEST INFRASTRUCTURE ONLY.  Nothing in the product path imports this package:
only ``tests/``, ``__graft_entry__.smoke()`` and the ``cpu_baseline`` leg of
``bench.py`` may use it, and only as the checker (or as the timed CPU
baseline), never as the thing that is measured or shipped.

What it is: a from-scratch PyTorch restatement (CPU, float64 by default,
dtype-parametric so the float32 variant can be timed as the CPU baseline) of
the reference's pure-JAX oracles.  Every function cites the reference
``file:line`` it follows (paths relative to the reference repo root).

  * ``gdn2``   -- ``atomic_ops/gdn2_wy_reference.py`` (chunked WY forward,
                  row-wise WY inverse, token-serial forward), the autodiff
                  backward that ``atomic_ops/kernel_trainable.py:38-55``
                  defines as the GDN2 gradient, and a hand restatement of the
                  B1..B5 backward chain (``kernel_trainable_B6.py:97-181``).
  * ``mamba2`` -- ``atomic_ops/mamba2_ssd_reference.py`` (chunked SSD
                  forward), a token-serial SSM, and the hand-derived MB0
                  backward of ``atomic_ops/mamba2_bwd_reference.py``.

How it is pinned (the reference ships no tests, fixtures or golden vectors,
and JAX is not installed, so the reference functions cannot be run):

  * GDN2 forward: chunked WY form against the independent token-serial
    recurrence; chunk-size invariance; state passing across a split
    sequence; ``(I + Akk) A = I``; closed forms (g=0, b=0, w=1 gives causal
    linear attention ``tril(scale Q K^T) V``; T=1 gives
    ``scale (q.k) (w*v)``).
  * GDN2 backward: torch autograd of the restated forward against central
    finite differences (float64), and against the independent hand-written
    B1..B5 chain.
  * Mamba2 forward: chunked SSD form against the token-serial SSM; A=0
    closed form (masked cumulative sum); chunk-size invariance; the
    ``state_prev = 0`` split identities.
  * Mamba2 backward: the MB0 restatement against torch autograd of the
    restated forward and against finite differences.

What stays unpinned (no reference execution possible): bit-level behaviour
in regimes where a clip or ``nan_to_num`` fires (|h| at 1e4, NaN/inf
inputs), where only a transcription review vouches for the restatement.
"""
