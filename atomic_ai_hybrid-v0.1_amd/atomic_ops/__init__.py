"""MI355X (gfx950) GDN2 WY chunk pipeline and Mamba2 SSD chunk scan.

Drop-in entry points with the reference's names and argument orders:
  kernel_trainable_B6.gdn2_pallas_forward_trainable(q, k, v, w, b, g, scale, h0=None)
  kernel_mamba2_trainable_B6.mamba2_pallas_forward_trainable_B6(dt, x, B, C, A, chunk_size, state0=None)
All computation runs in libatomic_hybrid.so (built by ../build.py); there is
no CPU or PyTorch fallback.
"""
