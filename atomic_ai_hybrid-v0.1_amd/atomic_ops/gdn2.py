"""PyTorch host side of the GDN2 WY chunk pipeline (device memory and streams
come from torch; every computation runs in libatomic_hybrid.so).

Layouts follow the reference (``atomic_ops/kernel_trainable_B6.py:187``):
q, k, b, g: [B, T, H, K]; v, w: [B, T, H, V]; h0 / h_final: [B, H, K, V];
o: [B, T, H, V] float32.
"""
from __future__ import annotations

import ctypes

import torch

from . import _lib

CHUNK = 64       # the default chunk_size; 128 and 256 are accepted too
RUN_CHUNK = 64   # the chunk length the kernels (and the workspace layout) use

_DT = {torch.float32: _lib.ATOMIC_F32, torch.bfloat16: _lib.ATOMIC_BF16}


def _ptr(t):
    return ctypes.c_void_p(t.data_ptr()) if t is not None else ctypes.c_void_p(0)


def _stream(device):
    return ctypes.c_void_p(torch.cuda.current_stream(device).cuda_stream)


def rows(t):
    """``(tensor, row_stride)`` of a [B, T, H, D] input as the library reads
    it (``_lib.row_view``)."""
    return _lib.row_view(t)


def _rows_of(args, tensors, first=0):
    """rows() of each tensor, their strides into args.row_stride[first:]."""
    out = []
    for i, t in enumerate(tensors):
        t2, s = rows(t)
        args.row_stride[first + i] = s
        out.append(t2)
    return out


def _check_inputs(q, k, v, w, b, g):
    if not q.is_cuda:
        raise ValueError("GDN2 inputs must be HIP device tensors")
    if q.dtype not in _DT:
        raise TypeError(f"unsupported dtype {q.dtype}")
    for name, t in (("k", k), ("b", b)):
        if t.shape != q.shape or t.dtype != q.dtype:
            raise ValueError(f"{name} must match q in shape and dtype")
    for name, t in (("v", v), ("w", w)):
        if t.shape[:3] != q.shape[:3] or t.dtype != q.dtype:
            raise ValueError(f"{name} must be [B,T,H,V] with q's dtype")
    if g.shape != q.shape or g.dtype != torch.float32:
        raise ValueError("g must be float32 with q's shape")


def make_args(q, v, scale, *, do_dtype=None, flags=0, chunk=CHUNK):
    B, T, H, K = q.shape
    V = v.shape[-1]
    if T % chunk != 0:
        # same constraint the reference asserts (gdn2_wy_reference.py:109-112)
        raise ValueError(f"seq_len={T} must be divisible by chunk_size={chunk}")
    return _lib.Gdn2Args(B, T, H, K, V, chunk, _DT[q.dtype],
                         _DT[do_dtype if do_dtype is not None else q.dtype], float(scale), flags)


def workspace_bytes(args):
    lib = _lib.load()
    n = lib.atomic_gdn2_workspace_size(ctypes.byref(args))
    if n == 0:
        raise _lib.AtomicError("atomic_gdn2_workspace_size: unsupported shape")
    return n


def new_workspace(args, device):
    return torch.empty(workspace_bytes(args), dtype=torch.uint8, device=device)


def workspace_layout(args):
    lib = _lib.load()
    lay = _lib.Gdn2Layout()
    _lib.check(lib.atomic_gdn2_workspace_layout(ctypes.byref(args), ctypes.byref(lay)),
               "atomic_gdn2_workspace_layout")
    return lay


def forward(q, k, v, w, b, g, scale, h0=None, *, save=False, workspace=None, chunk=CHUNK, timer=None,
            diag=None, sanitize_h0=False):
    """Returns ``(o, h_final, workspace)``.  With ``save`` the workspace keeps
    the per-chunk intermediates for :func:`backward`.  ``diag`` (an
    ``_lib.StageReports`` over ``_lib.GDN2_DIAG_STAGES``) receives the
    forward's per-stage reports.  ``sanitize_h0`` clips h0 to +-1e4 and
    nan_to_nums it first, as the reference's staged forward does
    (kernel_d_pipeline.py:54-55,101)."""
    _check_inputs(q, k, v, w, b, g)
    lib = _lib.load()
    B, T, H, K = q.shape
    V = v.shape[-1]
    flags = (_lib.GDN2_SAVE if save else 0) | (_lib.GDN2_SANITIZE_H0 if sanitize_h0 else 0)
    args = make_args(q, v, scale, flags=flags, chunk=chunk)
    q, k, v, w, b, g = _rows_of(args, (q, k, v, w, b, g))
    if timer is not None:
        args.profile = timer.arm()
    if diag is not None:
        args.diag = diag.ptr
    if workspace is None:
        workspace = new_workspace(args, q.device)
    if h0 is not None:
        h0 = h0.to(torch.float32).contiguous()
    o = torch.empty(B, T, H, V, dtype=torch.float32, device=q.device)
    h_final = torch.empty(B, H, K, V, dtype=torch.float32, device=q.device)
    rc = lib.atomic_gdn2_fwd(ctypes.byref(args), _ptr(q), _ptr(k), _ptr(v), _ptr(w), _ptr(b), _ptr(g),
                             _ptr(h0), _ptr(o), _ptr(h_final), _ptr(workspace),
                             ctypes.c_size_t(workspace.numel()), _stream(q.device))
    _lib.check(rc, "atomic_gdn2_fwd")
    return o, h_final, workspace


def forward_noalloc(q, k, v, w, b, g, scale, h0=None, *, o=None, h_final=None, chunk=CHUNK,
                    timer=None, diag=None):
    """The forward through ``atomic_gdn2_fwd_noalloc``: no workspace, the
    library's fixed device scratch instead.  ``o`` / ``h_final`` may be
    given (preallocated outputs).  Returns ``(o, h_final)``."""
    _check_inputs(q, k, v, w, b, g)
    lib = _lib.load()
    B, T, H, K = q.shape
    V = v.shape[-1]
    args = make_args(q, v, scale, chunk=chunk)
    q, k, v, w, b, g = _rows_of(args, (q, k, v, w, b, g))
    if timer is not None:
        args.profile = timer.arm()
    if diag is not None:
        args.diag = diag.ptr
    if h0 is not None:
        h0 = h0.to(torch.float32).contiguous()
    if o is None:
        o = torch.empty(B, T, H, V, dtype=torch.float32, device=q.device)
    if h_final is None:
        h_final = torch.empty(B, H, K, V, dtype=torch.float32, device=q.device)
    rc = lib.atomic_gdn2_fwd_noalloc(ctypes.byref(args), _ptr(q), _ptr(k), _ptr(v), _ptr(w), _ptr(b),
                                     _ptr(g), _ptr(h0), _ptr(o), _ptr(h_final), _stream(q.device))
    _lib.check(rc, "atomic_gdn2_fwd_noalloc")
    return o, h_final


def backward(q, k, v, w, b, g, scale, dO, dh_final=None, h0=None, *, workspace=None, reuse=False,
             chunk=CHUNK, timer=None, diag=None, sanitize_h0=False):
    """Gradients ``(dq, dk, dv, dw, db, dg, dh0)`` in the primals' dtypes
    (dg and dh0 float32).  ``reuse`` declares that ``workspace`` holds the
    intermediates of a ``forward(..., save=True)`` on the same inputs; the
    library checks that by the input addresses and row strides, so an input
    that has to be copied here (see ``rows``, or h0 not float32) turns reuse
    into a recompute.  ``sanitize_h0`` must match the forward's."""
    _check_inputs(q, k, v, w, b, g)
    lib = _lib.load()
    if dO.dtype not in _DT:
        dO = dO.to(torch.float32)
    args = make_args(q, v, scale, do_dtype=dO.dtype, chunk=chunk)
    seen = (q, k, v, w, b, g)
    q, k, v, w, b, g, dO = _rows_of(args, seen + (dO,))
    if any(x is not y for x, y in zip((q, k, v, w, b, g), seen)) or \
            (h0 is not None and (h0.dtype != torch.float32 or not h0.is_contiguous())):
        reuse = False
    args.flags = (_lib.GDN2_REUSE if reuse else 0) | (_lib.GDN2_SANITIZE_H0 if sanitize_h0 else 0)
    if timer is not None:
        args.profile = timer.arm()
    if diag is not None:
        args.diag = diag.ptr
    if workspace is None:
        workspace = new_workspace(args, q.device)
    if h0 is not None:
        h0 = h0.to(torch.float32).contiguous()
    if dh_final is not None:
        dh_final = dh_final.to(torch.float32).contiguous()
    B, T, H, K = q.shape
    # the gradients are dense
    dq, dk, db = (torch.empty(q.shape, dtype=q.dtype, device=q.device) for _ in range(3))
    dv, dw = (torch.empty(v.shape, dtype=v.dtype, device=v.device) for _ in range(2))
    dg = torch.empty(g.shape, dtype=g.dtype, device=g.device)
    dh0 = torch.empty(B, H, K, v.shape[-1], dtype=torch.float32, device=q.device)
    rc = lib.atomic_gdn2_bwd(ctypes.byref(args), _ptr(q), _ptr(k), _ptr(v), _ptr(w), _ptr(b), _ptr(g),
                             _ptr(h0), _ptr(dO), _ptr(dh_final), _ptr(dq), _ptr(dk), _ptr(dv), _ptr(dw),
                             _ptr(db), _ptr(dg), _ptr(dh0), _ptr(workspace),
                             ctypes.c_size_t(workspace.numel()), _stream(q.device))
    _lib.check(rc, "atomic_gdn2_bwd")
    return dq, dk, dv, dw, db, dg, dh0


def chunk_views(workspace, args):
    """Per-chunk intermediates inside ``workspace`` as tensors
    ``[B, H, NT, rows, cols]`` (for stage-level tests)."""
    lay = workspace_layout(args)
    B, H, C, K, V = args.batch, args.heads, RUN_CHUNK, args.dk, args.dv
    NT = args.seqlen // C
    dt = torch.bfloat16 if args.dtype == _lib.ATOMIC_BF16 else torch.float32
    es = 2 if dt == torch.bfloat16 else 4

    def view(off, rows, cols, dtype=dt, esz=es):
        n = B * H * NT * rows * cols
        return workspace[off:off + n * esz].view(dtype).view(B, H, NT, rows, cols)

    return dict(qg=view(lay.qg, C, K), kg=view(lay.kg, C, K), w_pseudo=view(lay.w_pseudo, C, K),
                u=view(lay.u, C, V), aqk=view(lay.aqk, C, C), ainv=view(lay.ainv, C, C),
                gc_last=view(lay.gc_last, 1, K, torch.float32, 4)[..., 0, :],
                h_pre_t=view(lay.h_pre_t, V, K), v_new_t=view(lay.v_new_t, V, C))
