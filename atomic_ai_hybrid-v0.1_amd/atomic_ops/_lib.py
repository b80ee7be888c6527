"""ctypes binding of libatomic_hybrid.so (the C ABI in include/atomic_hybrid.h).

The library is required: ``load()`` raises if it has not been built, and no
operation in this package has a CPU or PyTorch fallback.
"""
from __future__ import annotations

import ctypes
import os
import re

_HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(_HERE, "libatomic_hybrid.so")
HEADER = os.path.join(os.path.dirname(os.path.dirname(_HERE)), "include", "atomic_hybrid.h")

ATOMIC_OK = 0
ERRORS = {
    -1: "ATOMIC_ERR_SHAPE: unsupported or inconsistent dimensions",
    -2: "ATOMIC_ERR_DTYPE: unsupported dtype",
    -3: "ATOMIC_ERR_WORKSPACE: workspace missing or too small",
    -4: "ATOMIC_ERR_LAUNCH: kernel launch failed",
    -5: "ATOMIC_ERR_NULL: required pointer is NULL",
    -6: "ATOMIC_ERR_SCRATCH: does not fit the no-allocation entry point's fixed scratch "
        "(or asks it to keep intermediates)",
    -7: "ATOMIC_ERR_REUSE: the workspace does not hold the matching forward (REUSE)",
}
ATOMIC_F32, ATOMIC_BF16 = 0, 1
GDN2_SAVE, GDN2_REUSE, GDN2_SANITIZE_H0 = 1, 2, 4
ATOMIC_ERR_REUSE = -7


class Gdn2Args(ctypes.Structure):
    _fields_ = [("batch", ctypes.c_int32), ("seqlen", ctypes.c_int32), ("heads", ctypes.c_int32),
                ("dk", ctypes.c_int32), ("dv", ctypes.c_int32), ("chunk", ctypes.c_int32),
                ("dtype", ctypes.c_int32), ("do_dtype", ctypes.c_int32), ("scale", ctypes.c_float),
                ("flags", ctypes.c_int32), ("profile", ctypes.c_void_p), ("diag", ctypes.c_void_p),
                ("row_stride", ctypes.c_int64 * 7)]


def row_view(t):
    """``(tensor, row_stride)`` for a [B, T, ...] input as the library reads
    it: a view whose tokens are evenly spaced rows with the trailing dims
    dense inside a row (a slice of a wider [B, T, F] tensor; row stride s a
    multiple of 8, 16-byte aligned, batch stride T s) is passed as it is with
    its row stride s; a contiguous tensor with 0; anything else as a
    contiguous copy."""
    if t.is_contiguous():
        return t, 0
    shape, st = t.shape, t.stride()
    B, T = shape[0], shape[1]
    inner, ok = 1, True
    for d in range(len(shape) - 1, 1, -1):   # the trailing dims dense within a row
        ok &= shape[d] == 1 or st[d] == inner
        inner *= shape[d]
    s = st[1]
    if ok and (B == 1 or st[0] == T * s) and s >= inner and s % 8 == 0 and t.data_ptr() % 16 == 0:
        return t, s
    return t.contiguous(), 0


class Gdn2Layout(ctypes.Structure):
    _fields_ = [(n, ctypes.c_size_t) for n in
                ("qg", "kg", "w_pseudo", "u", "aqk", "ainv", "gc_last", "h_pre_t", "v_new_t", "total")]


class Mamba2Args(ctypes.Structure):
    _fields_ = [("batch", ctypes.c_int32), ("seqlen", ctypes.c_int32), ("heads", ctypes.c_int32),
                ("headdim", ctypes.c_int32), ("dstate", ctypes.c_int32), ("chunk", ctypes.c_int32),
                ("dtype", ctypes.c_int32), ("dy_dtype", ctypes.c_int32), ("flags", ctypes.c_int32),
                ("profile", ctypes.c_void_p), ("diag", ctypes.c_void_p), ("row_stride", ctypes.c_int64 * 5)]


class NormGateArgs(ctypes.Structure):
    _fields_ = [("rows", ctypes.c_int32), ("dim", ctypes.c_int32), ("variant", ctypes.c_int32),
                ("eps", ctypes.c_float), ("profile", ctypes.c_void_p)]


NORM_GATE_GDN2, NORM_GATE_MAMBA2 = 0, 1


class Mamba2PrologueArgs(ctypes.Structure):
    _fields_ = [("batch", ctypes.c_int32), ("seqlen", ctypes.c_int32), ("heads", ctypes.c_int32),
                ("headdim", ctypes.c_int32), ("dstate", ctypes.c_int32), ("dconv", ctypes.c_int32),
                ("profile", ctypes.c_void_p)]


class Mamba2ProjArgs(ctypes.Structure):
    _fields_ = [("batch", ctypes.c_int32), ("seqlen", ctypes.c_int32), ("heads", ctypes.c_int32),
                ("headdim", ctypes.c_int32), ("dstate", ctypes.c_int32), ("dconv", ctypes.c_int32),
                ("in_stride", ctypes.c_int64), ("profile", ctypes.c_void_p)]


class PrologueArgs(ctypes.Structure):
    _fields_ = [("batch", ctypes.c_int32), ("seqlen", ctypes.c_int32), ("heads", ctypes.c_int32),
                ("dhead", ctypes.c_int32), ("dconv", ctypes.c_int32), ("eps", ctypes.c_float),
                ("profile", ctypes.c_void_p)]

PROFILE_MAX = 16


class AtomicProfile(ctypes.Structure):
    _fields_ = [("start", ctypes.c_void_p * PROFILE_MAX), ("stop", ctypes.c_void_p * PROFILE_MAX),
                ("capacity", ctypes.c_int32), ("count", ctypes.c_int32),
                ("names", ctypes.c_char_p * PROFILE_MAX)]


class KernelTimer:
    """Caller-owned event pairs that the library records around each kernel
    it launches (on the launch stream).  ``durations()`` returns
    ``[(kernel_name, ms), ...]`` of the last call, after synchronising."""

    def __init__(self, device=None):
        import torch
        self._torch = torch
        self.start = [torch.cuda.Event(enable_timing=True) for _ in range(PROFILE_MAX)]
        self.stop = [torch.cuda.Event(enable_timing=True) for _ in range(PROFILE_MAX)]
        stream = torch.cuda.current_stream(device)
        for e in self.start + self.stop:   # create the underlying hipEvent_t
            e.record(stream)
        torch.cuda.synchronize(device)
        self.struct = AtomicProfile()
        for i in range(PROFILE_MAX):
            self.struct.start[i] = self.start[i].cuda_event
            self.struct.stop[i] = self.stop[i].cuda_event
        self.struct.capacity = PROFILE_MAX

    def arm(self):
        """Pointer for the ``profile`` field of an args struct."""
        self.struct.count = 0
        return ctypes.cast(ctypes.pointer(self.struct), ctypes.c_void_p)

    def durations(self):
        self._torch.cuda.synchronize()
        n = min(self.struct.count, PROFILE_MAX)
        return [(self.struct.names[i].decode(), self.start[i].elapsed_time(self.stop[i]))
                for i in range(n)]


class AtomicError(RuntimeError):
    """A negative status of the C ABI; ``code`` holds it (None for errors
    raised by the Python layer itself)."""

    def __init__(self, msg, code=None):
        super().__init__(msg)
        self.code = code


# Stage names of the args structs' `diag` reports, in the header's order
# (ATOMIC_GDN2_DIAG_* / ATOMIC_MAMBA2_DIAG_*), with the reference's tags for
# the GDN2 forward stages (kernel_d_pipeline.py:177-187,121-123).
GDN2_DIAG_STAGES = ("kernel_A_Aqk", "kernel_A_Akk", "kernel_B_wy_inverse_A", "kernel_C_w_pseudo",
                    "kernel_C_u", "kernel_C_kg", "kernel_C_qg", "kernel_D_o", "kernel_D_h_final",
                    "bwd_dv_new", "bwd_dh", "bwd_dAqk", "bwd_dAkk", "dq", "dk", "dv", "dw", "db", "dg",
                    "dh0")
GDN2_DIAG_FWD = 9
MAMBA2_DIAG_STAGES = ("cb", "chunk_states", "ssm_out", "state_final", "bwd_dstates", "ddt", "dx", "dB",
                      "dC", "dA", "dstate0")
MAMBA2_DIAG_FWD = 4
DIAG_LARGE = 1e6   # the reference's "suspiciously large but still finite" level


class StageReports:
    """Device buffer of ``atomic_stage_report`` entries (uint32 n_nonfinite,
    float max_abs) for an args struct's ``diag`` field."""

    def __init__(self, stages, device):
        import torch
        self.stages = stages
        self.buf = torch.zeros(len(stages), 2, dtype=torch.int32, device=device)

    @property
    def ptr(self):
        return ctypes.c_void_p(self.buf.data_ptr())

    def read(self, first=0, count=None):
        """``{stage: (n_nonfinite, max_abs)}`` for stages [first, first+count)
        (synchronises with the device)."""
        import torch
        host = self.buf.cpu()
        n = host[:, 0].tolist()
        mx = host[:, 1].view(torch.float32).tolist()
        end = len(self.stages) if count is None else first + count
        return {self.stages[i]: (n[i], mx[i]) for i in range(first, end)}

    def messages(self, tag, first=0, count=None):
        """The reference's report lines: a stage with non-finite entries, or
        finite but above 1e6 (kernel_d_pipeline.py:58-91)."""
        out = []
        for name, (bad, mx) in self.read(first, count).items():
            if bad:
                out.append(f"[GDN2-FWD-DIAG] non-finite at {tag}:{name}: n_nonfinite={bad} "
                           f"max_abs(finite part)={mx:.3e}")
            elif mx > DIAG_LARGE:
                out.append(f"[GDN2-FWD-DIAG] suspiciously large at {tag}:{name}: max_abs={mx:.3e}")
        return out


_P = ctypes.c_void_p
_SIGS = {
    "atomic_gdn2_workspace_size": (ctypes.c_size_t, [ctypes.POINTER(Gdn2Args)]),
    "atomic_gdn2_workspace_layout": (ctypes.c_int, [ctypes.POINTER(Gdn2Args), ctypes.POINTER(Gdn2Layout)]),
    "atomic_gdn2_fwd": (ctypes.c_int, [ctypes.POINTER(Gdn2Args)] + [_P] * 9 + [_P, ctypes.c_size_t, _P]),
    "atomic_gdn2_bwd": (ctypes.c_int, [ctypes.POINTER(Gdn2Args)] + [_P] * 16 + [_P, ctypes.c_size_t, _P]),
    "atomic_gdn2_fwd_noalloc": (ctypes.c_int, [ctypes.POINTER(Gdn2Args)] + [_P] * 9 + [_P]),
    "atomic_mamba2_workspace_size": (ctypes.c_size_t, [ctypes.POINTER(Mamba2Args)]),
    "atomic_mamba2_fwd": (ctypes.c_int, [ctypes.POINTER(Mamba2Args)] + [_P] * 8 + [_P, ctypes.c_size_t, _P]),
    "atomic_mamba2_bwd": (ctypes.c_int, [ctypes.POINTER(Mamba2Args)] + [_P] * 14 + [_P, ctypes.c_size_t, _P]),
    "atomic_mamba2_stage_workspace_size": (ctypes.c_size_t, [ctypes.POINTER(Mamba2Args)]),
    "atomic_mamba2_chunk_cumdecay": (ctypes.c_int, [ctypes.POINTER(Mamba2Args)] + [_P] * 3 + [_P]),
    "atomic_mamba2_intra_chunk_ssd": (ctypes.c_int, [ctypes.POINTER(Mamba2Args)] + [_P] * 7 + [_P, ctypes.c_size_t, _P]),
    "atomic_mamba2_inter_chunk_combine": (ctypes.c_int, [ctypes.POINTER(Mamba2Args)] + [_P] * 7 + [_P, ctypes.c_size_t, _P]),
    "atomic_mamba2_intra_chunk_ssd_bwd_workspace_size": (ctypes.c_size_t, [ctypes.POINTER(Mamba2Args)]),
    "atomic_mamba2_intra_chunk_ssd_bwd": (ctypes.c_int, [ctypes.POINTER(Mamba2Args)] + [_P] * 12
                                          + [_P, ctypes.c_size_t, _P]),
    "atomic_mamba2_bwd_scan_workspace_size": (ctypes.c_size_t, [ctypes.POINTER(Mamba2Args)]),
    "atomic_mamba2_bwd_scan": (ctypes.c_int, [ctypes.POINTER(Mamba2Args)] + [_P] * 14 + [_P, ctypes.c_size_t, _P]),
    "atomic_mamba2_da_backward_workspace_size": (ctypes.c_size_t, [ctypes.POINTER(Mamba2Args)]),
    "atomic_mamba2_da_backward": (ctypes.c_int, [ctypes.POINTER(Mamba2Args)] + [_P] * 5 + [_P, ctypes.c_size_t, _P]),
    "atomic_norm_gate_workspace_size": (ctypes.c_size_t, [ctypes.POINTER(NormGateArgs)]),
    "atomic_norm_gate_fwd": (ctypes.c_int, [ctypes.POINTER(NormGateArgs)] + [_P] * 4 + [_P]),
    "atomic_norm_gate_bwd": (ctypes.c_int, [ctypes.POINTER(NormGateArgs)] + [_P] * 7 + [_P, ctypes.c_size_t, _P]),
    "atomic_gdn2_prologue_workspace_size": (ctypes.c_size_t, [ctypes.POINTER(PrologueArgs)]),
    "atomic_gdn2_prologue_fwd": (ctypes.c_int, [ctypes.POINTER(PrologueArgs)] + [_P] * 15 + [_P]),
    "atomic_gdn2_prologue_bwd": (ctypes.c_int, [ctypes.POINTER(PrologueArgs)] + [_P] * 24 + [_P, ctypes.c_size_t, _P]),
    "atomic_mamba2_prologue_workspace_size": (ctypes.c_size_t, [ctypes.POINTER(Mamba2PrologueArgs)]),
    "atomic_mamba2_prologue_fwd": (ctypes.c_int, [ctypes.POINTER(Mamba2PrologueArgs)] + [_P] * 12 + [_P]),
    "atomic_mamba2_prologue_bwd": (ctypes.c_int, [ctypes.POINTER(Mamba2PrologueArgs)] + [_P] * 19 + [_P, ctypes.c_size_t, _P]),
    "atomic_gdn2_chunk_wy": (ctypes.c_int, [ctypes.POINTER(Gdn2Args)] + [_P] * 13 + [_P]),
    "atomic_gdn2_inter_chunk_combine": (ctypes.c_int, [ctypes.POINTER(Gdn2Args)] + [_P] * 9 + [_P]),
    "atomic_gdn2_inter_chunk_combine_with_state": (ctypes.c_int, [ctypes.POINTER(Gdn2Args)] + [_P] * 11 + [_P]),
    "atomic_gdn2_chunk_scores": (ctypes.c_int, [ctypes.POINTER(Gdn2Args)] + [_P] * 6 + [_P]),
    "atomic_gdn2_wy_solve": (ctypes.c_int, [ctypes.POINTER(Gdn2Args)] + [_P] * 2 + [_P]),
    "atomic_gdn2_recompute_wy": (ctypes.c_int, [ctypes.POINTER(Gdn2Args)] + [_P] * 12 + [_P]),
    "atomic_gdn2_dav_backward": (ctypes.c_int, [ctypes.POINTER(Gdn2Args)] + [_P] * 5 + [_P]),
    "atomic_gdn2_dhu_backward": (ctypes.c_int, [ctypes.POINTER(Gdn2Args)] + [_P] * 10 + [_P]),
    "atomic_gdn2_wy_dqkg_workspace_size": (ctypes.c_size_t, [ctypes.POINTER(Gdn2Args)]),
    "atomic_gdn2_wy_dqkg_backward": (ctypes.c_int, [ctypes.POINTER(Gdn2Args)] + [_P] * 19
                                     + [_P, ctypes.c_size_t, _P]),
    "atomic_gdn2_intra_backward": (ctypes.c_int, [ctypes.POINTER(Gdn2Args)] + [_P] * 10 + [_P]),
    "atomic_gdn2_reverse_cumsum_bwd": (ctypes.c_int, [ctypes.POINTER(Gdn2Args)] + [_P] * 2 + [_P]),
    "atomic_mamba2_proj_workspace_size": (ctypes.c_size_t, [ctypes.POINTER(Mamba2ProjArgs), ctypes.c_int]),
    "atomic_mamba2_proj_fwd": (ctypes.c_int, [ctypes.POINTER(Mamba2ProjArgs)] + [_P] * 16 + [_P, ctypes.c_size_t, _P]),
    "atomic_mamba2_proj_bwd": (ctypes.c_int, [ctypes.POINTER(Mamba2ProjArgs)] + [_P] * 24 + [_P, ctypes.c_size_t, _P]),
}

_lib = None


def header_functions():
    """Names of every function the public header declares."""
    with open(HEADER) as f:
        text = f.read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(atomic_[a-z0-9_]+)\s*\(", text)))


def load():
    """Load the built library (once).  Raises if it is missing."""
    global _lib
    if _lib is not None:
        return _lib
    if not os.path.exists(LIB_PATH):
        raise AtomicError(f"{LIB_PATH} is missing: build it with "
                          "`python atomic_ai_hybrid-v0.1_amd/build.py` (no fallback exists)")
    lib = ctypes.CDLL(LIB_PATH)
    for name, (res, args) in _SIGS.items():
        fn = getattr(lib, name, None)
        if fn is None:
            continue
        fn.restype = res
        fn.argtypes = args
    _lib = lib
    return lib


def check(rc, what):
    if rc != ATOMIC_OK:
        raise AtomicError(f"{what}: {ERRORS.get(rc, rc)}", rc)
