"""The REUSE contract is checked on the host: a backward asked to reuse a
workspace that no matching forward wrote returns ATOMIC_ERR_REUSE before
anything is launched (so these run without a GPU: the pointers are never
dereferenced)."""
import ctypes

from atomic_ops import _lib

FAKE = [ctypes.c_void_p(0x10000 + 0x1000 * i) for i in range(24)]


def test_gdn2_reuse_of_an_unsaved_workspace_is_refused():
    lib = _lib.load()
    a = _lib.Gdn2Args(1, 128, 2, 64, 64, 64, _lib.ATOMIC_BF16, _lib.ATOMIC_BF16, 1.0, _lib.GDN2_REUSE, None)
    n = lib.atomic_gdn2_workspace_size(ctypes.byref(a))
    assert n > 0
    ws = ctypes.c_void_p(0x7f0000000000)
    rc = lib.atomic_gdn2_bwd(ctypes.byref(a), *FAKE[:7], *FAKE[7:9], *FAKE[9:16], ws, ctypes.c_size_t(n),
                             ctypes.c_void_p(0))
    assert rc == -7 and "REUSE" in _lib.ERRORS[rc]


def test_mamba2_reuse_of_an_unsaved_workspace_is_refused():
    lib = _lib.load()
    a = _lib.Mamba2Args(1, 256, 2, 64, 128, 128, _lib.ATOMIC_BF16, _lib.ATOMIC_BF16, 2, None)
    n = lib.atomic_mamba2_workspace_size(ctypes.byref(a))
    assert n > 0
    ws = ctypes.c_void_p(0x7f1000000000)
    rc = lib.atomic_mamba2_bwd(ctypes.byref(a), *FAKE[:6], *FAKE[6:8], *FAKE[8:14], ws, ctypes.c_size_t(n),
                               ctypes.c_void_p(0))
    assert rc == -7
