"""The C ABI library loads and exports every function the public header
declares, and the ctypes structs match the header's layout (no GPU calls)."""
import ctypes
import re
import shutil
import subprocess

import pytest

from atomic_ops import _lib


def test_library_exports_every_header_function():
    lib = _lib.load()
    names = _lib.header_functions()
    assert names, "no functions found in include/atomic_hybrid.h"
    missing = [n for n in names if getattr(lib, n, None) is None]
    assert not missing, missing


def test_every_header_function_has_a_ctypes_signature():
    assert set(_lib.header_functions()) == set(_lib._SIGS)


STRUCTS = [(_lib.Gdn2Args, "atomic_gdn2_args"), (_lib.Mamba2Args, "atomic_mamba2_args"),
           (_lib.Gdn2Layout, "atomic_gdn2_layout"), (_lib.AtomicProfile, "atomic_profile"),
           (_lib.NormGateArgs, "atomic_norm_gate_args"), (_lib.PrologueArgs, "atomic_gdn2_prologue_args"),
           (_lib.Mamba2PrologueArgs, "atomic_mamba2_prologue_args"),
           (_lib.Mamba2ProjArgs, "atomic_mamba2_proj_args")]


def _header_fields(cname):
    with open(_lib.HEADER) as f:
        text = re.sub(r"/\*.*?\*/", "", f.read(), flags=re.S)
    body = re.search(r"typedef struct %s \{(.*?)\} %s;" % (cname, cname), text, re.S)
    assert body, cname
    names = []
    for stmt in body.group(1).split(";"):
        parts = [re.sub(r"\[.*?\]", "", p).strip() for p in stmt.split(",")]
        if not parts[0]:
            continue
        names.append(parts[0].split()[-1].lstrip("*"))
        names += [p.lstrip("*") for p in parts[1:]]
    return names


@pytest.mark.parametrize("struct,cname", STRUCTS)
def test_struct_fields_follow_the_header(struct, cname):
    assert _header_fields(cname) == [f[0] for f in struct._fields_]


def test_struct_offsets_match_the_c_compiler(tmp_path):
    """sizeof / offsetof of every header struct, from gcc, equal the ctypes
    layout."""
    gcc = shutil.which("gcc")
    if gcc is None:
        pytest.skip("gcc not available")
    lines = ['#include <stdio.h>', '#include <stddef.h>', '#include "%s"' % _lib.HEADER,
             "int main(void) {"]
    for struct, cname in STRUCTS:
        lines.append('printf("%s %%zu\\n", sizeof(%s));' % (cname, cname))
        for f in struct._fields_:
            lines.append('printf("%s.%s %%zu\\n", offsetof(%s, %s));' % (cname, f[0], cname, f[0]))
    lines.append("return 0; }")
    src = tmp_path / "layout.c"
    src.write_text("\n".join(lines))
    exe = tmp_path / "layout"
    subprocess.run([gcc, "-std=c11", str(src), "-o", str(exe)], check=True)
    out = dict(l.split() for l in subprocess.run([str(exe)], check=True, capture_output=True,
                                                  text=True).stdout.splitlines())
    for struct, cname in STRUCTS:
        assert int(out[cname]) == ctypes.sizeof(struct), cname
        for f in struct._fields_:
            assert int(out[f"{cname}.{f[0]}"]) == getattr(struct, f[0]).offset, (cname, f[0])


def test_workspace_size_rejects_bad_shapes_without_a_gpu():
    lib = _lib.load()
    ok = _lib.Gdn2Args(1, 128, 2, 128, 128, 64, _lib.ATOMIC_BF16, _lib.ATOMIC_BF16, 1.0, 0, None)
    assert lib.atomic_gdn2_workspace_size(ctypes.byref(ok)) > 0
    bad = _lib.Gdn2Args(1, 100, 2, 128, 128, 64, _lib.ATOMIC_BF16, _lib.ATOMIC_BF16, 1.0, 0, None)
    assert lib.atomic_gdn2_workspace_size(ctypes.byref(bad)) == 0
    # row strides: 0 (dense), or at least the dense row and a multiple of 8
    ok.row_stride[0] = 200
    assert lib.atomic_gdn2_workspace_size(ctypes.byref(ok)) == 0
    ok.row_stride[0] = 260
    assert lib.atomic_gdn2_workspace_size(ctypes.byref(ok)) == 0
    ok.row_stride[0] = 264
    assert lib.atomic_gdn2_workspace_size(ctypes.byref(ok)) > 0
    m_ok = _lib.Mamba2Args(1, 256, 2, 64, 128, 128, _lib.ATOMIC_BF16, _lib.ATOMIC_BF16, 0, None)
    assert lib.atomic_mamba2_workspace_size(ctypes.byref(m_ok)) > 0
    m_ok.row_stride[2] = 120          # below B's dense 128
    assert lib.atomic_mamba2_workspace_size(ctypes.byref(m_ok)) == 0
    m_ok.row_stride[2] = 136
    assert lib.atomic_mamba2_workspace_size(ctypes.byref(m_ok)) > 0
    m_f32 = _lib.Mamba2Args(1, 256, 2, 64, 128, 128, _lib.ATOMIC_F32, _lib.ATOMIC_BF16, 0, None)
    assert lib.atomic_mamba2_workspace_size(ctypes.byref(m_f32)) > 0
    m_bad = _lib.Mamba2Args(1, 256, 2, 64, 128, 128, 2, _lib.ATOMIC_BF16, 0, None)   # no such dtype
    assert lib.atomic_mamba2_workspace_size(ctypes.byref(m_bad)) == 0

    p_ok = _lib.Mamba2ProjArgs(1, 128, 4, 128, 64, 4, 1024, None)
    assert lib.atomic_mamba2_proj_workspace_size(ctypes.byref(p_ok), 0) > 0
    assert lib.atomic_mamba2_proj_workspace_size(ctypes.byref(p_ok), 1) > \
        lib.atomic_mamba2_proj_workspace_size(ctypes.byref(p_ok), 0)
    for bad in (_lib.Mamba2ProjArgs(1, 128, 4, 128, 32, 4, 1024, None),    # N not a multiple of 64
                _lib.Mamba2ProjArgs(1, 128, 4, 128, 64, 4, 500, None),     # stride below d_inner
                _lib.Mamba2ProjArgs(1, 128, 4, 128, 64, 4, 1026, None),    # stride not a multiple of 8
                _lib.Mamba2ProjArgs(1, 96, 4, 128, 64, 4, 1024, None)):    # L not a multiple of 128
        assert lib.atomic_mamba2_proj_workspace_size(ctypes.byref(bad), 1) == 0
