"""The C-ABI library loads and exports every entry point include/ssa_amd.h
declares (no compute: this runs without a GPU)."""
import ctypes
import os
import re

import pytest

from conftest import ROOT

HEADER = os.path.join(ROOT, "include", "ssa_amd.h")


def declared_functions():
    text = open(HEADER).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(ssa_[a-z0-9_]+)\s*\(", text)))


def test_header_declares_the_entry_points():
    names = declared_functions()
    for must in ["ssa_build_graph", "ssa_graph_workspace_bytes", "ssa_graph_out_width",
                 "ssa_bucket_sort", "ssa_bucket_sort_workspace_bytes", "ssa_merge_neighbors",
                 "ssa_sparse_gather_attention", "ssa_sparse_gather_attention_bwd",
                 "ssa_version", "ssa_last_error"]:
        assert must in names


def test_library_exports_every_declared_symbol():
    import torch  # noqa: F401  (binds the library to torch's HIP runtime)
    from ssa_amd import _lib
    L = _lib.lib()
    for name in declared_functions():
        assert hasattr(L, name), f"{name} declared in ssa_amd.h but not exported"


def test_version_and_error_text():
    from ssa_amd import _lib
    assert "gfx950" in _lib.version()
    assert isinstance(_lib.lib().ssa_last_error(), bytes)


def test_struct_layouts_match_the_header(tmp_path):
    """Every field of the ctypes mirrors sits at the offset the C compiler gives
    it in include/ssa_amd.h, and the structs have the same sizes."""
    import shutil
    import subprocess
    from ssa_amd import _lib
    gcc = shutil.which("gcc")
    if gcc is None:
        pytest.skip("no C compiler")
    mirrors = {"ssa_tensor4": _lib.Tensor4, "ssa_graph_args": _lib.GraphArgs,
               "ssa_apply_args": _lib.ApplyArgs, "ssa_apply_bwd_args": _lib.ApplyBwdArgs}
    lines = ['#include <stdio.h>', '#include <stddef.h>', '#include "ssa_amd.h"', 'int main(void) {']
    for cname, py in mirrors.items():
        lines.append(f'printf("{cname} size %zu\\n", sizeof({cname}));')
        for f in py._fields_:
            lines.append(f'printf("{cname} {f[0]} %zu\\n", offsetof({cname}, {f[0]}));')
    lines += ['return 0;', '}']
    src = tmp_path / "layout.c"
    src.write_text("\n".join(lines) + "\n")
    exe = tmp_path / "layout"
    inc = os.path.join(os.path.dirname(os.path.dirname(os.path.abspath(__file__))), "include")
    subprocess.check_call([gcc, "-std=c99", "-I", inc, str(src), "-o", str(exe)])
    got = {}
    for line in subprocess.check_output([str(exe)], text=True).splitlines():
        cname, field, val = line.split()
        got[(cname, field)] = int(val)
    for cname, py in mirrors.items():
        assert got[(cname, "size")] == ctypes.sizeof(py), cname
        for f in py._fields_:
            assert got[(cname, f[0])] == getattr(py, f[0]).offset, (cname, f[0])


def test_argument_errors_are_reported_without_a_gpu():
    """Shape validation happens on the host before any HIP call."""
    from ssa_amd import _lib
    a = _lib.GraphArgs()
    a.mode = 7
    rc = _lib.lib().ssa_build_graph(ctypes.byref(a), None, 0, None)
    assert rc == -1
    assert b"mode" in _lib.lib().ssa_last_error()
    assert _lib.lib().ssa_graph_out_width(ctypes.byref(a)) == -1
