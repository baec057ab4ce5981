"""The C-ABI library loads and exports every entry point include/ssa_amd.h
declares (no compute: this runs without a GPU)."""
import ctypes
import os
import re

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


def test_struct_sizes_match_c_layout():
    """ctypes mirrors of the header structs have the C layout sizes."""
    from ssa_amd import _lib
    assert ctypes.sizeof(_lib.Tensor4) == 40
    # every field of GraphArgs is 4 or 8 bytes with natural alignment
    assert ctypes.sizeof(_lib.GraphArgs) % 8 == 0
    assert _lib.GraphArgs.out_ties.offset + 8 == ctypes.sizeof(_lib.GraphArgs)


def test_argument_errors_are_reported_without_a_gpu():
    """Shape validation happens on the host before any HIP call."""
    from ssa_amd import _lib
    a = _lib.GraphArgs()
    a.mode = 7
    rc = _lib.lib().ssa_build_graph(ctypes.byref(a), None, 0, None)
    assert rc == -1
    assert b"mode" in _lib.lib().ssa_last_error()
    assert _lib.lib().ssa_graph_out_width(ctypes.byref(a)) == -1
