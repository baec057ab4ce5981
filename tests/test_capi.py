"""The C-ABI library loads and exports every entry point include/ssa_amd.h
declares (no compute: this runs without a GPU)."""
import ctypes
import os
import re

import pytest
import torch

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
                 "ssa_sparse_gather_attention_bwd_det", "ssa_build_graph_noalloc",
                 "ssa_project_build_graph", "ssa_checked_oob", "ssa_version", "ssa_last_error"]:
        assert must in names


def test_library_exports_every_declared_symbol():
    import torch  # noqa: F401  (binds the library to torch's HIP runtime)
    from ssa_amd import _lib
    L = _lib.lib()
    for name in declared_functions():
        assert hasattr(L, name), f"{name} declared in ssa_amd.h but not exported"


def test_checked_library_exports_every_declared_symbol():
    """The bounds-checked twin (built by `make checked`, as build() does) is
    the same C ABI."""
    import ctypes

    import torch  # noqa: F401
    from ssa_amd import _lib
    assert os.path.exists(_lib.CHECKED_LIB_PATH), "libssa_amd_checked.so is not built"
    L = ctypes.CDLL(_lib.CHECKED_LIB_PATH)
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
               "ssa_apply_args": _lib.ApplyArgs, "ssa_apply_bwd_args": _lib.ApplyBwdArgs,
               "ssa_project_graph_args": _lib.ProjectGraphArgs}
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


# ---------------------------------------------------------------------------- exact replay
# Words of one replayed row's arrays (rank keys, 16-bit key ids, two 16-bit
# stopper lists, leaf bits, the partition stack, the seen bitmap, glob scores); two
# rows share a workgroup's 160 KiB of LDS (minus 512 bytes of static data).
def _replay_words(W, M):
    words = ((M + 31) // 32 + 1) & ~1
    # rank keys, key ids (16-bit up to 65,536 keys, else 32-bit), two 16-bit
    # position lists, leaf bits, stack, seen bitmap
    cand = W if words > 2048 else (W + 1) // 2
    return (2 * W + cand + (W + 31) // 32 + 1 + 3 * 64 + words + 1) & ~1


def _replay_fits(W, M):
    return 2 * _replay_words(W, M) * 4 <= 160 * 1024 - 512


def _full_args(N, K, w=4, G=2, R=2, d=16):
    from ssa_amd import _lib
    lsh_k = max(K - (2 * w + 1 + G + 1), 8)
    a = _lib.GraphArgs()
    a.mode = _lib.GRAPH_FULL
    a.B, a.Hq, a.Hkv, a.N, a.M, a.d = 1, 1, 1, N, N, d
    a.q = _lib.Tensor4(1, _lib.SSA_F32, N * d, N * d, d)   # never dereferenced here
    a.k = _lib.Tensor4(1, _lib.SSA_F32, N * d, N * d, d)
    a.rand_proj = 1
    a.R, a.max_p, a.P, a.T, a.C, a.top_k = R, 12, 1, 0, 4 * lsh_k, lsh_k
    a.window, a.causal, a.is_cross, a.total_k = w, 1, 0, K
    a.glob, a.G = 1, G
    return a, lsh_k


def test_replay_beyond_lds_takes_a_workspace_region():
    """Tied rows are always replayed: when two replayed rows of kk + chunk
    slots no longer fit a workgroup's LDS, the workspace grows by a region for
    the replay's per-wave arrays (a jump at exactly that kk)."""
    from ssa_amd import _lib
    L = _lib.lib()
    N = 2048
    prev = None
    crossed = 0
    for K in range(1500, 1700, 4):
        a, kk = _full_args(N, K)
        Call = 2 * 4 * kk
        chunk = min(Call, max(256, 4 * kk))
        W = min(kk, Call) + chunk
        wsb = L.ssa_graph_workspace_bytes(ctypes.byref(a))
        assert wsb > 0, _lib.lib().ssa_last_error()
        fits = _replay_fits(W, N)
        if prev is not None and prev[1] and not fits:
            crossed += 1
            blocks = max(1, min(256, (64 << 20) // (2 * _replay_words(W, N) * 4)))
            region = blocks * 2 * _replay_words(W, N) * 4
            # everything else grows by a few KB per step of K
            assert wsb - prev[0] >= region
        prev = (wsb, fits)
    assert crossed == 1


def test_replay_limit_is_an_error_not_a_silent_skip():
    """kk + chunk above 65535 slots is refused (the replay's 16-bit positions)."""
    from ssa_amd import _lib
    a, kk = _full_args(32768, 14000)
    assert _lib.lib().ssa_graph_workspace_bytes(ctypes.byref(a)) < 0
    assert b"tie replay" in _lib.lib().ssa_last_error()


# ---------------------------------------------------------------------------- apply shapes
def _apply_operands(B=1, Hq=4, Hkv=2, N=8, M=8, d=16, K=5):
    q = torch.zeros(B, Hq, N, d)
    k = torch.zeros(B, Hkv, M, d)
    v = torch.zeros(B, Hkv, M, d)
    nb = torch.zeros(B, Hq, N, K, dtype=torch.long)
    va = torch.ones(B, Hq, N, K, dtype=torch.bool)
    return q, k, v, nb, va


@pytest.mark.parametrize("bad", ["broadcast_graph", "graph_rows", "short_v", "valid_shape",
                                 "head_dim", "batch", "heads"])
def test_apply_shape_mismatch_raises_before_any_launch(bad):
    """The gather attention refuses operands whose shapes disagree (a cached
    graph of another size, a broadcast (N, K) graph, a short v) on the host,
    before the device check and before any launch."""
    from ssa_amd import sparse_gather_attention
    q, k, v, nb, va = _apply_operands()
    if bad == "broadcast_graph":
        nb, va = nb[0, 0], va[0, 0]
    elif bad == "graph_rows":
        nb, va = nb[:, :, :6], va[:, :, :6]
    elif bad == "short_v":
        v = v[:, :, :5]
    elif bad == "valid_shape":
        va = va[..., :4]
    elif bad == "head_dim":
        k, v = k[..., :8], v[..., :8]
    elif bad == "batch":
        k, v = torch.cat([k, k]), torch.cat([v, v])
    elif bad == "heads":
        k, v = torch.zeros(1, 3, 8, 16), torch.zeros(1, 3, 8, 16)
    with pytest.raises(RuntimeError, match="sparse_gather_attention"):
        sparse_gather_attention(q, k, v, nb, 0.25, valid=va)


def test_apply_matching_shapes_reach_the_device_check():
    from ssa_amd import sparse_gather_attention
    q, k, v, nb, va = _apply_operands()
    with pytest.raises(RuntimeError, match="ROCm devices only"):
        sparse_gather_attention(q, k, v, nb, 0.25, valid=va)


@pytest.mark.parametrize("d,dtype,ok", [(96, 1, True), (80, 1, True), (112, 2, True), (48, 0, True),
                                        (12, 0, True), (12, 1, False), (100, 1, False),
                                        (264, 0, True), (320, 1, True), (512, 0, True),
                                        (516, 0, True), (520, 1, True), (1024, 1, True),
                                        (1028, 0, False), (2048, 1, False), (2, 0, False)])
def test_head_dim_rule(d, dtype, ok):
    """Head dims 4..1024 that are powers of two or whole 16-byte pieces of the
    element type are taken; others are refused with a message, before any
    launch."""
    from ssa_amd import _lib
    a, _ = _full_args(256, 64, d=d)
    a.q.dtype = a.k.dtype = dtype
    wsb = _lib.lib().ssa_graph_workspace_bytes(ctypes.byref(a))
    if ok:
        assert wsb > 0, _lib.lib().ssa_last_error()
    else:
        assert wsb < 0 and b"head dim" in _lib.lib().ssa_last_error()


# ---------------------------------------------------------------------------- size envelope
@pytest.mark.parametrize("M", [1048577, 2000000])
def test_key_length_beyond_the_sort_is_refused(M):
    """Keys beyond the bucket sort's 2^20 are refused by the library before
    any launch, and by the Python wrapper before it touches a device."""
    import torch

    from ssa_amd import _lib
    a, _ = _full_args(M, 64)
    assert _lib.lib().ssa_graph_workspace_bytes(ctypes.byref(a)) < 0
    assert b"key length" in _lib.lib().ssa_last_error()
    q = torch.zeros(1, 1, 8, 16)
    k = torch.zeros(1, 1, M, 16)
    with pytest.raises(RuntimeError, match="key length"):
        _lib.build_graph(q, k, torch.zeros(2, 12, 16), P=1, T=0, C=64, top_k=32, window=4,
                         causal=False, is_cross=True, total_k=64, glob=torch.zeros(2))


def test_key_length_refusals_name_their_limit():
    """Within the sort's range the library refuses, with the reason, what
    its structures cannot hold: a select row's seen bitmap beyond a
    workgroup's LDS (about 650,000 keys), and a list cut whose size field
    (min(C, M)) and key field (M - 1) need more than 32 bits together."""
    from ssa_amd import _lib
    L = _lib.lib()
    a, _ = _full_args(1 << 20, 64)
    assert L.ssa_graph_workspace_bytes(ctypes.byref(a)) < 0
    assert b"bytes of LDS" in L.ssa_last_error()
    a, _ = _full_args(300000, 64)
    a.N, a.causal, a.is_cross = 64, 0, 1        # 64 queries over the keys
    a.C = 8192                                  # 14 + 19 bits
    assert L.ssa_graph_workspace_bytes(ctypes.byref(a)) < 0
    assert b"32-bit fields" in L.ssa_last_error()
    a.C = 8191                                  # 13 + 19 bits
    assert L.ssa_graph_workspace_bytes(ctypes.byref(a)) > 0, L.ssa_last_error()


@pytest.mark.parametrize("M", [32769, 40000, 65536, 65537, 100003, 131072, 262144, 600000])
def test_key_lengths_beyond_16_bits_are_taken(M):
    a, _ = _full_args(M, 64)
    from ssa_amd import _lib
    assert _lib.lib().ssa_graph_workspace_bytes(ctypes.byref(a)) > 0, _lib.lib().ssa_last_error()


def test_any_number_of_globals_up_to_the_key_count():
    """Global tokens beyond a wavefront are taken (the empty-bucket list is
    walked 64 entries at a time); more globals than keys are refused by the
    library and by the Python wrapper."""
    import torch

    from ssa_amd import _lib
    for G in (64, 300, 1024):
        a, _ = _full_args(1024, 2000, G=G)
        assert _lib.lib().ssa_graph_workspace_bytes(ctypes.byref(a)) > 0, \
            _lib.lib().ssa_last_error()
    a, _ = _full_args(1024, 2000, G=1025)
    assert _lib.lib().ssa_graph_workspace_bytes(ctypes.byref(a)) < 0
    assert b"G=1025" in _lib.lib().ssa_last_error()
    with pytest.raises(RuntimeError, match="global tokens"):
        _lib.build_graph(torch.zeros(1, 1, 8, 16), torch.zeros(1, 1, 8, 16), torch.zeros(2, 12, 16),
                         P=1, T=0, C=64, top_k=32, window=4, causal=False, is_cross=False,
                         total_k=64, glob=torch.zeros(9))
