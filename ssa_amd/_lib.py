"""ctypes binding of libssa_amd.so (the C ABI declared in include/ssa_amd.h).

torch is imported first so that the HIP runtime torch ships
(libamdhip64.so.7) is the one the library binds to: device pointers and
stream handles then come from the same runtime instance.

Every wrapper raises RuntimeError when the library is missing or a call
fails; there is no CPU or torch fallback for the hot path.
"""
from __future__ import annotations

import contextlib
import ctypes
import os

import torch

_HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(_HERE, "libssa_amd.so")

SSA_F32, SSA_BF16, SSA_F16 = 0, 1, 2
GRAPH_FULL, GRAPH_LSH = 0, 1

_DTYPES = {torch.float32: SSA_F32, torch.bfloat16: SSA_BF16, torch.float16: SSA_F16}

c_i32 = ctypes.c_int32
c_i64 = ctypes.c_int64
c_vp = ctypes.c_void_p


class Tensor4(ctypes.Structure):
    _fields_ = [("ptr", c_vp), ("dtype", c_i32), ("sb", c_i64), ("sh", c_i64), ("sn", c_i64)]


class GraphArgs(ctypes.Structure):
    _fields_ = [
        ("mode", c_i32), ("B", c_i32), ("Hq", c_i32), ("Hkv", c_i32),
        ("N", c_i32), ("M", c_i32), ("d", c_i32),
        ("q", Tensor4), ("k", Tensor4),
        ("rand_proj", c_vp), ("R", c_i32), ("max_p", c_i32), ("P", c_i32), ("T", c_i32),
        ("C", c_i32), ("top_k", c_i32), ("window", c_i32), ("causal", c_i32),
        ("is_cross", c_i32), ("total_k", c_i32),
        ("glob", c_vp), ("G", c_i32),
        ("q_proj", c_vp), ("k_proj", c_vp),
        ("out_idx", c_vp), ("out_valid", c_vp), ("out_ties", c_vp),
        ("out_idx32", c_vp),
    ]


class ProjectGraphArgs(ctypes.Structure):
    _fields_ = [("x", c_vp), ("src", c_vp), ("wq", c_vp), ("wkv", c_vp),
                ("q_out", c_vp), ("kv_out", c_vp), ("d_model", c_i32), ("graph", GraphArgs)]


class ApplyArgs(ctypes.Structure):
    _fields_ = [
        ("B", c_i32), ("Hq", c_i32), ("Hkv", c_i32), ("N", c_i32), ("M", c_i32), ("d", c_i32),
        ("K", c_i32),
        ("q", Tensor4), ("k", Tensor4), ("v", Tensor4),
        ("neighbors", c_vp), ("valid", c_vp),
        ("scale", ctypes.c_float), ("fp32_weights", c_i32), ("dropout_p", ctypes.c_float),
        ("seed", ctypes.c_uint64),
        ("out", c_vp), ("out_sb", c_i64), ("out_sh", c_i64), ("out_sn", c_i64),
        ("neighbors32", c_vp), ("row_invalid", c_vp),
    ]


class ApplyBwdArgs(ctypes.Structure):
    _fields_ = [("fwd", ApplyArgs), ("dout", c_vp), ("dq", c_vp), ("dk", c_vp), ("dv", c_vp)]


_lib = None
_override = None
CHECKED_LIB_PATH = os.path.join(_HERE, "libssa_amd_checked.so")


def lib():
    """Load libssa_amd.so once; raise if it is not built.  Inside
    checked_library() the bounds-checked build serves instead."""
    global _lib
    if _override is not None:
        return _override
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise RuntimeError(
                f"ssa_amd: {LIB_PATH} is not built; run `make -C ssa_amd/csrc` "
                "(or __graft_entry__.build()).  There is no fallback path.")
        _lib = _configure(ctypes.CDLL(LIB_PATH))
    return _lib


_checked = None


@contextlib.contextmanager
def checked_library():
    """Route every call made inside the block through libssa_amd_checked.so:
    the same kernels with the graph build's data-dependent indices
    bounds-checked (an index outside its buffer is recorded and replaced by
    0).  Yields a function that returns and clears the record: None when
    nothing was out of bounds, else (site bits, last site, index, length)."""
    global _override, _checked
    if _checked is None:
        if not os.path.exists(CHECKED_LIB_PATH):
            raise RuntimeError(f"ssa_amd: {CHECKED_LIB_PATH} is not built; run "
                               "`make -C ssa_amd/csrc checked`")
        _checked = _configure(ctypes.CDLL(CHECKED_LIB_PATH))
    L = _checked

    def record():
        rec = (ctypes.c_uint32 * 4)()
        if L.ssa_checked_oob(rec) != 1:
            raise RuntimeError("ssa_amd: the checked library does not keep a record")
        return None if rec[0] == 0 else tuple(rec)
    prev = _override
    _override = L
    try:
        yield record
    finally:
        _override = prev


def _configure(L):
    """Declare the C ABI's signatures on a loaded library."""
    L.ssa_version.restype = ctypes.c_char_p
    L.ssa_last_error.restype = ctypes.c_char_p
    L.ssa_graph_out_width.restype = c_i64
    L.ssa_graph_out_width.argtypes = [ctypes.POINTER(GraphArgs)]
    L.ssa_graph_workspace_bytes.restype = c_i64
    L.ssa_graph_workspace_bytes.argtypes = [ctypes.POINTER(GraphArgs)]
    L.ssa_build_graph.restype = ctypes.c_int
    L.ssa_build_graph.argtypes = [ctypes.POINTER(GraphArgs), c_vp, c_i64, c_vp]
    L.ssa_build_graph_noalloc.restype = ctypes.c_int
    L.ssa_build_graph_noalloc.argtypes = [ctypes.POINTER(GraphArgs), c_vp]
    L.ssa_project_graph_supported.restype = ctypes.c_int
    L.ssa_project_graph_supported.argtypes = [ctypes.POINTER(ProjectGraphArgs)]
    L.ssa_project_graph_workspace_bytes.restype = c_i64
    L.ssa_project_graph_workspace_bytes.argtypes = [ctypes.POINTER(ProjectGraphArgs)]
    L.ssa_project_build_graph.restype = ctypes.c_int
    L.ssa_project_build_graph.argtypes = [ctypes.POINTER(ProjectGraphArgs), c_vp, c_i64, c_vp]
    L.ssa_project_gemm.restype = ctypes.c_int
    L.ssa_project_gemm.argtypes = [c_vp, c_i64, c_vp, c_i64, c_vp, c_i64, c_i32, c_i32, c_i32,
                                   c_vp]
    L.ssa_bucket_sort_workspace_bytes.restype = c_i64
    L.ssa_bucket_sort_workspace_bytes.argtypes = [c_i32, c_i32]
    L.ssa_bucket_sort.restype = ctypes.c_int
    L.ssa_bucket_sort.argtypes = [c_vp, c_i32, c_i32, c_i32, c_vp, c_vp, c_vp, c_vp, c_i64,
                                  c_vp]
    L.ssa_merge_neighbors.restype = ctypes.c_int
    L.ssa_merge_neighbors.argtypes = [c_vp, c_i32, c_vp, c_i32, c_vp, c_i32, c_i32, c_i32,
                                      c_i32, c_i32, c_vp, c_vp, c_vp, c_vp]
    L.ssa_sparse_gather_attention.restype = ctypes.c_int
    L.ssa_sparse_gather_attention.argtypes = [ctypes.POINTER(ApplyArgs), c_vp]
    L.ssa_measure_l2_read.restype = ctypes.c_int
    L.ssa_measure_l2_read.argtypes = [c_vp, c_i64, c_i32, c_i32, c_vp, c_vp]
    L.ssa_sparse_gather_attention_bwd.restype = ctypes.c_int
    L.ssa_sparse_gather_attention_bwd.argtypes = [ctypes.POINTER(ApplyBwdArgs), c_vp]
    L.ssa_sparse_gather_attention_bwd_det_workspace_bytes.restype = c_i64
    L.ssa_sparse_gather_attention_bwd_det_workspace_bytes.argtypes = [
        ctypes.POINTER(ApplyBwdArgs)]
    L.ssa_sparse_gather_attention_bwd_det.restype = ctypes.c_int
    L.ssa_sparse_gather_attention_bwd_det.argtypes = [ctypes.POINTER(ApplyBwdArgs), c_vp, c_i64,
                                                      c_vp]
    L.ssa_checked_oob.restype = ctypes.c_int
    L.ssa_checked_oob.argtypes = [ctypes.POINTER(ctypes.c_uint32)]
    return L


def version() -> str:
    return lib().ssa_version().decode()


def _check(rc: int, what: str):
    if rc != 0:
        msg = lib().ssa_last_error().decode()
        raise RuntimeError(f"ssa_amd.{what} failed ({rc}): {msg}")


def require_device(*tensors):
    for t in tensors:
        if t is not None and t.device.type != "cuda":
            raise RuntimeError(
                "ssa_amd runs the SparseAttention hot path on ROCm devices only "
                f"(got a tensor on {t.device}); move the module and inputs to 'cuda'.")


def _stream(t: torch.Tensor) -> int:
    return torch.cuda.current_stream(t.device).cuda_stream


def dtype_code(dt: torch.dtype) -> int:
    try:
        return _DTYPES[dt]
    except KeyError:
        raise RuntimeError(f"ssa_amd: dtype {dt} unsupported (float32, bfloat16, float16)")


def view4(t: torch.Tensor):
    """(B, H, L, d) tensor -> (Tensor4, keep-alive tensor) with a unit last stride."""
    if t.dim() != 4:
        raise RuntimeError(f"ssa_amd: expected a 4-D (B, H, L, d) tensor, got {tuple(t.shape)}")
    if t.stride(-1) != 1:
        t = t.contiguous()
    sb, sh, sn, _ = t.stride()
    return Tensor4(t.data_ptr(), dtype_code(t.dtype), sb, sh, sn), t


def _ptr(t):
    return None if t is None else t.data_ptr()


# --------------------------------------------------------------------------- graph build
# largest key length ssa_build_graph accepts (the library refuses some
# shorter ones whose lists or select rows do not fit its fields or LDS)
MAX_KEYS = 1 << 20


def _graph_args(q, k, rand_proj, *, P, T, C, top_k, window, causal, is_cross, total_k, glob,
                mode, q_proj, k_proj):
    """Checked ssa_graph_args for q (B,Hq,N,d), k (B,Hkv,M,d); returns (args,
    keep-alive tensors)."""
    if q.dim() != 4 or k.dim() != 4:
        raise RuntimeError(f"ssa_amd.build_graph: q {tuple(q.shape)} and k {tuple(k.shape)} must "
                           "be 4-D")
    B, Hq, N, d = q.shape
    Bk, Hkv, M, dk = k.shape
    if Bk != B or dk != d:
        raise RuntimeError(f"ssa_amd.build_graph: q {tuple(q.shape)} / k {tuple(k.shape)} mismatch")
    if Hkv < 1 or Hq % Hkv != 0:
        raise RuntimeError(f"ssa_amd.build_graph: {Hq} query heads are not a multiple of {Hkv} "
                           "kv heads")
    if rand_proj.dim() != 3 or rand_proj.shape[2] != d or not 1 <= P <= rand_proj.shape[1]:
        raise RuntimeError(f"ssa_amd.build_graph: hyperplanes {tuple(rand_proj.shape)} do not "
                           f"fit head dim {d} and {P} planes")
    R = rand_proj.shape[0]
    if q_proj is not None and tuple(q_proj.shape) != (B * Hq, R, N, P):
        raise RuntimeError(f"ssa_amd.build_graph: q_proj {tuple(q_proj.shape)} is not "
                           f"{(B * Hq, R, N, P)}")
    if k_proj is not None and tuple(k_proj.shape) != (B * Hkv, R, M, P):
        raise RuntimeError(f"ssa_amd.build_graph: k_proj {tuple(k_proj.shape)} is not "
                           f"{(B * Hkv, R, M, P)}")
    if not 1 <= M <= MAX_KEYS:
        raise RuntimeError(f"ssa_amd.build_graph: key length {M} unsupported (1..{MAX_KEYS}: the "
                           "bucket sort's limit)")
    if glob.numel() > M:
        raise RuntimeError(f"ssa_amd.build_graph: {glob.numel()} global tokens for {M} keys")
    require_device(q, k, rand_proj, glob)
    if q.dtype != k.dtype:
        raise RuntimeError("ssa_amd.build_graph: q and k dtypes differ")
    qa, qk = view4(q)
    ka, kk_ = view4(k)
    rp = rand_proj.detach().to(torch.float32).contiguous()
    g = glob.detach().to(device=q.device, dtype=torch.int64).contiguous()
    qp = q_proj.detach().to(torch.float32).contiguous() if q_proj is not None else None
    kp = k_proj.detach().to(torch.float32).contiguous() if k_proj is not None else None
    a = GraphArgs()
    a.mode = mode
    a.B, a.Hq, a.Hkv, a.N, a.M, a.d = B, Hq, Hkv, N, M, d
    a.q, a.k = qa, ka
    a.rand_proj = rp.data_ptr()
    a.R, a.max_p = rp.shape[0], rp.shape[1]
    a.P, a.T, a.C, a.top_k = P, T, C, top_k
    a.window, a.causal, a.is_cross, a.total_k = window, int(causal), int(is_cross), total_k
    a.glob, a.G = (g.data_ptr() if g.numel() else None), g.numel()
    a.q_proj, a.k_proj = _ptr(qp), _ptr(kp)
    return a, [qk, kk_, rp, g, qp, kp]


def _graph_outputs(a, width, mode, ids32, count_ties, device):
    """Allocate the graph outputs for width slots and point `a` at them."""
    B, Hq, N = a.B, a.Hq, a.N
    compact = ids32 and mode == GRAPH_FULL
    out = torch.empty((B, Hq, N, width), dtype=torch.int32 if compact else torch.int64,
                      device=device)
    valid = (torch.empty((B, Hq, N, width), dtype=torch.bool, device=device)
             if mode == GRAPH_FULL and not compact else None)
    ties = torch.zeros(1, dtype=torch.int32, device=device) if count_ties else None
    if compact:
        a.out_idx32 = out.data_ptr()
    else:
        a.out_idx, a.out_valid = out.data_ptr(), _ptr(valid)
    a.out_ties = _ptr(ties)
    return out, valid, ties


def kernel_head_dim(d: int, dtype: torch.dtype) -> int:
    """Head dim the kernels run at for rows of d elements: d itself when they
    take it (a power of two from 4, or whole 16-byte pieces of the element
    type), else d rounded up to whole pieces.  The added columns hold zeros,
    which add exact zeros to every dot product: scores, hash projections and
    outputs are those of the d columns (a zero sum may change sign, and the
    kernels rank -0 and +0 as one key)."""
    vec = 4 if dtype == torch.float32 else 8
    if d >= 4 and (d & (d - 1) == 0 or d % vec == 0):
        return d
    dp = (d + vec - 1) // vec * vec
    return dp if dp <= 1024 else d          # beyond: the library refuses d itself


def _pad_cols(t, dp):
    """t with its last dimension zero-padded to dp (t itself when it has dp)."""
    if t is None or t.shape[-1] == dp:
        return t
    return torch.nn.functional.pad(t, (0, dp - t.shape[-1]))


def build_graph(q, k, rand_proj, *, P, T, C, top_k, window, causal, is_cross, total_k, glob,
                mode=GRAPH_FULL, q_proj=None, k_proj=None, count_ties=False, ids32=False,
                noalloc=False):
    """Run ssa_build_graph.  q (B,Hq,N,d), k (B,Hkv,M,d) views on one device.

    Returns (out_idx, out_valid or None, ties or None).  With ids32 (FULL mode)
    out_idx is int32 with -1 in the invalid slots and out_valid is None.  With
    noalloc the build runs through ssa_build_graph_noalloc: no workspace is
    allocated (the library's fixed scratch array serves instead; the outputs
    are still allocated here).  Head dims the kernels do not take run
    zero-padded (kernel_head_dim)."""
    if q.dim() == 4 and k.dim() == 4 and q.shape[-1] == k.shape[-1]:
        dp = kernel_head_dim(q.shape[-1], q.dtype)
        q, k = _pad_cols(q, dp), _pad_cols(k, dp)
        if rand_proj.dim() == 3 and rand_proj.shape[-1] < dp:
            rand_proj = _pad_cols(rand_proj, dp)
    a, keep = _graph_args(q, k, rand_proj, P=P, T=T, C=C, top_k=top_k, window=window,
                          causal=causal, is_cross=is_cross, total_k=total_k, glob=glob, mode=mode,
                          q_proj=q_proj, k_proj=k_proj)
    L = lib()
    width = L.ssa_graph_out_width(ctypes.byref(a))
    if width < 0:
        _check(-1, "build_graph")
    wsb = 0 if noalloc else L.ssa_graph_workspace_bytes(ctypes.byref(a))
    if wsb < 0:
        _check(-1, "build_graph")
    out, valid, ties = _graph_outputs(a, width, mode, ids32, count_ties, q.device)
    if noalloc:
        ws = None
        with torch.cuda.device(q.device):
            _check(L.ssa_build_graph_noalloc(ctypes.byref(a), _stream(q)), "build_graph_noalloc")
    else:
        ws = torch.empty(max(int(wsb), 1), dtype=torch.uint8, device=q.device)
        _check(L.ssa_build_graph(ctypes.byref(a), ws.data_ptr(), int(wsb), _stream(q)),
               "build_graph")
    # keep inputs alive until the stream has consumed them
    keep.append(ws)
    del keep
    return out, valid, ties


def project_shape_ok(dtype, N, M, d_model, Hq, Hkv, d, R, P) -> bool:
    """The sizes ssa_project_build_graph takes (ssa_project_graph_supported
    checks them again with the pointers): bf16; head dim 32, 64 or 128; N and
    M multiples of 16; d_model a multiple of 64; Hq*d and 2*Hkv*d multiples
    of 256; the round set's hyperplanes in at most 12 // (d // 32) (and 4)
    tiles of 16."""
    if dtype != torch.bfloat16 or d not in (32, 64, 128):
        return False
    nt = (R * P + 15) // 16
    return (N % 16 == 0 and M % 16 == 0 and N >= 16 and M >= 16 and d_model % 64 == 0
            and (Hq * d) % 256 == 0 and (2 * Hkv * d) % 256 == 0 and nt <= min(4, 12 // (d // 32)))


def project_build_graph(x, src, wq, wkv, Hq, Hkv, d, rand_proj, *, P, T, C, top_k, window, causal,
                        is_cross, total_k, glob, mode=GRAPH_FULL, ids32=True, count_ties=False):
    """Run ssa_project_build_graph: q = x wq^T, [k v] = src wkv^T (bf16) and the
    graph on them, the hash in the projections' epilogue.

    x (B, N, d_model), src (B, M, d_model) contiguous bf16; wq (Hq*d, d_model),
    wkv (2*Hkv*d, d_model) contiguous bf16.  Returns (q, k, v, out_idx,
    out_valid, ties) with q (B, Hq, N, d) and k, v (B, Hkv, M, d) views of the
    projections' outputs, or None when the library does not take these sizes
    (the caller then projects and builds separately)."""
    B, N, dm = x.shape
    M = src.shape[1]
    if (x.dim() != 3 or src.dim() != 3 or src.shape[0] != B or src.shape[2] != dm
            or tuple(wq.shape) != (Hq * d, dm) or tuple(wkv.shape) != (2 * Hkv * d, dm)):
        raise RuntimeError(f"ssa_amd.project_build_graph: x {tuple(x.shape)}, src "
                           f"{tuple(src.shape)}, wq {tuple(wq.shape)}, wkv {tuple(wkv.shape)} do "
                           f"not fit {Hq} query / {Hkv} kv heads of dim {d}")
    if not project_shape_ok(x.dtype, N, M, dm, Hq, Hkv, d, rand_proj.shape[0], P):
        return None
    for t in (src, wq, wkv):
        if t.dtype != x.dtype:
            return None
    require_device(x, src, wq, wkv)
    x_, src_, wq_, wkv_ = (t.contiguous() for t in (x, src, wq, wkv))
    q_out = torch.empty((B, N, Hq * d), dtype=x.dtype, device=x.device)
    kv_out = torch.empty((B, M, 2 * Hkv * d), dtype=x.dtype, device=x.device)
    q4 = q_out.view(B, N, Hq, d).transpose(1, 2)
    kv4 = kv_out.view(B, M, 2 * Hkv, d).transpose(1, 2)
    k4, v4 = kv4[:, :Hkv], kv4[:, Hkv:]
    ga, keep = _graph_args(q4, k4, rand_proj, P=P, T=T, C=C, top_k=top_k, window=window,
                           causal=causal, is_cross=is_cross, total_k=total_k, glob=glob, mode=mode,
                           q_proj=None, k_proj=None)
    a = ProjectGraphArgs()
    a.x, a.src, a.wq, a.wkv = x_.data_ptr(), src_.data_ptr(), wq_.data_ptr(), wkv_.data_ptr()
    a.q_out, a.kv_out, a.d_model = q_out.data_ptr(), kv_out.data_ptr(), dm
    a.graph = ga
    L = lib()
    if not L.ssa_project_graph_supported(ctypes.byref(a)):
        return None
    width = L.ssa_graph_out_width(ctypes.byref(a.graph))
    wsb = L.ssa_project_graph_workspace_bytes(ctypes.byref(a))
    if width < 0 or wsb < 0:
        _check(-1, "project_build_graph")
    out, valid, ties = _graph_outputs(a.graph, width, mode, ids32, count_ties, x.device)
    ws = torch.empty(max(int(wsb), 1), dtype=torch.uint8, device=x.device)
    _check(L.ssa_project_build_graph(ctypes.byref(a), ws.data_ptr(), int(wsb), _stream(x)),
           "project_build_graph")
    keep += [x_, src_, wq_, wkv_, ws]
    del keep
    return q4, k4, v4, out, valid, ties


def project_gemm(x, w):
    """ssa_project_gemm: x (rows, K) w (cols, K)^T in bf16 on the library's
    projection GEMM (cols a multiple of 256, K of 64)."""
    require_device(x, w)
    if x.dtype != torch.bfloat16 or w.dtype != torch.bfloat16 or x.dim() != 2 or w.dim() != 2:
        raise RuntimeError("ssa_amd.project_gemm: 2-D bf16 operands")
    x_, w_ = x.contiguous(), w.contiguous()
    rows, K = x_.shape
    cols = w_.shape[0]
    if w_.shape[1] != K:
        raise RuntimeError(f"ssa_amd.project_gemm: x {tuple(x.shape)} w {tuple(w.shape)}")
    y = torch.empty((rows, cols), dtype=x.dtype, device=x.device)
    _check(lib().ssa_project_gemm(x_.data_ptr(), K, w_.data_ptr(), K, y.data_ptr(), cols, rows,
                                  cols, K, _stream(x)), "project_gemm")
    return y


def bucket_sort(ids: torch.Tensor, P: int):
    """ssa_bucket_sort on (rows, n) uint16-valued ids -> (perm int32, bstart, bsize)."""
    require_device(ids)
    ids16 = ids.to(torch.int32).to(torch.int16).contiguous()   # same bits as uint16 for < 2^15
    rows, n = ids16.shape
    perm = torch.empty((rows, n), dtype=torch.int32, device=ids.device)
    bstart = torch.empty((rows, 1 << P), dtype=torch.int32, device=ids.device)
    bsize = torch.empty((rows, 1 << P), dtype=torch.int32, device=ids.device)
    L = lib()
    wsb = max(int(L.ssa_bucket_sort_workspace_bytes(rows, n)), 1)
    ws = torch.empty(wsb, dtype=torch.uint8, device=ids.device)
    _check(L.ssa_bucket_sort(ids16.data_ptr(), rows, n, P, perm.data_ptr(), bstart.data_ptr(),
                             bsize.data_ptr(), ws.data_ptr(), wsb, _stream(ids)), "bucket_sort")
    return perm, bstart, bsize


def merge_neighbors(win, glob, lsh, has_self: bool, total_k: int):
    require_device(win, glob, lsh)
    B, H, N, Kl = lsh.shape
    w = win.to(torch.int64).contiguous()
    Kw = w.shape[1] if w.dim() == 2 else 0
    g = glob.to(torch.int64).contiguous()
    l = lsh.to(torch.int64).contiguous()
    Kall = Kw + g.numel() + Kl
    ks = min(total_k - 1, Kall) if has_self else min(total_k, Kall)
    Kout = (1 if has_self else 0) + ks
    out = torch.empty((B, H, N, Kout), dtype=torch.int64, device=lsh.device)
    valid = torch.empty((B, H, N, Kout), dtype=torch.bool, device=lsh.device)
    ws = torch.empty(16, dtype=torch.uint8, device=lsh.device)
    _check(lib().ssa_merge_neighbors(
        _ptr(w) if Kw else None, Kw, _ptr(g) if g.numel() else None, g.numel(),
        _ptr(l) if Kl else None, Kl, B * H, N, int(has_self), total_k, out.data_ptr(),
        valid.data_ptr(), ws.data_ptr(), _stream(lsh)), "merge_neighbors")
    return out, valid


# --------------------------------------------------------------------------- apply
def check_apply_shapes(q, k, v, neighbors, valid, out=None):
    """Raise RuntimeError unless the operands of the gather attention agree:
    q (B, Hq, N, d); k and v (B, Hkv, M, d) with Hq % Hkv == 0; neighbors
    (B, Hq, N, K); valid None or neighbors' shape; out (B, Hq, N, d).  The
    kernels index every row of these shapes, so a mismatch (a cached graph of
    another size, a broadcast (N, K) graph, a short v) is refused here, before
    any launch, where the reference's reshape would raise
    (sparse_attention.py:1137-1142)."""
    for name, t in (("q", q), ("k", k), ("v", v), ("neighbors", neighbors)):
        if t.dim() != 4:
            raise RuntimeError(f"ssa_amd.sparse_gather_attention: {name} must be 4-D, got "
                               f"shape {tuple(t.shape)}")
    B, Hq, N, d = q.shape
    Bk, Hkv, M, dk = k.shape
    if tuple(v.shape) != tuple(k.shape):
        raise RuntimeError(f"ssa_amd.sparse_gather_attention: v {tuple(v.shape)} and k "
                           f"{tuple(k.shape)} differ")
    if Bk != B or dk != d:
        raise RuntimeError(f"ssa_amd.sparse_gather_attention: k {tuple(k.shape)} does not match "
                           f"q {tuple(q.shape)} in batch or head dim")
    if Hkv < 1 or Hq % Hkv != 0:
        raise RuntimeError(f"ssa_amd.sparse_gather_attention: {Hq} query heads are not a "
                           f"multiple of {Hkv} kv heads")
    if M < 1:
        raise RuntimeError("ssa_amd.sparse_gather_attention: k has no keys")
    if tuple(neighbors.shape[:3]) != (B, Hq, N):
        raise RuntimeError(f"ssa_amd.sparse_gather_attention: neighbors {tuple(neighbors.shape)} "
                           f"do not match q {tuple(q.shape)} in (B, H, N)")
    if valid is not None and tuple(valid.shape) != tuple(neighbors.shape):
        raise RuntimeError(f"ssa_amd.sparse_gather_attention: valid {tuple(valid.shape)} and "
                           f"neighbors {tuple(neighbors.shape)} differ")
    if neighbors.dtype not in (torch.int64, torch.int32):
        raise RuntimeError(f"ssa_amd.sparse_gather_attention: neighbors dtype {neighbors.dtype} "
                           "(int64 or int32)")
    if out is not None and tuple(out.shape) != (B, Hq, N, d):
        raise RuntimeError(f"ssa_amd.sparse_gather_attention: out {tuple(out.shape)} does not "
                           f"match q {tuple(q.shape)}")


def _apply_args(q, k, v, neighbors, valid, scale, fp32w, dropout_p, seed, out, ids32=True):
    """int32 neighbours without a mask are passed as they are (a negative id
    is an invalid slot, as the int64 path treats it) when ids32 allows."""
    check_apply_shapes(q, k, v, neighbors, valid, out)
    B, Hq, N, d = q.shape
    _, Hkv, M, _ = k.shape
    K = neighbors.shape[-1]
    qa, qk = view4(q)
    ka, kk_ = view4(k)
    va, vk = view4(v)
    a = ApplyArgs()
    a.B, a.Hq, a.Hkv, a.N, a.M, a.d, a.K = B, Hq, Hkv, N, M, d, K
    a.q, a.k, a.v = qa, ka, va
    if ids32 and neighbors.dtype == torch.int32 and valid is None:
        nb, vl = neighbors.contiguous(), None
        a.neighbors32 = nb.data_ptr()
    else:
        nb = neighbors.to(torch.int64).contiguous()
        vl = valid.to(torch.bool).contiguous() if valid is not None else None
        a.neighbors, a.valid = nb.data_ptr(), _ptr(vl)
    a.scale, a.fp32_weights, a.dropout_p, a.seed = float(scale), int(fp32w), float(dropout_p), seed
    a.out = out.data_ptr()
    a.out_sb, a.out_sh, a.out_sn = out.stride(0), out.stride(1), out.stride(2)
    return a, (qk, kk_, vk, nb, vl)


def gather_attention_fwd(q, k, v, neighbors, valid, scale, fp32w=False, dropout_p=0.0, seed=0,
                         out=None, row_invalid=None):
    """row_invalid: optional (B*Hq*N,) int32, written with each query row's
    count of slots the graph marks invalid (valid false, or a negative int32
    id): the reference's padding statistic."""
    check_apply_shapes(q, k, v, neighbors, valid, out)
    require_device(q, k, v, neighbors, valid, row_invalid)
    if row_invalid is not None:
        B, Hq, N, _ = q.shape
        if (row_invalid.dtype != torch.int32 or row_invalid.numel() != B * Hq * N
                or not row_invalid.is_contiguous()):
            raise RuntimeError("ssa_amd.sparse_gather_attention: row_invalid must be a "
                               f"contiguous int32 tensor of {B * Hq * N} elements")
    if not (q.dtype == k.dtype == v.dtype):
        raise RuntimeError("ssa_amd.sparse_gather_attention: q, k, v dtypes differ")
    d = q.shape[-1]
    dp = kernel_head_dim(d, q.dtype)
    if dp != d:
        # head dims the kernels do not take: run zero-padded, keep the d columns
        o = gather_attention_fwd(_pad_cols(q, dp), _pad_cols(k, dp), _pad_cols(v, dp), neighbors,
                                 valid, scale, fp32w, dropout_p, seed, None, row_invalid)
        if out is None:
            return o[..., :d]
        out.copy_(o[..., :d])
        return out
    if out is None:
        B, Hq, N, d = q.shape
        out = torch.empty((B, N, Hq, d), dtype=q.dtype, device=q.device).transpose(1, 2)
    a, keep = _apply_args(q, k, v, neighbors, valid, scale, fp32w, dropout_p, seed, out)
    a.row_invalid = _ptr(row_invalid)
    _check(lib().ssa_sparse_gather_attention(ctypes.byref(a), _stream(q)),
           "sparse_gather_attention")
    del keep
    return out


def gather_attention_bwd(q, k, v, neighbors, valid, scale, fp32w, dropout_p, seed, dout,
                         deterministic=False):
    """dq, dk, dv (fp32).  deterministic: ssa_sparse_gather_attention_bwd_det,
    whose dK / dV sums are fixed-point and so the same bits on every run (a
    workspace is allocated here); else the fp32-atomic backward."""
    check_apply_shapes(q, k, v, neighbors, valid, dout)
    require_device(q, k, v, neighbors, valid, dout)
    d = q.shape[-1]
    dp = kernel_head_dim(d, q.dtype)
    if dp != d:
        # head dims the kernels do not take: run zero-padded, keep the d columns
        dq, dk, dv = gather_attention_bwd(_pad_cols(q, dp), _pad_cols(k, dp), _pad_cols(v, dp),
                                          neighbors, valid, scale, fp32w, dropout_p, seed,
                                          _pad_cols(dout, dp), deterministic)
        return dq[..., :d].contiguous(), dk[..., :d].contiguous(), dv[..., :d].contiguous()
    B, Hq, N, d = q.shape
    _, Hkv, M, _ = k.shape
    do = dout.to(torch.float32).contiguous()
    dq = torch.empty((B, Hq, N, d), dtype=torch.float32, device=q.device)
    dk = torch.zeros((B, Hkv, M, d), dtype=torch.float32, device=q.device)
    dv = torch.zeros((B, Hkv, M, d), dtype=torch.float32, device=q.device)
    dummy = torch.empty((B, N, Hq, d), dtype=q.dtype, device=q.device).transpose(1, 2)
    a, keep = _apply_args(q, k, v, neighbors, valid, scale, fp32w, dropout_p, seed, dummy,
                          ids32=False)
    b = ApplyBwdArgs()
    b.fwd = a
    b.dout, b.dq, b.dk, b.dv = do.data_ptr(), dq.data_ptr(), dk.data_ptr(), dv.data_ptr()
    L = lib()
    if deterministic:
        wsb = L.ssa_sparse_gather_attention_bwd_det_workspace_bytes(ctypes.byref(b))
        if wsb < 0:
            _check(int(wsb), "sparse_gather_attention_bwd_det")
        ws = torch.empty(max(int(wsb), 1), dtype=torch.uint8, device=q.device)
        _check(L.ssa_sparse_gather_attention_bwd_det(ctypes.byref(b), ws.data_ptr(), int(wsb),
                                                     _stream(q)),
               "sparse_gather_attention_bwd_det")
        del ws            # the allocator orders its reuse after this stream's work
    else:
        _check(L.ssa_sparse_gather_attention_bwd(ctypes.byref(b), _stream(q)),
               "sparse_gather_attention_bwd")
    del keep
    return dq, dk, dv


# --------------------------------------------------------------------------- measurement
def measure_l2_read(buf: torch.Tensor, blocks: int, iters: int, sink: torch.Tensor):
    """Launch ssa_measure_l2_read over `buf` (uint8, power-of-two size) on the
    current stream: blocks * buf.numel() * iters bytes delivered from the L2."""
    require_device(buf, sink)
    if sink.numel() * sink.element_size() < 4 * blocks:
        raise RuntimeError("ssa_amd.measure_l2_read: sink holds fewer than `blocks` uint32")
    _check(lib().ssa_measure_l2_read(buf.data_ptr(), buf.numel() * buf.element_size(), blocks,
                                     iters, sink.data_ptr(), _stream(buf)), "measure_l2_read")
