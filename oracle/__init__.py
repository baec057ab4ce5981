"""CPU oracle for the SSA SparseAttention forward hot path.

TEST INFRASTRUCTURE ONLY.  This package is the checker.  Only ``tests/``,
``__graft_entry__.smoke()`` and the ``cpu_baseline`` leg of ``bench.py`` may
import it.  The product package ``ssa_amd`` never imports it and has no CPU
fallback into it.

Two restatements live here:

* ``ssa_oracle.c`` (loaded through :mod:`ctypes` by the functions below): a
  plain-C, per-query restatement of the reference's algorithm
  (``sparse_attention.py`` of daedalus/SSA), including exact emulations of the
  library routines whose tie behaviour fixes the output bits (``torch.sort``
  unstable = introsort, ``torch.topk`` = introselect + introsort).
* :mod:`oracle.torch_port`: the reference's torch-op sequence restated on CPU,
  used as the timed CPU baseline (it issues the same library calls, so it
  times like the reference) and as a second, independent checker.

Parity status per function (what pins it) is listed in each docstring.
"""
from __future__ import annotations

import ctypes
import os
import subprocess

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
_SO = os.path.join(_HERE, "libssa_oracle.so")
_SRC = os.path.join(_HERE, "ssa_oracle.c")

_lib = None


def build(force: bool = False) -> str:
    """Compile ssa_oracle.c into oracle/libssa_oracle.so with gcc."""
    if force or not os.path.exists(_SO) or os.path.getmtime(_SO) < os.path.getmtime(_SRC):
        subprocess.check_call(["make", "-s", "-C", _HERE, "libssa_oracle.so"])
    return _SO


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(_SO):
            build()
        L = ctypes.CDLL(_SO)
        P = ctypes.c_void_p
        I64 = ctypes.c_int64
        L.ssa_oracle_sort_perm.argtypes = [P, ctypes.c_long, P]
        L.ssa_oracle_topk_row.argtypes = [P, ctypes.c_long, ctypes.c_long, P, P]
        L.ssa_oracle_hash.argtypes = [P, ctypes.c_long, ctypes.c_int, P, ctypes.c_int,
                                      ctypes.c_int, P, P, P]
        L.ssa_oracle_lsh_forward.restype = ctypes.c_long
        L.ssa_oracle_lsh_forward.argtypes = [
            P, P, ctypes.c_long, ctypes.c_long, ctypes.c_long, ctypes.c_long, ctypes.c_int,
            P, P, P, ctypes.c_int, ctypes.c_int, ctypes.c_int, ctypes.c_int, ctypes.c_int,
            ctypes.c_int, ctypes.c_int, P, ctypes.c_int, P, P, P, P, ctypes.c_long]
        L.ssa_oracle_merge.argtypes = [P, ctypes.c_long, P, ctypes.c_long, P, ctypes.c_long,
                                       ctypes.c_long, ctypes.c_long, ctypes.c_int,
                                       ctypes.c_long, P, P]
        L.ssa_oracle_apply.argtypes = [P, P, P, P, P, ctypes.c_long, ctypes.c_long,
                                       ctypes.c_long, ctypes.c_long, ctypes.c_int,
                                       ctypes.c_long, ctypes.c_float, ctypes.c_int,
                                       ctypes.c_int, P]
        L.ssa_oracle_set_mutation.argtypes = [ctypes.c_int]
        del I64
        _lib = L
    return _lib


class mutation:
    """Context manager that plants mistake `m` in the C oracle (see the MUT_*
    list in ssa_oracle.c) so a test can show that a pinning check catches it."""

    def __init__(self, m: int):
        self.m = m

    def __enter__(self):
        lib().ssa_oracle_set_mutation(self.m)
        return self

    def __exit__(self, *exc):
        lib().ssa_oracle_set_mutation(0)
        return False


def _p(a: np.ndarray):
    return a.ctypes.data_as(ctypes.c_void_p)


def _f32(a) -> np.ndarray:
    return np.ascontiguousarray(np.asarray(a, dtype=np.float32))


def _i64(a) -> np.ndarray:
    return np.ascontiguousarray(np.asarray(a, dtype=np.int64))


def sort_perm(keys) -> np.ndarray:
    """Permutation returned by ``torch.sort(keys)`` (unstable) on CPU.

    Follows sparse_attention.py:781.  Pinned by tests/test_oracle.py against
    ``torch.sort`` itself on many shapes and key distributions.
    """
    k = _i64(keys)
    out = np.empty_like(k)
    lib().ssa_oracle_sort_perm(_p(k), k.size, _p(out))
    return out


def topk_row(vals, k: int):
    """``torch.topk(vals, k)`` (largest, sorted) on one CPU row: (values, indices).

    Follows the call at sparse_attention.py:921.  Pinned by tests against
    ``torch.topk`` with heavy ties, NaN and -inf.
    """
    v = _f32(vals)
    ov = np.empty(k, np.float32)
    oi = np.empty(k, np.int64)
    lib().ssa_oracle_topk_row(_p(v), v.size, k, _p(ov), _p(oi))
    return ov, oi


def hash_rows(x, planes, T: int = 0):
    """fp32 projections, bucket ids and probe ids of rows ``x`` (rows, d) on
    planes (P, d).  Follows sparse_attention.py:575-646.  Pinned by closed
    forms (sign rule, bit order) and against ``LSHGraphBuilder._probe_ids``
    fixtures."""
    x = _f32(x)
    pl = _f32(planes)
    rows, d = x.shape
    P = pl.shape[0]
    proj = np.empty((rows, P), np.float32)
    ids = np.empty(rows, np.int64)
    probes = np.empty((rows, max(T, 1)), np.int64)
    lib().ssa_oracle_hash(_p(x), rows, d, _p(pl), P, T, _p(proj), _p(ids), _p(probes))
    return proj, ids, probes[:, :T]


def lsh_forward(q, k, planes, *, kv_rep: int, P: int, T: int, C: int, top_k: int,
                causal: bool, glob, q_proj=None, k_proj=None, want_perm: bool = False,
                q_step: int = 1):
    """LSHGraphBuilder.forward (sparse_attention.py:814-959).

    q: (BH, N, d), k: (BK, M, d) with BH = BK * kv_rep, planes: (R, maxP, d).
    Optional injected projections q_proj (BH, R, N, P) / k_proj (BK, R, M, P).
    Returns dict(idx (BH,N,kk) int64, val (BH,N,kk) f32, tie (BH,N) bool,
    n_ties, perm (BK,R,M) if want_perm).  q_step > 1 computes only the query
    rows n % q_step == 0; the other rows of idx / val / tie are zero.

    Pinned by golden fixtures generated from the reference (tests/golden).
    """
    q = _f32(q)
    k = _f32(k)
    pl = _f32(planes)
    BH, N, d = q.shape
    BK, M, _ = k.shape
    R, maxP, _ = pl.shape
    Tp = min(T, P)
    Call = R * (1 + Tp) * C
    kk = min(top_k, Call)
    g = _i64(glob)
    idx = np.zeros((BH, N, kk), np.int64)
    val = np.zeros((BH, N, kk), np.float32)
    tie = np.zeros((BH, N), np.uint8)
    perm = np.empty((BK, R, M), np.int64) if want_perm else None
    qp = _f32(q_proj) if q_proj is not None else None
    kp = _f32(k_proj) if k_proj is not None else None
    n_ties = lib().ssa_oracle_lsh_forward(
        _p(q), _p(k), BH, kv_rep, N, M, d,
        _p(qp) if qp is not None else None, _p(kp) if kp is not None else None,
        _p(pl), R, maxP, P, T, C, top_k, int(causal), _p(g), g.size,
        _p(idx), _p(val), _p(tie), _p(perm) if perm is not None else None, int(q_step))
    out = dict(idx=idx, val=val, tie=tie.astype(bool), n_ties=int(n_ties))
    if want_perm:
        out["perm"] = perm
    return out


def merge(win, glob, lsh, has_self: bool, total_k: int):
    """merge_neighbors (sparse_attention.py:966-1089) -> (neighbors, valid).

    win (N, Kw), glob (G,), lsh (BH, N, Kl).  Pinned by golden fixtures and
    by the closed form "[self] ++ ascending unique(pool - self)[:K-1]".
    """
    w = _i64(win)
    g = _i64(glob)
    l = _i64(lsh)
    BH, N, Kl = l.shape
    Kw = w.shape[1] if w.ndim == 2 else 0
    Kall = Kw + g.size + Kl
    ks = min(total_k - 1, Kall) if has_self else min(total_k, Kall)
    Kout = 1 + ks if has_self else ks
    out = np.empty((BH, N, Kout), np.int64)
    valid = np.empty((BH, N, Kout), np.uint8)
    lib().ssa_oracle_merge(_p(w), Kw, _p(g), g.size, _p(l), Kl, BH, N, int(has_self),
                           total_k, _p(out), _p(valid))
    return out, valid.astype(bool)


def apply(q, k, v, neighbors, valid, *, kv_rep: int, scale: float, mode: int,
          fp32_attn_weights: bool = False) -> np.ndarray:
    """sparse_gather_attention (sparse_attention.py:1096-1199) in float64.

    mode 0 = fp32 model dtype, 1 = bf16 (p rounded to bf16 before P.V),
    2 = fp16.  Returns (BH, N, d) float64; the caller rounds to the model
    dtype.  Pinned against dense softmax attention (torch, float64) when the
    neighbor list covers every key.
    """
    q = _f32(q)
    k = _f32(k)
    v = _f32(v)
    nb = _i64(neighbors)
    BH, N, d = q.shape
    BK, M, _ = k.shape
    K = nb.shape[-1]
    va = np.ascontiguousarray(np.asarray(valid, dtype=np.uint8)) if valid is not None else None
    out = np.empty((BH, N, d), np.float64)
    lib().ssa_oracle_apply(_p(q), _p(k), _p(v), _p(nb), _p(va) if va is not None else None,
                           BH, kv_rep, N, M, d, K, float(scale), mode,
                           int(fp32_attn_weights), _p(out))
    return out
