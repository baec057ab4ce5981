"""Drop-in host API of SSA's SparseAttention, backed by gfx950 HIP kernels.

Mirrors the Python surface of daedalus/SSA ``sparse_attention.py``: the same
class and function names, constructor arguments, attribute names, RNG
consumption order at construction (so seeded modules and checkpoints carry
identical weights and hyperplanes), ``state_dict`` keys, return contracts,
warnings and exceptions.  What changes is where the hot path runs:

* ``LSHGraphBuilder.forward``, ``merge_neighbors``, ``SparseAttention.build_graph``
  and ``sparse_gather_attention`` call libssa_amd.so through its C ABI
  (:mod:`ssa_amd._lib`).  They require ROCm tensors and raise otherwise --
  there is no CPU fallback.
* GQA/MQA: ``SparseAttention.forward`` hands the UN-expanded K/V
  (B, n_kv, M, d) to the kernels, which index kv head ``h // kv_rep``; the
  public ``_split_kv`` still returns the expanded tensor, and the graph /
  apply entry points accept either form.

Reference line citations point at the daedalus/SSA file.
"""
from __future__ import annotations

import math
import warnings
from dataclasses import dataclass
from typing import Optional, Tuple

import numpy as np
import torch
import torch.nn as nn
import torch.nn.functional as F

from . import _lib


# ---------------------------------------------------------------------------- config
@dataclass
class SSAConfig:
    """Hyper-parameters (sparse_attention.py:188-285; same fields and defaults)."""
    d_model: int = 512
    num_heads: int = 8
    num_kv_heads: Optional[int] = None
    num_neighbors: int = 128
    max_num_hashes: int = 12
    num_hash_rounds: int = 8
    lsh_num_probes: int = 0
    window_size: int = 8
    num_global_tokens: int = 2
    global_token_indices: Optional[list] = None
    dropout: float = 0.0
    causal: bool = False
    fp32_attn_weights: bool = False


# ---------------------------------------------------------------------------- diagnostics
class SubquadraticRegimeTracker:
    """Records (N, K, R, C) per call and reports whether K, R and C stayed
    constant (sparse_attention.py:292-350)."""

    def __init__(self):
        self.history: list = []

    def record(self, N: int, K: int, R: int, C: int) -> None:
        self.history.append((N, K, R, C))

    def check(self, warn: bool = True) -> bool:
        if len(self.history) < 2:
            return True
        ks = {h[1] for h in self.history}
        rs = {h[2] for h in self.history}
        cs = {h[3] for h in self.history}
        ok = len(ks) == 1 and len(rs) == 1 and len(cs) == 1
        if not ok and warn:
            ns = [h[0] for h in self.history]
            warnings.warn(
                f"SubquadraticRegimeTracker: K/R/C varied across {len(self.history)} calls "
                f"(N ranged {min(ns)}-{max(ns)}, K values seen: {sorted(ks)}, R values: "
                f"{sorted(rs)}, C values: {sorted(cs)}). The sub-quadratic complexity claim "
                f"only holds when K, R, C are constants independent of N.",
                stacklevel=2,
            )
        return ok


# ---------------------------------------------------------------------------- builders
class WindowGraphBuilder(nn.Module):
    """(N, 2w+1) positional window (sparse_attention.py:357-376).

    idx[n, o] = n + o for o in [-w, w]; causal maps o > 0 to n; clamped to
    [0, M-1].  The fused graph kernel computes the same window in closed form;
    this module serves callers that build the lists themselves."""

    def __init__(self, window_size: int, causal: bool = False):
        super().__init__()
        self.w = window_size
        self.causal = causal

    def forward(self, N: int, M: int, device) -> torch.Tensor:
        n = torch.arange(N, device=device).unsqueeze(1)
        o = torch.arange(-self.w, self.w + 1, device=device).unsqueeze(0)
        idx = n + o
        if self.causal:
            idx = torch.where(o > 0, n.expand_as(idx), idx)
        return idx.clamp(0, M - 1)


class GlobalGraphBuilder(nn.Module):
    """Global key ids (sparse_attention.py:384-415): ``arange(min(G, M))`` or
    the explicit indices clamped to [0, M-1] (non-persistent buffer)."""

    def __init__(self, num_global: int, indices: Optional[list] = None):
        super().__init__()
        if indices is not None:
            self.register_buffer("_fixed_idx", torch.tensor(indices, dtype=torch.long),
                                 persistent=False)
            self.G = len(indices)
            self._use_fixed = True
        else:
            self.G = num_global
            self._use_fixed = False

    def forward(self, M: int, device) -> torch.Tensor:
        if self._use_fixed:
            return self._fixed_idx.to(device).clamp(0, M - 1)
        return torch.arange(min(self.G, M), device=device)


class LSHGraphBuilder(nn.Module):
    """Multi-round random-hyperplane LSH candidate builder
    (sparse_attention.py:422-959).

    ``rand_proj`` (R, max_P, d) fp32 is drawn exactly as the reference draws
    it: per round ``randn(max_P, d)`` normalised by its row norm clamped at
    1e-12 (:511-520).  ``forward`` runs on the GPU kernels."""

    def __init__(self, d_head: int, lsh_candidates: int, num_rounds: int = 1,
                 max_num_hashes: int = 12, num_probes: int = 0):
        super().__init__()
        assert max_num_hashes <= 12, (
            f"max_num_hashes={max_num_hashes} would allow up to 2**{max_num_hashes}="
            f"{2 ** max_num_hashes:,} buckets per round per (batch,head) slice -- bucket "
            f"tables scale as O(2^P); increase num_hash_rounds instead.")
        self.max_P = max_num_hashes
        self.C = lsh_candidates
        self.R = num_rounds
        assert num_probes >= 0, f"num_probes must be >= 0, got {num_probes}"
        self.T = num_probes
        planes = []
        for _ in range(num_rounds):
            p = torch.randn(max_num_hashes, d_head)
            planes.append(p / p.norm(dim=-1, keepdim=True).clamp_min(1e-12))
        self.register_buffer("rand_proj", torch.stack(planes))

    @staticmethod
    def compute_effective_p(M: int, C: int, max_p: int, min_p: int = 1) -> int:
        """round(log2(M / C)) clamped to [min_p, max_p] (Python round,
        sparse_attention.py:522-557)."""
        if M <= 1 or C <= 0:
            return min_p
        return max(min_p, min(max_p, round(math.log2(max(M, 1) / max(C, 1)))))

    # Small host helpers kept for API parity (the reference's tests call them);
    # forward() does not use them -- the hash kernel computes the same values.
    def _hash_proj(self, x: torch.Tensor, round_idx: int, p_eff: int) -> torch.Tensor:
        """fp32 projections on the first p_eff planes of a round (:593-597)."""
        return x.float() @ self.rand_proj[round_idx, :p_eff].T

    def _hash(self, x: torch.Tensor, round_idx: int, p_eff: int) -> torch.Tensor:
        """Bucket id: bit j = (proj_j > 0), plane j = bit j (:559-591)."""
        bits = (self._hash_proj(x, round_idx, p_eff) > 0).long()
        return (bits << torch.arange(p_eff, device=x.device)).sum(-1)

    def _probe_ids(self, proj: torch.Tensor, p_eff: int, num_probes: int) -> list:
        """min(num_probes, p_eff) one-bit-flip neighbours of the base bucket,
        least confident (smallest |proj|, stable) bit first (:599-646)."""
        t_eff = min(num_probes, p_eff)
        if t_eff <= 0:
            return []
        bits = (proj > 0).long()
        base = (bits << torch.arange(p_eff, device=proj.device)).sum(-1)
        order = proj.abs().argsort(dim=-1, stable=True)
        out = []
        for t in range(t_eff):
            pos = order[..., t]
            out.append(base ^ (1 << pos))
        return out

    def forward(self, q: torch.Tensor, k: torch.Tensor, top_k: int, causal: bool = False,
                glob_fallback: Optional[torch.Tensor] = None, *, _proj=None) -> torch.Tensor:
        """(B, H, N, min(top_k, Call)) candidate key ids ordered by descending
        score (sparse_attention.py:814-959).  ``k`` may be (B, H, M, d) or the
        un-expanded (B, n_kv, M, d).  ``_proj=(q_proj, k_proj)`` injects fp32
        projections (parity testing)."""
        _lib.require_device(q, k)
        M = k.shape[2]
        if glob_fallback is None:
            glob_fallback = torch.zeros(1, dtype=torch.long, device=q.device)
        p_eff = self.compute_effective_p(M, self.C, self.max_P)
        qp, kp = _proj if _proj is not None else (None, None)
        out, _, _ = _lib.build_graph(
            q, k, self.rand_proj, P=p_eff, T=self.T, C=self.C, top_k=top_k, window=0,
            causal=causal, is_cross=False, total_k=1, glob=glob_fallback,
            mode=_lib.GRAPH_LSH, q_proj=qp, k_proj=kp)
        return out


# ---------------------------------------------------------------------------- merge
def merge_neighbors(win_idx: torch.Tensor, glob_idx: torch.Tensor, lsh_idx: torch.Tensor,
                    self_idx: Optional[torch.Tensor], total_k: int, N: int, B: int, H: int,
                    device) -> Tuple[torch.Tensor, torch.Tensor]:
    """Union of window, global and LSH ids per query (sparse_attention.py:966-1089):
    ``[self] ++ ascending unique(pool - {self})[:K-1]`` (self-attention) or
    ``ascending unique(pool)[:K]`` (cross), 0-padded with ``valid`` False.

    ``self_idx`` selects the mode; as in the reference it is the query
    position n for every (b, h)."""
    lsh = lsh_idx.reshape(B, H, N, -1)
    win = win_idx.reshape(N, -1) if win_idx.numel() else win_idx.reshape(N, 0)
    return _lib.merge_neighbors(win, glob_idx.reshape(-1), lsh, self_idx is not None, total_k)


# ---------------------------------------------------------------------------- apply
class _GatherAttention(torch.autograd.Function):
    @staticmethod
    def forward(ctx, q, k, v, neighbors, valid, scale, fp32w, dropout_p, seed, row_invalid=None):
        out = _lib.gather_attention_fwd(q, k, v, neighbors, valid, scale, fp32w, dropout_p, seed,
                                        row_invalid=row_invalid)
        ctx.save_for_backward(q, k, v, neighbors, valid)
        ctx.cfg = (scale, fp32w, dropout_p, seed)
        return out

    @staticmethod
    def backward(ctx, dout):
        # under torch.use_deterministic_algorithms(True) the backward whose
        # dK / dV sums are fixed-point (the same bits on every run); else the
        # faster one that adds them with fp32 atomics
        q, k, v, neighbors, valid = ctx.saved_tensors
        scale, fp32w, dropout_p, seed = ctx.cfg
        dq, dk, dv = _lib.gather_attention_bwd(q, k, v, neighbors, valid, scale, fp32w,
                                               dropout_p, seed, dout,
                                               deterministic=torch.are_deterministic_algorithms_enabled())
        return (dq.to(q.dtype), dk.to(k.dtype), dv.to(v.dtype), None, None, None, None, None,
                None, None)


def sparse_gather_attention(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor,
                            neighbors: torch.Tensor, scale: float,
                            valid: Optional[torch.Tensor] = None, dropout: float = 0.0,
                            training: bool = False, fp32_attn_weights: bool = False,
                            *, _row_invalid: Optional[torch.Tensor] = None) -> torch.Tensor:
    """Attention of each query over its K gathered neighbours
    (sparse_attention.py:1096-1199).  ``k``/``v`` may be (B, H, M, d) or the
    un-expanded (B, n_kv, M, d).  ``_row_invalid`` (the module's padding
    statistic): a (B*H*N,) int32 tensor the kernel fills with each row's count
    of invalid slots."""
    _lib.check_apply_shapes(q, k, v, neighbors, valid)
    _lib.require_device(q, k, v, neighbors, valid)
    p = float(dropout) if (training and dropout > 0.0) else 0.0
    seed = int(torch.randint(0, 2 ** 62, (1,)).item()) if p > 0.0 else 0
    return _GatherAttention.apply(q, k, v, neighbors, valid, float(scale),
                                  bool(fp32_attn_weights), p, seed, _row_invalid)


# ---------------------------------------------------------------------------- module
class SparseAttention(nn.Module):
    """O(N K) multi-head attention over a window + global + LSH neighbour graph
    (sparse_attention.py:1206-1510)."""

    def __init__(self, config: SSAConfig):
        super().__init__()
        assert config.d_model % config.num_heads == 0, (
            f"d_model ({config.d_model}) must be divisible by num_heads ({config.num_heads})")
        n_kv = config.num_kv_heads if config.num_kv_heads is not None else config.num_heads
        assert config.num_heads % n_kv == 0, (
            f"num_heads ({config.num_heads}) must be divisible by num_kv_heads ({n_kv})")
        self.config = config
        self.H = config.num_heads
        self.n_kv = n_kv
        self.kv_rep = config.num_heads // n_kv
        self.d_head = config.d_model // config.num_heads
        self.K = config.num_neighbors
        self.scale = self.d_head ** -0.5

        self.Wq = nn.Linear(config.d_model, self.H * self.d_head, bias=False)
        self.Wk = nn.Linear(config.d_model, n_kv * self.d_head, bias=False)
        self.Wv = nn.Linear(config.d_model, n_kv * self.d_head, bias=False)
        self.Wo = nn.Linear(self.H * self.d_head, config.d_model, bias=False)

        self.win_builder = WindowGraphBuilder(config.window_size, config.causal)
        self.glob_builder = GlobalGraphBuilder(config.num_global_tokens,
                                               config.global_token_indices)
        n_glob = (len(config.global_token_indices) if config.global_token_indices is not None
                  else config.num_global_tokens)
        guaranteed = 2 * config.window_size + 1 + n_glob + 1
        self.lsh_k = max(self.K - guaranteed, 8)
        if guaranteed > self.K:
            warnings.warn(
                f"SSAConfig: window+global+self budget ({guaranteed}) exceeds num_neighbors "
                f"({self.K}). lsh_k is floored at 8 and a large fraction of computed "
                f"candidates will be discarded as padding (harmless to correctness, wasteful "
                f"of compute). Consider reducing window_size or increasing num_neighbors.",
                stacklevel=2,
            )
        self.lsh_builder = LSHGraphBuilder(
            d_head=self.d_head, lsh_candidates=self.lsh_k * 4,
            num_rounds=config.num_hash_rounds, max_num_hashes=config.max_num_hashes,
            num_probes=config.lsh_num_probes)
        self.dp = config.dropout

    # -------------------------------------------------------------- layout helpers
    def _split_q(self, x):
        """(B, N, H*d) -> (B, H, N, d) view."""
        B, N, _ = x.shape
        return x.view(B, N, self.H, self.d_head).transpose(1, 2)

    def _split_kv_compact(self, x):
        """(B, M, n_kv*d) -> (B, n_kv, M, d) view (what the kernels consume)."""
        B, M, _ = x.shape
        return x.view(B, M, self.n_kv, self.d_head).transpose(1, 2)

    def _split_kv(self, x):
        """(B, M, n_kv*d) -> (B, H, M, d), each kv head repeated kv_rep times
        (the reference's layout, sparse_attention.py:1305-1315)."""
        kv = self._split_kv_compact(x)
        if self.kv_rep > 1:
            kv = kv.repeat_interleave(self.kv_rep, dim=1)
        return kv

    def _split(self, x):
        return self._split_q(x)

    def _merge(self, x):
        B, H, N, _ = x.shape
        return x.transpose(1, 2).contiguous().view(B, N, self.config.d_model)

    # -------------------------------------------------------------- graph / apply
    def build_graph(self, q: torch.Tensor, k: torch.Tensor, N: int, M: int, B: int, device,
                    causal: bool, is_cross: bool, *, _proj=None
                    ) -> Tuple[torch.Tensor, torch.Tensor]:
        """(neighbors int64, valid bool), both (B, H, N, K_out)
        (sparse_attention.py:1325-1390).  ``k`` may be expanded or not."""
        _lib.require_device(q, k)
        glob = self._glob_ids(M, q.device)
        p_eff = self.lsh_builder.compute_effective_p(M, self.lsh_builder.C, self.lsh_builder.max_P)
        qp, kp = _proj if _proj is not None else (None, None)
        out, valid, _ = _lib.build_graph(
            q, k, self.lsh_builder.rand_proj, P=p_eff, T=self.lsh_builder.T,
            C=self.lsh_builder.C, top_k=self.lsh_k, window=self.config.window_size,
            causal=causal, is_cross=is_cross, total_k=self.K, glob=glob,
            mode=_lib.GRAPH_FULL, q_proj=qp, k_proj=kp)
        return out, valid

    def _build_graph_ids32(self, q, k, N, M, B, causal, is_cross) -> torch.Tensor:
        """build_graph's graph as one int32 tensor, -1 where valid is False."""
        _lib.require_device(q, k)
        lb = self.lsh_builder
        out, _, _ = _lib.build_graph(
            q, k, lb.rand_proj, P=lb.compute_effective_p(M, lb.C, lb.max_P), T=lb.T, C=lb.C,
            top_k=self.lsh_k, window=self.config.window_size, causal=causal, is_cross=is_cross,
            total_k=self.K, glob=self._glob_ids(M, q.device), mode=_lib.GRAPH_FULL, ids32=True)
        return out

    def _glob_ids(self, M: int, device) -> torch.Tensor:
        """``glob_builder(M, device)``, kept per (M, device) so that a forward
        launches no arange: the ids depend on nothing else (explicit indices
        are keyed by their buffer's storage and version).  The kernels only
        read it."""
        fx = getattr(self.glob_builder, "_fixed_idx", None)
        key = (M, str(device), None if fx is None else (fx.data_ptr(), fx._version))
        cache = self.__dict__.setdefault("_globc", {})
        t = cache.get(key)
        if t is None:
            t = self.glob_builder(M, device)
            cache.clear()
            cache[key] = t
        return t

    def _fused_weight(self, mods):
        """The weights of `mods` stacked along the output dimension.  Under
        autograd they are concatenated on every call (gradients flow back to
        each projection); otherwise the stack is cached until a weight's
        storage or version changes."""
        ws = [m.weight for m in mods]
        if torch.is_grad_enabled() and any(w.requires_grad for w in ws):
            return torch.cat(ws, 0)
        key = tuple((w.data_ptr(), w._version, w.dtype, w.device) for w in ws)
        cache = self.__dict__.setdefault("_wcat", {})
        hit = cache.get(len(mods))
        if hit is None or hit[0] != key:
            with torch.no_grad():
                hit = (key, torch.cat(ws, 0))
            cache[len(mods)] = hit
        return hit[1]

    def _project(self, x, src, is_cross):
        """q (B, H, N, d), and k and v (B, n_kv, M, d) as views of one GEMM
        against the stacked Wk/Wv weights: the same products as Wq(x),
        Wk(src), Wv(src) (sparse_attention.py:1484-1486), without the GQA
        expansion."""
        hk = self.n_kv * self.d_head
        # q on its own, k and v stacked: measured faster at the bench workload
        # (4096 tokens, d_model 4096, 8 kv heads) than one GEMM for all three
        qx = self.Wq(x)
        y = F.linear(src, self._fused_weight((self.Wk, self.Wv)))
        kx, vx = y[..., :hk], y[..., hk:]
        return self._split_q(qx), self._split_kv_compact(kx), self._split_kv_compact(vx)

    # bf16 inference may project and build the graph in one library call whose
    # projections hash the rows they write (ssa_project_build_graph).  Off by
    # default: on the workloads measured, torch's projection GEMM plus the
    # build's own hash pass is as fast or faster (set True on an instance to
    # take the fused path)
    _fuse_projections = False

    def _project_build_fused(self, x, src, N, M, causal, is_cross):
        """(q, k, v, int32 graph) from ssa_project_build_graph, or None when the
        module or the sizes do not take that path (bf16 weights and inputs,
        head dims 32 / 64 / 128, N and M multiples of 16, ...)."""
        if not self._fuse_projections or x.dtype != torch.bfloat16 or x.device.type != "cuda":
            return None
        lb = self.lsh_builder
        P = lb.compute_effective_p(M, lb.C, lb.max_P)
        if not _lib.project_shape_ok(x.dtype, N, M, self.config.d_model, self.H, self.n_kv,
                                     self.d_head, lb.rand_proj.shape[0], P):
            return None
        r = _lib.project_build_graph(
            x, src, self.Wq.weight, self._fused_weight((self.Wk, self.Wv)), self.H, self.n_kv,
            self.d_head, lb.rand_proj, P=P, T=lb.T, C=lb.C, top_k=self.lsh_k,
            window=self.config.window_size, causal=causal, is_cross=is_cross, total_k=self.K,
            glob=self._glob_ids(M, x.device), mode=_lib.GRAPH_FULL, ids32=True)
        if r is None:
            return None
        q, k, v, out, _, _ = r
        return q, k, v, out

    def apply_graph(self, q: torch.Tensor, k: torch.Tensor, v: torch.Tensor,
                    neighbors: torch.Tensor, valid: torch.Tensor, *,
                    _row_invalid: Optional[torch.Tensor] = None) -> torch.Tensor:
        """sparse_gather_attention with this module's scale / dropout / fp32
        weights (sparse_attention.py:1392-1418)."""
        return sparse_gather_attention(q, k, v, neighbors, scale=self.scale, valid=valid,
                                       dropout=self.dp, training=self.training,
                                       fp32_attn_weights=self.config.fp32_attn_weights,
                                       _row_invalid=_row_invalid)

    def forward(self, x: torch.Tensor, key_value: Optional[torch.Tensor] = None,
                attention_mask: Optional[torch.Tensor] = None, return_stats: bool = False,
                *, _defer_stats: bool = False) -> Tuple[torch.Tensor, dict]:
        """(out (B, N, d_model), stats or {}) (sparse_attention.py:1420-1510).
        ``_defer_stats`` (for the layer stacks below): padding_fraction is left
        as a pending device count for ``_resolve_stats``, so a stack syncs with
        the host once instead of once per layer."""
        if attention_mask is not None:
            raise ValueError(
                "SparseAttention does not accept an external attention_mask. Use "
                "config.causal=True for autoregressive masking (handled internally by the "
                "graph builder). For padding, zero out padding positions in x before calling "
                "forward(), or set num_global_tokens to 0 so padding tokens are not forced "
                "into every query's neighbor set.")
        B, N, _ = x.shape
        is_cross = key_value is not None
        src = key_value if is_cross else x
        M = src.shape[1]
        causal = self.config.causal and not is_cross
        # the padding statistic: each row's invalid slots, counted by the
        # gather attention as it reads the graph
        row_inv = (torch.empty(B * self.H * N, dtype=torch.int32, device=x.device)
                   if return_stats else None)
        grad = torch.is_grad_enabled() and (
            x.requires_grad or src.requires_grad
            or any(m.weight.requires_grad for m in (self.Wq, self.Wk, self.Wv)))
        fused = None if grad else self._project_build_fused(x, src, N, M, causal, is_cross)
        if fused is not None:
            # bf16 inference: the projections hash the rows they write and the
            # build reads q and k only for scoring (one call into the library)
            q, k, v, neighbors = fused
            valid = None
            out = self.apply_graph(q, k, v, neighbors, None, _row_invalid=row_inv)
        elif grad:
            q, k, v = self._project(x, src, is_cross)
            neighbors, valid = self.build_graph(q, k, N, M, B, x.device, causal, is_cross)
            out = self.apply_graph(q, k, v, neighbors, valid, _row_invalid=row_inv)
        else:
            # no autograd: the same graph as int32 ids with -1 in the invalid
            # slots, which the gather attention reads as it is (a third of the
            # bytes of int64 ids and a mask, written once and read once)
            q, k, v = self._project(x, src, is_cross)
            neighbors, valid = self._build_graph_ids32(q, k, N, M, B, causal, is_cross), None
            out = self.apply_graph(q, k, v, neighbors, None, _row_invalid=row_inv)
        out_proj = self.Wo(self._merge(out))
        if not return_stats:
            return out_proj, {}
        peak_sparse = B * self.H * N * self.K * self.d_head
        peak_full = B * self.H * N * M * self.d_head
        pad = _PendingFraction(rows=row_inv, numel=neighbors.numel())
        return out_proj, {
            "neighbors_shape": tuple(neighbors.shape),
            "peak_sparse_elems": peak_sparse,
            "peak_full_elems": peak_full,
            "compression": peak_full / peak_sparse,
            "padding_fraction": pad if _defer_stats else pad.value(),
        }


class _PendingFraction:
    """Mean of a boolean mask as the reference's CPU ``.float().mean()``
    rounds it: the exact count divided by the element count in fp32 (the
    device's mean multiplies by a rounded reciprocal instead).  The count is
    taken on the device, from per-row counts (``rows``, numel elements in all)
    or from the mask as bytes summed in int32 while that cannot overflow (a
    bool tensor's own sum first copies it to int64); ``value()`` waits for it."""

    def __init__(self, invalid: Optional[torch.Tensor] = None, *,
                 rows: Optional[torch.Tensor] = None, numel: int = 0):
        if rows is not None:
            self.numel = numel
            self.count = rows.sum(dtype=torch.int64)
            return
        self.numel = invalid.numel()
        acc = torch.int32 if self.numel < (1 << 31) else torch.int64
        self.count = invalid.view(torch.uint8).sum(dtype=acc)

    def value(self) -> float:
        return float(np.float32(int(self.count.item())) / np.float32(max(self.numel, 1)))


def _resolve_stats(stats_list):
    """Replace pending padding fractions by their values (one host sync)."""
    for st in stats_list:
        pad = st.get("padding_fraction")
        if isinstance(pad, _PendingFraction):
            st["padding_fraction"] = pad.value()
    return stats_list


# ---------------------------------------------------------------------------- transformer
class SparseTransformerLayer(nn.Module):
    """Pre-LN block ``x + a + ff(norm2(x + a))`` (sparse_attention.py:1517-1533)."""

    def __init__(self, config: SSAConfig, ffn_mult: int = 4):
        super().__init__()
        d = config.d_model
        self.attn = SparseAttention(config)
        self.ff = nn.Sequential(
            nn.Linear(d, d * ffn_mult), nn.GELU(), nn.Dropout(config.dropout),
            nn.Linear(d * ffn_mult, d), nn.Dropout(config.dropout))
        self.norm1 = nn.LayerNorm(d)
        self.norm2 = nn.LayerNorm(d)

    def forward(self, x, return_stats: bool = False, *, _defer_stats: bool = False):
        a, stats = self.attn(self.norm1(x), return_stats=return_stats,
                             _defer_stats=_defer_stats)
        # x + a + ff(norm2(x + a)) evaluates (x + a) + ff(...): one x + a serves both
        h = x + a
        return h + self.ff(self.norm2(h)), stats


class SparseTransformer(nn.Module):
    """Optional embedding, a stack of SparseTransformerLayer, final LayerNorm
    (sparse_attention.py:1536-1550)."""

    def __init__(self, config: SSAConfig, num_layers: int = 6, vocab_size: int = 0):
        super().__init__()
        self.embed = nn.Embedding(vocab_size, config.d_model) if vocab_size else None
        self.layers = nn.ModuleList([SparseTransformerLayer(config) for _ in range(num_layers)])
        self.norm = nn.LayerNorm(config.d_model)

    def forward(self, x, return_stats: bool = False):
        if self.embed is not None:
            x = self.embed(x)
        stats_list = []
        for layer in self.layers:
            x, stats = layer(x, return_stats=return_stats, _defer_stats=True)
            stats_list.append(stats)
        return self.norm(x), _resolve_stats(stats_list)


# ---------------------------------------------------------------------------- graph reuse
def neighbor_overlap(neighbors_a: torch.Tensor, neighbors_b: torch.Tensor,
                     valid_a: torch.Tensor, valid_b: torch.Tensor) -> torch.Tensor:
    """Per-(b, h, n) Jaccard overlap of two valid neighbour sets
    (sparse_attention.py:1583-1615; offline diagnostic, torch ops)."""
    a = torch.where(valid_a, neighbors_a, torch.full_like(neighbors_a, -1))
    b = torch.where(valid_b, neighbors_b, torch.full_like(neighbors_b, -1))
    a_in_b = (a.unsqueeze(-1) == b.unsqueeze(-2)).any(dim=-1) & valid_a
    inter = a_in_b.sum(dim=-1).float()
    union = (valid_a.sum(dim=-1) + valid_b.sum(dim=-1)).float() - inter
    return inter / union.clamp_min(1.0)


def measure_cross_layer_overlap(model: "SparseTransformer", x: torch.Tensor) -> dict:
    """Adjacent-layer neighbour-set overlap of a SparseTransformer
    (sparse_attention.py:1618-1686)."""
    h = model.embed(x) if model.embed is not None else x
    graphs = []
    for layer in model.layers:
        normed = layer.norm1(h)
        attn = layer.attn
        B, N, _ = normed.shape
        q = attn._split_q(attn.Wq(normed))
        k = attn._split_kv_compact(attn.Wk(normed))
        v = attn._split_kv_compact(attn.Wv(normed))
        nb, va = attn.build_graph(q, k, N, N, B, normed.device, attn.config.causal, False)
        graphs.append((nb.detach(), va.detach()))
        out = attn.apply_graph(q, k, v, nb, va)
        a = attn.Wo(attn._merge(out))
        h = h + a
        h = h + layer.ff(layer.norm2(h))
    overlaps = [neighbor_overlap(graphs[i][0], graphs[i + 1][0], graphs[i][1], graphs[i + 1][1])
                for i in range(len(graphs) - 1)]
    return {
        "per_pair_overlap": overlaps,
        "mean_overlap_per_adjacent_pair": [ov.mean().item() for ov in overlaps],
        "num_layers": len(model.layers),
    }


class CachedGraphSparseTransformer(nn.Module):
    """Graph built once per ``reuse_every`` layers with the group's shared
    builders and re-applied to each layer's own q/k/v
    (sparse_attention.py:1688-1792)."""

    def __init__(self, config: SSAConfig, num_layers: int, reuse_every: int = 4,
                 ffn_mult: int = 4):
        super().__init__()
        assert reuse_every >= 1
        self.reuse_every = reuse_every
        self.config = config
        num_groups = math.ceil(num_layers / reuse_every)
        self.shared_attn_per_group = nn.ModuleList(
            [SparseAttention(config) for _ in range(num_groups)])
        self.group_of = [i // reuse_every for i in range(num_layers)]
        self.layers = nn.ModuleList(
            [SparseTransformerLayer(config, ffn_mult) for _ in range(num_layers)])
        self.norm = nn.LayerNorm(config.d_model)

    def forward(self, x, return_stats: bool = False):
        h = x
        stats_list = []
        cached = None
        cached_group = None
        for i, layer in enumerate(self.layers):
            group = self.group_of[i]
            recompute = group != cached_group
            normed = layer.norm1(h)
            attn = layer.attn
            B, N, _ = normed.shape
            q = attn._split_q(attn.Wq(normed))
            k = attn._split_kv_compact(attn.Wk(normed))
            v = attn._split_kv_compact(attn.Wv(normed))
            if recompute:
                nb, va = self.shared_attn_per_group[group].build_graph(
                    q, k, N, N, B, normed.device, attn.config.causal, is_cross=False)
                cached, cached_group = (nb, va), group
            else:
                nb, va = cached
            row_inv = (torch.empty(B * attn.H * N, dtype=torch.int32, device=normed.device)
                       if return_stats else None)
            out = attn.apply_graph(q, k, v, nb, va, _row_invalid=row_inv)
            a = attn.Wo(attn._merge(out))
            h = h + a
            h = h + layer.ff(layer.norm2(h))
            if return_stats:
                peak_sparse = B * attn.H * N * attn.K * attn.d_head
                peak_full = B * attn.H * N * N * attn.d_head
                stats_list.append({
                    "neighbors_shape": tuple(nb.shape),
                    "compression": peak_full / peak_sparse,
                    "padding_fraction": _PendingFraction(rows=row_inv, numel=va.numel()),
                    "graph_recomputed": recompute,
                })
            else:
                stats_list.append({})
        return self.norm(h), _resolve_stats(stats_list)
