"""The reference's SparseAttention forward restated as the same torch CPU op
sequence.  TEST INFRASTRUCTURE ONLY: used as the timed CPU baseline in
bench.py (it calls the same CPU library routines with the same shapes and
dtypes as daedalus/SSA sparse_attention.py, so it times like the reference
and produces the same bits) and as a second checker.

Each step cites the reference lines it follows.  Nothing here is used by the
product package.
"""
from __future__ import annotations

import math

import torch
import torch.nn.functional as F


def effective_p(M, C, max_p, min_p=1):
    """:522-557 (Python round)."""
    if M <= 1 or C <= 0:
        return min_p
    return max(min_p, min(max_p, round(math.log2(max(M, 1) / max(C, 1)))))


def _bucket_ids(proj, p):
    """:589-591 -- bit j = proj_j > 0, plane j = bit j."""
    return ((proj > 0).long() * (2 ** torch.arange(p))).sum(-1)


def _probe_sets(proj, p, T):
    """:599-646 -- one-bit flips of the base id, least |proj| first."""
    t_eff = min(T, p)
    if t_eff <= 0:
        return []
    bits = (proj > 0).long()
    pw = 2 ** torch.arange(p)
    base = (bits * pw).sum(-1)
    order = proj.abs().argsort(dim=-1)
    out = []
    for t in range(t_eff):
        pos = order[..., t]
        bit = torch.gather(bits, -1, pos.unsqueeze(-1)).squeeze(-1)
        out.append(base + pw[pos] * (1 - 2 * bit))
    return out


def _bucket_members(ids, bstart, bsize, perm, N, M, C, causal, glob):
    """:648-739 -- first C members of each query's bucket, overflow slots
    carry perm[M-1] and are invalid, causal future -> self, empty bucket ->
    glob ++ 0 (valid)."""
    BH = ids.shape[0]
    st = torch.gather(bstart, 1, ids)
    sz = torch.gather(bsize, 1, ids)
    pos = st.unsqueeze(-1) + torch.arange(C).view(1, 1, C)
    end = (st + sz - 1).clamp(max=M - 1)
    valid = pos <= end.unsqueeze(-1)
    pos = torch.where(valid, pos, torch.full_like(pos, M)).clamp(max=M).clamp(max=M - 1)
    cand = torch.gather(perm, 1, pos.reshape(BH, N * C)).view(BH, N, C)
    if causal:
        qpos = torch.arange(N).view(1, N, 1).expand(BH, N, C)
        cand = torch.where(cand > qpos, qpos, cand)
    empty = sz == 0
    if empty.any():
        G = glob.shape[0]
        fb = glob.view(1, 1, G).expand(BH, N, G)
        fb = fb[..., :C] if G >= C else torch.cat(
            [fb, torch.zeros(BH, N, C - G, dtype=torch.long)], -1)
        cand = torch.where(empty.unsqueeze(-1).expand_as(cand), fb, cand)
        valid = valid | empty.unsqueeze(-1).expand_as(valid)
    return cand, valid


def lsh_forward(q, k, rand_proj, top_k, causal, glob, C, R, max_p, T):
    """LSHGraphBuilder.forward (:814-959) on CPU tensors (k expanded to H heads)."""
    B, H, N, d = q.shape
    M = k.shape[2]
    BH = B * H
    p = effective_p(M, C, max_p)
    qf = q.reshape(BH, N, d)
    kf = k.reshape(BH, M, d)
    nb = 2 ** p
    cands, valids = [], []
    for r in range(R):
        planes = rand_proj[r, :p]
        qproj = qf.float() @ planes.T
        kid = _bucket_ids(kf.float() @ planes.T, p)
        qid = _bucket_ids(qproj, p)
        skid, perm = torch.sort(kid, dim=-1)
        bstart = torch.full((BH, nb), M, dtype=torch.long)
        bsize = torch.zeros((BH, nb), dtype=torch.long)
        bstart.scatter_reduce_(1, skid, torch.arange(M).unsqueeze(0).expand(BH, M),
                               reduce="amin", include_self=True)
        bsize.scatter_add_(1, skid, torch.ones_like(skid))
        for ids in [qid] + _probe_sets(qproj, p, T):
            c, v = _bucket_members(ids, bstart, bsize, perm, N, M, C, causal, glob)
            cands.append(c.to(torch.int32))
            valids.append(v)
    cand = torch.cat(cands, -1)
    valid = torch.cat(valids, -1)
    Call = cand.shape[-1]
    # first occurrence in stream order, regardless of validity (:879-890)
    sv, si = torch.sort(cand, dim=-1, stable=True)
    first = torch.ones_like(sv, dtype=torch.bool)
    first[..., 1:] = sv[..., 1:] != sv[..., :-1]
    keep_sorted = torch.gather(valid, -1, si) & first
    keep = torch.zeros_like(valid)
    keep.scatter_(-1, si, keep_sorted)
    valid = valid & keep
    # chunked fp32 rescore with a running top-k (:892-924)
    kk = min(top_k, Call)
    k2 = kf.reshape(BH * M, d)
    off = torch.arange(BH).unsqueeze(1) * M
    chunk = min(Call, max(256, kk * 4))
    best_s = torch.full((BH, N, kk), float("-inf"))
    best_i = torch.zeros(BH, N, kk, dtype=torch.int32)
    for s0 in range(0, Call, chunk):
        s1 = min(s0 + chunk, Call)
        cc = cand[:, :, s0:s1]
        rows = torch.index_select(k2, 0, (cc.reshape(BH, -1).long() + off).reshape(-1))
        sc = torch.einsum("bnd,bncd->bnc", qf.float(), rows.view(BH, N, s1 - s0, d).float())
        sc = sc.masked_fill(~valid[:, :, s0:s1], float("-inf"))
        best_s, sel = torch.cat([best_s, sc], -1).topk(kk, dim=-1)
        best_i = torch.gather(torch.cat([best_i, cc], -1), -1, sel)
    res = best_i.long()
    bad = torch.isneginf(best_s)
    if bad.any():                                              # :948-957
        G = glob.shape[0]
        fb = glob.view(1, 1, G).expand(BH, N, G)
        fb = fb[..., :kk] if G >= kk else torch.cat(
            [fb, torch.zeros(BH, N, kk - G, dtype=torch.long)], -1)
        res = torch.where(bad, fb, res)
    return res.view(B, H, N, kk)


def merge(win, glob, lsh, self_idx, total_k, N, B, H):
    """merge_neighbors (:966-1089)."""
    parts = [win.view(1, 1, N, -1).expand(B, H, N, -1), glob.view(1, 1, 1, -1).expand(B, H, N, -1),
             lsh]
    comb = torch.cat(parts, -1)
    tmax = comb.max()
    sent = tmax + 1
    if self_idx is not None:
        comb = comb.masked_fill(comb == self_idx.unsqueeze(-1), sent)
    srt, _ = torch.sort(comb, dim=-1)
    keep = torch.ones_like(srt, dtype=torch.bool)
    keep[..., 1:] = srt[..., 1:] != srt[..., :-1]
    ded, _ = torch.sort(srt.masked_fill(~keep, sent), dim=-1)
    if self_idx is not None:
        out = torch.cat([self_idx.unsqueeze(-1), ded[..., :total_k - 1]], -1)
    else:
        out = ded[..., :total_k]
    valid = out <= tmax
    if self_idx is not None:
        valid[..., 0] = True
    out = torch.where(out > tmax, torch.zeros_like(out), out)
    return out.clamp(0, tmax), valid


def apply(q, k, v, nb, scale, valid, fp32w=False):
    """sparse_gather_attention (:1096-1199), no dropout."""
    B, H, N, d = q.shape
    K = nb.shape[-1]
    M = k.shape[2]
    BH = B * H
    off = torch.arange(BH).unsqueeze(1) * M
    fi = (nb.reshape(BH, N * K) + off).reshape(-1)
    kg = torch.index_select(k.reshape(BH * M, d), 0, fi).view(B, H, N, K, d)
    vg = torch.index_select(v.reshape(BH * M, d), 0, fi).view(B, H, N, K, d)
    s = torch.einsum("bhnd,bhnkd->bhnk", q.float(), kg.float()) * scale
    s = s.masked_fill(~valid, float("-inf"))
    p = F.softmax(s, dim=-1)
    if fp32w:
        return torch.einsum("bhnk,bhnkd->bhnd", p, vg.float()).to(q.dtype)
    return torch.einsum("bhnk,bhnkd->bhnd", p.to(vg.dtype), vg)


def forward(x, Wq, Wk, Wv, Wo, rand_proj, *, H, n_kv, K, window, glob_n, R, max_p, T, causal,
            fp32w=False):
    """SparseAttention.forward (:1420-1491) for self-attention with default
    (first-G) global tokens.  Weights are (out, in) like nn.Linear."""
    B, N, _ = x.shape
    d = Wq.shape[0] // H
    rep = H // n_kv
    q = (x @ Wq.T).view(B, N, H, d).transpose(1, 2)
    k = (x @ Wk.T).view(B, N, n_kv, d).transpose(1, 2)
    v = (x @ Wv.T).view(B, N, n_kv, d).transpose(1, 2)
    if rep > 1:
        k = k.repeat_interleave(rep, dim=1)
        v = v.repeat_interleave(rep, dim=1)
    glob = torch.arange(min(glob_n, N))
    pos = torch.arange(N)
    off = torch.arange(-window, window + 1)
    win = pos.unsqueeze(1) + off.unsqueeze(0)
    if causal:
        win = torch.where((off > 0).unsqueeze(0).expand(N, -1), pos.unsqueeze(1).expand_as(win),
                          win)
    win = win.clamp(0, N - 1)
    lsh_k = max(K - (2 * window + 1 + glob_n + 1), 8)
    lsh = lsh_forward(q, k, rand_proj, lsh_k, causal, glob, 4 * lsh_k, R, max_p, T)
    self_idx = pos.view(1, 1, N).expand(B, H, N)
    nb, valid = merge(win, glob, lsh, self_idx, K, N, B, H)
    out = apply(q, k, v, nb, d ** -0.5, valid, fp32w)
    return out.transpose(1, 2).contiguous().view(B, N, H * d) @ Wo.T
