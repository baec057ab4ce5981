"""Write the golden vectors for the SparseAttention forward path.

Runs ONLY in the development container, where the reference checkout
(daedalus/SSA, ``sparse_attention.py``) is mounted read-only at
/root/reference.  It imports the reference, runs tiny configurations on the
CPU and stores inputs and outputs as compressed ``.npz`` fixtures next to this
script.  The fixtures are data (inputs, weights, outputs); nothing of the
reference's source travels with them.

What the vectors pin (the parts no closed form or library routine pins on its
own): the composition of LSHGraphBuilder.forward (stream order, first-
occurrence dedup including invalid fillers, causal substitution, empty-bucket
fallback, chunked top-k, -inf fallback), merge_neighbors, build_graph,
sparse_gather_attention, SparseAttention.forward with its stats, and the RNG
consumption order of seeded construction.

Usage:  python tests/golden/make_golden.py [--only-empty-ranked | --only-models | --only-proj]
"""
from __future__ import annotations

import dataclasses
import json
import os
import sys
import warnings

import numpy as np
import torch

REF = "/root/reference"
HERE = os.path.dirname(os.path.abspath(__file__))


def _np(t: torch.Tensor) -> np.ndarray:
    t = t.detach().cpu()
    if t.dtype in (torch.bfloat16, torch.float16):
        t = t.float()
    return t.numpy().copy()


# name, config kwargs, (B, N, M or None), dtype, extra
CASES = [
    ("self_base", dict(d_model=64, num_heads=2, num_neighbors=32, max_num_hashes=3,
                       num_hash_rounds=2, window_size=4, num_global_tokens=2), (2, 64, None),
     "float32", {}),
    ("causal", dict(d_model=64, num_heads=2, num_neighbors=16, max_num_hashes=2,
                    num_hash_rounds=3, window_size=3, num_global_tokens=1, causal=True),
     (1, 48, None), "float32", {}),
    ("cross", dict(d_model=64, num_heads=2, num_neighbors=32, max_num_hashes=3,
                   num_hash_rounds=2, window_size=4, num_global_tokens=2), (1, 40, 80),
     "float32", {}),
    ("gqa", dict(d_model=64, num_heads=4, num_kv_heads=2, num_neighbors=16, window_size=4,
                 num_global_tokens=2, max_num_hashes=3, num_hash_rounds=4), (2, 64, None),
     "float32", {}),
    ("mqa_causal", dict(d_model=64, num_heads=4, num_kv_heads=1, num_neighbors=16,
                        window_size=4, num_global_tokens=2, max_num_hashes=3,
                        num_hash_rounds=4, causal=True), (1, 96, None), "float32", {}),
    ("probes_causal", dict(d_model=32, num_heads=2, num_neighbors=32, max_num_hashes=6,
                           num_hash_rounds=2, window_size=2, num_global_tokens=1,
                           causal=True, lsh_num_probes=3), (1, 200, None), "float32", {}),
    ("globals_explicit", dict(d_model=64, num_heads=2, num_neighbors=24, window_size=2,
                              global_token_indices=[0, 5, 100], max_num_hashes=3,
                              num_hash_rounds=3, causal=True), (1, 64, None), "float32", {}),
    ("tiny_n_probes", dict(d_model=32, num_heads=2, num_neighbors=32, max_num_hashes=6,
                           num_hash_rounds=2, window_size=2, num_global_tokens=1,
                           lsh_num_probes=12), (1, 8, None), "float32", {}),
    ("oversize_window", dict(d_model=32, num_heads=2, num_neighbors=16, window_size=16,
                             num_global_tokens=2, max_num_hashes=3, num_hash_rounds=2),
     (1, 48, None), "float32", {}),
    ("cross_probes", dict(d_model=64, num_heads=4, num_kv_heads=2, num_neighbors=24,
                          max_num_hashes=4, num_hash_rounds=3, window_size=4,
                          num_global_tokens=2, lsh_num_probes=2), (2, 50, 130), "float32", {}),
    ("mid_causal_r8", dict(d_model=128, num_heads=2, num_neighbors=64, max_num_hashes=12,
                           num_hash_rounds=8, window_size=8, num_global_tokens=2,
                           causal=True), (1, 256, None), "float32", {}),
    ("dup_rows_ties", dict(d_model=32, num_heads=2, num_neighbors=24, max_num_hashes=4,
                           num_hash_rounds=3, window_size=2, num_global_tokens=1,
                           causal=True, lsh_num_probes=1), (1, 128, None), "float32",
     {"dup_rows": True}),
    ("bf16_gqa", dict(d_model=128, num_heads=4, num_kv_heads=2, num_neighbors=32,
                      window_size=4, num_global_tokens=2, max_num_hashes=12,
                      num_hash_rounds=4, causal=True), (1, 128, None), "bfloat16", {}),
    ("fp32w_dropout0", dict(d_model=32, num_heads=2, num_neighbors=12, max_num_hashes=2,
                            window_size=3, num_global_tokens=1, fp32_attn_weights=True),
     (1, 24, None), "float32", {}),
]

SEEDS = (0, 1)

# bf16 shapes the library's projection kernel takes (head dims 64, Hq*d and
# 2*Hkv*d multiples of 256, N and M multiples of 16): the q/k/v of these come
# from the fused projection + hash path in ssa_amd
PROJ_CASES = [
    ("bf16_proj_causal", dict(d_model=256, num_heads=4, num_kv_heads=2, num_neighbors=32,
                              window_size=2, num_global_tokens=2, max_num_hashes=4,
                              num_hash_rounds=4, lsh_num_probes=1, causal=True), (1, 256, None),
     "bfloat16", {}),
    ("bf16_proj_cross", dict(d_model=256, num_heads=4, num_kv_heads=2, num_neighbors=24,
                             window_size=2, num_global_tokens=2, max_num_hashes=6,
                             num_hash_rounds=3, lsh_num_probes=2), (1, 128, 256), "bfloat16",
     {}),
]


def run_case(sa, name, cfg_kw, shape, dtype, extra, seed):
    B, N, M = shape
    cfg = sa.SSAConfig(**cfg_kw)
    torch.manual_seed(seed)
    with warnings.catch_warnings():
        warnings.simplefilter("ignore")
        attn = sa.SparseAttention(cfg)
    attn.eval()
    init_state = {k: _np(v) for k, v in attn.state_dict().items()}
    dt = getattr(torch, dtype)
    if dtype != "float32":
        for p in attn.parameters():
            p.data = p.data.to(dt)
    gen = torch.Generator().manual_seed(1000 + seed)
    x = torch.randn(B, N, cfg.d_model, generator=gen)
    if extra.get("dup_rows"):
        # repeated token rows -> duplicate key rows -> exactly tied scores
        x[:, 1::3] = x[:, 0:1]
        x[:, 2::5] = x[:, 3:4]
    kv = torch.randn(B, M, cfg.d_model, generator=gen) if M is not None else None
    x = x.to(dt)
    kv = kv.to(dt) if kv is not None else None
    is_cross = kv is not None
    Mv = M if is_cross else N
    causal = cfg.causal and not is_cross
    with torch.no_grad():
        out, stats = attn(x, key_value=kv, return_stats=True)
        q = attn._split_q(attn.Wq(x))
        src = kv if is_cross else x
        k = attn._split_kv(attn.Wk(src))
        v = attn._split_kv(attn.Wv(src))
        glob = attn.glob_builder(Mv, "cpu")
        win = (torch.zeros(N, 0, dtype=torch.long) if is_cross
               else attn.win_builder(N, Mv, "cpu"))
        lsh = attn.lsh_builder(q, k, top_k=attn.lsh_k, causal=causal, glob_fallback=glob)
        nb, valid = attn.build_graph(q, k, N, Mv, B, "cpu", causal, is_cross)
        att = attn.apply_graph(q, k, v, nb, valid)
        # projections as the reference computes them, per round (fp32)
        p_eff = attn.lsh_builder.compute_effective_p(Mv, attn.lsh_builder.C,
                                                     attn.lsh_builder.max_P)
        qf = q.reshape(B * attn.H, N, -1)
        kf = k.reshape(B * attn.H, Mv, -1)
        qproj = torch.stack([attn.lsh_builder._hash_proj(qf, r, p_eff)
                             for r in range(attn.lsh_builder.R)], 1)
        kproj = torch.stack([attn.lsh_builder._hash_proj(kf, r, p_eff)
                             for r in range(attn.lsh_builder.R)], 1)
        probes = attn.lsh_builder._probe_ids(qproj[:, 0], p_eff, attn.lsh_builder.T)
        probes = (torch.stack(probes, -1) if probes
                  else torch.zeros(*qproj.shape[:1], N, 0, dtype=torch.long))
    rec = dict(
        x=_np(x), q=_np(q), k=_np(k), v=_np(v), glob=_np(glob), win=_np(win),
        lsh=_np(lsh), neighbors=_np(nb), valid=_np(valid), attn_out=_np(att), out=_np(out),
        qproj=_np(qproj), kproj=_np(kproj), probes0=_np(probes),
        **{"sd_" + k: v for k, v in init_state.items()},
    )
    if kv is not None:
        rec["kv"] = _np(kv)
    meta = dict(
        name=name, seed=seed, dtype=dtype, B=B, N=N, M=Mv, cross=is_cross, causal=causal,
        config={k: v for k, v in dataclasses.asdict(cfg).items()},
        p_eff=int(p_eff), lsh_k=int(attn.lsh_k), C=int(attn.lsh_builder.C),
        H=attn.H, n_kv=attn.n_kv, d_head=attn.d_head, scale=attn.scale,
        stats={k: (list(v) if isinstance(v, tuple) else v) for k, v in stats.items()},
        extra=extra,
    )
    return rec, meta


def lsh_empty_bucket_case(sa):
    """The empty-bucket fallback vector of the reference's own regression
    test: every key in bucket 0, every query in another bucket."""
    torch.manual_seed(42)
    lsh = sa.LSHGraphBuilder(d_head=4, max_num_hashes=1, lsh_candidates=4)
    k = torch.zeros(1, 1, 8, 4)
    q = torch.ones(1, 1, 4, 4)
    glob = torch.tensor([0, 1])
    out = lsh(q, k, top_k=2, causal=False, glob_fallback=glob)
    return dict(q=_np(q), k=_np(k), glob=_np(glob), out=_np(out),
                rand_proj=_np(lsh.rand_proj)), dict(C=4, top_k=2, max_P=1, R=1)


def lsh_empty_bucket_ranked_case(sa):
    """Empty bucket whose glob ++ 0 list must compete on score: query 0 meets
    an empty bucket in round 0 (every key has a negative first coordinate) and
    a populated one in round 1; keys 5 (the global token) and 0 score above
    every round-1 candidate, so they are selected only if the empty-bucket
    list is built.  Hyperplanes are set to unit vectors after construction."""
    torch.manual_seed(7)
    lsh = sa.LSHGraphBuilder(d_head=4, max_num_hashes=1, lsh_candidates=4, num_rounds=2)
    with torch.no_grad():
        lsh.rand_proj.zero_()
        lsh.rand_proj[0, 0, 0] = 1.0
        lsh.rand_proj[1, 0, 1] = 1.0
    k = torch.tensor([[-1., -1, 0, 4], [-1, 1, 0, 0], [-1, 1, 0, 0], [-1, 1, 0, 0],
                      [-1, 1, 0, 0], [-1, -1, 0, 5], [-1, 1, 0, 0], [-1, 1, 0, 0]])
    q = torch.tensor([[1., 1, 0, 1], [-1, 1, 0, 1]])
    glob = torch.tensor([5])
    out = lsh(q.view(1, 1, 2, 4), k.view(1, 1, 8, 4), top_k=2, causal=False, glob_fallback=glob)
    return dict(q=_np(q), k=_np(k), glob=_np(glob), out=_np(out),
                rand_proj=_np(lsh.rand_proj)), dict(C=4, top_k=2, max_P=1, R=2)


# ---------------------------------------------------------------------------- models
# Tiny SparseTransformer / CachedGraphSparseTransformer configurations: per
# layer they store the layer's input, q / k (expanded, as the reference holds
# them) / v, the fp32 hash projections as the reference computes them, the
# graph, the attention output and the layer's output; plus the final output,
# the stats list and the construction state_dict.
MODEL_CFG = dict(d_model=32, num_heads=4, num_kv_heads=2, num_neighbors=16, window_size=2,
                 num_global_tokens=2, max_num_hashes=4, num_hash_rounds=3, lsh_num_probes=1,
                 causal=True)
MODEL_SHAPE = (2, 96)          # batch, tokens
MODEL_DIR = os.path.join(HERE, "models")


def _projections(builder, q, k, N, M):
    """fp32 hash projections of q and k per round, (BH, R, L, P), as the
    reference computes them (sparse_attention.py:593-597)."""
    lb = builder.lsh_builder
    p_eff = lb.compute_effective_p(M, lb.C, lb.max_P)
    B, H = q.shape[:2]
    qf = q.reshape(B * H, N, -1)
    kf = k.reshape(B * H, M, -1)
    qp = torch.stack([lb._hash_proj(qf, r, p_eff) for r in range(lb.R)], 1)
    kp = torch.stack([lb._hash_proj(kf, r, p_eff) for r in range(lb.R)], 1)
    return qp, kp, p_eff


def _stats_json(stats_list):
    return [{k: (list(v) if isinstance(v, tuple) else v) for k, v in st.items()}
            for st in stats_list]


def model_case(sa, kind, dtype, seed):
    """kind: 'transformer' (2-layer SparseTransformer with a 50-token
    vocabulary, token ids in) or 'cached' (3-layer
    CachedGraphSparseTransformer, reuse_every=2, embeddings in)."""
    cfg = sa.SSAConfig(**MODEL_CFG)
    B, N = MODEL_SHAPE
    torch.manual_seed(seed)
    with warnings.catch_warnings():
        warnings.simplefilter("ignore")
        if kind == "transformer":
            model = sa.SparseTransformer(cfg, num_layers=2, vocab_size=50)
        else:
            model = sa.CachedGraphSparseTransformer(cfg, num_layers=3, reuse_every=2)
    model.eval()
    init_state = {k: _np(v) for k, v in model.state_dict().items()}
    dt = getattr(torch, dtype)
    if dtype != "float32":
        # parameters only: the hyperplane buffers stay fp32 (the reference's
        # fp32 hash matmul needs them so)
        for p in model.parameters():
            p.data = p.data.to(dt)
    gen = torch.Generator().manual_seed(2000 + seed)
    rec = {}
    with torch.no_grad():
        if kind == "transformer":
            ids = torch.randint(0, 50, (B, N), generator=gen)
            rec["ids"] = ids.numpy()
            out, stats = model(ids, return_stats=True)
            h = model.embed(ids)
        else:
            x = torch.randn(B, N, cfg.d_model, generator=gen).to(dt)
            rec["x"] = _np(x)
            out, stats = model(x, return_stats=True)
            h = x
        # the layer loop again, step by step, with the reference's own methods
        cached, cached_group = None, None
        for li, layer in enumerate(model.layers):
            attn = layer.attn
            normed = layer.norm1(h)
            q = attn._split_q(attn.Wq(normed))
            k = attn._split_kv(attn.Wk(normed))
            v = attn._split_kv(attn.Wv(normed))
            if kind == "transformer":
                builder, recompute = attn, True
            else:
                group = model.group_of[li]
                builder, recompute = model.shared_attn_per_group[group], group != cached_group
            qp, kp, p_eff = _projections(builder, q, k, N, N)
            if recompute:
                nb, va = builder.build_graph(q, k, N, N, B, "cpu", cfg.causal, False)
                if kind == "cached":
                    cached, cached_group = (nb, va), group
            else:
                nb, va = cached
            att = attn.apply_graph(q, k, v, nb, va)
            a = attn.Wo(attn._merge(att))
            h_next = h + a + layer.ff(layer.norm2(h + a))
            if kind == "transformer":
                ref_next, _ = layer(h)
                assert torch.equal(ref_next, h_next), "layer loop restated differently"
            for key, val in (("in", h), ("q", q), ("k", k), ("v", v), ("qproj", qp),
                             ("kproj", kp), ("neighbors", nb), ("valid", va),
                             ("attn_out", att), ("out", h_next)):
                rec[f"l{li}_{key}"] = _np(val)
            rec[f"l{li}_recompute"] = np.array(recompute)
            h = h_next
        assert torch.equal(model.norm(h), out), "model output restated differently"
    rec["out"] = _np(out)
    rec.update({"sd_" + k: v for k, v in init_state.items()})
    meta = dict(kind=kind, seed=seed, dtype=dtype, B=B, N=N, config=MODEL_CFG,
                num_layers=len(model.layers), stats=_stats_json(stats),
                group_of=list(getattr(model, "group_of", [])))
    return rec, meta


def write_models(sa):
    os.makedirs(MODEL_DIR, exist_ok=True)
    names = []
    for kind in ("transformer", "cached"):
        for dtype in ("float32", "bfloat16"):
            for seed in SEEDS:
                rec, meta = model_case(sa, kind, dtype, seed)
                fn = f"{kind}_{'fp32' if dtype == 'float32' else 'bf16'}_seed{seed}.npz"
                np.savez_compressed(os.path.join(MODEL_DIR, fn), meta=json.dumps(meta), **rec)
                names.append(fn)
                print("wrote models/" + fn, flush=True)
    with open(os.path.join(MODEL_DIR, "index.json"), "w") as f:
        json.dump(names, f, indent=1)


def main():
    sys.path.insert(0, REF)
    import sparse_attention as sa  # the reference module (read-only checkout)

    if "--only-models" in sys.argv:
        write_models(sa)
        return
    if "--only-proj" in sys.argv:
        with open(os.path.join(HERE, "index.json")) as f:
            index = json.load(f)
        for name, cfg_kw, shape, dtype, extra in PROJ_CASES:
            for seed in SEEDS:
                rec, meta = run_case(sa, name, cfg_kw, shape, dtype, extra, seed)
                fn = f"{name}_s{seed}.npz"
                np.savez_compressed(os.path.join(HERE, fn), meta=json.dumps(meta), **rec)
                if fn not in index:
                    index.append(fn)
                print("wrote", fn, "lsh", rec["lsh"].shape, "nb", rec["neighbors"].shape)
        with open(os.path.join(HERE, "index.json"), "w") as f:
            json.dump(index, f, indent=1)
        return
    if "--only-empty-ranked" in sys.argv:
        rec, meta = lsh_empty_bucket_ranked_case(sa)
        np.savez_compressed(os.path.join(HERE, "lsh_empty_bucket_ranked.npz"),
                            meta=json.dumps(meta), **rec)
        print("wrote lsh_empty_bucket_ranked.npz", rec["out"].tolist())
        return
    index = []
    for name, cfg_kw, shape, dtype, extra in CASES + PROJ_CASES:
        for seed in SEEDS:
            rec, meta = run_case(sa, name, cfg_kw, shape, dtype, extra, seed)
            fn = f"{name}_s{seed}.npz"
            np.savez_compressed(os.path.join(HERE, fn), meta=json.dumps(meta), **rec)
            index.append(fn)
            print("wrote", fn, "lsh", rec["lsh"].shape, "nb", rec["neighbors"].shape)
    rec, meta = lsh_empty_bucket_case(sa)
    np.savez_compressed(os.path.join(HERE, "lsh_empty_bucket.npz"), meta=json.dumps(meta), **rec)
    index.append("lsh_empty_bucket.npz")
    rec, meta = lsh_empty_bucket_ranked_case(sa)
    np.savez_compressed(os.path.join(HERE, "lsh_empty_bucket_ranked.npz"), meta=json.dumps(meta),
                        **rec)
    index.append("lsh_empty_bucket_ranked.npz")
    with open(os.path.join(HERE, "index.json"), "w") as f:
        json.dump(index, f, indent=1)
    write_models(sa)


if __name__ == "__main__":
    main()
