"""The reference suite's module-level properties, run on the GPU against the
drop-in module (tests/*.py of daedalus/SSA, restated for device tensors)."""
import warnings

import pytest
import torch

from conftest import has_gpu

pytestmark = [pytest.mark.gpu,
              pytest.mark.skipif(not has_gpu(), reason="needs a ROCm GPU")]

DEV = "cuda"


def _cfg(**kw):
    from ssa_amd import SSAConfig
    return SSAConfig(**kw)


BASE = dict(d_model=128, num_heads=2, num_neighbors=32, max_num_hashes=3, window_size=4,
            num_global_tokens=2, dropout=0.0, causal=False)
CAUSAL = dict(d_model=64, num_heads=2, num_neighbors=16, max_num_hashes=2, window_size=3,
              num_global_tokens=1, causal=True)


def _attn(**kw):
    from ssa_amd import SparseAttention
    with warnings.catch_warnings():
        warnings.simplefilter("ignore")
        return SparseAttention(_cfg(**kw)).to(DEV)


def test_transformer_shapes_and_stats():
    from ssa_amd import SparseTransformer
    m = SparseTransformer(_cfg(**BASE), num_layers=2).to(DEV)
    x = torch.randn(2, 64, 128, device=DEV)
    out, stats = m(x, return_stats=True)
    assert out.shape == x.shape
    s = stats[0]
    assert s["neighbors_shape"] == (2, 2, 64, 32)
    assert s["compression"] > 1.0
    assert set(s) == {"neighbors_shape", "peak_sparse_elems", "peak_full_elems", "compression",
                      "padding_fraction"}
    out2, stats2 = m(x)
    assert all(st == {} for st in stats2)


def test_cross_attention_shapes_and_range():
    a = _attn(**BASE).eval()
    qx = torch.randn(1, 48, 128, device=DEV)
    kv = torch.randn(1, 96, 128, device=DEV)
    out, stats = a(qx, key_value=kv, return_stats=True)
    assert out.shape == qx.shape
    assert stats["neighbors_shape"][:3] == (1, 2, 48)
    with torch.no_grad():
        q = a._split_q(a.Wq(qx))
        k = a._split_kv(a.Wk(kv))
        nb, va = a.build_graph(q, k, 48, 96, 1, DEV, False, True)
    assert (nb[va] < 96).all() and (nb[va] >= 0).all()


def test_cross_attention_output_width_quirk():
    """Cross-attention width is min(K, G + lsh_k), not K (merge slices the
    deduplicated G + lsh_k columns)."""
    a = _attn(d_model=64, num_heads=4, num_neighbors=64, window_size=4, num_global_tokens=2,
              max_num_hashes=3, num_hash_rounds=6)
    a.lsh_k = 52  # as in the 4-head, K=64, w=4 cross config: 64 - (9 + 2 + 1)
    qx = torch.randn(1, 40, 64, device=DEV)
    kv = torch.randn(1, 120, 64, device=DEV)
    _, st = a(qx, key_value=kv, return_stats=True)
    assert st["neighbors_shape"][-1] == 54


def test_neighbor_graph_no_duplicates_and_self_first():
    a = _attn(**BASE).eval()
    x = torch.randn(1, 64, 128, device=DEV)
    with torch.no_grad():
        q = a._split_q(a.Wq(x))
        k = a._split_kv(a.Wk(x))
        nb, va = a.build_graph(q, k, 64, 64, 1, DEV, False, False)
    assert (nb[0, :, :, 0] == torch.arange(64, device=DEV)).all()
    for h in range(2):
        for i in range(64):
            s = nb[0, h, i, 1:][va[0, h, i, 1:]].tolist()
            assert len(s) == len(set(s)) and i not in s


def test_empty_bucket_fallback_uses_global_tokens():
    from ssa_amd import LSHGraphBuilder
    torch.manual_seed(42)
    lsh = LSHGraphBuilder(d_head=4, max_num_hashes=1, lsh_candidates=4).to(DEV)
    k = torch.zeros(1, 1, 8, 4, device=DEV)
    # a query on the positive side of the single plane -> bucket 1, empty
    q = lsh.rand_proj[0, 0].view(1, 1, 1, 4).expand(1, 1, 4, 4).contiguous()
    nb = lsh(q, k, top_k=2, causal=False, glob_fallback=torch.tensor([0, 1], device=DEV))
    assert not (nb == 7).all()
    assert set(nb[0, 0, 0].tolist()) <= {0, 1}


def test_empty_bucket_list_competes_on_score_reference_vector():
    """Reference vector: the glob ++ 0 list of an empty bucket outscores the
    populated round (query 0 -> [5, 0]).  Query 1 has a k-th place tie among
    keys 1, 2, 3 (equal scores) that the reference's top-k resolves to key 2."""
    import os
    import numpy as np
    from ssa_amd import LSHGraphBuilder
    z = np.load(os.path.join(os.path.dirname(__file__), "golden", "lsh_empty_bucket_ranked.npz"))
    lsh = LSHGraphBuilder(d_head=4, max_num_hashes=1, lsh_candidates=4, num_rounds=2).to(DEV)
    with torch.no_grad():
        lsh.rand_proj.copy_(torch.from_numpy(z["rand_proj"]))
    q = torch.from_numpy(z["q"]).view(1, 1, 2, 4).to(DEV)
    k = torch.from_numpy(z["k"]).view(1, 1, 8, 4).to(DEV)
    nb = lsh(q, k, top_k=2, causal=False, glob_fallback=torch.from_numpy(z["glob"]).to(DEV))
    assert nb.cpu().view(2, 2).tolist() == z["out"].reshape(2, 2).tolist()


def test_cross_attention_more_queries_than_keys():
    a = _attn(d_model=16, num_heads=1, num_neighbors=4, max_num_hashes=1, window_size=1,
              num_global_tokens=1)
    out, _ = a(torch.randn(1, 10, 16, device=DEV), key_value=torch.randn(1, 3, 16, device=DEV))
    assert out.shape == (1, 10, 16) and not out.isnan().any()


def test_causal_no_future_leak_lsh_and_graph():
    from ssa_amd import LSHGraphBuilder
    N = 64
    lsh = LSHGraphBuilder(d_head=8, max_num_hashes=2, lsh_candidates=8).to(DEV)
    q = torch.randn(1, 1, N, 8, device=DEV)
    k = torch.randn(1, 1, N, 8, device=DEV)
    nb = lsh(q, k, top_k=4, causal=True, glob_fallback=torch.zeros(1, dtype=torch.long,
                                                                     device=DEV))
    assert (nb[0, 0] <= torch.arange(N, device=DEV).unsqueeze(1)).all()
    a = _attn(d_model=32, num_heads=2, num_neighbors=32, max_num_hashes=6, num_hash_rounds=2,
              window_size=2, num_global_tokens=1, causal=True, lsh_num_probes=3).eval()
    x = torch.randn(1, 200, 32, device=DEV)
    with torch.no_grad():
        q = a._split_q(a.Wq(x))
        k = a._split_kv(a.Wk(x))
        nb, va = a.build_graph(q, k, 200, 200, 1, DEV, True, False)
    pos = torch.arange(200, device=DEV).view(1, 1, 200, 1)
    assert ((nb <= pos) | ~va).all()
    out, _ = a(x)
    assert not out.isnan().any()


def test_causal_global_leak_is_kept():
    """Explicit global ids are never causally filtered (reference behaviour)."""
    a = _attn(d_model=32, num_heads=2, num_neighbors=24, window_size=2,
              global_token_indices=[0, 1, 40], max_num_hashes=3, causal=True).eval()
    x = torch.randn(1, 64, 32, device=DEV)
    with torch.no_grad():
        q = a._split_q(a.Wq(x))
        k = a._split_kv(a.Wk(x))
        nb, va = a.build_graph(q, k, 64, 64, 1, DEV, True, False)
    assert (nb[0, :, 0][va[0, :, 0]] == 40).any()


@pytest.mark.parametrize("nkv", [1, 2, 4])
def test_gqa_mqa_forward_and_grad(nkv):
    a = _attn(d_model=64, num_heads=4, num_kv_heads=nkv, num_neighbors=16, window_size=4,
              num_global_tokens=2, max_num_hashes=3)
    x = torch.randn(2, 24, 64, device=DEV, requires_grad=True)
    out, _ = a(x)
    assert out.shape == x.shape
    out.sum().backward()
    assert not x.grad.isnan().any()
    assert a.Wk.weight.grad.norm().item() > 0


def test_build_apply_split_matches_forward():
    for kw, cross in [(BASE, False), (BASE, True), (CAUSAL, False)]:
        a = _attn(**kw).eval()
        x = torch.randn(2, 48, kw["d_model"], device=DEV)
        kv = torch.randn(2, 80, kw["d_model"], device=DEV) if cross else None
        with torch.no_grad():
            ref, _ = a(x, key_value=kv)
            src = kv if cross else x
            q = a._split_q(a.Wq(x))
            k = a._split_kv(a.Wk(src))
            v = a._split_kv(a.Wv(src))
            M = src.shape[1]
            nb, va = a.build_graph(q, k, 48, M, 2, DEV, kw["causal"] and not cross, cross)
            out = a.Wo(a._merge(a.apply_graph(q, k, v, nb, va)))
        assert torch.allclose(ref, out, atol=1e-6)


def test_forward_without_autograd_uses_int32_graph_bit_identically():
    """forward() without autograd builds the graph as int32 ids (-1 = invalid):
    the same ids as build_graph where valid, and the same output, bit for bit,
    as build_graph + apply_graph on the int64 graph (bf16 and fp32, self and
    cross); the stats read the same padding fraction."""
    from ssa_amd import _lib
    for dtype in (torch.float32, torch.bfloat16):
        for kw, cross in [(BASE, False), (CAUSAL, False), (BASE, True)]:
            a = _attn(**kw).eval()
            for p_ in a.parameters():
                p_.data = p_.data.to(dtype)
            x = torch.randn(2, 48, kw["d_model"], device=DEV).to(dtype)
            kv = torch.randn(2, 80, kw["d_model"], device=DEV).to(dtype) if cross else None
            src = kv if cross else x
            M = src.shape[1]
            causal = kw["causal"] and not cross
            with torch.no_grad():
                out, stats = a(x, key_value=kv, return_stats=True)
                q = a._split_q(a.Wq(x))
                k = a._split_kv_compact(a.Wk(src))
                v = a._split_kv_compact(a.Wv(src))
                nb, va = a.build_graph(q, k, 48, M, 2, DEV, causal, cross)
                ids = a._build_graph_ids32(q, k, 48, M, 2, causal, cross)
                ref = a.Wo(a._merge(a.apply_graph(q, k, v, nb, va)))
                via32 = _lib.gather_attention_fwd(q, k, v, ids, None, a.scale)
                via64 = _lib.gather_attention_fwd(q, k, v, nb, va, a.scale)
            assert ids.dtype == torch.int32
            assert torch.equal(ids.long(), torch.where(va, nb, torch.full_like(nb, -1)))
            assert torch.equal(out, ref)
            assert torch.equal(via32, via64)
            assert stats["padding_fraction"] == (~va).cpu().float().mean().item()   # the reference's CPU mean
            assert stats["neighbors_shape"] == tuple(nb.shape)


def test_gradients_reach_all_projections():
    a = _attn(d_model=32, num_heads=2, num_neighbors=12, max_num_hashes=2, window_size=3,
              num_global_tokens=1)
    x = torch.randn(2, 24, 32, device=DEV, requires_grad=True)
    out, _ = a(x)
    out.sum().backward()
    for W in (a.Wq, a.Wk, a.Wv, a.Wo):
        assert W.weight.grad is not None and W.weight.grad.norm().item() > 0


def test_dropout_train_vs_eval():
    a = _attn(d_model=32, num_heads=2, num_neighbors=16, max_num_hashes=2, window_size=3,
              num_global_tokens=1, dropout=0.5)
    x = torch.randn(1, 24, 32, device=DEV)
    a.train()
    o1, _ = a(x)
    o2, _ = a(x)
    assert not torch.allclose(o1, o2)
    a.eval()
    o3, _ = a(x)
    o4, _ = a(x)
    assert torch.equal(o3, o4)


def test_fp32_attn_weights_close_in_fp32():
    from ssa_amd import SparseAttention
    kw = dict(d_model=32, num_heads=2, num_neighbors=12, max_num_hashes=2, window_size=3,
              num_global_tokens=1)
    torch.manual_seed(123)
    a = SparseAttention(_cfg(**kw, fp32_attn_weights=False)).to(DEV)
    torch.manual_seed(123)
    b = SparseAttention(_cfg(**kw, fp32_attn_weights=True)).to(DEV)
    x = torch.randn(1, 24, 32, device=DEV)
    assert torch.allclose(a(x)[0], b(x)[0], atol=1e-5)


def test_bf16_module_parameters_only_cast():
    """bf16 recipe: parameters cast, rand_proj kept fp32."""
    a = _attn(d_model=128, num_heads=4, num_kv_heads=2, num_neighbors=32, window_size=4,
              num_global_tokens=2, causal=True)
    for p in a.parameters():
        p.data = p.data.to(torch.bfloat16)
    x = (torch.randn(1, 128, 128, device=DEV) * 0.02).to(torch.bfloat16)
    out, st = a(x, return_stats=True)
    assert out.dtype == torch.bfloat16 and torch.isfinite(out.float()).all()
    assert a.lsh_builder.rand_proj.dtype == torch.float32


def test_cached_graph_transformer_pattern_and_grad():
    from ssa_amd import CachedGraphSparseTransformer
    m = CachedGraphSparseTransformer(_cfg(**BASE), num_layers=6, reuse_every=3).to(DEV)
    x = torch.randn(2, 48, 128, device=DEV, requires_grad=True)
    out, stats = m(x, return_stats=True)
    assert out.shape == x.shape
    assert [s["graph_recomputed"] for s in stats] == [True, False, False, True, False, False]
    out.sum().backward()
    assert not x.grad.isnan().any() and x.grad.norm().item() > 0


def test_neighbor_overlap_known_answers_and_cross_layer_report():
    from ssa_amd import SparseTransformer, measure_cross_layer_overlap, neighbor_overlap
    a = torch.tensor([[[[0, 1, 2, 3]]]], device=DEV)
    b = torch.tensor([[[[2, 3, 4, 5]]]], device=DEV)
    v = torch.ones(1, 1, 1, 4, dtype=torch.bool, device=DEV)
    assert abs(neighbor_overlap(a, b, v, v).item() - 2 / 6) < 1e-6
    m = SparseTransformer(_cfg(**BASE), num_layers=4).to(DEV)
    rep = measure_cross_layer_overlap(m, torch.randn(2, 32, 128, device=DEV))
    assert len(rep["mean_overlap_per_adjacent_pair"]) == 3
    assert sum(rep["mean_overlap_per_adjacent_pair"]) / 3 < 0.9


def test_vocab_embedding_path():
    from ssa_amd import SparseTransformer
    m = SparseTransformer(_cfg(d_model=32, num_heads=2, num_neighbors=12, max_num_hashes=2,
                               window_size=3, num_global_tokens=1), num_layers=2,
                          vocab_size=100).to(DEV)
    ids = torch.randint(0, 100, (2, 24), device=DEV)
    out, _ = m(ids)
    out.sum().backward()
    assert out.shape == (2, 24, 32) and not m.embed.weight.grad.isnan().any()


def _recall(nb, va, q, k, true_k=32):
    dense = q[0, 0] @ k[0, 0].T
    top = dense.topk(true_k, dim=-1).indices
    hit = (nb[0, 0].unsqueeze(-1) == top.unsqueeze(1)) & va[0, 0].unsqueeze(-1)
    return (hit.any(1).sum(-1).float() / true_k).mean().item()


def test_recall_beats_random_and_grows_with_probes():
    from ssa_amd import SparseAttention
    rs = []
    for T in (0, 1, 3):
        torch.manual_seed(0)
        a = SparseAttention(_cfg(d_model=64, num_heads=2, num_neighbors=64, max_num_hashes=12,
                                 num_hash_rounds=4, lsh_num_probes=T, window_size=8,
                                 num_global_tokens=4)).to(DEV).eval()
        x = torch.randn(1, 2048, 64, device=DEV)
        with torch.no_grad():
            q = a._split_q(a.Wq(x))
            k = a._split_kv(a.Wk(x))
            nb, va = a.build_graph(q, k, 2048, 2048, 1, DEV, False, False)
        rs.append(_recall(nb, va, q, k))
    assert rs[0] > 2 * 64 / 2048
    assert rs[1] > rs[0] and rs[2] > rs[1], rs


@pytest.mark.parametrize("causal,cross", [(True, False), (False, False), (False, True)])
def test_forward_equals_build_then_apply(causal, cross):
    """forward (fused projections, graph as int32 ids) equals build_graph +
    apply_graph on the same projections, and the int32 graph equals the
    int64 + valid one."""
    kw = dict(d_model=256, num_heads=4, num_kv_heads=2, num_neighbors=48, max_num_hashes=6,
              window_size=5, num_global_tokens=2, causal=causal)
    torch.manual_seed(3)
    a = _attn(**kw).eval()
    B, N, M = 2, 300, (420 if cross else 300)
    x = torch.randn(B, N, 256, device=DEV)
    src = torch.randn(B, M, 256, device=DEV) if cross else x
    with torch.no_grad():
        q, k, v = a._project(x, src, cross)
        nb1, va1 = a.build_graph(q, k, N, M, B, DEV, causal, cross)
        ids = a._build_graph_ids32(q, k, N, M, B, causal, cross)
        out_fwd, _ = a(x, key_value=src if cross else None)
        out_ref = a.Wo(a._merge(a.apply_graph(q, k, v, nb1, va1)))
    torch.cuda.synchronize()
    assert torch.equal(ids >= 0, va1)
    assert torch.equal(ids.long().clamp_min(0), nb1)
    assert torch.equal(out_fwd, out_ref)


def test_fused_projection_matches_separate_projections():
    """q, k, v from one fused GEMM equal Wq(x), Wk(x), Wv(x) to fp32 rounding,
    and gradients reach every projection."""
    kw = dict(d_model=256, num_heads=4, num_kv_heads=2, num_neighbors=32, max_num_hashes=4,
              window_size=3, num_global_tokens=1, causal=True)
    torch.manual_seed(5)
    a = _attn(**kw)
    x = torch.randn(2, 96, 256, device=DEV)
    for cross in (False, True):
        src = torch.randn(2, 80, 256, device=DEV) if cross else x
        with torch.no_grad():
            q, k, v = a._project(x, src, cross)
            q2 = a._split_q(a.Wq(x))
            k2 = a._split_kv_compact(a.Wk(src))
            v2 = a._split_kv_compact(a.Wv(src))
        for u, w in ((q, q2), (k, k2), (v, v2)):
            assert torch.allclose(u, w, rtol=1e-5, atol=1e-5)
    a.train()
    out, _ = a(x)
    out.float().pow(2).mean().backward()
    for m in (a.Wq, a.Wk, a.Wv, a.Wo):
        assert m.weight.grad is not None and torch.isfinite(m.weight.grad).all()
        assert m.weight.grad.abs().sum() > 0
