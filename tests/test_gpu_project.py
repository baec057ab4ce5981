"""GPU parity of the projections with the hash in their epilogue
(ssa_project_build_graph / ssa_project_gemm).

* The GEMM alone: every element is the fp32-accumulated product rounded once
  to bf16 (within the rounding of the fp32 sum), checked against float64.
* Exact-arithmetic tier: x, the weights and the hyperplanes hold small
  integers, so the projections, the hyperplane projections and every score
  are exact in any order: q / k / v must equal the integer products and the
  graph must equal the oracle's on those q, k bit for bit.
* Reference vectors (bf16_proj_*): the reference's own x, weights and
  hyperplanes; the fused q / k / v must equal the reference's bf16 projections
  and the fused graph the reference's graph.
* The module's fused forward against its separate projections + build.
"""
import os

import numpy as np
import pytest
import torch

import oracle
from conftest import GOLDEN, has_gpu, load_golden, row_rel_err

pytestmark = [pytest.mark.gpu,
              pytest.mark.skipif(not has_gpu(), reason="needs a ROCm GPU")]

DEV = "cuda"


class _nowarn:
    def __enter__(self):
        import warnings
        self.c = warnings.catch_warnings()
        self.c.__enter__()
        warnings.simplefilter("ignore")

    def __exit__(self, *a):
        self.c.__exit__(*a)


def _bf16_ulp(a):
    """bf16 unit in the last place of |a| (float64 array)."""
    e = np.floor(np.log2(np.maximum(np.abs(a), 2.0 ** -126)))
    return 2.0 ** (e - 7)


# ------------------------------------------------------------------ the GEMM
@pytest.mark.parametrize("rows,cols,K", [(256, 256, 64), (272, 512, 128), (1024, 768, 320),
                                         (4096, 1024, 256), (48, 256, 1024)])
def test_project_gemm_is_the_rounded_fp32_product(rows, cols, K):
    from ssa_amd import _lib
    g = torch.Generator().manual_seed(rows + cols + K)
    x = torch.randn(rows, K, generator=g).to(torch.bfloat16)
    w = (torch.randn(cols, K, generator=g) * 0.05).to(torch.bfloat16)
    y = _lib.project_gemm(x.to(DEV), w.to(DEV)).float().cpu().numpy().astype(np.float64)
    xd, wd = x.double().numpy(), w.double().numpy()
    exact = xd @ wd.T
    # fp32 accumulation error bound plus half an ulp of the final rounding
    bound = K * 2.0 ** -24 * (np.abs(xd) @ np.abs(wd).T) + 0.5 * _bf16_ulp(exact)
    assert np.all(np.abs(y - exact) <= bound * 1.0001)
    # and the value torch's bf16 linear computes (the same fp32 accumulation and
    # one rounding; only where both sums round alike)
    ref = torch.nn.functional.linear(x.to(DEV), w.to(DEV)).float().cpu().numpy()
    same = float((ref == y).mean())
    print(f"equal to torch's F.linear on {same:.6f} of the elements")
    assert same > 0.999


# ------------------------------------------------------------------ exact tier
PROJ_CASES = [
    # name, B, H, n_kv, N, M, d, R, maxP, T, K, w, G, causal, cross
    ("causal_gqa_d64", 1, 4, 2, 128, 128, 64, 3, 4, 1, 24, 2, 2, True, False),
    ("mqa_d128_probes", 2, 2, 1, 96, 96, 128, 2, 6, 2, 32, 2, 1, True, False),
    ("cross_d32", 2, 8, 4, 64, 160, 32, 3, 4, 1, 20, 4, 2, False, True),
    ("globals_d64", 1, 4, 2, 128, 128, 64, 3, 3, 0, 24, 2, [0, 5, 100], True, False),
    ("wide_d64_r8", 1, 8, 2, 256, 256, 64, 8, 4, 0, 48, 4, 2, True, False),
    ("self_d128_nc", 1, 4, 1, 64, 64, 128, 4, 3, 1, 24, 3, 2, False, False),
]


def _ints(shape, lo, hi, gen, density=1.0):
    v = torch.randint(lo, hi + 1, shape, generator=gen).float()
    if density < 1.0:
        v = v * (torch.rand(shape, generator=gen) < density).float()
    return v


def _proj_module(case, seed):
    from ssa_amd import SSAConfig, SparseAttention
    (_, B, H, nkv, N, M, d, R, maxP, T, K, w, G, causal, cross) = case
    cfg = SSAConfig(d_model=H * d, num_heads=H, num_kv_heads=nkv, num_neighbors=K,
                    max_num_hashes=maxP, num_hash_rounds=R, lsh_num_probes=T, window_size=w,
                    num_global_tokens=G if isinstance(G, int) else 2,
                    global_token_indices=G if isinstance(G, list) else None, causal=causal)
    torch.manual_seed(seed)
    with _nowarn():
        attn = SparseAttention(cfg)
    return attn


@pytest.mark.parametrize("case", PROJ_CASES, ids=lambda c: c[0])
@pytest.mark.parametrize("seed", [0, 1])
def test_fused_projection_graph_exact_tier_matches_oracle(case, seed):
    from ssa_amd import _lib
    (_, B, H, nkv, N, M, d, R, maxP, T, K, w, G, causal, cross) = case
    attn = _proj_module(case, seed)
    attn._fuse_projections = True
    dm = H * d
    gen = torch.Generator().manual_seed(300 + seed)
    # |x . w| <= 1 per term over d_model <= 512 terms: every projection is an
    # integer of magnitude <= 256, exact in bf16; hyperplanes in [-6, 6]
    x = _ints((B, N, dm), -1, 1, gen)
    src = _ints((B, M, dm), -1, 1, gen) if cross else x
    with torch.no_grad():
        for lin in (attn.Wq, attn.Wk, attn.Wv):
            lin.weight.copy_(_ints(tuple(lin.weight.shape), -1, 1, gen, density=0.25))
        rp = _ints(tuple(attn.lsh_builder.rand_proj.shape), -6, 6, gen)
        attn.lsh_builder.rand_proj.copy_(rp)
    q_ref = (x @ attn.Wq.weight.T)
    k_ref = (src @ attn.Wk.weight.T)
    v_ref = (src @ attn.Wv.weight.T)
    assert float(max(q_ref.abs().max(), k_ref.abs().max(), v_ref.abs().max())) <= 256
    attn = attn.to(DEV)
    for p in attn.parameters():
        p.data = p.data.to(torch.bfloat16)
    causal_eff = causal and not cross
    xd = x.to(DEV, torch.bfloat16)
    sd = src.to(DEV, torch.bfloat16) if cross else xd
    with torch.no_grad():
        r = attn._project_build_fused(xd, sd, N, M, causal_eff, cross)
    assert r is not None, "these sizes take the fused path"
    q, k, v, nb32 = r
    torch.cuda.synchronize()
    # the projections: exact integers
    assert torch.equal(q.float().cpu(), q_ref.view(B, N, H, d).transpose(1, 2))
    assert torch.equal(k.float().cpu(), k_ref.view(B, M, nkv, d).transpose(1, 2))
    assert torch.equal(v.float().cpu(), v_ref.view(B, M, nkv, d).transpose(1, 2))
    # the graph: the oracle's on the same q, k
    lb = attn.lsh_builder
    P = lb.compute_effective_p(M, lb.C, maxP)
    glob = attn.glob_builder(M, "cpu")
    ref = oracle.lsh_forward(q.float().cpu().reshape(B * H, N, d).numpy(),
                             k.float().cpu().reshape(B * nkv, M, d).numpy(), rp.numpy(),
                             kv_rep=H // nkv, P=P, T=T, C=lb.C, top_k=attn.lsh_k,
                             causal=causal_eff, glob=glob.numpy())
    win = (np.zeros((N, 0), np.int64) if cross else attn.win_builder(N, M, "cpu").numpy())
    rnb, rva = oracle.merge(win, glob.numpy(), ref["idx"], has_self=not cross, total_k=K)
    exp = np.where(rva, rnb, -1)
    got = nb32.cpu().numpy().reshape(B * H, N, -1)
    np.testing.assert_array_equal(got, exp)
    # and the separate build on the fused q, k gives the same graph
    with torch.no_grad():
        sep = attn._build_graph_ids32(q, k, N, M, B, causal_eff, cross)
    torch.cuda.synchronize()
    np.testing.assert_array_equal(sep.cpu().numpy().reshape(B * H, N, -1), exp)


# ------------------------------------------------------------------ reference vectors
PROJ_FILES = sorted(p for p in (os.path.join(GOLDEN, f) for f in os.listdir(GOLDEN))
                    if os.path.basename(p).startswith("bf16_proj_"))


@pytest.mark.parametrize("path", PROJ_FILES, ids=os.path.basename)
def test_fused_projection_graph_on_reference_vectors(path):
    """The reference's x, weights (cast to bf16 as its own bf16 runs cast
    them) and hyperplanes: the fused q / k / v equal the reference's bf16
    projections and the fused graph equals the reference's neighbours."""
    from ssa_amd import SSAConfig, SparseAttention
    z, m = load_golden(path)
    B, N, M, H, nkv, d = m["B"], m["N"], m["M"], m["H"], m["n_kv"], m["d_head"]
    cfg = SSAConfig(**m["config"])
    with _nowarn():
        attn = SparseAttention(cfg)
    attn._fuse_projections = True
    sd = {k[3:]: torch.from_numpy(z[k]) for k in z.keys() if k.startswith("sd_")}
    attn.load_state_dict(sd, strict=False)
    attn = attn.to(DEV)
    for p in attn.parameters():
        p.data = p.data.to(torch.bfloat16)
    x = torch.from_numpy(z["x"]).to(DEV, torch.bfloat16)
    src = torch.from_numpy(z["kv"]).to(DEV, torch.bfloat16) if m["cross"] else x
    with torch.no_grad():
        r = attn._project_build_fused(x, src, N, M, m["causal"], m["cross"])
    assert r is not None, "these sizes take the fused path"
    q, k, v, nb32 = r
    torch.cuda.synchronize()
    rep = H // nkv
    zq = z["q"]
    zk = z["k"].reshape(B, H, M, d)[:, ::rep]          # the reference's expanded layout
    zv = z["v"].reshape(B, H, M, d)[:, ::rep]
    for name, got, exp in (("q", q, zq), ("k", k, zk), ("v", v, zv)):
        g = got.float().cpu().numpy()
        diff = int((g != exp).sum())
        print(f"{name}: {diff} of {g.size} elements differ from the reference's projection")
        # the reference's CPU bf16 GEMM and this one both accumulate in fp32 and
        # round once; only a sum that lands on a rounding boundary may differ,
        # and then by one ulp
        assert diff <= g.size // 1000
        assert np.all(np.abs(g - exp) <= _bf16_ulp(exp.astype(np.float64)) * 1.0001)
        if name == "q":
            q_same = diff == 0
        if name == "k":
            k_same = diff == 0
    got = nb32.cpu().numpy().reshape(B * H, N, -1)
    exp = np.where(z["valid"], z["neighbors"], -1).reshape(B * H, N, -1)
    if q_same and k_same:
        np.testing.assert_array_equal(got, exp)
    else:
        # the graph of the fused q, k: the oracle's, with the reference's
        # hyperplanes (only rows touched by a differing element may differ from
        # the reference's own)
        lb = attn.lsh_builder
        P = m["p_eff"]
        ref = oracle.lsh_forward(q.float().cpu().reshape(B * H, N, d).numpy(),
                                 k.float().cpu().reshape(B * nkv, M, d).numpy(),
                                 z["sd_lsh_builder.rand_proj"], kv_rep=rep, P=P, T=lb.T,
                                 C=lb.C, top_k=attn.lsh_k, causal=m["causal"],
                                 glob=z["glob"])
        rnb, rva = oracle.merge(z["win"], z["glob"], ref["idx"], has_self=not m["cross"],
                                total_k=attn.K)
        np.testing.assert_array_equal(got, np.where(rva, rnb, -1))


# ------------------------------------------------------------------ module forward
@pytest.mark.parametrize("shape", [
    # d_model, H, n_kv, B, N, K, w, R, T, causal
    (1024, 16, 4, 2, 2048, 128, 16, 8, 1, True),
    (4096, 32, 8, 1, 1024, 128, 16, 8, 0, True),
    (512, 4, 2, 2, 512, 64, 4, 6, 2, False),
], ids=["transformer_layer", "bench_heads", "d128_noncausal"])
def test_fused_forward_matches_separate_projections(shape):
    from ssa_amd import SSAConfig, SparseAttention
    dm, H, nkv, B, N, K, w, R, T, causal = shape
    cfg = SSAConfig(d_model=dm, num_heads=H, num_kv_heads=nkv, num_neighbors=K, window_size=w,
                    num_global_tokens=2, num_hash_rounds=R, lsh_num_probes=T, causal=causal)
    torch.manual_seed(3)
    with _nowarn():
        attn = SparseAttention(cfg)
    attn = attn.to(DEV)
    for p in attn.parameters():
        p.data = p.data.to(torch.bfloat16)
    attn.eval()
    g = torch.Generator(device="cpu").manual_seed(7)
    x = torch.randn(B, N, dm, generator=g).to(DEV, torch.bfloat16)
    M = N
    lb = attn.lsh_builder
    attn._fuse_projections = True
    with torch.no_grad():
        r = attn._project_build_fused(x, x, N, M, causal, False)
        assert r is not None
        q, k, v, nb_f = r
        out_f, st_f = attn(x, return_stats=True)
        attn._fuse_projections = False
        out_s, st_s = attn(x, return_stats=True)
        q_s, k_s, v_s = attn._project(x, x, False)
        nb_s = attn._build_graph_ids32(q, k, N, M, B, causal, False)
        nb_t = attn._build_graph_ids32(q_s, k_s, N, M, B, causal, False)
    torch.cuda.synchronize()
    # the projections: torch's bf16 linear computes the same rounded sums
    for a_, b_ in ((q, q_s), (k, k_s), (v, v_s)):
        same = float((a_ == b_).float().mean())
        assert same > 0.999
    # the graph of the fused q, k, built separately: the hyperplane projections
    # are summed in another order there, so a row may differ only where one of
    # its query's projections lies within the fp32 rounding of zero
    gf, gs = nb_f.cpu().numpy(), nb_s.cpu().numpy()
    diff_rows = int((gf != gs).any(-1).sum())
    rows = gf.shape[0] * gf.shape[1] * gf.shape[2]
    print(f"{diff_rows} of {rows} rows differ between the fused and the separate build")
    assert diff_rows <= max(2, rows // 10000)
    assert st_f["padding_fraction"] == pytest.approx(st_s["padding_fraction"], abs=1e-3)
    # the forward outputs agree on every token whose graph rows (all heads) the
    # separate path, on torch's projections, built alike
    same_tok = (nb_f.cpu() == nb_t.cpu()).all(-1).all(1).numpy()       # (B, N)
    assert same_tok.mean() > 0.99
    of = out_f.float().cpu().numpy()[same_tok]
    os_ = out_s.float().cpu().numpy()[same_tok]
    assert row_rel_err(of, os_) < 2e-2
