"""GPU parity of the HIP kernels against the oracle (and the golden vectors).

Bar: neighbor ids / valid masks / permutations bit-exact; attention output
within 1e-5 relative (fp32) and 2e-2 (bf16/fp16), per query row: the row's
largest deviation over the row's largest reference magnitude.

Two input tiers (sparse_attention.py cannot fix fp32 summation order):
* exact-arithmetic inputs (small integers): every fp32 projection and score is
  exact in any order, so the whole graph must match the oracle bit for bit,
  including the many rows whose kk-th LSH score is tied (small integers tie
  often): those are resolved by the GPU's replay of the reference's
  nth_element / sort, and the LSH lists must come out in the same order;
* the reference's own vectors with the reference's fp32 projections injected:
  neighbor lists must match the reference's.
"""
import os

import numpy as np
import pytest
import torch

import oracle
from conftest import golden_files, has_gpu, load_golden, row_rel_err

pytestmark = [pytest.mark.gpu,
              pytest.mark.skipif(not has_gpu(), reason="needs a ROCm GPU")]

DEV = "cuda"
REL = {torch.float32: 1e-5, torch.bfloat16: 2e-2, torch.float16: 2e-2}
MODE = {torch.float32: 0, torch.bfloat16: 1, torch.float16: 2}


def _ints(shape, lo, hi, gen):
    return torch.randint(lo, hi + 1, shape, generator=gen).float()


# ------------------------------------------------------------------ bucket sort
# rows beyond 32768 keys take the sort with 32-bit positions and the row in
# the workspace (40001: odd, so rows start at unaligned key offsets)
@pytest.mark.parametrize("rows,n,P", [(3, 17, 1), (2, 1024, 1), (4, 4096, 3), (2, 8192, 4),
                                      (2, 16384, 6), (1, 32768, 5), (2, 300, 12), (5, 16, 2),
                                      (2, 5, 1), (2, 40001, 7), (2, 65536, 5), (1, 131072, 9),
                                      (1, 524288, 11), (1, 1048576, 12)])
@pytest.mark.parametrize("dist", ["uniform", "skewed", "sorted", "reversed", "constant"])
def test_bucket_sort_is_torch_sort(rows, n, P, dist):
    from ssa_amd import _lib
    rng = np.random.default_rng(rows * 1000 + n + P)
    if dist == "uniform":
        k = rng.integers(0, 2 ** P, (rows, n))
    elif dist == "skewed":
        k = np.minimum(rng.geometric(0.3, (rows, n)) - 1, 2 ** P - 1)
    elif dist == "sorted":
        k = np.sort(rng.integers(0, 2 ** P, (rows, n)), axis=-1)
    elif dist == "reversed":
        k = np.sort(rng.integers(0, 2 ** P, (rows, n)), axis=-1)[:, ::-1]
    else:
        k = np.full((rows, n), 2 ** P - 1)
    k = torch.from_numpy(np.ascontiguousarray(k).astype(np.int64))
    perm, bstart, bsize = _lib.bucket_sort(k.to(DEV), P)
    ref = torch.sort(k, dim=-1)[1]
    assert torch.equal(perm.cpu().long(), ref)
    cnt = torch.stack([torch.bincount(k[r], minlength=2 ** P) for r in range(rows)])
    assert torch.equal(bsize.cpu().long(), cnt)
    starts = torch.cumsum(cnt, -1) - cnt
    assert torch.equal(bstart.cpu().long(), starts)


# ------------------------------------------------------------------ graph, exact tier
GRAPH_CASES = [
    # name, B, H, n_kv, N, M, d, R, maxP, T, K, w, G(explicit or count), causal, cross
    ("self_small", 1, 2, 2, 64, 64, 16, 2, 3, 0, 32, 4, 2, False, False),
    ("causal_gqa", 2, 4, 2, 96, 96, 16, 3, 4, 0, 24, 3, 2, True, False),
    ("mqa_causal_probes", 1, 4, 1, 200, 200, 32, 2, 6, 3, 32, 2, 1, True, False),
    ("cross_probes", 2, 4, 2, 50, 130, 16, 3, 4, 2, 24, 4, 2, False, True),
    ("explicit_globals", 1, 2, 2, 64, 64, 16, 3, 3, 1, 24, 2, [0, 5, 100], True, False),
    ("tiny_n", 1, 2, 2, 8, 8, 16, 2, 6, 12, 32, 2, 1, False, False),
    ("oversize_window", 1, 2, 2, 48, 48, 16, 2, 3, 0, 16, 16, 2, False, False),
    ("mid_r8", 1, 2, 2, 512, 512, 64, 8, 12, 0, 64, 8, 2, True, False),
    ("big_bucket_bits", 1, 2, 1, 1024, 1024, 32, 2, 12, 1, 40, 2, 2, False, False),
    # head dims that are not powers of two (the next instance's kernels, the
    # elements past d zero)
    ("head_dim_96", 1, 4, 2, 160, 160, 96, 3, 4, 1, 32, 4, 2, True, False),
    ("head_dim_80_cross", 2, 2, 1, 60, 100, 80, 2, 4, 1, 24, 4, 2, False, True),
    ("head_dim_112", 1, 2, 2, 128, 128, 112, 2, 4, 0, 24, 3, 2, True, False),
    ("head_dim_48", 1, 2, 1, 96, 96, 48, 2, 3, 0, 20, 2, 1, False, False),
    # the smallest and the largest matrix-core rescore instances
    ("head_dim_8", 1, 2, 2, 80, 80, 8, 2, 3, 0, 16, 2, 1, True, False),
    ("head_dim_128", 1, 2, 1, 256, 256, 128, 2, 4, 1, 32, 4, 2, True, False),
    # more global tokens than a wavefront holds: the empty-bucket list glob ++ 0
    # taken 64 entries at a time (101 of them, and 100 explicit ones over C=112)
    ("many_globals", 1, 2, 2, 256, 256, 16, 3, 4, 1, 160, 4, 100, True, False),
    ("many_globals_cross", 1, 2, 1, 80, 300, 16, 2, 4, 1, 128, 4, list(range(0, 300, 3)),
     False, True),
    # head dims beyond 256: the 512 instances, elements past d zero
    ("head_dim_320", 1, 2, 1, 96, 96, 320, 2, 3, 0, 24, 2, 2, True, False),
    ("head_dim_512_cross", 1, 2, 2, 40, 70, 512, 2, 3, 1, 20, 2, 1, False, True),
    # beyond 512: the 1024 instances
    ("head_dim_640", 1, 2, 1, 64, 64, 640, 2, 3, 0, 20, 2, 1, True, False),
    ("head_dim_1024_cross", 1, 2, 2, 40, 70, 1024, 2, 3, 1, 20, 2, 1, False, True),
    # more than 2048 (head, round, id set) instances in one head chunk: the
    # tiles ordered by a launch of their own instead of inside the scatter
    ("many_instances", 10, 32, 8, 32, 32, 8, 8, 3, 0, 16, 2, 1, True, False),
    # head dims the kernels do not take (neither a power of two nor whole
    # 16-byte pieces: 6 in every type, 20 in bf16 / f16, 125): run zero-padded
    ("head_dim_6", 1, 2, 1, 64, 64, 6, 2, 3, 0, 20, 2, 1, True, False),
    ("head_dim_3", 1, 2, 1, 48, 48, 3, 2, 3, 1, 20, 2, 1, True, False),
    ("head_dim_20", 1, 2, 2, 80, 80, 20, 2, 3, 1, 24, 2, 1, True, False),
    ("head_dim_125_cross", 1, 2, 1, 40, 70, 125, 2, 3, 1, 20, 2, 1, False, True),
    # key lengths beyond 32768: the bucket sort with 32-bit positions, the
    # cut entries' 16-bit fields read unsigned
    ("long_keys_causal", 1, 1, 1, 65536, 65536, 16, 2, 12, 0, 32, 2, 2, True, False),
    ("long_keys_cross", 1, 2, 1, 512, 40000, 16, 2, 6, 1, 32, 2, 2, False, True),
    # key ids beyond 16 bits: the cut entries' fields split at the width of C
    # (lists of 224 members ranked through the bitmap and the cut's rank table),
    # 7-bit slots in the short-list sort, 32-bit ids in the per-wave replay, and
    # (at 262,144 keys) two select rows per workgroup
    ("keys_131072_causal", 1, 1, 1, 131072, 131072, 16, 2, 12, 0, 64, 2, 2, True, False),
    ("keys_100003_cross_probes", 1, 2, 1, 300, 100003, 16, 2, 12, 1, 32, 2, 2, False, True),
    ("keys_262144_cross", 1, 2, 2, 200, 262144, 16, 2, 12, 0, 64, 2, 2, False, True),
]


def _graph_case(case, seed, dtype=torch.float32, lsh_only=False):
    from ssa_amd import SSAConfig, SparseAttention
    (_, B, H, nkv, N, M, d, R, maxP, T, K, w, G, causal, cross) = case
    cfg = SSAConfig(d_model=H * d, num_heads=H, num_kv_heads=nkv, num_neighbors=K,
                    max_num_hashes=maxP, num_hash_rounds=R, lsh_num_probes=T, window_size=w,
                    num_global_tokens=G if isinstance(G, int) else 2,
                    global_token_indices=G if isinstance(G, list) else None, causal=causal)
    torch.manual_seed(seed)
    with _nowarn():
        attn = SparseAttention(cfg)
    gen = torch.Generator().manual_seed(100 + seed)
    q = _ints((B, H, N, d), -6, 6, gen)
    k = _ints((B, nkv, M, d), -6, 6, gen)
    rp = _ints(tuple(attn.lsh_builder.rand_proj.shape), -6, 6, gen)
    attn.lsh_builder.rand_proj.copy_(rp)
    attn = attn.to(DEV)
    P = attn.lsh_builder.compute_effective_p(M, attn.lsh_builder.C, maxP)
    glob = attn.glob_builder(M, "cpu")
    qd, kd = q.to(DEV, dtype), k.to(DEV, dtype)
    with torch.no_grad():
        if lsh_only:
            got = attn.lsh_builder(qd, kd, attn.lsh_k, causal and not cross, glob.to(DEV))
            got_v = None
        else:
            got, got_v = attn.build_graph(qd, kd, N, M, B, DEV, causal and not cross, cross)
    torch.cuda.synchronize()
    ref = oracle.lsh_forward(q.reshape(B * H, N, d).numpy(), k.reshape(B * nkv, M, d).numpy(),
                             rp.numpy(), kv_rep=H // nkv, P=P, T=T, C=attn.lsh_builder.C,
                             top_k=attn.lsh_k, causal=causal and not cross, glob=glob.numpy())
    return attn, got, got_v, ref, (B, H, N, M, K, w, cross, causal, glob)


class _nowarn:
    def __enter__(self):
        import warnings
        self.c = warnings.catch_warnings()
        self.c.__enter__()
        warnings.simplefilter("ignore")

    def __exit__(self, *a):
        self.c.__exit__(*a)


@pytest.mark.parametrize("case", GRAPH_CASES, ids=lambda c: c[0])
@pytest.mark.parametrize("seed", [0, 1])
def test_full_graph_exact_tier_matches_oracle(case, seed):
    attn, got, got_v, ref, (B, H, N, M, K, w, cross, causal, glob) = _graph_case(case, seed)
    win = (np.zeros((N, 0), np.int64) if cross
           else attn.win_builder(N, M, "cpu").numpy())
    rnb, rva = oracle.merge(win, glob.numpy(), ref["idx"], has_self=not cross, total_k=K)
    g_nb = got.cpu().numpy().reshape(B * H, N, -1)
    g_va = got_v.cpu().numpy().reshape(B * H, N, -1)
    assert g_nb.shape == rnb.shape
    np.testing.assert_array_equal(g_nb, rnb)
    np.testing.assert_array_equal(g_va, rva)


@pytest.mark.parametrize("case", GRAPH_CASES[:5], ids=lambda c: c[0])
def test_lsh_builder_exact_tier_matches_oracle(case):
    attn, got, _, ref, (B, H, N, M, K, w, cross, causal, glob) = _graph_case(case, 3,
                                                                            lsh_only=True)
    g = got.cpu().numpy().reshape(B * H, N, -1)
    r = ref["idx"]
    assert g.shape == r.shape
    # same lists in the same order, tied rows included
    print(f"  {case[0]}: {ref['n_ties']} rows with a tied kk-th score", flush=True)
    np.testing.assert_array_equal(g, r)


# num_neighbors 1400: kk = 1388, so best ++ chunk spans 6,940 slots; about
# 120 rows tie at the kk-th score (small integers), which the workgroup
# replay takes with two waves' arrays in LDS
HUGE_K = ("huge_k_replay_workspace", 1, 1, 1, 2048, 2048, 16, 2, 3, 0, 1400, 4, 2, True, False)
# num_neighbors 1700 over 4,096 keys: kk = 1688 and 8,440 slots, which no
# longer fit LDS twice; 1,634 tied rows, more than the workgroup replay takes,
# so the per-wave replay runs from its workspace region
HUGE_K_WAVE = ("huge_k_per_wave_replay_workspace", 1, 1, 1, 4096, 4096, 16, 2, 3, 0, 1700, 4, 2,
               True, False)
# the same replay with 32-bit key ids: 4,096 queries over 70,000 keys
# (cross-attention), kk = 1698, cut fields of 13 + 17 bits
HUGE_K_WAVE_WIDE = ("huge_k_per_wave_replay_wide_ids", 1, 1, 1, 4096, 70000, 16, 2, 3, 0, 1700, 4,
                    2, False, True)


def test_full_graph_exact_tier_huge_k_replay_outside_lds():
    attn, got, got_v, ref, (B, H, N, M, K, w, cross, causal, glob) = _graph_case(HUGE_K, 0)
    print(f"  huge K: {ref['n_ties']} rows with a tied kk-th score", flush=True)
    assert ref["n_ties"] > 0
    win = attn.win_builder(N, M, "cpu").numpy()
    rnb, rva = oracle.merge(win, glob.numpy(), ref["idx"], has_self=True, total_k=K)
    np.testing.assert_array_equal(got.cpu().numpy().reshape(B * H, N, -1), rnb)
    np.testing.assert_array_equal(got_v.cpu().numpy().reshape(B * H, N, -1), rva)


def test_full_graph_exact_tier_huge_k_per_wave_replay_workspace():
    attn, got, got_v, ref, (B, H, N, M, K, w, cross, causal, glob) = _graph_case(HUGE_K_WAVE, 0)
    print(f"  huge K, per-wave replay: {ref['n_ties']} rows with a tied kk-th score", flush=True)
    assert ref["n_ties"] > 1024
    win = attn.win_builder(N, M, "cpu").numpy()
    rnb, rva = oracle.merge(win, glob.numpy(), ref["idx"], has_self=True, total_k=K)
    np.testing.assert_array_equal(got.cpu().numpy().reshape(B * H, N, -1), rnb)
    np.testing.assert_array_equal(got_v.cpu().numpy().reshape(B * H, N, -1), rva)


def test_full_graph_exact_tier_huge_k_per_wave_replay_wide_ids():
    attn, got, got_v, ref, (B, H, N, M, K, w, cross, causal, glob) = _graph_case(HUGE_K_WAVE_WIDE, 0)
    print(f"  huge K over {M} keys, per-wave replay: {ref['n_ties']} rows with a tied kk-th score",
          flush=True)
    assert ref["n_ties"] > 1024
    win = np.zeros((N, 0), np.int64)
    rnb, rva = oracle.merge(win, glob.numpy(), ref["idx"], has_self=False, total_k=K)
    np.testing.assert_array_equal(got.cpu().numpy().reshape(B * H, N, -1), rnb)
    np.testing.assert_array_equal(got_v.cpu().numpy().reshape(B * H, N, -1), rva)


def test_lsh_builder_exact_tier_huge_k_replay_outside_lds():
    attn, got, _, ref, (B, H, N, M, K, w, cross, causal, glob) = _graph_case(HUGE_K, 1,
                                                                            lsh_only=True)
    np.testing.assert_array_equal(got.cpu().numpy().reshape(B * H, N, -1), ref["idx"])


def test_graph_build_captured_in_a_graph_replays_the_eager_graph():
    """A build captured into a HIP graph (one stream under capture) gives the
    eager graph on every replay, with eager builds in between."""
    from ssa_amd import SSAConfig, SparseAttention
    torch.manual_seed(5)
    cfg = SSAConfig(d_model=256, num_heads=4, num_kv_heads=2, num_neighbors=48, window_size=4,
                    num_global_tokens=2, num_hash_rounds=4, lsh_num_probes=1, causal=True)
    with _nowarn():
        attn = SparseAttention(cfg).to(DEV).eval()
    x = torch.randn(2, 300, 256, device=DEV)
    with torch.no_grad():
        q, k, _ = attn._project(x, x, False)
        eager = attn._build_graph_ids32(q, k, 300, 300, 2, True, False)
        side = torch.cuda.Stream()
        side.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(side):
            attn._build_graph_ids32(q, k, 300, 300, 2, True, False)
        torch.cuda.current_stream().wait_stream(side)
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g):
            out = attn._build_graph_ids32(q, k, 300, 300, 2, True, False)
        for _ in range(3):
            out.fill_(7)
            g.replay()
            torch.cuda.synchronize()
            assert torch.equal(out, eager)
            again = attn._build_graph_ids32(q, k, 300, 300, 2, True, False)
            torch.cuda.synchronize()
            assert torch.equal(again, eager)


# Tied-row counts on either side of the replay's two paths (a 256-CU device):
# up to four tied rows per workgroup take the workgroup replay (several rows
# per workgroup past 256), more take the per-wave replay
MANY_TIES = [
    # 428 tied rows
    ("many_ties_workgroup_replay", 1, 4, 2, 512, 512, 16, 4, 6, 1, 32, 4, 2, True, False, 256, 1024),
    # 1339 tied rows
    ("many_ties_per_wave_replay", 2, 8, 2, 384, 384, 8, 3, 5, 1, 24, 4, 2, True, False, 1024, 6144),
]


@pytest.mark.parametrize("case", MANY_TIES, ids=lambda c: c[0])
def test_graph_exact_tier_many_tied_rows(case):
    lo, hi = case[-2:]
    attn, got, got_v, ref, (B, H, N, M, K, w, cross, causal, glob) = _graph_case(case[:-2], 0)
    print(f"  {case[0]}: {ref['n_ties']} rows with a tied kk-th score", flush=True)
    assert lo < ref["n_ties"] <= hi
    win = attn.win_builder(N, M, "cpu").numpy()
    rnb, rva = oracle.merge(win, glob.numpy(), ref["idx"], has_self=True, total_k=K)
    np.testing.assert_array_equal(got.cpu().numpy().reshape(B * H, N, -1), rnb)
    np.testing.assert_array_equal(got_v.cpu().numpy().reshape(B * H, N, -1), rva)
    _, got, _, ref, _ = _graph_case(case[:-2], 0, lsh_only=True)
    np.testing.assert_array_equal(got.cpu().numpy().reshape(B * H, N, -1), ref["idx"])


@pytest.mark.parametrize("case", GRAPH_CASES, ids=lambda c: c[0])
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16], ids=["bf16", "f16"])
def test_graph_16bit_inputs_exact_tier(case, dtype):
    """bf16 and fp16 q/k holding small integers are exact: same graph as fp32
    (the matrix-core rescore of either 16-bit type, aux and exact-key paths,
    every head-dim instance)."""
    attn, got, got_v, ref, (B, H, N, M, K, w, cross, causal, glob) = _graph_case(
        case, 5, dtype=dtype)
    win = (np.zeros((N, 0), np.int64) if cross else attn.win_builder(N, M, "cpu").numpy())
    rnb, rva = oracle.merge(win, glob.numpy(), ref["idx"], has_self=not cross, total_k=K)
    np.testing.assert_array_equal(got.cpu().numpy().reshape(B * H, N, -1), rnb)
    np.testing.assert_array_equal(got_v.cpu().numpy().reshape(B * H, N, -1), rva)


# ------------------------------------------------------------------ graph, reference vectors
@pytest.mark.parametrize("path", golden_files(), ids=os.path.basename)
def test_graph_on_reference_vectors_with_injected_projections(path):
    from ssa_amd import SSAConfig, SparseAttention
    z, m = load_golden(path)
    B, N, M, H, d = m["B"], m["N"], m["M"], m["H"], m["d_head"]
    cfg = SSAConfig(**m["config"])
    with _nowarn():
        attn = SparseAttention(cfg)
    attn.lsh_builder.rand_proj.copy_(torch.from_numpy(z["sd_lsh_builder.rand_proj"]))
    attn = attn.to(DEV)
    dt = torch.bfloat16 if m["dtype"] == "bfloat16" else torch.float32
    q = torch.from_numpy(z["q"]).to(DEV, dt)
    k_exp = torch.from_numpy(z["k"]).to(DEV, dt)            # reference layout (B, H, M, d)
    R, P = z["sd_lsh_builder.rand_proj"].shape[0], m["p_eff"]
    qp = torch.from_numpy(z["qproj"]).reshape(B * H, R, N, P).to(DEV)
    kp = torch.from_numpy(z["kproj"]).reshape(B * H, R, M, P).to(DEV)
    with torch.no_grad():
        lsh = attn.lsh_builder(q, k_exp, attn.lsh_k, m["causal"],
                               torch.from_numpy(z["glob"]).to(DEV), _proj=(qp, kp))
        nb, va = attn.build_graph(q, k_exp, N, M, B, DEV, m["causal"], m["cross"],
                                  _proj=(qp, kp))
    torch.cuda.synchronize()
    # the reference's lists, in its order (ties resolved by the replay)
    g_l = lsh.cpu().numpy().reshape(B * H, N, -1)
    z_l = z["lsh"].reshape(B * H, N, -1)
    np.testing.assert_array_equal(g_l, z_l)
    g_nb = nb.cpu().numpy().reshape(B * H, N, -1)
    z_nb = z["neighbors"].reshape(B * H, N, -1)
    np.testing.assert_array_equal(g_nb, z_nb)
    np.testing.assert_array_equal(va.cpu().numpy().reshape(B * H, N, -1),
                                  z["valid"].reshape(B * H, N, -1))


# ------------------------------------------------------------------ apply
APPLY_CASES = [
    # B, H, n_kv, N, M, d, K
    (1, 2, 2, 33, 40, 16, 12),
    (2, 4, 2, 64, 64, 64, 32),
    (1, 8, 1, 50, 70, 128, 128),
    (1, 2, 1, 17, 300, 128, 256),
    (1, 2, 2, 9, 9, 8, 5),
    (1, 2, 2, 20, 30, 32, 64),
    (1, 2, 1, 10, 40, 256, 24),
    (1, 4, 2, 12, 20, 4, 10),
    (1, 1, 1, 3, 500, 128, 2500),
    (1, 4, 2, 40, 50, 96, 24),
    (1, 2, 1, 30, 60, 80, 33),
    (1, 2, 2, 20, 30, 112, 16),
    (2, 2, 2, 9, 15, 48, 12),
    (1, 2, 1, 11, 40, 200, 20),
    (1, 2, 1, 9, 40, 320, 24),
    (1, 4, 2, 7, 30, 512, 16),
    (1, 2, 1, 7, 30, 640, 12),
    (1, 2, 2, 5, 20, 1024, 10),
    (1, 2, 1, 9, 30, 6, 12),
    (1, 2, 1, 9, 30, 2, 12),
    (1, 2, 2, 8, 25, 3, 10),
    (1, 2, 2, 8, 25, 20, 10),
    (1, 2, 1, 7, 30, 125, 12),
]


def _apply_inputs(case, dtype, seed=0):
    B, H, nkv, N, M, d, K = case
    g = torch.Generator().manual_seed(seed)
    q = torch.randn(B, H, N, d, generator=g).to(dtype)
    k = torch.randn(B, nkv, M, d, generator=g).to(dtype)
    v = torch.randn(B, nkv, M, d, generator=g).to(dtype)
    nb = torch.randint(0, M, (B, H, N, K), generator=g)
    va = torch.rand(B, H, N, K, generator=g) > 0.3
    va[..., 0] = True
    return q, k, v, nb, va


@pytest.mark.parametrize("case", APPLY_CASES)
@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16, torch.float16])
@pytest.mark.parametrize("fp32w", [False, True])
def test_apply_matches_oracle(case, dtype, fp32w):
    from ssa_amd import sparse_gather_attention
    B, H, nkv, N, M, d, K = case
    q, k, v, nb, va = _apply_inputs(case, dtype)
    scale = d ** -0.5
    with torch.no_grad():
        out = sparse_gather_attention(q.to(DEV), k.to(DEV), v.to(DEV), nb.to(DEV), scale,
                                      valid=va.to(DEV), fp32_attn_weights=fp32w)
    torch.cuda.synchronize()
    ref = oracle.apply(q.float().reshape(B * H, N, d).numpy(),
                       k.float().reshape(B * nkv, M, d).numpy(),
                       v.float().reshape(B * nkv, M, d).numpy(), nb.reshape(B * H, N, K).numpy(),
                       va.reshape(B * H, N, K).numpy(), kv_rep=H // nkv, scale=scale,
                       mode=MODE[dtype], fp32_attn_weights=fp32w)
    ref = torch.from_numpy(ref).to(dtype).float().numpy()   # reference output dtype
    got = out.float().cpu().numpy().reshape(B * H, N, d)
    err = row_rel_err(got, ref)
    assert err <= REL[dtype], err


# rows of more slots than LDS holds (K > 4096): the kernels that compute the
# scores again in each pass instead of keeping them
LONG_CASES = [(1, 2, 1, 6, 12000, 64, 5000), (1, 2, 2, 5, 9000, 128, 8191),
              (1, 1, 1, 3, 20000, 96, 16384)]


@pytest.mark.parametrize("case", LONG_CASES, ids=lambda c: f"K{c[-1]}_d{c[5]}")
@pytest.mark.parametrize("dtype,fp32w", [(torch.float32, False), (torch.bfloat16, False),
                                         (torch.bfloat16, True), (torch.float16, False)])
def test_apply_long_rows_match_oracle(case, dtype, fp32w):
    test_apply_matches_oracle(case, dtype, fp32w)


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("det", [False, True], ids=["atomic", "deterministic"])
def test_apply_long_rows_backward_matches_autograd(dtype, det):
    """K = 5000 slots per row (beyond LDS), GQA 4 / 2 heads: every row of
    dq / dk / dv against float64 autograd, both backward kernels."""
    from ssa_amd import sparse_gather_attention
    B, H, nkv, N, M, d, K = 1, 4, 2, 8, 6000, 64, 5000
    q, k, v, nb, va = _apply_inputs((B, H, nkv, N, M, d, K), dtype, 13)
    g = torch.Generator().manual_seed(14)
    dout = torch.randn(B, H, N, d, generator=g)
    prev = torch.are_deterministic_algorithms_enabled()
    try:
        torch.use_deterministic_algorithms(det)
        qd, kd, vd = (t.to(DEV).requires_grad_(True) for t in (q, k, v))
        out = sparse_gather_attention(qd, kd, vd, nb.to(DEV), d ** -0.5, valid=va.to(DEV))
        out.backward(dout.to(DEV, dtype))
        torch.cuda.synchronize()
    finally:
        torch.use_deterministic_algorithms(prev)
    qr, kr, vr = (t.double().requires_grad_(True) for t in (q, k, v))
    ke = kr.repeat_interleave(H // nkv, 1)
    ve = vr.repeat_interleave(H // nkv, 1)
    idx = nb.unsqueeze(-1).expand(B, H, N, K, d)
    kg = torch.gather(ke.unsqueeze(2).expand(B, H, N, M, d), 3, idx)
    vg = torch.gather(ve.unsqueeze(2).expand(B, H, N, M, d), 3, idx)
    s = (qr.unsqueeze(3) * kg).sum(-1) * d ** -0.5
    p = torch.softmax(s.masked_fill(~va, float("-inf")), -1)
    o = (p.unsqueeze(-1) * vg).sum(3)
    o.backward(dout.to(dtype).double())       # the upstream gradient the device got
    for name, got, exp in [("dq", qd.grad, qr.grad), ("dk", kd.grad, kr.grad),
                           ("dv", vd.grad, vr.grad)]:
        _check_grad_rows(name, got, exp, dtype)


def test_apply_expanded_kv_equals_grouped_kv():
    from ssa_amd import sparse_gather_attention
    case = (1, 4, 2, 40, 40, 64, 24)
    q, k, v, nb, va = _apply_inputs(case, torch.float32, 3)
    a = [t.to(DEV) for t in (q, k, v, nb, va)]
    with torch.no_grad():
        o1 = sparse_gather_attention(a[0], a[1], a[2], a[3], 0.125, valid=a[4])
        o2 = sparse_gather_attention(a[0], a[1].repeat_interleave(2, 1),
                                     a[2].repeat_interleave(2, 1), a[3], 0.125, valid=a[4])
    assert torch.equal(o1, o2)


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("ids32", [False, True])
def test_apply_counts_invalid_slots_per_row(dtype, ids32):
    """row_invalid: each row's slots the graph marks invalid (valid false, or
    a negative int32 id): the reference's padding statistic, ~valid summed
    per row (sparse_attention.py:1508); an out-of-range or negative int64 id
    marked valid is skipped by the attention but not counted.  Same output
    as without it."""
    from ssa_amd import _lib
    case = (2, 4, 2, 50, 60, 64, 37)
    q, k, v, nb, va = _apply_inputs(case, dtype, 5)
    nb[0, 1, 3, 4] = 60            # out of range
    nb[1, 2, 7, 9] = -5            # negative
    a = [t.to(DEV) for t in (q, k, v)]
    if ids32:
        ids = torch.where(va, nb, torch.full_like(nb, -1)).to(torch.int32).to(DEV)
        nbd, vad = ids, None
        bad = ids < 0
    else:
        nbd, vad = nb.to(DEV), va.to(DEV)
        bad = ~vad
    rows = torch.full((2 * 4 * 50,), -7, dtype=torch.int32, device=DEV)
    with torch.no_grad():
        o1 = _lib.gather_attention_fwd(a[0], a[1], a[2], nbd, vad, 0.125, row_invalid=rows)
        o2 = _lib.gather_attention_fwd(a[0], a[1], a[2], nbd, vad, 0.125)
    torch.cuda.synchronize()
    assert torch.equal(o1, o2)
    assert torch.equal(rows.cpu(), bad.reshape(-1, 37).sum(-1).to(torch.int32).cpu())


def test_module_padding_fraction_is_the_mask_mean():
    """SparseAttention's padding_fraction (from the per-row counts) equals the
    reference's (~valid).float().mean() on the graph it built."""
    from ssa_amd import SSAConfig, SparseAttention
    torch.manual_seed(0)
    cfg = SSAConfig(d_model=64, num_heads=4, num_kv_heads=2, num_neighbors=40, window_size=3,
                    num_global_tokens=2, num_hash_rounds=2, causal=True)
    with _nowarn():
        attn = SparseAttention(cfg).to(DEV).eval()
    x = torch.randn(2, 96, 64, device=DEV)
    with torch.no_grad():
        _, st = attn(x, return_stats=True)
        q, k, _ = attn._project(x, x, False)
        _, valid = attn.build_graph(q, k, 96, 96, 2, x.device, True, False)
    ref = float((~valid).cpu().float().mean())
    assert st["padding_fraction"] == ref


def test_apply_fp32_head_dim_12_matches_oracle():
    """fp32 takes head dims in whole 4-element pieces (12: the 16 instance)."""
    from ssa_amd import sparse_gather_attention
    case = (1, 2, 1, 17, 25, 12, 9)
    B, H, nkv, N, M, d, K = case
    q, k, v, nb, va = _apply_inputs(case, torch.float32, 2)
    with torch.no_grad():
        out = sparse_gather_attention(q.to(DEV), k.to(DEV), v.to(DEV), nb.to(DEV), d ** -0.5,
                                      valid=va.to(DEV))
    ref = oracle.apply(q.reshape(B * H, N, d).numpy(), k.reshape(B * nkv, M, d).numpy(),
                       v.reshape(B * nkv, M, d).numpy(), nb.reshape(B * H, N, K).numpy(),
                       va.reshape(B * H, N, K).numpy(), kv_rep=H // nkv, scale=d ** -0.5, mode=0)
    assert row_rel_err(out.cpu().numpy().reshape(B * H, N, d), ref) <= REL[torch.float32]


# per-row bar of the gradients: each row of dq (a query) or of dk / dv (a key)
# against the row's own largest reference magnitude, like the forward; a row
# no query reaches must come out exactly zero.  The reference takes the
# upstream gradient the device got (rounded to the dtype); 16-bit gradients
# are rounded once more on the way out (2^-8 relative at most).  fp32: 5e-5
# (about 400 ulps): a key row reached by few queries can sum nearly
# cancelling terms, whose fp32 rounding then stands out against the row's
# largest value (1.2e-5 in the backward shape sweep)
GRAD_REL = {torch.float32: 5e-5, torch.bfloat16: 1e-2, torch.float16: 1e-2}


def _check_grad_rows(name, got, exp, dtype):
    g = got.detach().double().cpu().numpy()
    r = exp.detach().double().cpu().numpy()
    g2, r2 = g.reshape(-1, g.shape[-1]), r.reshape(-1, r.shape[-1])
    zero = np.abs(r2).max(-1) == 0
    assert not np.abs(g2[zero]).any(), f"{name}: gradient in a row no query reaches"
    e = row_rel_err(g2[~zero], r2[~zero]) if (~zero).any() else 0.0
    print(f"  {name}: {int((~zero).sum())} rows, worst row error {e:.2e}", flush=True)
    assert e <= GRAD_REL[dtype], (name, e)


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("case", [(1, 4, 2, 24, 30, 32, 16), (1, 4, 2, 24, 30, 96, 16),
                                  (1, 2, 1, 10, 30, 320, 12), (1, 2, 2, 6, 20, 512, 8),
                                  (1, 2, 1, 5, 20, 1024, 8), (1, 2, 1, 6, 20, 125, 8)],
                         ids=["d32", "d96", "d320", "d512", "d1024", "d125"])
def test_apply_backward_matches_autograd_reference(dtype, case):
    from ssa_amd import sparse_gather_attention
    B, H, nkv, N, M, d, K = case
    q, k, v, nb, va = _apply_inputs(case, dtype, 5)
    g = torch.Generator().manual_seed(9)
    dout = torch.randn(B, H, N, d, generator=g)
    qd, kd, vd = (t.to(DEV).requires_grad_(True) for t in (q, k, v))
    out = sparse_gather_attention(qd, kd, vd, nb.to(DEV), d ** -0.5, valid=va.to(DEV))
    out.backward(dout.to(DEV, dtype))
    # float64 CPU reference of the same function (gather, masked softmax, P.V)
    qr, kr, vr = (t.double().requires_grad_(True) for t in (q, k, v))
    ke = kr.repeat_interleave(H // nkv, 1)
    ve = vr.repeat_interleave(H // nkv, 1)
    idx = nb.unsqueeze(-1).expand(B, H, N, K, d)
    kg = torch.gather(ke.unsqueeze(2).expand(B, H, N, M, d), 3, idx)
    vg = torch.gather(ve.unsqueeze(2).expand(B, H, N, M, d), 3, idx)
    s = (qr.unsqueeze(3) * kg).sum(-1) * d ** -0.5
    s = s.masked_fill(~va, float("-inf"))
    p = torch.softmax(s, -1)
    o = (p.unsqueeze(-1) * vg).sum(3)
    o.backward(dout.to(dtype).double())       # the upstream gradient the device got
    for name, got, exp in [("dq", qd.grad, qr.grad), ("dk", kd.grad, kr.grad),
                           ("dv", vd.grad, vr.grad)]:
        _check_grad_rows(name, got, exp, dtype)


# ------------------------------------------------------------------ dropout
@pytest.mark.parametrize("dtype,fp32w", [(torch.float32, False), (torch.bfloat16, False),
                                         (torch.bfloat16, True)])
def test_dropout_keep_rate_scaling_and_backward(dtype, fp32w):
    """Training-mode dropout on the attention weights (sparse_attention.py:
    1193-1194) over 1,048,576 slots.  V rows are one-hot, so each output
    element is the weight of one key: the output shows every slot's weight
    with and without dropout.
    * the kept fraction is within 5 sigma of 1 - p (overall and per slot);
    * a dropped weight is 0 and a kept one is the weight times 1 / (1 - p),
      both in the weights' dtype (torch's dropout multiplies by a noise
      tensor of that dtype holding 1 / (1 - p));
    * the backward of the same call (same seed) matches float64 autograd of
      the forward with the mask read off its output."""
    from ssa_amd import sparse_gather_attention
    B, H, N, M, d, K = 1, 2, 4096, 128, 128, 128
    p = 0.25
    scale = d ** -0.5
    g = torch.Generator().manual_seed(11)
    q = torch.randn(B, H, N, d, generator=g).to(dtype)
    k = torch.randn(B, H, M, d, generator=g).to(dtype)
    v = torch.eye(M, d).expand(B, H, M, d).contiguous().to(dtype)
    nb = torch.argsort(torch.rand(B, H, N, K, generator=g), -1)   # every key once per row
    qd, kd, vd, nbd = (t.to(DEV) for t in (q, k, v, nb))
    with torch.no_grad():
        w0 = sparse_gather_attention(qd, kd, vd, nbd, scale, fp32_attn_weights=fp32w)
    torch.manual_seed(1234)
    qg, kg_, vg_ = (t.clone().requires_grad_(True) for t in (qd, kd, vd))
    out = sparse_gather_attention(qg, kg_, vg_, nbd, scale, dropout=p, training=True,
                                  fp32_attn_weights=fp32w)
    G = torch.randn(B, H, N, d, generator=g).to(DEV, dtype)
    out.backward(G)
    torch.cuda.synchronize()
    w0c, w1 = w0.float().cpu(), out.detach().float().cpu()
    assert (w0c > 0).all()
    keep = w1 != 0
    n = keep.numel()
    rate = keep.float().mean().item()
    sig = (p * (1 - p) / n) ** 0.5
    assert abs(rate - (1 - p)) < 5 * sig, (rate, sig)
    per_slot = keep.reshape(-1, d).float().mean(0)
    sig1 = (p * (1 - p) / (n // d)) ** 0.5
    assert (per_slot - (1 - p)).abs().max().item() < 5 * sig1
    s32 = torch.tensor(1.0, dtype=torch.float32) / torch.tensor(1.0 - p, dtype=torch.float32)
    if fp32w:
        # fp32 weights scaled in fp32, the output rounded once to bf16; the
        # undropped output is itself the weight rounded to bf16, so the two
        # differ by at most two bf16 roundings (2^-8 relative each)
        rel = ((w1[keep] - w0c[keep] * s32) / (w0c[keep] * s32)).abs().max().item()
        assert rel <= 2 ** -7, rel
    else:
        s_dt = s32.to(dtype)
        expect = (w0.cpu() * s_dt).float()          # product in fp32, rounded to dtype
        expect = expect.to(dtype).float()
        assert torch.equal(w1[keep], expect[keep])
    # backward against float64 autograd (on the device) with the observed
    # mask: slot j of a row holds key nb[j], whose output column shows it
    mask = torch.gather(keep.double(), 3, nb).to(DEV)
    qr, kr, vr = (t.to(DEV).double().requires_grad_(True) for t in (q, k, v))
    flat = (nbd + torch.arange(B * H, device=DEV).view(B, H, 1, 1) * M).reshape(-1)
    kgat = kr.reshape(B * H * M, d).index_select(0, flat).view(B, H, N, K, d)
    vgat = vr.reshape(B * H * M, d).index_select(0, flat).view(B, H, N, K, d)
    sc = (qr.unsqueeze(3) * kgat).sum(-1) * scale
    pr = torch.softmax(sc, -1) * mask * float(s32)
    o = (pr.unsqueeze(-1) * vgat).sum(3)
    o.backward(G.double())
    for name, got, exp in [("dq", qg.grad, qr.grad), ("dk", kg_.grad, kr.grad),
                           ("dv", vg_.grad, vr.grad)]:
        _check_grad_rows(name, got, exp, dtype)


@pytest.mark.parametrize("dtype,fp32w", [(torch.bfloat16, False), (torch.bfloat16, True),
                                         (torch.float32, False)])
def test_apply_backward_at_bench_head_shape(dtype, fp32w):
    """Backward at the bf16 GQA bench shape (N=4096, K=128, d=128), two kv
    groups (8 query heads), against float64 autograd of the same function
    computed on the device."""
    from ssa_amd import sparse_gather_attention
    B, H, nkv, N, M, d, K = 1, 8, 2, 4096, 4096, 128, 128
    g = torch.Generator().manual_seed(21)
    q = (torch.randn(B, H, N, d, generator=g) * 0.5).to(dtype)
    k = (torch.randn(B, nkv, M, d, generator=g) * 0.5).to(dtype)
    v = torch.randn(B, nkv, M, d, generator=g).to(dtype)
    nb = torch.randint(0, M, (B, H, N, K), generator=g)
    va = torch.rand(B, H, N, K, generator=g) > 0.2
    va[..., 0] = True
    dout = torch.randn(B, H, N, d, generator=g)
    qd, kd, vd = (t.to(DEV).requires_grad_(True) for t in (q, k, v))
    out = sparse_gather_attention(qd, kd, vd, nb.to(DEV), d ** -0.5, valid=va.to(DEV),
                                  fp32_attn_weights=fp32w)
    out.backward(dout.to(DEV, dtype))
    qr, kr, vr = (t.to(DEV).double().requires_grad_(True) for t in (q, k, v))
    nbd, vad = nb.to(DEV), va.to(DEV)
    ke = kr.repeat_interleave(H // nkv, 1)
    ve = vr.repeat_interleave(H // nkv, 1)
    flat = (nbd + torch.arange(B * H, device=DEV).view(B, H, 1, 1) * M).reshape(-1)
    kg = ke.reshape(B * H * M, d).index_select(0, flat).view(B, H, N, K, d)
    vg = ve.reshape(B * H * M, d).index_select(0, flat).view(B, H, N, K, d)
    s = (qr.unsqueeze(3) * kg).sum(-1) * d ** -0.5
    p = torch.softmax(s.masked_fill(~vad, float("-inf")), -1)
    o = (p.unsqueeze(-1) * vg).sum(3)
    o.backward(dout.to(dtype).to(DEV).double())   # the upstream gradient the device got
    for name, got, exp in [("dq", qd.grad, qr.grad), ("dk", kd.grad, kr.grad),
                           ("dv", vd.grad, vr.grad)]:
        _check_grad_rows(name, got, exp, dtype)


# ------------------------------------------------------------------ deterministic backward
@pytest.mark.parametrize("dtype,dropout", [(torch.float32, 0.0), (torch.bfloat16, 0.0),
                                           (torch.bfloat16, 0.2)])
def test_deterministic_backward_same_bits_and_matches_autograd(dtype, dropout):
    """Under torch.use_deterministic_algorithms(True) the backward takes
    ssa_sparse_gather_attention_bwd_det: dK / dV summed as fixed-point
    integers per key row, so three runs give the same bits; every row of
    dq / dk / dv matches float64 autograd (with the dropout mask read off the
    output, as in the dropout test) to the per-row bar.  GQA (8 query heads
    over 2 kv heads), N=M=2048, K=128, d=128, every key reached by several
    queries and some by hundreds."""
    from ssa_amd import sparse_gather_attention
    B, H, nkv, N, M, d, K = 1, 8, 2, 2048, 2048, 128, 128
    g = torch.Generator().manual_seed(31)
    q = (torch.randn(B, H, N, d, generator=g) * 0.5).to(dtype)
    k = (torch.randn(B, nkv, M, d, generator=g) * 0.5).to(dtype)
    v = torch.randn(B, nkv, M, d, generator=g).to(dtype)
    nb = torch.randint(0, M, (B, H, N, K), generator=g)
    nb[..., :4] = torch.arange(4)                   # four keys every query reads
    va = torch.rand(B, H, N, K, generator=g) > 0.2
    va[..., 0] = True
    dout = torch.randn(B, H, N, d, generator=g)
    prev = torch.are_deterministic_algorithms_enabled()
    grads, outs = [], []
    try:
        torch.use_deterministic_algorithms(True)
        for _ in range(3):
            qd, kd, vd = (t.to(DEV).requires_grad_(True) for t in (q, k, v))
            torch.manual_seed(77)
            out = sparse_gather_attention(qd, kd, vd, nb.to(DEV), d ** -0.5, valid=va.to(DEV),
                                          dropout=dropout, training=dropout > 0)
            out.backward(dout.to(DEV, dtype))
            torch.cuda.synchronize()
            grads.append((qd.grad.clone(), kd.grad.clone(), vd.grad.clone()))
            outs.append(out.detach().clone())
    finally:
        torch.use_deterministic_algorithms(prev)
    for gr in grads[1:]:
        for a, b_ in zip(gr, grads[0]):
            assert torch.equal(a, b_)
    # with dropout the reference is the fp32-atomic backward of the same seed
    # (itself checked against float64 autograd by the dropout test); without,
    # float64 autograd
    if dropout > 0:
        qd, kd, vd = (t.to(DEV).requires_grad_(True) for t in (q, k, v))
        torch.manual_seed(77)
        out = sparse_gather_attention(qd, kd, vd, nb.to(DEV), d ** -0.5, valid=va.to(DEV),
                                      dropout=dropout, training=True)
        out.backward(dout.to(DEV, dtype))
        torch.cuda.synchronize()
        assert torch.equal(out.detach(), outs[0])
        for name, got, exp in [("dq", grads[0][0], qd.grad), ("dk", grads[0][1], kd.grad),
                               ("dv", grads[0][2], vd.grad)]:
            _check_grad_rows(name, got.float(), exp.double(), dtype)
        return
    qr, kr, vr = (t.to(DEV).double().requires_grad_(True) for t in (q, k, v))
    nbd, vad = nb.to(DEV), va.to(DEV)
    ke = kr.repeat_interleave(H // nkv, 1)
    ve = vr.repeat_interleave(H // nkv, 1)
    flat = (nbd + torch.arange(B * H, device=DEV).view(B, H, 1, 1) * M).reshape(-1)
    kg = ke.reshape(B * H * M, d).index_select(0, flat).view(B, H, N, K, d)
    vg = ve.reshape(B * H * M, d).index_select(0, flat).view(B, H, N, K, d)
    s = (qr.unsqueeze(3) * kg).sum(-1) * d ** -0.5
    p = torch.softmax(s.masked_fill(~vad, float("-inf")), -1)
    o = (p.unsqueeze(-1) * vg).sum(3)
    o.backward(dout.to(dtype).to(DEV).double())   # the upstream gradient the device got
    for name, got, exp in [("dq", grads[0][0], qr.grad), ("dk", grads[0][1], kr.grad),
                           ("dv", grads[0][2], vr.grad)]:
        _check_grad_rows(name, got, exp, dtype)


# ------------------------------------------------------------------ merge
@pytest.mark.parametrize("has_self", [True, False])
@pytest.mark.parametrize("K", [8, 24, 200])
def test_merge_kernel_matches_oracle(has_self, K):
    from ssa_amd import merge_neighbors
    g = torch.Generator().manual_seed(K)
    B, H, N, Kl = 2, 3, 40, 20
    win = (torch.arange(N).unsqueeze(1) + torch.arange(-3, 4).unsqueeze(0)).clamp(0, N - 1)
    if not has_self:
        win = win[:, :0]
    glob = torch.tensor([0, 7, 7])
    lsh = torch.randint(0, N, (B, H, N, Kl), generator=g)
    self_idx = torch.arange(N).view(1, 1, N).expand(B, H, N) if has_self else None
    nb, va = merge_neighbors(win.to(DEV), glob.to(DEV), lsh.to(DEV),
                             self_idx.to(DEV) if has_self else None, K, N, B, H, DEV)
    rnb, rva = oracle.merge(win.numpy(), glob.numpy(), lsh.reshape(B * H, N, Kl).numpy(),
                            has_self=has_self, total_k=K)
    np.testing.assert_array_equal(nb.cpu().numpy().reshape(B * H, N, -1), rnb)
    np.testing.assert_array_equal(va.cpu().numpy().reshape(B * H, N, -1), rva)


# ------------------------------------------------------------------ module vs reference vectors
@pytest.mark.parametrize("path", golden_files(), ids=os.path.basename)
def test_apply_graph_on_reference_vectors(path):
    """The reference's own graph applied by our kernel reproduces its output."""
    from ssa_amd import SSAConfig, SparseAttention
    z, m = load_golden(path)
    with _nowarn():
        attn = SparseAttention(SSAConfig(**m["config"])).to(DEV).eval()
    dt = torch.bfloat16 if m["dtype"] == "bfloat16" else torch.float32
    q, k, v = (torch.from_numpy(z[n]).to(DEV, dt) for n in ("q", "k", "v"))
    nb = torch.from_numpy(z["neighbors"]).to(DEV)
    va = torch.from_numpy(z["valid"]).to(DEV)
    with torch.no_grad():
        out = attn.apply_graph(q, k, v, nb, va)
    err = row_rel_err(out.float().cpu().numpy(), z["attn_out"])
    assert err <= REL[dt], err
