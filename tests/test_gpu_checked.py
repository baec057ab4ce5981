"""The graph build under the bounds-checked library (libssa_amd_checked.so,
the same kernels built with SSA_CHECKED): every data-dependent index of the
select, tie replay and merge paths -- key ids, sorted-list and bucket
positions, tie rows, output slots -- stays inside what it indexes, and the
graphs equal the product library's.  Cases: exact-tier inputs (small
integers: many tied rows, both tie replays, replay arrays outside LDS) in
fp32 and bf16, the bench workload (bf16 GQA, N=4096, K=128, 32 / 8 heads,
head dim 128) in both modes, and the 32k MQA workload's shape on four query
heads (512-key select buffer, probes, explicit globals)."""
import math
import warnings

import pytest
import torch

from conftest import has_gpu
from ssa_amd import _lib

pytestmark = [pytest.mark.gpu,
              pytest.mark.skipif(not has_gpu(), reason="needs a ROCm GPU")]

DEV = "cuda"


def test_product_library_keeps_no_record():
    import ctypes
    rec = (ctypes.c_uint32 * 4)()
    assert _lib.lib().ssa_checked_oob(rec) == 0
    with _lib.checked_library() as record:
        record()
        assert record() is None


def _both(fn):
    """fn() under the product library, then under the checked one; the
    checked run must record no index outside its buffer."""
    ref = fn()
    torch.cuda.synchronize()
    with _lib.checked_library() as record:
        record()                              # clear what earlier tests left
        got = fn()
        torch.cuda.synchronize()
        rec = record()
    assert rec is None, f"index out of bounds: site bits {rec[0]:#x}, last site {rec[1]}, " \
                        f"index {rec[2]}, length {rec[3]}"
    return ref, got


def _kw(N, M, K, w, G, T, R, causal, cross=False, glob=None):
    lsh_k = max(K - ((0 if cross else 2 * w + 1) + G + (0 if cross else 1)), 8)
    C = 4 * lsh_k
    P = max(1, min(12, round(math.log2(M / C)))) if M > C else 1
    g = torch.arange(min(G, M)) if glob is None else torch.tensor(glob)
    return dict(P=P, T=T, C=C, top_k=lsh_k, window=w, causal=causal, is_cross=cross,
                total_k=K, glob=g.to(DEV))


# name, B, Hq, Hkv, N, M, d, R, T, K, window, G, causal, cross, dtype
INT_CASES = [
    ("causal_gqa", 2, 4, 2, 96, 96, 16, 3, 0, 24, 3, 2, True, False, torch.float32),
    ("cross_probes", 2, 4, 2, 50, 130, 16, 3, 2, 24, 4, 2, False, True, torch.float32),
    ("many_ties_workgroup", 1, 4, 2, 512, 512, 16, 4, 1, 32, 4, 2, True, False, torch.float32),
    ("many_ties_per_wave", 2, 8, 2, 384, 384, 8, 3, 1, 24, 4, 2, True, False, torch.float32),
    ("many_ties_bf16", 1, 4, 2, 512, 512, 64, 4, 1, 32, 4, 2, True, False, torch.bfloat16),
    ("huge_k", 1, 1, 1, 2048, 2048, 16, 2, 0, 1400, 4, 2, True, False, torch.float32),
    ("huge_k_per_wave", 1, 1, 1, 4096, 4096, 16, 2, 0, 1700, 4, 2, True, False, torch.float32),
    ("long_keys", 1, 1, 1, 65536, 65536, 16, 2, 0, 32, 2, 2, True, False, torch.float32),
    ("keys_131072", 1, 1, 1, 131072, 131072, 16, 2, 0, 64, 2, 2, True, False, torch.float32),
    ("keys_262144_cross", 1, 2, 2, 200, 262144, 16, 2, 1, 64, 2, 2, False, True, torch.float32),
    ("huge_k_wide_ids", 1, 1, 1, 4096, 70000, 16, 2, 0, 1700, 4, 2, False, True, torch.float32),
    ("many_globals", 1, 2, 2, 256, 256, 16, 3, 1, 160, 4, 100, True, False, torch.bfloat16),
]


@pytest.mark.parametrize("case", INT_CASES, ids=lambda c: c[0])
@pytest.mark.parametrize("mode", [_lib.GRAPH_FULL, _lib.GRAPH_LSH], ids=["full", "lsh"])
def test_checked_build_exact_tier(case, mode):
    _, B, Hq, Hkv, N, M, d, R, T, K, w, G, causal, cross, dt = case
    g = torch.Generator().manual_seed(3)
    q = torch.randint(-6, 7, (B, Hq, N, d), generator=g).to(dt).to(DEV)
    k = torch.randint(-6, 7, (B, Hkv, M, d), generator=g).to(dt).to(DEV)
    rp = torch.randint(-6, 7, (R, 12, d), generator=g).float().to(DEV)
    kw = _kw(N, M, K, w, G, T, R, causal and not cross, cross)
    print(f"  {case[0]} mode {mode}", flush=True)
    ref, got = _both(lambda: _lib.build_graph(q, k, rp, mode=mode, count_ties=True, **kw))
    print(f"  tied rows {int(ref[2].item())}", flush=True)
    assert torch.equal(got[0], ref[0])
    if mode == _lib.GRAPH_FULL:
        assert torch.equal(got[1], ref[1])
    assert int(got[2].item()) == int(ref[2].item())


@pytest.mark.parametrize("mode", [_lib.GRAPH_FULL, _lib.GRAPH_LSH], ids=["full", "lsh"])
def test_checked_build_bench_workload(mode):
    """The bf16 GQA workload (N=4096, K=128, 32 q / 8 kv heads, d 128, window
    16, 2 globals, 8 rounds, causal) from the module's own projections."""
    from ssa_amd import SSAConfig, SparseAttention
    cfg = SSAConfig(d_model=4096, num_heads=32, num_kv_heads=8, num_neighbors=128,
                    window_size=16, num_global_tokens=2, num_hash_rounds=8, max_num_hashes=12,
                    lsh_num_probes=0, causal=True)
    torch.manual_seed(0)
    with warnings.catch_warnings():
        warnings.simplefilter("ignore")
        attn = SparseAttention(cfg)
    for W in (attn.Wq, attn.Wk, attn.Wv, attn.Wo):
        torch.nn.init.xavier_uniform_(W.weight)
    attn = attn.to(DEV)
    for p in attn.parameters():
        p.data = p.data.to(torch.bfloat16)
    attn.eval()
    g = torch.Generator().manual_seed(1000)
    x = (torch.randn(1, 4096, 4096, generator=g) * 0.02).to(torch.bfloat16).to(DEV)
    with torch.no_grad():
        q = attn._split_q(attn.Wq(x))
        k = attn._split_kv_compact(attn.Wk(x))
    lb = attn.lsh_builder
    P = lb.compute_effective_p(4096, lb.C, lb.max_P)
    kw = dict(P=P, T=lb.T, C=lb.C, top_k=attn.lsh_k, window=16, causal=True, is_cross=False,
              total_k=128, glob=attn.glob_builder(4096, DEV))
    ref, got = _both(lambda: _lib.build_graph(q, k, lb.rand_proj, mode=mode, count_ties=True,
                                              ids32=mode == _lib.GRAPH_FULL, **kw))
    assert torch.equal(got[0], ref[0])
    assert int(got[2].item()) == int(ref[2].item())


def test_checked_build_mqa_32k_shape():
    """N=32768 over one kv head (four of its query heads), K=256, window 32,
    globals [0, 1, 16384], 8 rounds, 2 probes, causal: the 512-key select
    buffer and the probe lists."""
    g = torch.Generator().manual_seed(5)
    N, d = 32768, 128
    q = (torch.randn(1, 4, N, d, generator=g)).to(torch.bfloat16).to(DEV)
    k = (torch.randn(1, 1, N, d, generator=g)).to(torch.bfloat16).to(DEV)
    rp = torch.randn(8, 12, d, generator=g)
    rp = (rp / rp.norm(dim=-1, keepdim=True)).to(DEV)
    kw = _kw(N, N, 256, 32, 3, 2, 8, True, glob=[0, 1, 16384])
    ref, got = _both(lambda: _lib.build_graph(q, k, rp, count_ties=True, ids32=True, **kw))
    assert torch.equal(got[0], ref[0])
    assert int(got[2].item()) == int(ref[2].item())
