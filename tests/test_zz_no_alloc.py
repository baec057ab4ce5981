"""ssa_build_graph_noalloc (the graph build over the library's fixed scratch
array) against ssa_build_graph (the build over a caller-allocated workspace):
bit-identical graphs on two calls in a row, the second one smaller, and a
clear error for a problem that does not fit the array.  Both entry points are
called through the C ABI."""
import pytest
import torch

from ssa_amd import _lib

pytestmark = pytest.mark.gpu
DEV = "cuda:0"


def _inputs(B, Hq, Hkv, N, d, dtype, seed):
    g = torch.Generator().manual_seed(seed)
    q = torch.randn(B, Hq, N, d, generator=g).to(dtype).to(DEV)
    k = torch.randn(B, Hkv, N, d, generator=g).to(dtype).to(DEV)
    rp = torch.randn(8, 12, d, generator=g)
    rp = (rp / rp.norm(dim=-1, keepdim=True)).to(DEV)
    return q, k, rp


def _kw(N, K=128, w=16, G=2, T=0, R=8, causal=True, mode=_lib.GRAPH_FULL):
    lsh_k = max(K - (2 * w + 1 + G + 1), 8)
    C = 4 * lsh_k
    import math
    P = max(1, min(12, round(math.log2(N / C)))) if N > 1 else 1
    return dict(P=P, T=T, C=C, top_k=lsh_k, window=w, causal=causal, is_cross=False,
                total_k=K, glob=torch.arange(min(G, N), device=DEV), mode=mode)


@pytest.mark.parametrize("mode", [_lib.GRAPH_FULL, _lib.GRAPH_LSH])
def test_noalloc_build_matches_workspace_build(mode):
    cases = [
        # 8 heads of 25 MB of score rows each: built in head chunks that fit
        dict(B=1, Hq=8, Hkv=2, N=4096, d=64, dtype=torch.bfloat16, seed=1),
        # then a smaller problem on the same scratch array
        dict(B=2, Hq=4, Hkv=4, N=512, d=32, dtype=torch.float32, seed=2),
    ]
    for c in cases:
        print(f"noalloc case {c} mode {mode}", flush=True)
        q, k, rp = _inputs(c["B"], c["Hq"], c["Hkv"], c["N"], c["d"], c["dtype"], c["seed"])
        kw = _kw(c["N"], mode=mode)
        ref_idx, ref_valid, ref_ties = _lib.build_graph(q, k, rp[:, :, :c["d"]].contiguous(),
                                                        count_ties=True, **kw)
        got_idx, got_valid, got_ties = _lib.build_graph(q, k, rp[:, :, :c["d"]].contiguous(),
                                                        count_ties=True, noalloc=True, **kw)
        torch.cuda.synchronize()
        assert torch.equal(got_idx, ref_idx)
        if mode == _lib.GRAPH_FULL:
            assert torch.equal(got_valid, ref_valid)
        assert int(got_ties.item()) == int(ref_ties.item())


def test_noalloc_int32_graph_matches():
    q, k, rp = _inputs(1, 4, 1, 2048, 128, torch.bfloat16, 3)
    kw = _kw(2048)
    ref, _, _ = _lib.build_graph(q, k, rp, ids32=True, **kw)
    got, _, _ = _lib.build_graph(q, k, rp, ids32=True, noalloc=True, **kw)
    torch.cuda.synchronize()
    assert torch.equal(got, ref)


def test_noalloc_refuses_a_problem_beyond_the_scratch_array():
    # one head's score rows alone (N * R * C * 2 bytes) exceed 64 MiB
    q, k, rp = _inputs(1, 1, 1, 32768, 16, torch.float32, 4)
    kw = _kw(32768, K=256)
    with pytest.raises(RuntimeError, match="scratch array"):
        _lib.build_graph(q, k, rp[:, :, :16].contiguous(), noalloc=True, **kw)
