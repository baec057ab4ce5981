"""ssa_build_graph_noalloc (the graph build over the library's fixed scratch
array) against ssa_build_graph (the build over a caller-allocated workspace):
bit-identical graphs on two calls in a row, the second one smaller, a tie
replay whose arrays go to the scratch array, a captured build replayed, calls
on two streams ordered, and a clear error for a problem that does not fit the
array.  Both entry points are called through the C ABI."""
import numpy as np
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


def _int_inputs(N, d, R, seed):
    g = torch.Generator().manual_seed(seed)
    q = torch.randint(-6, 7, (1, 1, N, d), generator=g).float()
    k = torch.randint(-6, 7, (1, 1, N, d), generator=g).float()
    rp = torch.randint(-6, 7, (R, 3, d), generator=g).float()
    return q, k, rp


def test_noalloc_tie_replay_outside_lds_matches_workspace_build():
    """kk = 1688 over 3 rounds of 6,752 candidates: the per-wave replay's
    arrays (kk + chunk = 8,440 slots) do not fit LDS, so they go to the
    scratch array, sized to it (fewer replay blocks, each looping over its
    rows); about 1,000 rows tie at the kk-th score (small integers), more than
    the workgroup replay takes within the scratch array's budget.  The graph
    equals the workspace build's, and the LSH lists equal the oracle's."""
    import oracle
    N, d, R = 2048, 16, 3
    q, k, rp = _int_inputs(N, d, R, 7)
    kw = dict(P=1, T=0, C=4 * 1688, top_k=1688, window=4, causal=False, is_cross=False,
              total_k=1700, glob=torch.arange(2, device=DEV))
    qd, kd, rpd = q.to(DEV), k.to(DEV), rp.to(DEV)
    ref_idx, ref_valid, ref_ties = _lib.build_graph(qd, kd, rpd, count_ties=True, **kw)
    got_idx, got_valid, got_ties = _lib.build_graph(qd, kd, rpd, count_ties=True, noalloc=True,
                                                    **kw)
    torch.cuda.synchronize()
    print(f"  tied rows {int(got_ties.item())}", flush=True)
    assert int(got_ties.item()) == int(ref_ties.item()) > 512
    assert torch.equal(got_idx, ref_idx)
    assert torch.equal(got_valid, ref_valid)
    lsh, _, _ = _lib.build_graph(qd, kd, rpd, noalloc=True, mode=_lib.GRAPH_LSH, **kw)
    torch.cuda.synchronize()
    exp = oracle.lsh_forward(q.reshape(1, N, d).numpy(), k.reshape(1, N, d).numpy(), rp.numpy(),
                             kv_rep=1, P=1, T=0, C=4 * 1688, top_k=1688, causal=False,
                             glob=np.arange(2))
    assert exp["n_ties"] == int(got_ties.item())
    np.testing.assert_array_equal(lsh.cpu().numpy().reshape(1, N, -1), exp["idx"])


def test_noalloc_build_captured_in_a_graph_replays_the_eager_graph():
    """The build without allocation captured into a HIP graph (after one eager
    call has set up the device) gives the eager graph on every replay, with
    eager builds through both entry points in between."""
    q, k, rp = _inputs(2, 4, 2, 300, 64, torch.bfloat16, 5)
    kw = _kw(300, K=48, w=4, G=2, T=1, R=4)
    rp = rp[:4, :, :64].contiguous()
    eager, _, _ = _lib.build_graph(q, k, rp, ids32=True, noalloc=True, **kw)
    ws, _, _ = _lib.build_graph(q, k, rp, ids32=True, **kw)
    torch.cuda.synchronize()
    assert torch.equal(eager, ws)
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        _lib.build_graph(q, k, rp, ids32=True, noalloc=True, **kw)
    torch.cuda.current_stream().wait_stream(side)
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        out, _, _ = _lib.build_graph(q, k, rp, ids32=True, noalloc=True, **kw)
    for i in range(3):
        out.fill_(7)
        g.replay()
        torch.cuda.synchronize()
        assert torch.equal(out, eager), f"replay {i}"
        again, _, _ = _lib.build_graph(q, k, rp, ids32=True, noalloc=True, **kw)
        other, _, _ = _lib.build_graph(q, k, rp, ids32=True, **kw)
        torch.cuda.synchronize()
        assert torch.equal(again, eager) and torch.equal(other, eager)


def test_noalloc_calls_on_two_streams_are_ordered():
    """Two builds without allocation issued on two streams with no host sync
    between them: each call waits for the previous call's work on the GPU, so
    both graphs equal the workspace builds of the same problems."""
    probs = []
    for seed, (Hq, Hkv, N, d) in [(11, (8, 2, 4096, 64)), (12, (4, 4, 2048, 128))]:
        q, k, rp = _inputs(1, Hq, Hkv, N, d, torch.bfloat16, seed)
        kw = _kw(N)
        rp = rp[:, :, :d].contiguous()
        ref, _, _ = _lib.build_graph(q, k, rp, ids32=True, **kw)
        probs.append((q, k, rp, kw, ref))
    torch.cuda.synchronize()
    streams = [torch.cuda.Stream(), torch.cuda.Stream()]
    for rnd in range(3):
        order = [0, 1] if rnd % 2 == 0 else [1, 0]
        outs = {}
        for s in streams:
            s.wait_stream(torch.cuda.current_stream())
        for i in order:
            q, k, rp, kw, _ = probs[i]
            with torch.cuda.stream(streams[i]):
                outs[i], _, _ = _lib.build_graph(q, k, rp, ids32=True, noalloc=True, **kw)
        torch.cuda.synchronize()
        for i in order:
            assert torch.equal(outs[i], probs[i][4]), f"round {rnd}, problem {i}"
