"""Deterministic sweeps of graph-build and gather-attention shapes against
the oracle (and of the backward against float64 autograd).

96 configurations (and 24 more over wider ranges) drawn from seeded
generators over batch size, kv heads and group size, query and key lengths,
head dims (including ones the kernels run zero-padded), hash rounds, planes, probes, neighbour counts, window, global
tokens, causal / cross-attention and fp32 / bf16 / fp16 inputs.  q, k and the
hyperplanes hold small integers, so every projection and score is exact in
every type: the merged graph (neighbours and valid mask) must equal the
oracle's bit for bit, and so must the LSH mode's neighbour lists, in order,
tied kk-th scores included (the GPU replays the reference's top-k on those
rows).
"""
import numpy as np
import pytest
import torch

import oracle
from conftest import has_gpu
from test_gpu_parity import _graph_case
from test_gpu_parity import test_apply_matches_oracle as _apply_check
from test_gpu_parity import test_apply_backward_matches_autograd_reference as _bwd_check

pytestmark = [pytest.mark.gpu,
              pytest.mark.skipif(not has_gpu(), reason="needs a ROCm GPU")]


def _sweep_cases(n=96, seed=2024):
    rng = np.random.default_rng(seed)
    dtypes = [torch.float32, torch.bfloat16, torch.float16]
    cases = []
    for i in range(n):
        cross = bool(rng.random() < 0.3)
        causal = (not cross) and bool(rng.random() < 0.6)
        nkv = int(rng.choice([1, 2, 4]))
        H = nkv * int(rng.choice([1, 2, 4]))
        B = int(rng.choice([1, 2]))
        N = int(rng.integers(8, 400))
        M = int(rng.integers(8, 700)) if cross else N
        d = int(rng.choice([6, 16, 20, 32, 48, 64, 96, 128]))
        R = int(rng.integers(1, 5))
        maxP = int(rng.integers(2, 9))
        T = int(rng.integers(0, 4))
        w = int(rng.integers(0, 9))
        G = int(rng.integers(0, 4))
        K = int(rng.integers(2 * w + G + 10, 2 * w + G + 80))
        dt = dtypes[int(rng.integers(0, 3))]
        cases.append(((f"sweep{i}", B, H, nkv, N, M, d, R, maxP, T, K, w, G, causal, cross), dt))
    return cases


CASES = _sweep_cases()


@pytest.mark.parametrize("case,dtype", CASES, ids=[c[0][0] for c in CASES])
def test_graph_shape_sweep_matches_oracle(case, dtype):
    attn, got, got_v, ref, (B, H, N, M, K, w, cross, causal, glob) = _graph_case(
        case, 11, dtype=dtype)
    win = (np.zeros((N, 0), np.int64) if cross else attn.win_builder(N, M, "cpu").numpy())
    rnb, rva = oracle.merge(win, glob.numpy(), ref["idx"], has_self=not cross, total_k=K)
    np.testing.assert_array_equal(got.cpu().numpy().reshape(B * H, N, -1), rnb)
    np.testing.assert_array_equal(got_v.cpu().numpy().reshape(B * H, N, -1), rva)


def _wide_cases(n=24, seed=777):
    """Wider ranges: up to 2,499 queries and 2,999 keys, 8 kv heads, head dims
    4 to 256, up to 8 rounds, 12 planes, 16-wide windows and 5 globals."""
    rng = np.random.default_rng(seed)
    dtypes = [torch.float32, torch.bfloat16, torch.float16]
    cases = []
    for i in range(n):
        cross = bool(rng.random() < 0.3)
        causal = (not cross) and bool(rng.random() < 0.6)
        nkv = int(rng.choice([1, 2, 4, 8]))
        H = nkv * int(rng.choice([1, 2, 4]))
        B = int(rng.choice([1, 2, 3]))
        N = int(rng.integers(8, 2500))
        M = int(rng.integers(8, 3000)) if cross else N
        d = int(rng.choice([4, 6, 8, 16, 20, 32, 48, 64, 80, 96, 112, 128, 256]))
        R = int(rng.integers(1, 9))
        maxP = int(rng.integers(2, 13))
        T = int(rng.integers(0, 4))
        w = int(rng.integers(0, 17))
        G = int(rng.integers(0, 6))
        K = int(rng.integers(2 * w + G + 10, 2 * w + G + 200))
        cases.append(((f"wide{i}", B, H, nkv, N, M, d, R, maxP, T, K, w, G, causal, cross),
                      dtypes[int(rng.integers(0, 3))]))
    return cases


WIDE_CASES = _wide_cases()


@pytest.mark.parametrize("case,dtype", WIDE_CASES, ids=[c[0][0] for c in WIDE_CASES])
def test_graph_wide_sweep_matches_oracle(case, dtype):
    test_graph_shape_sweep_matches_oracle(case, dtype)


@pytest.mark.parametrize("case,dtype", CASES[::2], ids=[c[0][0] for c in CASES[::2]])
def test_lsh_shape_sweep_matches_oracle(case, dtype):
    attn, got, _, ref, (B, H, N, M, K, w, cross, causal, glob) = _graph_case(
        case, 13, dtype=dtype, lsh_only=True)
    np.testing.assert_array_equal(got.cpu().numpy().reshape(B * H, N, -1), ref["idx"])




def _apply_sweep_cases(n=48, seed=77):
    """(B, Hq, Hkv, N, M, d, K) for the gather attention, with dtype and
    fp32_attn_weights: random group sizes, head dims 4 to 1024 (including
    ones run zero-padded), K from 1 to 600."""
    rng = np.random.default_rng(seed)
    dtypes = [torch.float32, torch.bfloat16, torch.float16]
    dims = [4, 6, 8, 16, 20, 24, 32, 40, 64, 72, 96, 128, 160, 256, 320, 512, 640, 1024]
    cases = []
    for i in range(n):
        nkv = int(rng.choice([1, 2, 4]))
        H = nkv * int(rng.choice([1, 2, 4]))
        B = int(rng.choice([1, 2]))
        N = int(rng.integers(1, 40))
        M = int(rng.integers(1, 300))
        d = int(rng.choice(dims))
        K = int(rng.integers(1, 600))
        cases.append(((B, H, nkv, N, M, d, K), dtypes[int(rng.integers(0, 3))],
                      bool(rng.random() < 0.3)))
    return cases


APPLY_CASES = _apply_sweep_cases()


@pytest.mark.parametrize("case,dtype,fp32w", APPLY_CASES,
                         ids=[f"apply{i}" for i in range(len(APPLY_CASES))])
def test_apply_shape_sweep_matches_oracle(case, dtype, fp32w):
    """Every query row within the per-row bar of the oracle's float64 apply
    (1e-5 relative in fp32, 2e-2 in bf16 / fp16; 30% of slots masked, slot 0
    valid)."""
    _apply_check(case, dtype, fp32w)


def _bwd_sweep_cases(n=24, seed=91):
    """(B, Hq, Hkv, N, M, d, K) for the backward, small enough for the float64
    autograd reference (which materialises the gathered rows)."""
    rng = np.random.default_rng(seed)
    dims = [4, 6, 16, 20, 32, 48, 64, 96, 128, 200, 256]
    cases = []
    for i in range(n):
        nkv = int(rng.choice([1, 2]))
        H = nkv * int(rng.choice([1, 2, 4]))
        cases.append(((int(rng.choice([1, 2])), H, nkv, int(rng.integers(1, 16)),
                       int(rng.integers(2, 120)), int(rng.choice(dims)),
                       int(rng.integers(1, 100))),
                      [torch.float32, torch.bfloat16][int(rng.integers(0, 2))]))
    return cases


BWD_CASES = _bwd_sweep_cases()


@pytest.mark.parametrize("case,dtype", BWD_CASES,
                         ids=[f"bwd{i}" for i in range(len(BWD_CASES))])
def test_apply_backward_shape_sweep_matches_autograd(case, dtype):
    """dq, dk, dv per row against float64 autograd of the same function."""
    _bwd_check(dtype, case)

