"""Pins the CPU oracle before anything is checked against it.

* library routines: the oracle's introsort / introselect emulations against
  ``torch.sort`` / ``torch.topk`` themselves (the routines the reference calls);
* golden vectors written by importing the reference (tests/golden);
* closed forms: sign-at-zero rule, bit order, probe flips, merge layout;
* apply against dense softmax attention when the neighbor list covers every key.
"""
import os

import numpy as np
import pytest
import torch

import oracle
from conftest import golden_files, load_golden

RNG = np.random.default_rng(1234)


# --------------------------------------------------------------------------- sort
@pytest.mark.parametrize("rows,M,P", [(2, 1024, 1), (2, 4096, 3), (1, 32768, 5), (4, 512, 1),
                                      (2, 8192, 4), (4, 40, 2), (4, 17, 1), (2, 300, 12),
                                      (1, 65536, 12), (3, 3, 1), (2, 16, 2), (2, 33, 3)])
@pytest.mark.parametrize("dist", ["uniform", "skewed", "sorted", "reversed", "constant"])
def test_sort_perm_matches_torch_sort(rows, M, P, dist):
    """torch.sort(int64 rows, stable=False) == introsort permutation."""
    if dist == "uniform":
        k = RNG.integers(0, 2 ** P, (rows, M))
    elif dist == "skewed":
        k = np.minimum(RNG.geometric(0.3, (rows, M)) - 1, 2 ** P - 1)
    elif dist == "sorted":
        k = np.sort(RNG.integers(0, 2 ** P, (rows, M)), axis=-1)
    elif dist == "reversed":
        k = np.sort(RNG.integers(0, 2 ** P, (rows, M)), axis=-1)[:, ::-1]
    else:
        k = np.zeros((rows, M))
    k = np.ascontiguousarray(k.astype(np.int64))
    ref = torch.sort(torch.from_numpy(k), dim=-1)[1].numpy()
    for r in range(rows):
        np.testing.assert_array_equal(oracle.sort_perm(k[r]), ref[r])


def _equal_keys_final_slot(n, i):
    """Final slot of the element at position i of an introsort segment of n
    equal keys: the closed form the device's segment sort applies to such
    segments (ssa_sort.hip, eq_final_pos), restated."""
    base = 0
    while n > 16:
        h = n // 2
        i = h if i == 0 else (0 if i == h else i)       # median of three: first <-> middle
        if i != 0 and 2 * i != n:                        # the scan swaps k and n - k
            i = n - i
        c = (n + 1) // 2                                 # and cuts at ceil(n / 2)
        if i < c:
            n = c
        else:
            base, i, n = base + c, i - c, n - c
    return base + i


@pytest.mark.parametrize("n", list(range(1, 70)) + [255, 256, 257, 511, 1000, 1023, 1024, 4096,
                                                     5000, 32768])
def test_equal_key_segment_permutation_closed_form(n):
    """A segment of equal keys sorts (torch.sort's introsort) into a
    permutation fixed by its length alone, which the closed form gives."""
    # 2-D like the reference's rows (a 1-D sort of 32768+ int keys takes a radix path)
    ref = torch.sort(torch.zeros((1, n), dtype=torch.int64), dim=-1)[1].numpy()[0]
    np.testing.assert_array_equal(oracle.sort_perm(np.zeros(n, dtype=np.int64)), ref)
    mine = np.empty(n, dtype=np.int64)
    for i in range(n):
        mine[_equal_keys_final_slot(n, i)] = i
    np.testing.assert_array_equal(mine, ref)


def test_sort_is_not_stable_so_emulation_matters():
    k = RNG.integers(0, 8, (1, 4096)).astype(np.int64)
    uns = torch.sort(torch.from_numpy(k), dim=-1)[1].numpy()
    st = torch.sort(torch.from_numpy(k), dim=-1, stable=True)[1].numpy()
    assert not np.array_equal(uns, st)
    np.testing.assert_array_equal(oracle.sort_perm(k[0]), uns[0])


# --------------------------------------------------------------------------- topk
@pytest.mark.parametrize("n,k", [(460, 92), (540, 108), (308, 52), (935, 187), (3000, 3),
                                 (100, 10), (1000, 2), (5, 5), (64, 1)])
@pytest.mark.parametrize("dist", ["continuous", "levels2", "levels5", "levels1000", "neginf",
                                  "nan"])
def test_topk_row_matches_torch_topk(n, k, dist):
    if dist == "continuous":
        v = RNG.standard_normal(n).astype(np.float32)
    elif dist.startswith("levels"):
        v = RNG.integers(0, int(dist[6:]), n).astype(np.float32)
    elif dist == "neginf":
        v = RNG.standard_normal(n).astype(np.float32)
        v[RNG.random(n) < 0.7] = -np.inf
    else:
        v = RNG.standard_normal(n).astype(np.float32)
        v[RNG.random(n) < 0.1] = np.nan
    rv, ri = torch.from_numpy(v).topk(k)
    mv, mi = oracle.topk_row(v, k)
    np.testing.assert_array_equal(mi, ri.numpy())
    np.testing.assert_array_equal(mv, rv.numpy())


# --------------------------------------------------------------------------- hash
def test_hash_sign_rule_and_bit_order():
    """bit j = (proj_j > 0) with plane j as bit j; +0, -0 and NaN give 0."""
    planes = np.eye(4, dtype=np.float32)
    x = np.array([[1, 0, 0, 0], [0, 1, 0, 0], [0, 0, 0, 1], [1, 1, 1, 1], [0, 0, 0, 0],
                  [-0.0, -1, 2, 0], [np.nan, 1, 0, 0]], np.float32)
    _, ids, _ = oracle.hash_rows(x, planes)
    # a NaN coordinate makes every projection NaN (NaN * 0 = NaN) -> id 0
    assert ids.tolist() == [1, 2, 8, 15, 0, 4, 0]


def test_probe_ids_flip_least_confident_bits_of_base():
    planes = np.eye(4, dtype=np.float32)
    x = np.array([[0.5, -0.1, 2.0, -3.0]], np.float32)   # |proj| order: 1, 0, 2, 3
    _, ids, probes = oracle.hash_rows(x, planes, T=3)
    base = 0b0101
    assert ids[0] == base
    assert probes[0].tolist() == [base + 2, base - 1, base - 4]


def test_probe_ties_keep_plane_order():
    planes = np.eye(3, dtype=np.float32)
    x = np.array([[1.0, -1.0, 1.0]], np.float32)          # all |proj| equal -> 0, 1, 2
    _, ids, probes = oracle.hash_rows(x, planes, T=3)
    assert ids[0] == 0b101
    assert probes[0].tolist() == [0b100, 0b111, 0b001]


# --------------------------------------------------------------------------- golden
@pytest.mark.parametrize("path", golden_files(), ids=os.path.basename)
def test_oracle_lsh_merge_apply_match_golden(path):
    z, m = load_golden(path)
    B, N, M, H, d = m["B"], m["N"], m["M"], m["H"], m["d_head"]
    cfg = m["config"]
    q = z["q"].reshape(B * H, N, d)
    k = z["k"].reshape(B * H, M, d)
    rp = z["sd_lsh_builder.rand_proj"]
    R, P = rp.shape[0], m["p_eff"]
    res = oracle.lsh_forward(q, k, rp, kv_rep=1, P=P, T=cfg["lsh_num_probes"], C=m["C"],
                             top_k=m["lsh_k"], causal=m["causal"], glob=z["glob"],
                             q_proj=z["qproj"].reshape(B * H, R, N, P),
                             k_proj=z["kproj"].reshape(B * H, R, M, P))
    np.testing.assert_array_equal(res["idx"], z["lsh"].reshape(B * H, N, -1))
    nb, va = oracle.merge(z["win"], z["glob"], res["idx"], has_self=not m["cross"],
                          total_k=cfg["num_neighbors"])
    np.testing.assert_array_equal(nb, z["neighbors"].reshape(B * H, N, -1))
    np.testing.assert_array_equal(va, z["valid"].reshape(B * H, N, -1))
    mode = 1 if m["dtype"] == "bfloat16" else 0
    ao = oracle.apply(q, k, z["v"].reshape(B * H, M, d), nb, va, kv_rep=1, scale=m["scale"],
                      mode=mode, fp32_attn_weights=cfg["fp32_attn_weights"])
    ref = z["attn_out"].reshape(B * H, N, d)
    if mode == 1:   # reference output is bf16: compare after rounding to bf16
        ao = torch.from_numpy(ao).to(torch.bfloat16).float().numpy()
        tol = 2e-2
    else:
        tol = 1e-5
    assert np.abs(ao - ref).max() <= tol * np.abs(ref).max()


def test_oracle_golden_tie_cases_exercise_the_tie_path():
    """The duplicate-row vectors contain k-th-place ties that only the exact
    introselect replay reproduces; make sure the oracle flags them."""
    path = [p for p in golden_files() if "dup_rows_ties_s0" in p][0]
    z, m = load_golden(path)
    B, N, M, H, d = m["B"], m["N"], m["M"], m["H"], m["d_head"]
    rp = z["sd_lsh_builder.rand_proj"]
    R, P = rp.shape[0], m["p_eff"]
    res = oracle.lsh_forward(z["q"].reshape(B * H, N, d), z["k"].reshape(B * H, M, d), rp,
                             kv_rep=1, P=P, T=m["config"]["lsh_num_probes"], C=m["C"],
                             top_k=m["lsh_k"], causal=m["causal"], glob=z["glob"],
                             q_proj=z["qproj"].reshape(B * H, R, N, P),
                             k_proj=z["kproj"].reshape(B * H, R, M, P))
    assert res["n_ties"] > 10


def test_oracle_empty_bucket_vector():
    z = np.load(os.path.join(os.path.dirname(__file__), "golden", "lsh_empty_bucket.npz"))
    res = oracle.lsh_forward(z["q"].reshape(1, 4, 4), z["k"].reshape(1, 8, 4), z["rand_proj"],
                             kv_rep=1, P=1, T=0, C=4, top_k=2, causal=False, glob=z["glob"])
    np.testing.assert_array_equal(res["idx"], z["out"].reshape(1, 4, 2))


def test_oracle_empty_bucket_list_competes_on_score():
    """Reference vector where the glob ++ 0 list of an empty bucket outscores
    the populated round: query 0 selects [5, 0]; query 1 has a tie at the
    k-th place among keys 1..3 that the reference resolves to key 2."""
    z = np.load(os.path.join(os.path.dirname(__file__), "golden", "lsh_empty_bucket_ranked.npz"))
    res = oracle.lsh_forward(z["q"].reshape(1, 2, 4), z["k"].reshape(1, 8, 4), z["rand_proj"],
                             kv_rep=1, P=1, T=0, C=4, top_k=2, causal=False, glob=z["glob"])
    np.testing.assert_array_equal(res["idx"], z["out"].reshape(1, 2, 2))


def test_oracle_projection_path_matches_injected_on_exact_inputs():
    """With exact-arithmetic inputs (small integers) the oracle's own fp32
    projections equal any summation order, so computed == injected."""
    BH, N, d, R, P = 2, 64, 16, 3, 2
    q = RNG.integers(-8, 9, (BH, N, d)).astype(np.float32)
    k = RNG.integers(-8, 9, (BH, N, d)).astype(np.float32)
    rp = RNG.integers(-8, 9, (R, 4, d)).astype(np.float32)
    qp = np.einsum("bnd,rpd->brnp", q, rp[:, :P]).astype(np.float32)
    kp = np.einsum("bnd,rpd->brnp", k, rp[:, :P]).astype(np.float32)
    kw = dict(kv_rep=1, P=P, T=1, C=12, top_k=9, causal=True, glob=[0, 1])
    a = oracle.lsh_forward(q, k, rp, **kw)
    b = oracle.lsh_forward(q, k, rp, q_proj=qp, k_proj=kp, **kw)
    np.testing.assert_array_equal(a["idx"], b["idx"])


# --------------------------------------------------------------------------- merge
def test_merge_closed_form():
    """[self] ++ ascending unique(pool - {self})[:K-1], zero padding invalid."""
    N, K = 40, 20
    win = np.clip(np.arange(N)[:, None] + np.arange(-3, 4)[None], 0, N - 1)
    glob = np.array([0, 1])
    lsh = RNG.integers(0, N, (3, N, 9))
    nb, va = oracle.merge(win, glob, lsh, has_self=True, total_k=K)
    for bh in range(3):
        for n in range(N):
            pool = sorted((set(win[n].tolist()) | {0, 1} | set(lsh[bh, n].tolist())) - {n})
            exp = [n] + pool[:K - 1]
            cnt = len(exp)
            assert nb[bh, n, :cnt].tolist() == exp
            assert va[bh, n, :cnt].all() and not va[bh, n, cnt:].any()
            assert (nb[bh, n, cnt:] == 0).all()


def test_merge_cross_width_is_min_k_g_plus_lsh():
    lsh = RNG.integers(0, 50, (2, 7, 52))
    nb, va = oracle.merge(np.zeros((7, 0), np.int64), np.array([0, 1]), lsh, has_self=False,
                          total_k=64)
    assert nb.shape[-1] == 54


# --------------------------------------------------------------------------- apply
@pytest.mark.parametrize("mode", [0, 1])
def test_apply_equals_dense_attention_when_graph_is_complete(mode):
    BH, N, M, d = 3, 17, 23, 16
    q = RNG.standard_normal((BH, N, d)).astype(np.float32)
    k = RNG.standard_normal((BH, M, d)).astype(np.float32)
    v = RNG.standard_normal((BH, M, d)).astype(np.float32)
    nb = np.stack([RNG.permutation(M) for _ in range(BH * N)]).reshape(BH, N, M)
    scale = d ** -0.5
    out = oracle.apply(q, k, v, nb, None, kv_rep=1, scale=scale, mode=mode)
    s = torch.from_numpy(q).double() @ torch.from_numpy(k).double().transpose(1, 2) * scale
    ref = torch.softmax(s, -1) @ torch.from_numpy(v).double()
    tol = 1e-12 if mode == 0 else 2e-2
    assert np.abs(out - ref.numpy()).max() <= tol * np.abs(ref.numpy()).max()


# --------------------------------------------------------------------------- planted mistakes
def _golden_graph_matches(path) -> bool:
    z, m = load_golden(path)
    B, N, M, H, d = m["B"], m["N"], m["M"], m["H"], m["d_head"]
    cfg = m["config"]
    rp = z["sd_lsh_builder.rand_proj"]
    R, P = rp.shape[0], m["p_eff"]
    res = oracle.lsh_forward(z["q"].reshape(B * H, N, d), z["k"].reshape(B * H, M, d), rp,
                             kv_rep=1, P=P, T=cfg["lsh_num_probes"], C=m["C"],
                             top_k=m["lsh_k"], causal=m["causal"], glob=z["glob"],
                             q_proj=z["qproj"].reshape(B * H, R, N, P),
                             k_proj=z["kproj"].reshape(B * H, R, M, P))
    nb, va = oracle.merge(z["win"], z["glob"], res["idx"], has_self=not m["cross"],
                          total_k=cfg["num_neighbors"])
    return (np.array_equal(res["idx"], z["lsh"].reshape(B * H, N, -1))
            and np.array_equal(nb, z["neighbors"].reshape(B * H, N, -1))
            and np.array_equal(va, z["valid"].reshape(B * H, N, -1)))


def _pinning_failures():
    """Names of the oracle's pinning checks that fail (golden vectors, library
    routines, closed forms)."""
    failed = []
    checks = [("sign rule", test_hash_sign_rule_and_bit_order),
              ("probe flips", test_probe_ids_flip_least_confident_bits_of_base),
              ("probe ties", test_probe_ties_keep_plane_order),
              ("empty bucket vector", test_oracle_empty_bucket_vector),
              ("ranked empty bucket vector", test_oracle_empty_bucket_list_competes_on_score),
              ("merge closed form", test_merge_closed_form),
              ("sort vs torch.sort", lambda: test_sort_perm_matches_torch_sort(2, 4096, 3,
                                                                              "uniform"))]
    for name, fn in checks:
        try:
            fn()
        except AssertionError:
            failed.append(name)
    for path in golden_files():
        if not _golden_graph_matches(path):
            failed.append(os.path.basename(path))
    return failed


MUTATIONS = {1: "stable sort", 2: "fillers do not mark their key", 3: "sign rule >= 0",
             4: "no causal substitution", 5: "no empty-bucket list", 6: "-inf slots -> 0",
             7: "cumulative probe flips", 8: "one unchunked top-k", 9: "self kept in merge pool"}


def test_faithful_oracle_passes_every_pinning_check():
    assert _pinning_failures() == []


@pytest.mark.parametrize("mut", sorted(MUTATIONS), ids=lambda m: MUTATIONS[m])
def test_planted_mistake_fails_a_pinning_check(mut):
    """Each plausible mistake in the restatement is caught by at least one of
    the checks that pin the oracle."""
    with oracle.mutation(mut):
        failed = _pinning_failures()
    assert failed, f"planted mistake '{MUTATIONS[mut]}' passes every pinning check"


# ---------------------------------------------------------------------------- CPU baseline
def _self_attention_fixtures():
    out = []
    for path in golden_files():
        z, m = load_golden(path)
        if not m["cross"] and m["config"]["global_token_indices"] is None:
            out.append(path)
    return out


@pytest.mark.parametrize("path", _self_attention_fixtures(), ids=os.path.basename)
def test_cpu_baseline_port_reproduces_reference_forward(path):
    """oracle/torch_port.forward, the timed CPU baseline, issues the reference's
    torch op sequence: its output is bit-identical to the reference's own
    SparseAttention.forward on every self-attention fixture."""
    import torch
    from oracle import torch_port
    z, m = load_golden(path)
    c = m["config"]
    dt = getattr(torch, m["dtype"])
    W = {n: torch.from_numpy(z["sd_" + n + ".weight"]).to(dt) for n in ("Wq", "Wk", "Wv", "Wo")}
    x = torch.from_numpy(z["x"]).to(dt)
    with torch.no_grad():
        out = torch_port.forward(
            x, W["Wq"], W["Wk"], W["Wv"], W["Wo"],
            torch.from_numpy(z["sd_lsh_builder.rand_proj"]), H=m["H"], n_kv=m["n_kv"],
            K=c["num_neighbors"], window=c["window_size"], glob_n=c["num_global_tokens"],
            R=c["num_hash_rounds"], max_p=c["max_num_hashes"], T=c["lsh_num_probes"],
            causal=m["causal"], fp32w=c["fp32_attn_weights"])
    assert torch.equal(out.float(), torch.from_numpy(z["out"]))


# ---------------------------------------------------------------------------- chunked top-k
def _chunked_topk(sc, ids, kk, chunk):
    """The reference's running top-k over stream chunks (sparse_attention.py:904-922)."""
    bs = np.full(kk, -np.inf, np.float32)
    bi = np.zeros(kk, np.int64)
    for s0 in range(0, len(sc), chunk):
        v, idx = oracle.topk_row(np.concatenate([bs, sc[s0:s0 + chunk]]), kk)
        bi = np.concatenate([bi, ids[s0:s0 + chunk]])[np.asarray(idx)]
        bs = np.asarray(v, np.float32)
    return bs, bi


def _decomposed_topk(sc, ids, kk, chunk, only_cut_ties):
    """The same result chunk by chunk from the states' sorted keys alone: a
    chunk replays on the previous state's keys with positions as payload only
    when equal finite keys reach its first kk + 1 merged places (for a set,
    only when that key is the final kk-th one); otherwise the sorted merge is
    its map.  Finite output slots are then followed back through the maps."""
    nch = (len(sc) + chunk - 1) // chunk
    S = np.full(kk, -np.inf, np.float32)
    maps, tied, states = [], [], []
    for s in range(nch):
        merged = np.concatenate([S, sc[s * chunk:(s + 1) * chunk]])
        order = sorted((i for i in range(len(merged)) if np.isfinite(merged[i])),
                       key=lambda i: (-merged[i], i >= kk))
        top = order[:kk + 1]
        tied.append({merged[top[t]] for t in range(min(kk, len(top) - 1))
                     if merged[top[t]] == merged[top[t + 1]]})
        states.append(S.copy())
        maps.append(top[:kk] + [0] * (kk - min(kk, len(top))))
        an = min(kk, len(order))
        S = np.full(kk, -np.inf, np.float32)
        S[:an] = merged[order[:an]]
    fcount = int(np.isfinite(S).sum())
    replayed = 0
    for s in range(nch):
        if only_cut_ties:
            need = fcount == kk and S[kk - 1] in tied[s]
        else:
            need = bool(tied[s])
        if need:
            _, idx = oracle.topk_row(np.concatenate([states[s], sc[s * chunk:(s + 1) * chunk]]), kk)
            maps[s] = list(np.asarray(idx))
            replayed += 1
    out = []
    for t in range(fcount):
        pos, slot = t, -1
        for s in range(nch - 1, -1, -1):
            tg = maps[s][pos]
            if tg >= kk:
                slot = s * chunk + tg - kk
                break
            pos = tg
        out.append(ids[slot])
    return S, np.array(out, np.int64), replayed


@pytest.mark.parametrize("only_cut_ties", [False, True])
def test_chunked_topk_decomposes_into_independent_chunks(only_cut_ties):
    """The workgroup tie replay's decomposition: per chunk on the states' keys,
    then followed back; the ordered list exactly, or the set (cut-key rule)."""
    rng = np.random.default_rng(11)
    replayed = chunks = 0
    for _ in range(150):
        kk = int(rng.choice([3, 8, 16, 32]))
        chunk = int(rng.choice([4 * kk, 256, 5 * kk + 3]))
        n = int(rng.integers(chunk // 2, 6 * chunk))
        sc = rng.integers(0, int(rng.choice([5, 20, 100, 1000])), n).astype(np.float32)
        sc[rng.random(n) < rng.choice([0.0, 0.3, 0.7])] = -np.inf
        ids = rng.permutation(10 * n)[:n].astype(np.int64)
        bs, bi = _chunked_topk(sc, ids, kk, chunk)
        S, out, r = _decomposed_topk(sc, ids, kk, chunk, only_cut_ties)
        f = int(np.isfinite(bs).sum())
        np.testing.assert_array_equal(S[:f], bs[:f])
        assert len(out) == f
        if only_cut_ties:
            assert sorted(out.tolist()) == sorted(bi[:f].tolist())
        else:
            np.testing.assert_array_equal(out, bi[:f])
        replayed += r
        chunks += (n + chunk - 1) // chunk
    assert 0 < replayed < chunks
