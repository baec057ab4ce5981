"""SparseTransformer and CachedGraphSparseTransformer against the reference's
own vectors (tests/golden/models, written by tests/golden/make_golden.py).

Per layer, with the reference's q / k / v and fp32 hash projections injected:
* the graph the layer builds (its own builders, or its group's shared ones in
  the cached model) equals the reference's bit for bit;
* a reused graph is the one its group's first layer built;
* the gather attention over the reference's graph matches the reference's
  attention output, and the whole layer (Wo, residual, LayerNorm, FFN) its
  output, per row within 1e-5 (fp32) or 2e-2 (bf16) of the row's largest
  magnitude.
End to end: the model's output and stats list from the same seed and inputs.
"""
import glob
import json
import os
import warnings

import numpy as np
import pytest
import torch

from conftest import GOLDEN, has_gpu

pytestmark = [pytest.mark.gpu, pytest.mark.skipif(not has_gpu(), reason="needs a ROCm GPU")]

DEV = "cuda"
MODELS = sorted(glob.glob(os.path.join(GOLDEN, "models", "*.npz")))
TOL = {"float32": 1e-5, "bfloat16": 2e-2}


def _load(path):
    z = np.load(path)
    return z, json.loads(str(z["meta"]))


def _model(z, m):
    from ssa_amd import CachedGraphSparseTransformer, SSAConfig, SparseTransformer
    cfg = SSAConfig(**m["config"])
    torch.manual_seed(m["seed"])
    with warnings.catch_warnings():
        warnings.simplefilter("ignore")
        if m["kind"] == "transformer":
            model = SparseTransformer(cfg, num_layers=m["num_layers"], vocab_size=50)
        else:
            model = CachedGraphSparseTransformer(cfg, num_layers=m["num_layers"], reuse_every=2)
    # seeded construction draws the reference's weights and hyperplanes
    sd = model.state_dict()
    ref_keys = sorted(k[3:] for k in z.files if k.startswith("sd_"))
    assert sorted(sd.keys()) == ref_keys
    for key in ref_keys:
        np.testing.assert_array_equal(sd[key].numpy(), z["sd_" + key], err_msg=key)
    model = model.to(DEV)
    dt = getattr(torch, m["dtype"])
    for p in model.parameters():
        p.data = p.data.to(dt)
    return model.eval(), dt


def _rows_close(got, ref, tol, what):
    """max over rows of |got - ref|_inf / |ref|_inf (rows: the last dim)."""
    g = got.detach().float().cpu().numpy().reshape(-1, got.shape[-1]).astype(np.float64)
    r = np.asarray(ref, np.float64).reshape(-1, got.shape[-1])
    scale = np.maximum(np.abs(r).max(-1), 1e-30)
    err = (np.abs(g - r).max(-1) / scale).max()
    assert err <= tol, f"{what}: worst row relative error {err:.3g} > {tol}"
    return err


def _t(z, key, dt=None):
    t = torch.from_numpy(np.ascontiguousarray(z[key])).to(DEV)
    return t.to(dt) if dt is not None else t


@pytest.mark.parametrize("path", MODELS, ids=os.path.basename)
def test_every_layer_matches_reference(path):
    z, m = _load(path)
    model, dt = _model(z, m)
    B, N = m["B"], m["N"]
    tol = TOL[m["dtype"]]
    built = None
    worst = 0.0
    with torch.no_grad():
        for li, layer in enumerate(model.layers):
            attn = layer.attn
            q, k, v = _t(z, f"l{li}_q", dt), _t(z, f"l{li}_k", dt), _t(z, f"l{li}_v", dt)
            nb_ref, va_ref = _t(z, f"l{li}_neighbors"), _t(z, f"l{li}_valid")
            recompute = bool(z[f"l{li}_recompute"])
            assert recompute == (m["kind"] == "transformer" or
                                 m["stats"][li]["graph_recomputed"])
            if m["kind"] == "transformer":
                builder = attn
            else:
                builder = model.shared_attn_per_group[model.group_of[li]]
            if recompute:
                proj = (_t(z, f"l{li}_qproj"), _t(z, f"l{li}_kproj"))
                nb, va = builder.build_graph(q, k, N, N, B, DEV, attn.config.causal, False,
                                             _proj=proj)
                assert torch.equal(nb, nb_ref), f"layer {li}: neighbours differ"
                assert torch.equal(va, va_ref), f"layer {li}: valid masks differ"
                built = (nb, va)
            else:
                # the reference reuses its group's graph
                assert torch.equal(built[0], nb_ref) and torch.equal(built[1], va_ref)
            out = attn.apply_graph(q, k, v, nb_ref, va_ref)
            worst = max(worst, _rows_close(out, z[f"l{li}_attn_out"], tol,
                                           f"layer {li} attention"))
            h = _t(z, f"l{li}_in", dt)
            a = attn.Wo(attn._merge(out))
            h_next = h + a + layer.ff(layer.norm2(h + a))
            worst = max(worst, _rows_close(h_next, z[f"l{li}_out"], tol, f"layer {li} output"))
    print(f"  {os.path.basename(path)}: worst row error {worst:.2e}", flush=True)


def _capture_graphs(model, kind):
    """Record the graph every layer's attention uses during a forward, as
    (neighbors, valid) per layer in layer order."""
    seen = []
    if kind == "transformer":
        for layer in model.layers:
            attn = layer.attn
            orig = attn._build_graph_ids32

            def wrap(*a, _orig=orig, **kw):
                ids = _orig(*a, **kw)
                seen.append((ids.long().clamp_min(0), ids >= 0))
                return ids
            attn._build_graph_ids32 = wrap
    else:
        for builder in model.shared_attn_per_group:
            orig = builder.build_graph

            def wrap(*a, _orig=orig, **kw):
                nb, va = _orig(*a, **kw)
                seen.append((nb, va))
                return nb, va
            builder.build_graph = wrap
    return seen


# Tokens of each bf16 fixture (B * N = 192) affected by a graph difference,
# bounded near what the device's GEMMs give (0, 0, 8 and 0 measured, about
# twice that allowed); fp32 must have none.
AFFECTED_MAX = {"cached_bf16_seed0": 4, "cached_bf16_seed1": 4,
                "transformer_bf16_seed0": 16, "transformer_bf16_seed1": 4}


@pytest.mark.parametrize("path", MODELS, ids=os.path.basename)
def test_model_forward_matches_reference(path):
    """The whole model from the same seed and inputs.  Its layers' q and k come
    from the device's GEMMs, whose rounding differs from the reference's CPU
    GEMMs, so in bf16 a hash bit or a near-tied score can come out the other
    way.  Every layer's graph is therefore compared with the reference's, and
    a token counts as affected when its own graph differs in some layer or it
    attends to a token that was affected in the layer before; every token
    that is not affected must match the reference's output.  fp32 must match
    everywhere, stats included."""
    z, m = _load(path)
    model, dt = _model(z, m)
    tol = TOL[m["dtype"]]
    seen = _capture_graphs(model, m["kind"])
    with torch.no_grad():
        x = _t(z, "ids") if m["kind"] == "transformer" else _t(z, "x", dt)
        out, stats = model(x, return_stats=True)
    torch.cuda.synchronize()
    B, N, L = m["B"], m["N"], m["num_layers"]
    assert len(stats) == L
    # the graph each layer used
    if m["kind"] == "transformer":
        graphs = seen
    else:
        graphs, gi = [], -1
        for li in range(L):
            if bool(z[f"l{li}_recompute"]):
                gi += 1
            graphs.append(seen[gi])
    assert len(graphs) == L
    affected = np.zeros((B, N), bool)
    n_diff = 0
    for li in range(L):
        nb, va = (t.cpu().numpy() for t in graphs[li])
        rnb, rva = z[f"l{li}_neighbors"], z[f"l{li}_valid"]
        differs = ((nb != rnb) | (va != rva)).any(-1).any(1)          # (B, N) over heads
        n_diff += int(differs.sum())
        # tokens reading an affected key through a valid slot
        reads = np.zeros((B, N), bool)
        for b in range(B):
            bad = np.flatnonzero(affected[b])
            if bad.size:
                hit = np.isin(nb[b], bad) & va[b]
                reads[b] = hit.any(-1).any(0)
        affected = affected | differs | reads
    if m["dtype"] == "float32":
        assert n_diff == 0, f"{n_diff} token graphs differ in fp32"
    for got, ref in zip(stats, m["stats"]):
        assert set(got) == set(ref)
        for key, val in ref.items():
            gv = list(got[key]) if isinstance(got[key], tuple) else got[key]
            if key == "padding_fraction" and n_diff:
                assert abs(gv - val) <= 0.01, (key, gv, val)
            else:
                assert gv == val, (key, gv, val)
    keep = ~affected
    name = os.path.basename(path)[:-4]
    print(f"  {name}: token graphs differing {n_diff}, tokens affected "
          f"{int(affected.sum())} of {B * N}", flush=True)
    assert int(affected.sum()) <= AFFECTED_MAX.get(name, 0), "more tokens affected than measured"
    err = _rows_close(out[torch.from_numpy(keep).to(DEV)],
                      z["out"][keep], tol, "model output (unaffected tokens)")
    print(f"  output worst row error {err:.2e}", flush=True)
