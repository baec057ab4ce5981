"""Benchmark: SparseAttention forward tokens/s on one MI355X.

Workload (default): bf16 GQA SparseAttention, d_model=4096, 32 query heads /
8 kv heads (d_head=128), batch 1, N=4096, K=128, window 16, 2 global tokens,
8 hash rounds, causal.  Weights: seeded construction, Wq/Wk/Wv/Wo re-drawn
with xavier_uniform_ in that order, parameters cast to bf16 (the hyperplanes
stay fp32); x = 0.02 * N(0, 1) in bf16 from a generator seeded 1000.

One "step" = one SparseAttention.forward (projections, graph build, gather
attention, output projection) on inputs already resident in HBM.

Also reported:
* roofline of the gather-attention kernel, priced against the resource that
  bounds it: the L2-to-CU delivery rate (`bound` "l2", below).  Its
  algorithmic bytes per launch B*H*N*(2*K_out*d + 2*d)*2 (K and V row
  gathers, q read, out write) over the kernel's average duration, measured
  with events on the launch stream, are kept as `algorithmic_rate`; over the
  8 TB/s HBM peak they exceed 1 (`algorithmic_rate_over_hbm_peak`) because the
  gathered rows repeat and the L2 serves them;
* recall@32 of the graph against exact dense top-32 (head 0 and all heads);
* cpu_baseline: the reference's torch op sequence (oracle/torch_port.py) on
  the host cores over the whole workload (about 20 s a run on 16 cores,
  about 50 GB of host memory);
* roofline.traffic / hbm_frac: HBM bytes per apply launch from the committed
  rocprofv3 FETCH_SIZE/WRITE_SIZE summary (profiles/hbm_traffic_bf16_gqa_n4096.md)
  and the share of the 8 TB/s peak they use;
* roofline.achieved / peak / frac: bytes the CUs' L1 caches requested from
  the L2 per launch (TCP_TCC_READ_REQ from the committed summary
  profiles/l2_traffic_bf16_gqa_n4096.md, times the bytes per request measured
  on a plain copy) over the launch time, against the L2-to-CU rate measured
  live here with ssa_measure_l2_read (every CU streaming an L2-resident
  buffer with 16-byte loads); roofline.published_peak is the L2's read width
  as AMD describes the XCD (16 channels x 128 B per clock, 8 XCDs) at the
  2.4 GHz peak engine clock.

`--workload NAME` measures one of the other workload shapes instead (no CPU
baseline): fp32_b2_n1024, mqa_n32768, cross_fp32, cross_bf16, transformer6.
Each is built as the full-size GPU tests build it (seeded construction, the
same input recipe) and reports forward tokens/s plus the apply kernel's
event-timed roofline.

Usage: python bench.py [--gpus 1] [--steps 20] [--warmup 5] [--no-cpu]
                       [--workload NAME]
"""
import argparse
import json
import os
import sys
import time
import warnings

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

PEAK_HBM = 8.0e12
# L2 read width of the 8 XCDs: 16 channels x 128 B per clock each, at 2.4 GHz
PEAK_L2_PUBLISHED = 8 * 16 * 128 * 2.4e9


def build_module(dev):
    import torch
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
    attn = attn.to(dev)
    for p in attn.parameters():
        p.data = p.data.to(torch.bfloat16)
    attn.eval()
    g = torch.Generator().manual_seed(1000)
    x = (torch.randn(1, 4096, 4096, generator=g) * 0.02).to(torch.bfloat16).to(dev)
    return cfg, attn, x


# The other workload shapes: (description, SSAConfig fields, B, N, M (cross), dtype,
# x scale, xavier re-init)
OTHER = {
    "fp32_b2_n1024": ("SparseAttention fp32 causal, d_model=512, 8 heads (d_head=64), B=2, "
                      "N=1024, K=128, window=8, 2 global tokens, R=8",
                      dict(d_model=512, num_heads=8, num_neighbors=128, window_size=8,
                           num_global_tokens=2, num_hash_rounds=8, max_num_hashes=12,
                           lsh_num_probes=0, causal=True), 2, 1024, None, "f32", 1.0),
    "mqa_n32768": ("SparseAttention bf16 MQA causal, d_model=4096, 32 q heads / 1 kv head "
                   "(d_head=128), B=1, N=32768, K=256, window=32, globals [0,1,16384], R=8, "
                   "2 probes",
                   dict(d_model=4096, num_heads=32, num_kv_heads=1, num_neighbors=256,
                        window_size=32, global_token_indices=[0, 1, 16384], num_hash_rounds=8,
                        max_num_hashes=12, lsh_num_probes=2, causal=True),
                   1, 32768, None, "bf16", 1.0),
    "cross_fp32": ("SparseAttention fp32 cross-attention, d_model=1024, 16 heads (d_head=64), "
                   "B=4, 2048 queries over 512 keys, K=64, window=4, 2 global tokens, R=6",
                   dict(d_model=1024, num_heads=16, num_neighbors=64, window_size=4,
                        num_global_tokens=2, num_hash_rounds=6, max_num_hashes=12,
                        lsh_num_probes=0, causal=False), 4, 2048, 512, "f32", 1.0),
    "cross_bf16": ("SparseAttention bf16 cross-attention, d_model=1024, 16 heads (d_head=64), "
                   "B=4, 2048 queries over 512 keys, K=64, window=4, 2 global tokens, R=6",
                   dict(d_model=1024, num_heads=16, num_neighbors=64, window_size=4,
                        num_global_tokens=2, num_hash_rounds=6, max_num_hashes=12,
                        lsh_num_probes=0, causal=False), 4, 2048, 512, "bf16", 1.0),
    "transformer6": ("SparseTransformer, 6 layers, d_model=1024, 16 q heads / 4 kv heads, "
                     "vocab 32000, B=2, N=8192, K=128, window=16, R=8, 1 probe, causal, bf16, "
                     "return_stats=True",
                     dict(d_model=1024, num_heads=16, num_kv_heads=4, num_neighbors=128,
                          window_size=16, num_hash_rounds=8, lsh_num_probes=1, causal=True),
                     2, 8192, None, "bf16", None),
}


def _set_fuse(model, on):
    """Whether bf16 forwards take the library's projections with the hash in
    their epilogue or (the default) torch's projections and a separate hash."""
    from ssa_amd import SparseAttention
    for m in model.modules():
        if isinstance(m, SparseAttention):
            m._fuse_projections = on


def _timed(fn, steps, warmup):
    import torch
    for _ in range(warmup):
        fn()
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(steps):
        fn()
    torch.cuda.synchronize()
    return (time.perf_counter() - t0) / steps


def _stage_times(attn, q, k, v, N, M, B, causal, cross, reps):
    """build and apply as forward runs them without autograd (int32 ids), each
    bracketed by events on the launch stream."""
    import torch
    st = torch.cuda.current_stream()
    evs = [[torch.cuda.Event(enable_timing=True) for _ in range(3)] for _ in range(reps)]
    for e in evs:
        e[0].record(st)
        ids = attn._build_graph_ids32(q, k, N, M, B, causal, cross)
        e[1].record(st)
        attn.apply_graph(q, k, v, ids, None)
        e[2].record(st)
    torch.cuda.synchronize()
    t_build = sum(e[0].elapsed_time(e[1]) for e in evs) / reps
    t_apply = sum(e[1].elapsed_time(e[2]) for e in evs) / reps
    return t_build, t_apply, ids.shape[-1]


def other_workload(name, args):
    import torch
    from ssa_amd import SSAConfig, SparseAttention, SparseTransformer
    desc, cfg_kw, B, N, M, dt, xscale = OTHER[name]
    dtype = torch.float32 if dt == "f32" else torch.bfloat16
    dev = "cuda:0"
    torch.manual_seed(0)
    g = torch.Generator().manual_seed(1000)
    with warnings.catch_warnings():
        warnings.simplefilter("ignore")
        if name == "transformer6":
            model = SparseTransformer(SSAConfig(**cfg_kw), num_layers=6, vocab_size=32000)
        else:
            model = SparseAttention(SSAConfig(**cfg_kw))
    model = model.to(dev)
    for p in model.parameters():
        p.data = p.data.to(dtype)
    model.eval()
    _set_fuse(model, args.fuse)
    with torch.no_grad():
        if name == "transformer6":
            ids = torch.randint(0, 32000, (B, N), generator=g).to(dev)
            t = _timed(lambda: model(ids, return_stats=True), args.steps, args.warmup)
            # the stage timing and roofline of layer 0's attention, on its own input
            attn = model.layers[0].attn
            src = xin = model.layers[0].norm1(model.embed(ids))
        else:
            attn = model
            xin = (torch.randn(B, N, cfg_kw["d_model"], generator=g) * xscale).to(dtype).to(dev)
            src = (torch.randn(B, M, cfg_kw["d_model"], generator=g).to(dtype).to(dev)
                   if M else xin)
            kv = src if M else None
            t = _timed(lambda: model(xin, key_value=kv), args.steps, args.warmup)
        Mk = src.shape[1]
        cross = M is not None
        causal = cfg_kw.get("causal", False) and not cross
        q = attn._split_q(attn.Wq(xin))
        k = attn._split_kv_compact(attn.Wk(src))
        v = attn._split_kv_compact(attn.Wv(src))
        t_build, t_apply, K_out = _stage_times(attn, q, k, v, N, Mk, B, causal, cross,
                                               max(args.steps, 5))
    esize = 4 if dtype == torch.float32 else 2
    bytes_apply = B * attn.H * N * (2 * K_out * attn.d_head + 2 * attn.d_head) * esize
    l2_rate, l2_setup = measure_l2_peak(dev)
    l2_share = _l2_profile_value("l2share", "l2_read_kernel")
    l2_peak = l2_rate * (l2_share if l2_share is not None else 1.0)
    l2_setup["l2_share"] = l2_share
    l2_bytes = workload_l2_bytes(name)
    line = {
        "metric": "sparse-attn fwd tokens/sec at N=4096,K=128; % HBM roofline; recall@32",
        "value": B * N / t, "unit": "tokens/s", "n_gpus": 1, "steps": args.steps,
        "warmup": args.warmup, "ms_per_step": t * 1000.0, "higher_is_better": True,
        "scaling": "weak", "vs_baseline": None, "dtype": dt, "data": "synthetic",
        "config": {"workload": desc, "global_batch": B, "seq_len": N,
                   "parallelism": "single GPU"},
        "roofline": l2_roofline(
            "apply (" + ("layer 0, " if name == "transformer6" else "") + "gather attention)",
            t_apply, l2_bytes, l2_peak, l2_setup, bytes_apply, None),
        "t_build_ms": t_build, "t_apply_ms": t_apply, "k_out": K_out,
        "cpu_baseline": None,
    }
    print(json.dumps(line), flush=True)


def recall_at_32(q, k, nb, va, rep, causal_variant=False):
    """Reference method (tests/test_quality_and_scaling.py:80-95): dense unscaled
    top-32 per query vs the valid neighbours; returns (head 0, all-head mean)."""
    import torch
    B, H, N, d = q.shape
    res = []
    for h in range(H):
        qs = q[0, h].float()
        ks = k[0, h // rep].float()
        s = qs @ ks.T
        if causal_variant:
            s = s.masked_fill(torch.ones_like(s, dtype=torch.bool).triu(1), float("-inf"))
        top = s.topk(32, dim=-1).indices
        hit = ((nb[0, h].unsqueeze(-1) == top.unsqueeze(1)) & va[0, h].unsqueeze(-1)).any(1)
        if causal_variant:
            tk = torch.clamp(torch.arange(N, device=q.device) + 1, max=32).float()
            valid_top = torch.isfinite(torch.gather(s, 1, top))
            r = (hit & valid_top).sum(-1).float() / tk
        else:
            r = hit.sum(-1).float() / 32.0
        res.append(r.mean().item())
    return res[0], sum(res) / len(res)


def select_read_stats(attn, q, k, N):
    """What select_kernel reads per query row at this workload (causal self
    attention, B=1), from the same hashing, permutation and cut rules on the
    device: per (row, list) the members below the query (the sorted list's
    prefix), the 64-member chunks that cover them, and the bytes those chunks
    load (4 B member id + 2 B score code per lane, whole chunks) against the
    bytes of the members themselves.  The permutation is torch.sort's on the
    host (the reference's, which the library reproduces)."""
    import torch
    lb = attn.lsh_builder
    C, R = lb.C, lb.rand_proj.shape[0]
    P = lb.compute_effective_p(N, C, lb.max_P)
    Hq, Hkv, rep = attn.H, attn.n_kv, attn.kv_rep
    planes = lb.rand_proj[:, :P].float()                                   # (R, P, d)
    w = (2 ** torch.arange(P, device=q.device)).view(1, 1, P)
    members = torch.zeros(Hq, N, device=q.device)
    chunks = torch.zeros(Hq, N, device=q.device)
    nlists = 0
    for r in range(R):
        kid = ((k[0].float() @ planes[r].T > 0).long() * w).sum(-1)        # (Hkv, M)
        qid = ((q[0].float() @ planes[r].T > 0).long() * w).sum(-1)        # (Hq, N)
        for g in range(Hkv):
            perm = torch.sort(kid[g].cpu(), dim=-1)[1].to(q.device)        # the reference's order
            skey = kid[g][perm]
            for h in range(g * rep, (g + 1) * rep):
                cut = torch.zeros(N, device=q.device)
                for u in range(2 ** P):
                    sel = perm[skey == u][:C]                               # the list: first C members
                    lst = torch.sort(sel)[0]
                    rows = qid[h] == u
                    n = torch.arange(N, device=q.device)[rows]
                    cut[rows] = torch.searchsorted(lst, n).float()          # members below the query
                members[h] += cut
                chunks[h] += torch.ceil(cut / 64)
        nlists += 1
    loaded = chunks * 64 * 6
    needed = members * 6
    return {"lists_per_row": nlists, "members_per_row": members.mean().item(),
            "chunks_per_row": chunks.mean().item(),
            "chunk_fill": (members.sum() / (chunks.sum() * 64)).item(),
            "bytes_loaded_per_row": loaded.mean().item(),
            "bytes_of_members_per_row": needed.mean().item(),
            "cut_and_aux_bytes_per_row": nlists * 20 + (attn.config.num_global_tokens + 3) * 4}


# the apply kernel the bf16 workload launches (16-bit packed path)
APPLY_KERNEL = "apply_fwd16_kernel"


def measured_traffic(kernel):
    """HBM bytes per launch of `kernel` from the committed rocprofv3 FETCH_SIZE /
    WRITE_SIZE summary (a line `traffic <kernel> <bytes>`), or None."""
    path = os.path.join(ROOT, "profiles", "hbm_traffic_bf16_gqa_n4096.md")
    try:
        with open(path) as f:
            for line in f:
                parts = line.strip().strip("`").split()
                if len(parts) == 3 and parts[0] == "traffic" and parts[1] == kernel:
                    return int(parts[2])
    except OSError:
        pass
    return None


def _l2_profile_value(tag, kernel):
    """A `<tag> <kernel> <value>` line of the committed rocprofv3 summary
    profiles/l2_traffic_bf16_gqa_n4096.md, or None."""
    path = os.path.join(ROOT, "profiles", "l2_traffic_bf16_gqa_n4096.md")
    try:
        with open(path) as f:
            for line in f:
                parts = line.strip().strip("`").split()
                if len(parts) == 3 and parts[0] == tag and parts[1] == kernel:
                    return float(parts[2])
    except OSError:
        pass
    return None


def l2_bytes_per_launch(kernel):
    """Bytes the CUs' L1 caches requested from the L2 per launch of `kernel`
    (TCP_TCC_READ_REQ x 128 bytes), or None."""
    v = _l2_profile_value("l2bytes", kernel)
    return None if v is None else int(v)


def workload_l2_bytes(workload):
    """L2-to-CU bytes per gather-attention launch of another workload shape
    from the committed summary profiles/l2_traffic_workloads.md (a line
    `l2bytes <workload> <bytes>`), or None."""
    path = os.path.join(ROOT, "profiles", "l2_traffic_workloads.md")
    try:
        with open(path) as f:
            for line in f:
                parts = line.strip().strip("`").split()
                if len(parts) == 3 and parts[0] == "l2bytes" and parts[1] == workload:
                    return int(parts[2])
    except OSError:
        pass
    return None


def l2_roofline(kernel, t_apply_ms, l2_bytes, l2_peak, l2_setup, alg_bytes, hbm_bytes):
    """The gather kernel's roofline.  Its K/V rows repeat across queries and
    the L2 serves them (97% hits), so its bound is the L2-to-CU delivery
    rate: the bytes its L1 caches requested from the L2 per launch over the
    launch time, against that rate measured live (ssa_measure_l2_read).  HBM
    carries about 2% of the algorithmic bytes (hbm_frac, from the measured
    FETCH_SIZE + WRITE_SIZE); the algorithmic bytes over the HBM peak are
    kept under their own name, and exceed 1."""
    t = t_apply_ms / 1000.0
    ach = l2_bytes / t if l2_bytes is not None else None
    return {"bound": "l2", "resource": "L2 to CU",
            "achieved": ach / 1e9 if ach is not None else None,
            "peak": l2_peak / 1e9, "unit": "GB/s",
            "frac": ach / l2_peak if ach is not None else None,
            "traffic": hbm_bytes,
            "kernel": kernel, "ms_per_launch": t_apply_ms,
            "l2_bytes_per_launch": l2_bytes,
            "peak_kernel": "ssa_measure_l2_read", "peak_setup": l2_setup,
            "published_peak": PEAK_L2_PUBLISHED / 1e9,
            "published_frac": ach / PEAK_L2_PUBLISHED if ach is not None else None,
            "hbm_frac": hbm_bytes / t / PEAK_HBM if hbm_bytes is not None else None,
            "algorithmic_bytes_per_launch": alg_bytes,
            "algorithmic_rate": alg_bytes / t / 1e9,
            "algorithmic_rate_over_hbm_peak": alg_bytes / t / PEAK_HBM}


def measure_l2_peak(dev, reps=5):
    """Load rate (bytes/s) of ssa_measure_l2_read with 8 workgroups of 256
    threads per CU, each streaming the same 1 MiB buffer 8 times (the buffer
    stays in every XCD's 4 MiB L2; a CU's L1 is 32 KiB), timed with events on
    the launch stream; the best of `reps` launches after one warm-up."""
    import torch
    from ssa_amd import _lib
    nbytes, iters = 1 << 20, 8
    cus = torch.cuda.get_device_properties(dev).multi_processor_count
    blocks = 8 * cus
    buf = torch.randint(0, 255, (nbytes,), dtype=torch.uint8, device=dev)
    sink = torch.zeros(blocks, dtype=torch.int32, device=dev)
    st = torch.cuda.current_stream()
    _lib.measure_l2_read(buf, blocks, iters, sink)
    best = None
    for _ in range(reps):
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record(st)
        _lib.measure_l2_read(buf, blocks, iters, sink)
        e1.record(st)
        torch.cuda.synchronize()
        t = e0.elapsed_time(e1) / 1000.0
        best = t if best is None or t < best else best
    return blocks * nbytes * iters / best, {"blocks": blocks, "buffer_bytes": nbytes,
                                            "iters": iters, "cus": cus}


def host_info():
    model, mem = "", None
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    model = line.split(":", 1)[1].strip()
                    break
        with open("/proc/meminfo") as f:
            for line in f:
                if line.startswith("MemTotal"):
                    mem = int(line.split()[1]) * 1024
                    break
    except OSError:
        pass
    return model, mem


def cpu_baseline(attn_gpu):
    """Time the reference's CPU op sequence on the whole workload: one warm-up
    on one kv-head group, then two runs over all of it (every head, no
    scaling); the faster run is the figure."""
    import torch
    from oracle import torch_port
    cfg = attn_gpu.config
    # the cores this process may use: its CPU affinity, which on a shared GPU
    # host is the job's share (os.cpu_count() counts every core of the host)
    try:
        nthreads = len(os.sched_getaffinity(0))
    except AttributeError:
        nthreads = os.cpu_count() or 1
    omp = os.environ.get("OMP_NUM_THREADS")
    if omp:
        nthreads = min(nthreads, int(omp))
    torch.set_num_threads(nthreads)
    rep = attn_gpu.kv_rep
    d = attn_gpu.d_head
    groups = cfg.num_heads // rep
    rp = attn_gpu.lsh_builder.rand_proj.detach().cpu()
    g = torch.Generator().manual_seed(1000)
    x = (torch.randn(1, 4096, 4096, generator=g) * 0.02).to(torch.bfloat16)

    def run(ng):
        Wq = attn_gpu.Wq.weight[: ng * rep * d].detach().cpu()
        Wk = attn_gpu.Wk.weight[: ng * d].detach().cpu()
        Wv = attn_gpu.Wv.weight[: ng * d].detach().cpu()
        Wo = attn_gpu.Wo.weight[:, : ng * rep * d].detach().cpu()
        kw = dict(H=ng * rep, n_kv=ng, K=cfg.num_neighbors, window=cfg.window_size,
                  glob_n=cfg.num_global_tokens, R=cfg.num_hash_rounds,
                  max_p=cfg.max_num_hashes, T=cfg.lsh_num_probes, causal=cfg.causal)
        t0 = time.perf_counter()
        with torch.no_grad():
            torch_port.forward(x, Wq, Wk, Wv, Wo, rp, **kw)
        return time.perf_counter() - t0

    tw = run(1)
    print(f"# cpu warm-up (1 of {groups} kv groups): {tw:.2f} s", file=sys.stderr, flush=True)
    times = []
    for i in range(2):
        times.append(run(groups))
        print(f"# cpu run {i} (whole workload): {times[-1]:.2f} s", file=sys.stderr, flush=True)
    t = min(times)
    model, mem = host_info()
    return {"value": 4096 / t, "unit": "tokens/s", "cores": torch.get_num_threads(),
            "kind": "port",
            "sample": f"the whole workload ({cfg.num_heads} query heads, {groups} kv heads, "
                      f"N=4096, projections included) through the reference's torch CPU op "
                      f"sequence (oracle/torch_port.py, bit-identical to the reference on its "
                      f"fixtures) on {torch.get_num_threads()} threads; faster of two runs "
                      f"({times[0]:.2f} s, {times[1]:.2f} s) after a warm-up on one kv group; "
                      f"no scaling; CPU: {model}",
            "os_cpu_count": os.cpu_count(), "omp_num_threads": os.environ.get("OMP_NUM_THREADS"),
            "host_ram_bytes": mem}


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--no-recall", action="store_true")
    ap.add_argument("--select-stats", action="store_true",
                    help="also report what select_kernel reads per query row (select_reads)")
    ap.add_argument("--workload", default="gqa_n4096",
                    choices=["gqa_n4096"] + sorted(OTHER),
                    help="gqa_n4096 (default): the bf16 GQA N=4096 workload above")
    ap.add_argument("--fuse", action="store_true",
                    help="bf16 models: the library's projections with the hash in their "
                         "epilogue (ssa_project_build_graph) instead of torch's projections and "
                         "the build's hash pass")
    ap.add_argument("--calibrate-copy", action="store_true",
                    help="first run a plain bf16 copy kernel (x*1, 256 MiB in, 256 MiB out) "
                         "5 times, as the reference point for rocprofv3 FETCH_SIZE/WRITE_SIZE")
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py: measures one GPU; --gpus {args.gpus} is not supported (the sparse "
              "forward would shard by kv-head group, with no exchange inside attention).",
              file=sys.stderr)
        sys.exit(2)
    import torch
    dev = "cuda:0"
    if args.workload != "gqa_n4096":
        other_workload(args.workload, args)
        return
    if args.calibrate_copy:
        n = 128 << 20
        src = torch.ones(n, dtype=torch.bfloat16, device=dev)
        dst = torch.empty_like(src)
        for _ in range(5):
            torch.mul(src, 1, out=dst)
        torch.cuda.synchronize()
        print(f"# copy calibration: 5 x (read {2 * n} B, write {2 * n} B)", file=sys.stderr,
              flush=True)
        del src, dst
    cfg, attn, x = build_module(dev)
    _set_fuse(attn, args.fuse)
    B, N = x.shape[0], x.shape[1]
    H, d, K = attn.H, attn.d_head, attn.K
    print("# workload built", file=sys.stderr, flush=True)

    with torch.no_grad():
        for _ in range(args.warmup):
            attn(x)
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        for _ in range(args.steps):
            attn(x)
        torch.cuda.synchronize()
        t1 = time.perf_counter()
    ms = (t1 - t0) * 1000.0 / args.steps
    value = B * N / ((t1 - t0) / args.steps)
    print(f"# forward {ms:.3f} ms/step", file=sys.stderr, flush=True)

    # per-stage timing with events on the launch stream (torch's current stream):
    # build then apply as forward runs them without autograd (the graph as int32
    # ids, -1 = invalid), each stage bracketed by its own events so that the
    # apply launches see the same cache state as in forward
    with torch.no_grad():
        q = attn._split_q(attn.Wq(x))
        k = attn._split_kv_compact(attn.Wk(x))
        v = attn._split_kv_compact(attn.Wv(x))
        st = torch.cuda.current_stream()
        reps = max(args.steps, 10)
        evs = [[torch.cuda.Event(enable_timing=True) for _ in range(3)] for _ in range(reps)]
        for e in evs:
            e[0].record(st)
            ids = attn._build_graph_ids32(q, k, N, N, B, True, False)
            e[1].record(st)
            out = attn.apply_graph(q, k, v, ids, None)
            e[2].record(st)
        torch.cuda.synchronize()
        # apply alone, back to back on one graph: K/V rows, q and the index
        # table stay cache-resident, so this is the gather path's warm rate
        ew = [torch.cuda.Event(enable_timing=True) for _ in range(2)]
        out = attn.apply_graph(q, k, v, ids, None)
        ew[0].record(st)
        for _ in range(reps):
            out = attn.apply_graph(q, k, v, ids, None)
        ew[1].record(st)
        torch.cuda.synchronize()
    t_apply_warm = ew[0].elapsed_time(ew[1]) / reps
    t_build = sum(e[0].elapsed_time(e[1]) for e in evs) / reps
    t_apply = sum(e[1].elapsed_time(e[2]) for e in evs) / reps
    K_out = ids.shape[-1]
    bytes_apply = B * H * N * (2 * K_out * d + 2 * d) * 2
    traffic = measured_traffic(APPLY_KERNEL)
    print(f"# build {t_build:.3f} ms, apply {t_apply:.3f} ms", file=sys.stderr, flush=True)
    l2_rate, l2_setup = measure_l2_peak(dev)
    # the share of the reference kernel's loads that the L2 served (the rest
    # hit in L1), from the same counters as the apply kernel's L2 bytes
    l2_share = _l2_profile_value("l2share", "l2_read_kernel")
    l2_peak = l2_rate * (l2_share if l2_share is not None else 1.0)
    l2_setup["l2_share"] = l2_share
    l2_bytes = l2_bytes_per_launch(APPLY_KERNEL)
    print(f"# L2-to-CU delivery {l2_peak / 1e12:.2f} TB/s", file=sys.stderr, flush=True)

    # rows whose k-th LSH score is tied (selection decided by the tie rule)
    from ssa_amd import _lib
    with torch.no_grad():
        lb = attn.lsh_builder
        p_eff = lb.compute_effective_p(N, lb.C, lb.max_P)
        _, _, ties = _lib.build_graph(q, k, lb.rand_proj, P=p_eff, T=lb.T, C=lb.C,
                                      top_k=attn.lsh_k, window=cfg.window_size, causal=True,
                                      is_cross=False, total_k=K, glob=attn.glob_builder(N, dev),
                                      count_ties=True)
        tie_rows = int(ties.item())

    rec = None
    if not args.no_recall:
        with torch.no_grad():
            nb, va = ids.long().clamp_min(0), ids >= 0      # build_graph's (neighbors, valid)
            r0, rall = recall_at_32(q, k, nb, va, attn.kv_rep)
            c0, call = recall_at_32(q, k, nb, va, attn.kv_rep, causal_variant=True)
        rec = {"head0": r0, "all_heads": rall, "causal_head0": c0, "causal_all_heads": call}

    line = {
        "metric": "sparse-attn fwd tokens/sec at N=4096,K=128; % HBM roofline; recall@32",
        "value": value, "unit": "tokens/s", "n_gpus": 1, "steps": args.steps,
        "warmup": args.warmup, "ms_per_step": ms, "higher_is_better": True,
        "scaling": "weak", "vs_baseline": None, "dtype": "bf16", "data": "synthetic",
        "config": {"workload": "SparseAttention bf16 GQA forward, d_model=4096, 32 q heads / "
                               "8 kv heads (d_head=128), B=1, N=4096, K=128, window=16, "
                               "2 global tokens, R=8, causal",
                   "global_batch": B, "seq_len": N, "parallelism": "single GPU"},
        "roofline": l2_roofline(APPLY_KERNEL, t_apply, l2_bytes, l2_peak, l2_setup,
                                bytes_apply, traffic),
        "t_build_ms": t_build, "t_apply_ms": t_apply, "t_apply_warm_ms": t_apply_warm,
        "k_out": K_out,
        "tie_rows": tie_rows, "query_rows": B * H * N,
        "recall_at_32": rec,
    }
    if args.select_stats:
        with torch.no_grad():
            line["select_reads"] = select_read_stats(attn, q, k, N)
    if not args.no_cpu:
        cb = cpu_baseline(attn)
        line["cpu_baseline"] = cb
        line["speedup_vs_cpu"] = value / cb["value"]
    else:
        line["cpu_baseline"] = None
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
