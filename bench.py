"""HBA layer forward benchmark on one MI355X.

Step = one HBA attention layer forward at 32K context (B=1, n=32768, 14 query
/ 2 KV heads, d=64, 4 sinks, RoPE window 1024, 64-token blocks, 4 slots,
top-16, bf16, 16 needle blocks per KV head): key preparation, slot summaries,
flat block selection and the union attention, all HIP kernels, inputs resident
in HBM.  `value` = tokens/s of that forward.  The JSON line also carries the
roofline of the dominant kernel (the union attention, MFMA-bound), the
per-stage times, the 32K decode step (B=32 sequences, paged bf16 cache) as
µs/step against the HBM roofline, and the CPU baseline: the reference's naive
dense and gathered paths restated in torch (oracle/hba_cpu_torch.py), one
4096-token fp32 layer forward on the host's cores, in a child process.

  python bench.py [--gpus 1] [--steps K] [--warmup W] [--no-cpu] [--no-decode]
  python bench.py --copy-probe MIB      # plain device copy, for counter calibration
  python bench.py --config hier128k     # hierarchical selection at 128K vs the flat scan
  python bench.py --config donor        # 28/4-head d=128 layer at 64K, B=2, + 64 decode steps
"""
import argparse
import json
import os
import platform
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
for _p in (ROOT, os.path.join(ROOT, "hierarchical-block-attention_amd")):
    if _p not in sys.path:
        sys.path.insert(0, _p)

PEAK_BF16_TFLOPS = 2500.0     # MI355X dense bf16 MFMA
PEAK_HBM_GBS = 8000.0         # MI355X HBM3E

WORKLOAD = dict(workload="hba_layer_fwd_32k", batch=1, seq_len=32768, q_heads=14, kv_heads=2,
                head_dim=64, sinks=4, window=1024, block=64, slots=4, top_k=16, needles=16,
                qknorm="sharp gains d**0.25", selection="flat")
DECODE = dict(batch=32, len_lo=16384, len_hi=32768, seed=0)

# The union attention is one launch (hba_attn_fwd): each workgroup streams its
# 64 queries' sink and routed blocks, then their window tiles, through one LDS
# ring in one softmax state.  Its time is taken with HIP events around the op.
ATTN_KERNELS = "hba_attn_fwd = attn_routed_kernel<64,2,false,true> (sinks + routed blocks, then window tiles)"
# HBM (beyond-L2) bytes per hba_attn_fwd call on this workload: rocprofv3 --pmc
# FETCH_SIZE and WRITE_SIZE of the launch, each divided by the counter's
# reading per byte of a plain device copy (python bench.py --copy-probe 1024);
# profiles/hba_attn_32k_traffic.md.
ATTN_TRAFFIC_BYTES = 500836152


def cpu_model():
    try:
        with open("/proc/cpuinfo") as fh:
            for line in fh:
                if line.startswith("model name"):
                    return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return platform.processor()


def layer_setup(dev):
    import torch
    import hba_amd
    from hba_amd import synth
    w = WORKLOAD
    cfg = hba_amd.HBAConfig(n_heads=w["q_heads"], n_kv=w["kv_heads"], head_dim=w["head_dim"],
                            sinks=w["sinks"], window=w["window"], block=w["block"], slots=w["slots"],
                            k_blocks=w["top_k"])
    x = synth.layer_inputs(w["batch"], w["seq_len"], w["q_heads"], w["kv_heads"], w["head_dim"],
                           m=w["slots"], dtype=torch.bfloat16, device=dev, seed=0, sharp=True,
                           needles=True, window=w["window"])
    prm = synth.Params(x["q_gain"], x["k_gain"], x["probes"], x["proj"])
    cos, sin = hba_amd.rope_tables(w["seq_len"], w["head_dim"], cfg.rope_theta, dev)
    return cfg, x, prm, cos, sin


def run_layer_overlapped(cfg, x, prm, cos, sin):
    """One layer forward as forward_stages(overlap=True) runs it in bf16: the
    keys and block summaries in one launch, then the attention as two
    launches, the window on a second stream concurrent with score_select, the
    sinks + routed launch after both."""
    import torch
    from hba_amd import ops
    qeps = keps = 1e-6
    q = x["q"]
    n, Hkv, d = q.shape[1], x["k"].shape[2], q.shape[3]
    from hba_amd.config import union_scale
    scale = union_scale(cfg, d, n)
    kc, kr, vt, S0 = ops.prep_keys_summarize(x["k"], x["v"], prm.k.gain, keps, cos, sin, prm.probes, prm.proj)
    main = torch.cuda.current_stream()
    side = ops.side_stream(q.device)
    out, ws = ops.attn_buffers(q, Hkv)
    side.wait_stream(main)
    with torch.cuda.stream(side):
        ops.attn_window_(q, prm.q.gain, prm.k.gain, qeps, kr, vt, cos, sin, cfg.sinks, cfg.window, scale, out, ws)
    for t in (out, ws, kr, vt):
        t.record_stream(side)
    idx, val, cnt = ops.score_select(q, prm.q.gain, qeps, S0, cfg.window, cfg.k_blocks, scale)
    main.wait_stream(side)
    return ops.attn_routed_(q, prm.q.gain, prm.k.gain, qeps, kc, vt, idx, cnt, cfg.sinks, scale, out, ws)


def run_layer(cfg, x, prm, cos, sin, ev=None):
    """One layer forward, stages in sequence on one stream; with `ev` (dict of
    event pairs) each stage is bracketed."""
    from hba_amd import ops
    qeps = keps = 1e-6

    def mark(name, i):
        if ev is not None:
            ev[name][i].record()
    n = x["q"].shape[1]
    d = x["q"].shape[3]
    from hba_amd.config import union_scale
    scale = union_scale(cfg, d, n)
    mark("prep", 0)
    kc, kr, vt, S0 = ops.prep_keys_summarize(x["k"], x["v"], prm.k.gain, keps, cos, sin, prm.probes, prm.proj)
    mark("prep", 1)
    mark("select", 0)
    idx, val, cnt = ops.score_select(x["q"], prm.q.gain, qeps, S0, cfg.window, cfg.k_blocks, scale)
    mark("select", 1)
    mark("attn", 0)
    out = ops.attn_fwd(x["q"], prm.q.gain, prm.k.gain, qeps, kc, kr, vt, cos, sin, idx, cnt, cfg.sinks, cfg.window,
                       scale)
    mark("attn", 1)
    return out


def bench_layer(dev, steps, warmup):
    import torch
    from hba_amd import synth
    cfg, x, prm, cos, sin = layer_setup(dev)
    for _ in range(warmup):
        run_layer(cfg, x, prm, cos, sin)
        run_layer_overlapped(cfg, x, prm, cos, sin)
    torch.cuda.synchronize()
    # the same layer with the attention as two launches, the window overlapped
    # with the selection (forward_stages(overlap=True))
    t4 = torch.cuda.Event(enable_timing=True)
    t5 = torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    t4.record()
    for s in range(steps):
        run_layer_overlapped(cfg, x, prm, cos, sin)
    t5.record()
    torch.cuda.synchronize()
    ms_split = t4.elapsed_time(t5) / steps
    # the stages in sequence, each bracketed by events: the per-stage times
    # and the attention op's own duration (roofline)
    names = ("prep", "select", "attn")   # prep: the keys and the block summaries, one launch
    evs = [{k: (torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)) for k in names}
           for _ in range(steps)]
    t2 = torch.cuda.Event(enable_timing=True)
    t3 = torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    t2.record()
    for s in range(steps):
        run_layer(cfg, x, prm, cos, sin, evs[s])
    t3.record()
    torch.cuda.synchronize()
    ms_seq = t2.elapsed_time(t3) / steps
    # the step, timed last (the two loops above keep the GPU at its working
    # clocks): the layer as forward_stages runs it, every stage in sequence on
    # one stream, the attention one launch
    for _ in range(warmup):
        run_layer(cfg, x, prm, cos, sin)
    t0 = torch.cuda.Event(enable_timing=True)
    t1 = torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    wall0 = time.perf_counter()
    t0.record()
    for s in range(steps):
        run_layer(cfg, x, prm, cos, sin)
    t1.record()
    torch.cuda.synchronize()
    wall = time.perf_counter() - wall0
    ms = t0.elapsed_time(t1) / steps
    stage = {k: sum(e[k][0].elapsed_time(e[k][1]) for e in evs) / steps for k in names}
    w = WORKLOAD
    n = w["seq_len"]
    attn_flop = synth.attention_flops(w["batch"], n, w["q_heads"], w["head_dim"], w["sinks"],
                                      w["window"], w["block"], w["top_k"])
    score_flop = synth.scoring_flops(w["batch"], n, w["kv_heads"], w["head_dim"], w["slots"],
                                     w["block"], w["window"])
    summ_flop = synth.summarizer_flops(w["batch"], n, w["kv_heads"], w["head_dim"], w["slots"],
                                       w["block"])
    return dict(ms=ms, ms_marked=ms_seq, ms_split=ms_split, wall_s=wall, stage_ms=stage, attn_flop=attn_flop, score_flop=score_flop,
                summ_flop=summ_flop, tokens=w["batch"] * n,
                mean_keys=synth.mean_keys(n, w["sinks"], w["window"], w["block"], w["top_k"]),
                cfg=cfg, x=x, prm=prm, cos=cos, sin=sin)


def decode_bytes(lens, Hkv, d, m, S, W, k, Hq, esize=2):
    """Algorithmic HBM bytes of one decode step: per (sequence, KV head) the K
    and V rows of the attended union plus the candidate summaries; plus q and o."""
    from hba_amd.synth import ncand
    tot = 0
    for L in lens:
        i = L - 1
        nc = ncand(i, 64, W)
        keys = min(S, i + 1) + max(0, i - max(S, i - W + 1) + 1) + min(k, nc) * 64
        tot += Hkv * (keys * 2 * d * esize + nc * m * d * esize)
    tot += 2 * len(lens) * Hq * d * esize
    return tot


DECODE_PAIR_MIN = 128   # (sequence, KV head) pairs from which the library runs decode_pair_kernel
DECODE_STEPS_PER_GRAPH = 10


def bench_decode(dev, iters=200, batch=None):
    import torch
    import hba_amd
    from hba_amd import ops, synth
    Bd = batch or DECODE["batch"]
    Hq, Hkv, d, m, S, W, k = 14, 2, 64, 4, 4, 1024, 16
    cfg = hba_amd.HBAConfig(n_heads=Hq, n_kv=Hkv, head_dim=d, slots=m, sinks=S, window=W, k_blocks=k)
    lens = synth.decode_lengths(Bd, DECODE["len_lo"], DECODE["len_hi"], seed=DECODE["seed"])
    Lmax = max(lens)
    cache = hba_amd.PagedKVCache(cfg, Bd, Lmax, torch.bfloat16, dev)
    cache._free = synth.shuffled_pages(len(cache._free), seed=1)
    g = torch.Generator().manual_seed(0)
    probes = torch.randn(Hkv, m, d, generator=g) * d ** -0.5
    proj = torch.eye(d).unsqueeze(0).repeat(Hkv, 1, 1) + torch.randn(Hkv, d, d, generator=g) * 0.02
    gq = torch.full((Hq,), d ** 0.25, device=dev)
    gk = torch.full((Hkv,), d ** 0.25, device=dev)
    prm = synth.Params(gq, gk, probes.to(dev), proj.to(dev))
    cos, sin = hba_amd.rope_tables(Lmax, d, cfg.rope_theta, dev)
    for s, L in enumerate(lens):
        kraw = torch.randn(1, L, Hkv, d, generator=g).to(torch.bfloat16).to(dev)
        vraw = torch.randn(1, L, Hkv, d, generator=g).to(torch.bfloat16).to(dev)
        kc, kr, _ = ops.prep_keys(kraw, vraw, gk, 1e-6, cos, sin)
        cache.load(s, kc[0].transpose(0, 1), kr[0].transpose(0, 1), vraw[0], prm)
        del kraw, vraw, kc, kr
    q = torch.randn(Bd, Hq, d, generator=g).to(torch.bfloat16).to(dev)
    scales = cache.scales()
    eager = hba_amd.hba_decode_step(q, cache, cfg, prm, cos, sin, scales=scales)[0]
    torch.cuda.synchronize()
    stream = torch.cuda.Stream()
    stream.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(stream):
        for _ in range(2):
            hba_amd.hba_decode_step(q, cache, cfg, prm, cos, sin, scales=scales)
    torch.cuda.current_stream().wait_stream(stream)
    torch.cuda.synchronize()

    def timed_graph(nsteps):
        # nsteps identical decode steps captured in one graph (as a serving
        # loop captures every layer of a token): per-step device time without
        # the host's per-replay launch cost
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph):
            for _ in range(nsteps):
                gout = hba_amd.hba_decode_step(q, cache, cfg, prm, cos, sin, scales=scales)[0]
        for _ in range(5):
            graph.replay()
        torch.cuda.synchronize()
        ok = bool(torch.equal(gout, eager))
        reps = max(1, iters // nsteps)
        e0 = torch.cuda.Event(enable_timing=True)
        e1 = torch.cuda.Event(enable_timing=True)
        e0.record()
        for _ in range(reps):
            graph.replay()
        e1.record()
        torch.cuda.synchronize()
        return e0.elapsed_time(e1) * 1000.0 / (reps * nsteps), ok and bool(torch.equal(gout, eager))

    def timed_cold(reps=40, direct=False):
        # one step, each after 512 MB have streamed through the GPU (more
        # than its 256 MB Infinity Cache and the L2s) and with a fresh query:
        # the step reads its pages, summaries and page table from HBM.  The
        # streaming runs outside the timed events; the step is timed alone,
        # launched directly (direct) or as a one-step graph replay (its
        # launch included, as in the one-step warm figure).
        qbuf = torch.empty_like(q)
        graph = torch.cuda.CUDAGraph()
        qbuf.copy_(q)
        with torch.cuda.graph(graph):
            hba_amd.hba_decode_step(qbuf, cache, cfg, prm, cos, sin, scales=scales)
        gq = torch.Generator(device=dev).manual_seed(5)
        fresh = [torch.randn(q.shape, generator=gq, device=dev).to(q.dtype) for _ in range(8)]
        flush = torch.zeros(128 << 20, dtype=torch.float32, device=dev)   # 512 MB
        e0 = torch.cuda.Event(enable_timing=True)
        e1 = torch.cuda.Event(enable_timing=True)
        times = []
        for r in range(reps + 3):
            flush.add_(1.0)
            qbuf.copy_(fresh[r % len(fresh)])
            e0.record()
            if direct:   # enqueued while the flush runs, so no host gap falls between the events
                hba_amd.hba_decode_step(qbuf, cache, cfg, prm, cos, sin, scales=scales)
            else:
                graph.replay()
            e1.record()
            torch.cuda.synchronize()
            if r >= 3:
                times.append(e0.elapsed_time(e1) * 1000.0)
        del flush
        return sorted(times)[len(times) // 2]

    us_warm, ok = timed_graph(DECODE_STEPS_PER_GRAPH)
    us1, ok1 = timed_graph(1)
    ok = ok and ok1
    us_graph = timed_cold()
    us = timed_cold(direct=True)
    nbytes = decode_bytes(lens, Hkv, d, m, S, W, k, Hq)
    gbs = nbytes / (us * 1e-6) / 1e9
    pair = Bd * Hkv >= DECODE_PAIR_MIN and os.environ.get("HBA_DECODE_KERNEL") != "fused"
    kern = ("decode_pair_kernel: one launch, one workgroup per (sequence, KV head) (scores, top-k in "
            "LDS, window, sink and routed pages, LSE merge)") if pair else (
           "decode_fused_kernel: one launch (page scores and chunk top-k with the window "
           "and sink pages; the last score workgroup of a (sequence, KV head) merges the lists "
           "and runs the routed pages; the last workgroup merges the partial states)")
    return dict(us_per_step=round(us, 3), algorithmic_bytes=nbytes, achieved_GBs=round(gbs, 1),
                hbm_frac=round(gbs / PEAK_HBM_GBS, 4), graph_replay_matches_eager=ok,
                timing="cold: median over 40 steps, each launched directly on the stream (hba_decode_step) "
                       "after 512 MB streamed through the GPU (caches flushed) and with a fresh query; the same "
                       "step as a one-step HIP-graph replay in us_per_step_cold_graph_replay",
                us_per_step_cold_graph_replay=round(us_graph, 3),
                us_per_step_warm_10_step_graph=round(us_warm, 3),
                warm_GBs=round(nbytes / (us_warm * 1e-6) / 1e9, 1),
                us_per_step_warm_one_step_graph=round(us1, 3),
                batch=Bd, context="L ~ U[16384, 32768], paged bf16, shuffled page table", kernels=kern)


CPU_WORKLOAD = dict(batch=1, seq_len=4096, q_heads=14, kv_heads=2, head_dim=64, sinks=4, window=1024, block=64,
                    slots=4, top_k=16, dtype="fp32", qknorm="gains 1", seed=0)
CPU_FLOP = 2.233e10   # algorithmic FLOP of one forward at this workload (mean 1515 keys per query)


def cpu_leg(reps=5):
    """The CPU baseline itself, run in a child process that never touches the
    GPU: one HBA layer forward at the 4096-token fp32 workload through the
    oracle's torch restatements of the reference's naive dense path
    (attention.py:306-356) and, timed separately, its gathered path
    (:610-713), on the host's cores; 1 warmup, then the median of `reps`.
    Prints one JSON line with its own peak RSS."""
    import resource
    import statistics
    import torch
    import hba_amd
    import oracle.hba_cpu_torch as T
    import oracle.hba_oracle as O
    from hba_amd import synth
    threads = min(os.cpu_count() or 1, int(os.environ.get("OMP_NUM_THREADS", os.cpu_count() or 1)))
    torch.set_num_threads(threads)
    w = CPU_WORKLOAD
    cfg = hba_amd.HBAConfig(n_heads=w["q_heads"], n_kv=w["kv_heads"], head_dim=w["head_dim"], sinks=w["sinks"],
                            window=w["window"], block=w["block"], slots=w["slots"], k_blocks=w["top_k"])
    x = synth.layer_inputs(1, w["seq_len"], w["q_heads"], w["kv_heads"], w["head_dim"], m=w["slots"],
                           dtype=torch.float32, seed=w["seed"], sharp=False)
    cos, sin = (torch.from_numpy(t) for t in O.rope_tables(w["seq_len"], w["head_dim"], cfg.rope_theta))
    args = (x["q"], x["k"], x["v"], cos, sin, cfg, x["probes"], x["proj"], x["q_gain"], x["k_gain"], 1e-6)
    res = {}
    with torch.no_grad():
        for name, fn in (("dense", T.dense_forward), ("gathered", T.gathered_forward)):
            fn(*args)
            ts = []
            for _ in range(reps):
                t0 = time.perf_counter()
                fn(*args)
                ts.append(time.perf_counter() - t0)
            res[name] = statistics.median(ts)
    res["threads"] = torch.get_num_threads()
    res["peak_rss_MiB"] = round(resource.getrusage(resource.RUSAGE_SELF).ru_maxrss / 1024.0, 1)
    print(json.dumps(res))


def cpu_baseline():
    """cpu_leg in a child process (its peak RSS is its own), reported beside
    the GPU numbers: value = tokens/s of the naive dense path; the gathered
    path's time, threads, CPU model, peak RSS and GFLOP/s alongside."""
    import subprocess
    r = subprocess.run([sys.executable, os.path.abspath(__file__), "--cpu-leg"], capture_output=True, text=True,
                       timeout=900)
    if r.returncode != 0:
        return {"value": None, "unit": "tokens/s", "error": r.stderr[-400:]}
    d = json.loads(r.stdout.strip().splitlines()[-1])
    n = CPU_WORKLOAD["seq_len"]
    return {"value": round(n / d["dense"], 1), "unit": "tokens/s", "cores": d["threads"], "kind": "port",
            "sample": f"the whole forward, not a sample: one HBA layer at seq 4096, 14/2 heads, d=64, fp32, "
                      f"W=1024, k=16, seed 0, through the oracle's torch restatement of the reference's naive "
                      f"dense path (attention.py:306-356), torch CPU on {d['threads']} threads, 1 warmup + "
                      f"median of 5; host {cpu_model()}",
            "workload": dict(CPU_WORKLOAD),
            "dense_s_per_forward": round(d["dense"], 4),
            "gathered_s_per_forward": round(d["gathered"], 4),
            "gathered_tokens_per_s": round(n / d["gathered"], 1),
            "gflops_dense": round(CPU_FLOP / d["dense"] / 1e9, 2),
            "gflops_gathered": round(CPU_FLOP / d["gathered"] / 1e9, 2),
            "peak_rss_MiB": d["peak_rss_MiB"]}


def _timed(fn, reps=5):
    """Mean ms of fn() over reps calls (HIP events on the current stream), after
    warm calls for at least 0.2 s (the clocks ramp over the first ~30 ms of work)."""
    import torch
    t0 = time.perf_counter()
    while True:
        out = fn()
        torch.cuda.synchronize()
        if time.perf_counter() - t0 > 0.2:
            break
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record()
    for _ in range(reps):
        out = fn()
    e1.record()
    torch.cuda.synchronize()
    return e0.elapsed_time(e1) / reps, out


def bench_equiv32k(dev):
    """Dense uniform-RoPE causal attention (the equiv=True mode) at 32K: B=1,
    14/2 heads, d=64, QKNorm with the sharp gains, bf16: key preparation plus
    the window kernel with no sinks and a whole-sequence window.  FLOP counted
    as 4*d per (query, head, key <= query)."""
    import torch
    import hba_amd
    from hba_amd import synth
    w = WORKLOAD
    n, Hq, Hkv, d = w["seq_len"], w["q_heads"], w["kv_heads"], w["head_dim"]
    cfg = hba_amd.HBAConfig(n_heads=Hq, n_kv=Hkv, head_dim=d)
    x = synth.layer_inputs(1, n, Hq, Hkv, d, dtype=torch.bfloat16, device=dev, seed=0, sharp=True)
    prm = synth.Params(x["q_gain"], x["k_gain"], x["probes"], x["proj"])
    cos, sin = hba_amd.rope_tables(n, d, cfg.rope_theta, dev)
    ms, _ = _timed(lambda: hba_amd.equiv_attention(x["q"], x["k"], x["v"], cos, sin, cfg, prm), reps=5)
    flop = 4.0 * d * Hq * n * (n + 1) / 2
    tflops = flop / (ms * 1e-3) / 1e12
    return {"metric": "dense causal uniform-RoPE attention (equiv mode) tokens/s at 32K",
            "config": {"workload": "hba_equiv_32k", "batch": 1, "seq_len": n, "q_heads": Hq, "kv_heads": Hkv,
                       "head_dim": d},
            "tokens_per_s": round(n / (ms * 1e-3), 1), "ms": round(ms, 4), "flop": flop,
            "achieved_TFLOPs": round(tflops, 1), "mfma_frac": round(tflops / PEAK_BF16_TFLOPS, 4)}


def bench_bwd32k(dev, reps=5):
    """Backward of the HBA layer at 32K (the layer32k workload, bf16): the
    forward through hba_attention_dense with q, k, v and the QKNorm gains
    requiring grad, then hba_attn_bwd timed alone (HIP events around each
    out.backward, graph retained; the median of the timed calls, since a call
    can carry a one-off host stall of the caching allocator).  FLOP counted
    as 10*d per attended (query, head, key): S, dP, dQ, dK and dV, 2.5x the
    forward's count."""
    import torch
    import hba_amd
    from hba_amd import synth
    cfg, x, prm, cos, sin = layer_setup(dev)
    cfg.aux_w = 0.0          # the attention backward alone; the aux-KL is timed below
    q, k, v = (x[t].clone().requires_grad_(True) for t in ("q", "k", "v"))
    gq = x["q_gain"].clone().requires_grad_(True)
    gk = x["k_gain"].clone().requires_grad_(True)
    qkn = synth.Params(gq, gk, x["probes"], x["proj"])
    out = hba_amd.hba_attention_dense(q, k, v, cos, sin, cfg, qkn, qkn)[0]
    dout = torch.randn(out.shape, generator=torch.Generator().manual_seed(1)).to(out.dtype).to(dev)
    for _ in range(2):
        out.backward(dout, retain_graph=True)
    torch.cuda.synchronize()
    ev = [torch.cuda.Event(enable_timing=True) for _ in range(reps + 1)]
    ev[0].record()
    for r in range(reps):
        out.backward(dout, retain_graph=True)
        ev[r + 1].record()
    torch.cuda.synchronize()
    ms = float(sorted(ev[r].elapsed_time(ev[r + 1]) for r in range(reps))[reps // 2])
    w = WORKLOAD
    # attention_flops counts 4*d per attended (query, head, key); the backward 10*d
    flop = 2.5 * synth.attention_flops(w["batch"], w["seq_len"], w["q_heads"], w["head_dim"], w["sinks"],
                                       w["window"], w["block"], w["top_k"])
    tflops = flop / (ms * 1e-3) / 1e12
    # the summarizer's aux-KL (teacher, KL, gradients into probes and proj) at the same size
    pr = x["probes"].clone().requires_grad_(True)
    pj = x["proj"].clone().requires_grad_(True)
    summ = synth.Params(gq, gk, pr, pj)
    qd, kd, vd = x["q"], x["k"], x["v"]
    for _ in range(2):
        hba_amd.aux_kl(qd, kd, vd, cos, sin, cfg, summ, qkn)
    torch.cuda.synchronize()
    ea = [torch.cuda.Event(enable_timing=True) for _ in range(4)]
    ea[0].record()
    for r in range(3):
        hba_amd.aux_kl(qd, kd, vd, cos, sin, cfg, summ, qkn)
        ea[r + 1].record()
    torch.cuda.synchronize()
    aux_ms = float(sorted(ea[r].elapsed_time(ea[r + 1]) for r in range(3))[1])
    n_, Bk_, W_ = w["seq_len"], w["block"], w["window"]
    cand_keys = sum(max(0, (i - W_ + 1) // Bk_ - 1) * Bk_ for i in range(n_) if i - W_ + 1 >= 2 * Bk_)
    teacher_flop = 2.0 * w["head_dim"] * w["q_heads"] * cand_keys * w["batch"]
    return {"metric": "HBA layer backward tokens/s at 32K (dq, dk, dv, QKNorm gain grads; selection fixed)",
            "config": {"workload": "hba_layer_bwd_32k", "batch": 1, "seq_len": w["seq_len"], "q_heads": w["q_heads"],
                       "kv_heads": w["kv_heads"], "head_dim": w["head_dim"], "top_k": w["top_k"]},
            "tokens_per_s": round(w["seq_len"] / (ms * 1e-3), 1), "ms": round(ms, 3), "flop": flop,
            "achieved_TFLOPs": round(tflops, 2), "mfma_frac": round(tflops / PEAK_BF16_TFLOPS, 5),
            "timing": f"median of {reps} backward calls",
            "aux_kl": {"ms": round(aux_ms, 3), "teacher_flop": teacher_flop,
                       "teacher_TFLOPs": round(teacher_flop / (aux_ms * 1e-3) / 1e12, 2),
                       "what": "hba_aux_kl: QKNorm'd queries, block scores, the teacher's block LSEs on MFMA over "
                               "every candidate key, the KL rows, d aux / d probes and d proj (median of 3)"},
            "kernels": "bwd_kt (transposed keys) + bwd_dq_union_kernel (32 queries per workgroup, each staged "
                       "64-key block's K, V and K^T tiles shared through an LDS ring, MFMA) + "
                       "bwd_pick_bits (the selection as routed-row bits per key block) + bwd_dkv_mfma (8 waves "
                       "per KV head, 64-key block and 4096-row range, 64-pair tiles on MFMA; a second launch for "
                       "the sink keys) + bwd_dkv_fin (rope^T, QKNorm backward)"}


def bench_hier128k(dev):
    """Hierarchical tree selection at 128K (B=1, 14/2 heads, d=64, 2048 blocks,
    super-summaries over 16 blocks, beam 8, top-16, log-length temperature
    active, needles as in the 32K workload): flat and hierarchical selection
    timed, their set agreement over all queries and the last one, the
    comparisons per query, and the union attention over the hierarchical
    selection."""
    import torch
    import hba_amd
    from hba_amd import ops, synth
    from hba_amd.config import union_scale
    from hba_amd.synth import ncand
    n, Hq, Hkv, d, m, S, W, k, F, beam = 131072, 14, 2, 64, 4, 4, 1024, 16, 16, 8
    cfg = hba_amd.HBAConfig(n_heads=Hq, n_kv=Hkv, head_dim=d, sinks=S, window=W, block=64, slots=m, k_blocks=k,
                            fanout=F, beam=beam)
    x = synth.layer_inputs(1, n, Hq, Hkv, d, m=m, dtype=torch.bfloat16, device=dev, seed=0, sharp=True,
                           needles=True, window=W)
    prm = synth.Params(x["q_gain"], x["k_gain"], x["probes"], x["proj"])
    cos, sin = hba_amd.rope_tables(n, d, cfg.rope_theta, dev)
    scale = union_scale(cfg, d, n)
    t_prep, (kc, kr, vt) = _timed(lambda: ops.prep_keys(x["k"], x["v"], prm.k.gain, 1e-6, cos, sin))
    t_summ, S0 = _timed(lambda: ops.summarize(kc, prm.probes, prm.proj))
    t_flat, (fi, fv, fc) = _timed(lambda: ops.score_select(x["q"], prm.q.gain, 1e-6, S0, W, k, scale))
    t_sup, S1 = _timed(lambda: ops.build_super(S0, F))
    t_hier, (hi, hv, hc) = _timed(lambda: ops.hier_select(x["q"], prm.q.gain, 1e-6, S0, S1, W, k, F, beam, scale))
    t_attn, _ = _timed(lambda: ops.attn_fwd(x["q"], prm.q.gain, prm.k.gain, 1e-6, kc, kr, vt, cos, sin, hi, hc,
                                            S, W, scale), reps=3)
    # set agreement |flat & hier| / |flat| per (KV head, query) with a non-empty flat set
    fi, fc, hi, hc = fi[0].cpu(), fc[0].cpu(), hi[0].cpu(), hc[0].cpu()
    agree = tot = 0
    last = []
    for g in range(Hkv):
        fs = fi[g].clone()
        fs[torch.arange(k)[None, :] >= fc[g][:, None]] = -1
        hs = hi[g].clone()
        hs[torch.arange(k)[None, :] >= hc[g][:, None]] = -2
        inter = (fs[:, :, None] == hs[:, None, :]).any(-1).sum(-1)
        ok = fc[g] > 0
        agree += int(inter[ok].sum())
        tot += int(fc[g][ok].sum())
        last.append(float(inter[-1]) / max(1, int(fc[g][-1])))
    nsup = (n // 64 + F - 1) // F
    return {"metric": "HBA hierarchical selection at 128K: time vs flat scan, set agreement",
            "config": {"workload": "hba_hier_select_128k", "batch": 1, "seq_len": n, "q_heads": Hq, "kv_heads": Hkv,
                       "head_dim": d, "fanout": F, "beam": beam, "top_k": k, "needles": 16,
                       "temperature": round(scale / union_scale(cfg, d, 32768), 6)},
            "ms": {"prep": round(t_prep, 4), "summ": round(t_summ, 4), "flat_select": round(t_flat, 4),
                   "build_super": round(t_sup, 4), "hier_select": round(t_hier, 4),
                   "attn_on_hier": round(t_attn, 4)},
            "hier_vs_flat_select_speedup": round(t_flat / (t_sup + t_hier), 3),
            "agreement_all_queries": round(agree / max(1, tot), 4),
            "agreement_last_query": round(sum(last) / len(last), 4),
            "comparisons_per_query": {"hier": nsup + beam * F, "flat": int(ncand(n - 1, 64, W)),
                                      "ratio": round(ncand(n - 1, 64, W) / (nsup + beam * F), 2)}}


def bench_donor(dev, steps=64):
    """Donor-shaped layer: B=2, n=65536, 28/4 heads, d=128, 8 sinks, window
    1024, top-16, bf16, N(0,1) inputs from a seed: the prefill forward (stages
    timed), then a batched decode continuation from that cache, each token
    appending one new key/value per sequence and decoding its query: `steps`
    tokens through cache.append + hba_decode_step, then `steps` through a
    DecodeLoop (two launches per token straight through the C-ABI), then
    `steps` replayed from a DecodeLoop's HIP graph."""
    import torch
    import hba_amd
    from hba_amd import ops, synth
    from hba_amd.config import union_scale
    B, n, Hq, Hkv, d, m, S, W, k = 2, 65536, 28, 4, 128, 4, 8, 1024, 16
    cfg = hba_amd.HBAConfig(n_heads=Hq, n_kv=Hkv, head_dim=d, sinks=S, window=W, block=64, slots=m, k_blocks=k)
    x = synth.layer_inputs(B, n, Hq, Hkv, d, m=m, dtype=torch.bfloat16, device=dev, seed=0, sharp=True,
                           needles=False, window=W)
    prm = synth.Params(x["q_gain"], x["k_gain"], x["probes"], x["proj"])
    Lmax = n + 4 * steps + 3          # the tokens appended below: 1 + steps + 2 (1 + steps) + steps
    cos, sin = hba_amd.rope_tables(Lmax, d, cfg.rope_theta, dev)
    scale = union_scale(cfg, d, n)
    t_prep, (kc, kr, vt, S0) = _timed(lambda: ops.prep_keys_summarize(x["k"], x["v"], prm.k.gain, 1e-6, cos, sin,
                                                                      prm.probes, prm.proj), reps=3)
    t_sel, (idx, val, cnt) = _timed(lambda: ops.score_select(x["q"], prm.q.gain, 1e-6, S0, W, k, scale), reps=3)
    t_attn, _ = _timed(lambda: ops.attn_fwd(x["q"], prm.q.gain, prm.k.gain, 1e-6, kc, kr, vt, cos, sin, idx, cnt,
                                            S, W, scale), reps=3)
    t_layer = t_prep + t_sel + t_attn
    flop = (synth.attention_flops(B, n, Hq, d, S, W, 64, k) + synth.scoring_flops(B, n, Hkv, d, m, 64, W) +
            synth.summarizer_flops(B, n, Hkv, d, m, 64))
    # decode continuation from the prefill cache
    cache = hba_amd.PagedKVCache(cfg, B, Lmax, torch.bfloat16, dev)
    for s_ in range(B):
        cache.load(s_, kc[s_].transpose(0, 1), kr[s_].transpose(0, 1), x["v"][s_], prm)
    del kc, kr, vt, idx, val, cnt
    g = torch.Generator().manual_seed(1)
    qs = torch.randn(steps, B, Hq, d, generator=g).to(torch.bfloat16).to(dev)
    ks = torch.randn(steps, B, Hkv, d, generator=g).to(torch.bfloat16).to(dev)
    vs = torch.randn(steps, B, Hkv, d, generator=g).to(torch.bfloat16).to(dev)
    cache.append(ks[0], vs[0], prm, prm, cos, sin)          # first calls of the ops, one token
    hba_amd.hba_decode_step(qs[0], cache, cfg, prm, cos, sin)
    torch.cuda.synchronize()
    ev = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)) for _ in range(steps)]
    t0 = torch.cuda.Event(enable_timing=True)
    t1 = torch.cuda.Event(enable_timing=True)
    t0.record()
    for st in range(steps):
        cache.append(ks[st], vs[st], prm, prm, cos, sin)
        ev[st][0].record()
        hba_amd.hba_decode_step(qs[st], cache, cfg, prm, cos, sin)
        ev[st][1].record()
    t1.record()
    torch.cuda.synchronize()
    step_us = sorted(a.elapsed_time(b) * 1000.0 for a, b in ev)
    loop_us = {}
    replay_us = []
    for mode in ("direct", "graph"):
        lp = hba_amd.DecodeLoop(cache, cfg, prm, prm, cos, sin, graph=(mode == "graph"))
        lp.step(qs[0], ks[0], vs[0])                    # first call (graph upload), one token
        torch.cuda.synchronize()
        t2 = torch.cuda.Event(enable_timing=True)
        t3 = torch.cuda.Event(enable_timing=True)
        t2.record()
        for st in range(steps):
            lp.step(qs[st], ks[st], vs[st])
        t3.record()
        torch.cuda.synchronize()
        loop_us[mode] = round(t2.elapsed_time(t3) * 1000.0 / steps, 2)
    # the graph's replay alone: its inputs written into the static buffers
    # first (a serving loop's upstream kernels write them there), events
    # around each replay
    rev = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)) for _ in range(steps)]
    for st in range(steps):
        lp.q.copy_(qs[st])
        lp.k.copy_(ks[st])
        lp.v.copy_(vs[st])
        rev[st][0].record()
        lp.step()
        rev[st][1].record()
    torch.cuda.synchronize()
    replay_us = sorted(a_.elapsed_time(b_) * 1000.0 for a_, b_ in rev)
    return {"metric": "HBA donor-shaped layer: prefill tokens/s; decode continuation us/step",
            "config": {"workload": "hba_layer_fwd_donor_64k_d128", "batch": B, "seq_len": n, "q_heads": Hq,
                       "kv_heads": Hkv, "head_dim": d, "sinks": S, "window": W, "top_k": k, "decode_steps": steps},
            "prefill": {"tokens_per_s": round(B * n / (t_layer * 1e-3), 1), "ms": round(t_layer, 4),
                        "stage_ms": {"prep_and_summaries": round(t_prep, 4), "select": round(t_sel, 4),
                                     "attn": round(t_attn, 4)},
                        "mfma_frac": round(flop / (t_layer * 1e-3) / 1e12 / PEAK_BF16_TFLOPS, 4)},
            "decode": {"step_us_median": round(step_us[len(step_us) // 2], 2),
                       "step_us_min": round(step_us[0], 2),
                       "append_plus_step_us": round(t0.elapsed_time(t1) * 1000.0 / steps, 2),
                       "loop_token_us": loop_us["direct"], "loop_graph_token_us": loop_us["graph"],
                       "graph_replay_token_us_median": round(replay_us[len(replay_us) // 2], 2),
                       "loop_graph_note": "loop_graph_token_us includes step()'s three input copies into the "
                                          "graph's static buffers; graph_replay_token_us is the replay alone",
                       "lengths": [n + 1, n + 4 * steps + 3]}}


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=50,
                    help="untimed layer steps first; the step time is steady from about 40 on (clocks ramp)")
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--no-decode", action="store_true")
    ap.add_argument("--cpu-leg", action="store_true",
                    help="internal: run only the CPU baseline (no GPU use) and print its JSON")
    ap.add_argument("--copy-probe", type=int, default=0, metavar="MIB",
                    help="only run 3 plain device copies of MIB MiB (counter calibration) and exit")
    ap.add_argument("--config", choices=["layer32k", "hier128k", "donor", "equiv32k", "bwd32k", "decode32k",
                                         "decode32k_b128"],
                    default="layer32k",
                    help="layer32k: the headline line (default); hier128k / donor / equiv32k / bwd32k / "
                         "decode32k / decode32k_b128 (the decode step at 128 sequences): the other "
                         "measured workloads, one JSON line each")
    a = ap.parse_args()
    if a.cpu_leg:
        cpu_leg()
        return
    if a.copy_probe:
        import torch
        src = torch.empty(a.copy_probe << 20, dtype=torch.uint8, device="cuda:0").fill_(1)
        dst = torch.empty_like(src)
        for _ in range(3):
            dst.copy_(src)
        torch.cuda.synchronize()
        print(json.dumps({"copy_probe_MiB": a.copy_probe, "copies": 3}))
        return
    world = int(os.environ.get("WORLD_SIZE", a.gpus))
    if a.gpus != 1 or world != 1:
        print(json.dumps({"error": "this benchmark runs on exactly one GPU: the HBA operator is "
                                   "measured on one MI355X (multi-GPU sharding is design-only)",
                          "n_gpus": a.gpus}))
        sys.exit(2)
    import torch
    dev = torch.device("cuda:0")
    if a.config != "layer32k":
        line = {"hier128k": bench_hier128k, "donor": bench_donor, "equiv32k": bench_equiv32k,
                "bwd32k": bench_bwd32k,
                "decode32k": lambda d: {"metric": "HBA decode step µs (B=32, 16-32K paged bf16 cache)",
                                        **bench_decode(d)},
                "decode32k_b128": lambda d: {"metric": "HBA decode step µs (B=128, 16-32K paged bf16 cache)",
                                             **bench_decode(d, iters=100, batch=128)}}[a.config](dev)
        line.update({"n_gpus": 1, "dtype": "bf16", "data": "synthetic"})
        print(json.dumps(line))
        return
    res = bench_layer(dev, a.steps, a.warmup)
    ms = res["ms"]
    attn_ms = res["stage_ms"]["attn"]
    achieved = res["attn_flop"] / (attn_ms * 1e-3) / 1e12
    dec = None if a.no_decode else bench_decode(dev)
    cpu = None if a.no_cpu else cpu_baseline()
    total_flop = res["attn_flop"] + res["score_flop"] + res["summ_flop"]
    line = {
        "metric": "HBA layer fwd tokens/s at 32K (% MFMA roofline); decode µs/step (% HBM BW)",
        "value": round(res["tokens"] / (ms * 1e-3), 1),
        "unit": "tokens/s",
        "n_gpus": 1,
        "steps": a.steps,
        "warmup": a.warmup,
        "ms_per_step": round(ms, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic",
        "config": dict(WORKLOAD),
        "roofline": {"bound": "mfma", "kernel": ATTN_KERNELS,
                     "achieved": round(achieved, 2), "peak": PEAK_BF16_TFLOPS, "unit": "TFLOP/s",
                     "frac": round(achieved / PEAK_BF16_TFLOPS, 4), "traffic": ATTN_TRAFFIC_BYTES,
                     "algorithmic_flop_per_launch": res["attn_flop"],
                     "mean_keys_per_query": round(res["mean_keys"], 1)},
        "layer_frac_of_mfma_roofline": round(total_flop / (ms * 1e-3) / 1e12 / PEAK_BF16_TFLOPS, 4),
        "stage_ms": {k: round(v, 4) for k, v in res["stage_ms"].items()},
        "schedule": {"step": "prep_keys_summarize (keys and block summaries, one launch), score_select, "
                             "hba_attn_fwd (one launch) in sequence on one stream",
                     "ms_per_step_two_launch_attn_window_overlapped": round(res["ms_split"], 4),
                     "ms_per_step_with_stage_events": round(res["ms_marked"], 4)},
        "decode": dec,
        "cpu_baseline": cpu,
    }
    print(json.dumps(line))


if __name__ == "__main__":
    main()
