"""HIP kernels against the oracle at the benchmarked workloads' own sizes, so
that every code path those workloads take is compared (through the C-ABI):

  fp32 4096      n = 4096, W = 1024, k = 16, 14/2 heads, fp32: selection
                 bit-exact, every output row within 1e-5 (gains 1 and d**0.25)
  bf16 32K       n = 32768, needles, sharp gains: 256 sampled rows (selection
                 on the kernel's own scores bit-exact, attention within 2e-2)
  decode 16-32K  32K-token sequences (8 score chunks of 64 candidate pages)
                 batched with short ones, bf16 and fp32: picks bit-exact,
                 outputs within tolerance of the prefill row L-1
  hier 128K      128 supers, beam 8, temperature on: 256 sampled rows
                 (parent bitmask of 4 words per query)
  d128 decode    28/4 heads, d = 128, 8 sinks: 70 append + decode steps over a
                 page boundary from L ~ 6000 (2 score chunks); every append
                 bit-exact, every step against the oracle
  reference      the fp32 path against outputs written by the reference
                 itself (tests/golden/golden_d64.npz)
"""
import numpy as np
import pytest
import torch

import make_golden as MG
import oracle.hba_oracle as O

pytestmark = pytest.mark.gpu

hba_amd = pytest.importorskip("hba_amd")
from hba_amd import ops, synth  # noqa: E402

TOL = {"f32": 1e-5, "bf16": 2e-2}
TDT = {"f32": torch.float32, "bf16": torch.bfloat16}


@pytest.fixture(scope="module")
def dev():
    if not torch.cuda.is_available():
        pytest.fail("GPU tests need a visible gfx950 device")
    return torch.device("cuda:0")


def f(t):
    return t.detach().float().cpu().numpy()


def sample_rows(n, extra=(), count=160, seed=0):
    rs = np.random.RandomState(seed)
    return np.unique(np.concatenate([np.arange(0, 8), np.arange(n - 64, n),
                                     np.linspace(0, n - 1, count).astype(np.int64),
                                     rs.randint(0, n, 32), np.asarray(extra, np.int64)])).astype(np.int64)


def margin_flips(k_idx, k_cnt, o_scores, kk, rel=1e-5):
    """Kernel picks vs the oracle's declared-order scores o_scores [r, nb]: the
    same sets except blocks within `rel` of the k-th score (near-ties at the
    k boundary, the reference's own flip rule gates.py:183-203).  Returns the
    number of rows that differ."""
    bad = 0
    for r in range(o_scores.shape[0]):
        row = o_scores[r]
        fin = np.isfinite(row)
        c = min(kk, int(fin.sum()))
        assert int(k_cnt[r]) == c
        if c == 0:
            continue
        order = np.lexsort((np.arange(row.size), -np.where(fin, row, -np.inf)))
        ref = set(order[:c].tolist())
        got = set(k_idx[r, :c].tolist())
        if got != ref:
            kth = row[order[c - 1]]
            for blk in got ^ ref:
                assert abs(row[blk] - kth) <= rel * max(1.0, abs(kth)), (r, blk, row[blk], kth)
            bad += 1
    return bad


# --------------------------------------------------------- fp32 at 4096 ----
@pytest.mark.parametrize("sharp", [False, True])
def test_fp32_4096_selection_exact_and_every_row(dev, sharp):
    """B = 1, n = 4096, 14/2 heads, d = 64, S = 4, W = 1024, k = 16, fp32,
    seed 0: summaries within fp32 rounding of the float64 restatement, the
    flat selection bit-exact against the oracle's declared order, and every
    one of the 4096 output rows within 1e-5 of the float64 union softmax;
    the dense drop-in (route_topk's scale) on the same rows."""
    n, Hq, Hkv, d = 4096, 14, 2, 64
    cfg = hba_amd.HBAConfig(n_heads=Hq, n_kv=Hkv, head_dim=d, window=1024, sinks=4, k_blocks=16, slots=4)
    x = synth.layer_inputs(1, n, Hq, Hkv, d, m=4, dtype=torch.float32, device=dev, seed=0, sharp=sharp)
    prm = synth.Params(x["q_gain"], x["k_gain"], x["probes"], x["proj"])
    cos, sin = hba_amd.rope_tables(n, d, cfg.rope_theta, dev)
    r = hba_amd.forward_stages(x["q"], x["k"], x["v"], cos, sin, cfg, prm, prm)
    out_d, aux = hba_amd.hba_attention_dense(x["q"], x["k"], x["v"], cos, sin, cfg, prm, prm)
    torch.cuda.synchronize()
    S0 = f(r["S0"])[0]
    P = O.prepare(f(x["q"])[0], f(x["k"])[0], f(x["v"])[0], f(cos), f(sin), cfg, f(x["probes"]), f(x["proj"]),
                  f(x["q_gain"]), f(x["k_gain"]), 1e-6, "f32", S0=S0)
    ref_S0 = O.summarize(P.kc, f(x["probes"]), f(x["proj"]), 64)
    assert np.abs(S0 - ref_S0).max() <= 2e-5 * max(1.0, np.abs(ref_S0).max())
    o_idx, o_val, o_cnt = O.flat_select(P.qg, P.S0, r["sel_scale"], 16, 64, cfg.window)
    for key, want in (("idx", o_idx), ("val", o_val), ("cnt", o_cnt)):
        assert np.array_equal(r[key][0].cpu().numpy(), want), key
    rows = np.arange(n)
    ref = O.attn_rows(P.qc, P.qr, P.kc, P.kr, P.v, o_idx, o_cnt, r["scale"], cfg.sinks, cfg.window, 64, rows)
    err = np.abs(f(r["out"])[0] - ref).max()
    assert err <= 1e-5, err
    # dense: route_topk's scale has no temperature; at n <= native_ctx it is the same selection
    assert np.abs(f(out_d)[0] - ref).max() <= 1e-5
    # and its aux-KL (aux_w = 1) against the oracle's, on the same summaries
    aref = O.aux_kl(P.qc[None], P.kc[None], f(x["probes"]), f(x["proj"]), Hkv, r["scale"],
                    hba_amd.route_scale(cfg, d), 64, cfg.window, S0_scores=S0[None], dtype="f32")[0]
    assert abs(float(aux) - aref) <= 1e-5 * abs(aref), (float(aux), aref)


# ---------------------------------------------------------- bf16 at 32K ----
def test_bf16_32k_needles_sampled_rows(dev):
    """The benchmark's layer (n = 32768, 14/2 heads, d = 64, bf16, sharp gains,
    16 needle blocks per KV head) through forward_stages: on 256 sampled rows
    (the last 64, the needle queries, a spread), the top-k of the kernel's own
    scores is bit-exact, its scores are the declared-order fp32 scores up to
    GEMM rounding, its picks are the oracle's up to k-boundary near-ties, and
    the attention rows are within 2e-2 (mean 1e-3, 99.9 % within 4e-3) of the float64
    union softmax."""
    n, Hq, Hkv, d, W, k = 32768, 14, 2, 64, 1024, 16
    cfg = hba_amd.HBAConfig(n_heads=Hq, n_kv=Hkv, head_dim=d, window=W, sinks=4, k_blocks=k, slots=4)
    x = synth.layer_inputs(1, n, Hq, Hkv, d, m=4, dtype=torch.bfloat16, device=dev, seed=0, sharp=True,
                           needles=True, window=W)
    prm = synth.Params(x["q_gain"], x["k_gain"], x["probes"], x["proj"])
    cos, sin = hba_amd.rope_tables(n, d, cfg.rope_theta, dev)
    r = hba_amd.forward_stages(x["q"], x["k"], x["v"], cos, sin, cfg, prm, prm)
    idx, val, cnt, scores = ops.score_select_with_scores(x["q"], x["q_gain"], 1e-6, r["S0"], W, k, r["sel_scale"])
    torch.cuda.synchronize()
    assert torch.equal(idx, r["idx"]) and torch.equal(cnt, r["cnt"]) and torch.equal(val, r["val"])
    rows = sample_rows(n, [p for (p, _) in x["needles"].values()])
    P = O.prepare(f(x["q"])[0], f(x["k"])[0], f(x["v"])[0], f(cos), f(sin), cfg, f(x["probes"]), f(x["proj"]),
                  f(x["q_gain"]), f(x["k_gain"]), 1e-6, "bf16", S0=f(r["S0"])[0])
    sc = scores[0][:, torch.from_numpy(rows).to(dev)].cpu().numpy()
    ki, kv, kc_ = (t[0][:, torch.from_numpy(rows).to(dev)].cpu().numpy() for t in (idx, val, cnt))
    for g in range(Hkv):
        ti, tv, tc = O.topk(sc[g], k)
        assert np.array_equal(ti, ki[g]) and np.array_equal(tv, kv[g]) and np.array_equal(tc, kc_[g])
        osc = O.block_scores(P.qg[g], P.S0[g], rows, r["sel_scale"], 64, W)
        fin = np.isfinite(osc)
        assert np.array_equal(np.isfinite(sc[g]), fin)
        assert np.abs(sc[g][fin] - osc[fin]).max() <= 2e-6 * max(1.0, np.abs(osc[fin]).max())
        assert margin_flips(ki[g], kc_[g], osc, k) <= 2
    ref = O.attn_rows(P.qc, P.qr, P.kc, P.kr, P.v, r["idx"][0].cpu().numpy(), r["cnt"][0].cpu().numpy(),
                      r["scale"], cfg.sinks, W, 64, rows)
    err = np.abs(f(r["out"])[0][rows] - ref)
    # the bar is 2e-2; the distribution sits near one bf16 rounding of the output
    assert err.max() <= TOL["bf16"], err.max()
    assert err.mean() <= 1e-3 and np.quantile(err, 0.999) <= 4e-3, (err.mean(), np.quantile(err, 0.999))


# ------------------------------------------------------------- decode ------
def lean_cache(dev, dt, lens, Hq=14, Hkv=2, d=64, m=4, W=1024, S=4, k=16, seed=0, extra=0, **cfgkw):
    """A paged cache holding len(lens) sequences of N(0,1) keys and values
    (QKNorm'd and rotated by hba_prep_keys, on a shuffled page table), drawn
    per sequence so that long contexts need no [B, Lmax] draw.  Returns the
    cache, the parameters, the tables and the host copies the oracle reads."""
    cfg = hba_amd.HBAConfig(n_heads=Hq, n_kv=Hkv, head_dim=d, slots=m, window=W, sinks=S, k_blocks=k, **cfgkw)
    Bd, Lmax = len(lens), max(lens) + extra
    g = torch.Generator().manual_seed(seed)
    probes = torch.randn(Hkv, m, d, generator=g) * d ** -0.5
    proj = torch.eye(d).unsqueeze(0).repeat(Hkv, 1, 1) + torch.randn(Hkv, d, d, generator=g) * 0.02
    gq = torch.full((Hq,), d ** 0.25)
    gk = torch.full((Hkv,), d ** 0.25)
    prm = synth.Params(gq.to(dev), gk.to(dev), probes.to(dev), proj.to(dev))
    cos, sin = hba_amd.rope_tables(Lmax + 64, d, cfg.rope_theta, dev)
    cache = hba_amd.PagedKVCache(cfg, Bd, Lmax + 64, TDT[dt], dev)
    cache._free = synth.shuffled_pages(len(cache._free), seed=seed + 1)
    kcs, vs = [], []
    for s, L in enumerate(lens):
        kraw = torch.randn(1, L, Hkv, d, generator=g).to(TDT[dt]).to(dev)
        vraw = torch.randn(1, L, Hkv, d, generator=g).to(TDT[dt]).to(dev)
        kc, kr, _ = ops.prep_keys(kraw, vraw, prm.k.gain, 1e-6, cos, sin)
        cache.load(s, kc[0].transpose(0, 1), kr[0].transpose(0, 1), vraw[0], prm)
        kcs.append(f(kc[0].transpose(0, 1)))
        vs.append(f(vraw[0]))
    return cfg, cache, prm, cos, sin, kcs, vs, g


def check_decode(cache, cfg, prm, cos, sin, kcs, vs, qd, dt, out, sidx, scnt):
    d = cfg.head_dim
    for s, L in enumerate(cache.lens):
        pt = cache._table[s][: L // 64]
        S0s = f(cache.summ_pages[torch.tensor(pt, dtype=torch.long)]).transpose(1, 0, 2, 3)
        scale = hba_amd.union_scale(cfg, d, L)
        ref, (idx, val, cnt) = O.decode_row(f(qd[s]), kcs[s], vs[s], f(cos), f(sin), cfg, S0s, f(prm.q.gain),
                                            1e-6, dt, scale)
        assert np.array_equal(scnt[s].cpu().numpy(), cnt), (s, L)
        for g in range(cfg.n_kv):
            assert list(sidx[s, g, : cnt[g]].cpu().numpy()) == list(idx[g, : cnt[g]]), (s, L, g)
        err = np.abs(f(out[s]) - ref).max()
        assert err <= TOL[dt], (s, L, err)


@pytest.mark.parametrize("dt,kern", [("bf16", "fused"), ("bf16", "pair"), ("f32", "fused")])
def test_decode_16k_32k_batch(dev, dt, kern, monkeypatch):
    """The decode workload's lengths (L ~ U[16384, 32768], seed 0) plus one
    sequence of exactly 32768 tokens (8 score chunks of 64 candidate pages)
    and two short ones, whose chunks past their last candidate are empty; in
    bf16 on both kernels."""
    monkeypatch.setenv("HBA_DECODE_KERNEL", kern)
    lens = synth.decode_lengths(6, 16384, 32768, seed=0) + [32768, 70, 1500]
    cfg, cache, prm, cos, sin, kcs, vs, g = lean_cache(dev, dt, lens)
    qd = torch.randn(len(lens), 14, 64, generator=g).to(TDT[dt]).to(dev)
    out, sidx, scnt = hba_amd.hba_decode_step(qd, cache, cfg, prm, cos, sin)
    torch.cuda.synchronize()
    check_decode(cache, cfg, prm, cos, sin, kcs, vs, qd, dt, out, sidx, scnt)


@pytest.mark.parametrize("kern", ["fused", "pair"])
def test_decode_d128_continuation_over_a_page_boundary(dev, kern, monkeypatch):
    """The donor shape's decode continuation: 28/4 heads, d = 128, 8 sinks,
    two sequences loaded at ~6000 tokens (2 score chunks), then 70 steps that
    each append one token per sequence (kv_append, bit-exact) and decode a
    new query against the oracle; the pages that fill get their summaries.
    native_ctx = 4096 makes the log-length temperature differ per sequence.
    On both bf16 decode kernels."""
    monkeypatch.setenv("HBA_DECODE_KERNEL", kern)
    lens = [6000, 5950]
    cfg, cache, prm, cos, sin, kcs, vs, g = lean_cache(dev, "bf16", lens, Hq=28, Hkv=4, d=128, S=8, extra=80,
                                                       native_ctx=4096)
    gk = f(prm.k.gain)
    filled = 0
    for step in range(70):
        kn = torch.randn(2, 4, 128, generator=g).to(torch.bfloat16).to(dev)
        vn = torch.randn(2, 4, 128, generator=g).to(torch.bfloat16).to(dev)
        qd = torch.randn(2, 28, 128, generator=g).to(torch.bfloat16).to(dev)
        cache.append(kn, vn, prm, prm, cos, sin)
        out, sidx, scnt = hba_amd.hba_decode_step(qd, cache, cfg, prm, cos, sin)
        torch.cuda.synchronize()
        for s in range(2):
            pos = cache.lens[s] - 1
            page = cache._table[s][pos // 64]
            want = O.qknorm(f(kn)[s], gk, 1e-6, "bf16")
            assert np.array_equal(f(cache.key_rows(page)[:, pos % 64]), want), (step, s)
            rot = O.apply_rope(want[None], f(cos), f(sin), "bf16", positions=np.array([pos]))[0]
            assert np.array_equal(f(cache.key_rows(page, rotated=True)[:, pos % 64]), rot), (step, s)
            assert np.array_equal(f(cache.value_rows(page)[:, pos % 64]), f(vn)[s]), (step, s)
            kcs[s] = np.concatenate([kcs[s], want[None]], 0)
            vs[s] = np.concatenate([vs[s], f(vn)[s][None]], 0)
            if cache.lens[s] % 64 == 0:            # the page just filled: its summary
                kpage = f(cache.key_rows(page)).transpose(1, 0, 2)
                sref = O.summarize(kpage, f(prm.probes), f(prm.proj), 64)[:, 0]
                assert np.abs(f(cache.summ_pages[page]) - sref).max() <= 2 ** -7 * max(1, np.abs(sref).max())
                filled += 1
        check_decode(cache, cfg, prm, cos, sin, kcs, vs, qd, "bf16", out, sidx, scnt)
    assert filled == 3                             # at 6016 (6000 -> 6070); at 5952 and 6016 (5950 -> 6020)


# ------------------------------------------------------- hier at 128K ------
def check_hier_rows(qg, S0, S1, F, beam, kk, scale, W, rows, ki, kv, kc_, sc, sup):
    """The bf16 GEMM path of hier_select on sampled rows of one KV head: the
    super and child sets it scored follow the oracle's rules, both score
    arrays agree with the declared-order scores up to GEMM rounding, and the
    picks are the oracle's top-k of the kernel's own child scores."""
    nb, m, d = S0.shape
    ns = S1.shape[0]
    beff = min(beam, ns)
    kout = min(kk, beff * F)
    bmax = np.array([O.cand_bmax(int(i), 64, W) for i in rows])
    lo = np.arange(ns) * F
    hi = np.minimum(lo + F - 1, nb - 1)
    valid = (bmax[:, None] >= 1) & (lo[None, :] <= bmax[:, None]) & (hi[None, :] >= 1)
    assert np.array_equal(np.isfinite(sup), valid)
    ex = (qg[rows].astype(np.float64) @ S1.reshape(-1, d).T.astype(np.float64)).reshape(len(rows), ns, m)
    ex = ex.max(-1) * scale
    assert np.abs(sup[valid] - ex[valid]).max() <= 2e-6 * max(1.0, np.abs(ex[valid]).max())
    pi, pv, pc = O.topk(sup, beff)
    kept = np.zeros((len(rows), nb), dtype=bool)
    for r in range(len(rows)):
        for p in pi[r, : pc[r]]:
            kept[r, p * F: min(nb, p * F + F)] = True
    blk = np.arange(nb)
    cand = (blk[None, :] >= 1) & (blk[None, :] <= bmax[:, None])
    assert np.array_equal(np.isfinite(sc), kept & cand)
    osc = O.block_scores(qg, S0, rows, scale, 64, W)
    fin = np.isfinite(sc)
    assert np.abs(sc[fin] - osc[fin]).max() <= 2e-6 * max(1.0, np.abs(osc[fin]).max())
    ti, tv, tc = O.topk(sc, kout)
    pad = kk - kout
    ti = np.concatenate([ti, np.full((len(rows), pad), -1, np.int32)], 1)
    tv = np.concatenate([tv, np.full((len(rows), pad), -np.inf, np.float32)], 1)
    assert np.array_equal(ti, ki) and np.array_equal(tv, kv) and np.array_equal(tc, kc_)


@pytest.mark.parametrize("dt", ["bf16", "f32"])
def test_hier_select_128k(dev, dt):
    """n = 131072 (2048 blocks, 128 supers of F = 16, beam 8, top-16), 14/2
    heads, d = 64, needles, the log-length temperature at 4x native context
    (tau = 1 + 0.1 ln 4): fp32 picks bit-exact against the oracle's
    hier_select on 256 sampled rows; bf16 through the dumps of the scores the
    kernel ranked."""
    n, Hq, Hkv, d, W, k, F, beam = 131072, 14, 2, 64, 1024, 16, 16, 8
    cfg = hba_amd.HBAConfig(n_heads=Hq, n_kv=Hkv, head_dim=d, window=W, sinks=4, k_blocks=k, slots=4, fanout=F,
                            beam=beam)
    x = synth.layer_inputs(1, n, Hq, Hkv, d, m=4, dtype=TDT[dt], device=dev, seed=0, sharp=True, needles=True,
                           window=W)
    cos, sin = hba_amd.rope_tables(n, d, cfg.rope_theta, dev)
    scale = hba_amd.union_scale(cfg, d, n)
    assert abs(scale * d - (1 + 0.1 * np.log(4))) < 1e-6
    kc, kr, vt = ops.prep_keys(x["k"], x["v"], x["k_gain"], 1e-6, cos, sin)
    del kr, vt
    S0 = ops.summarize(kc, x["probes"], x["proj"])
    S1 = ops.build_super(S0, F)
    assert S1.shape[2] == 128
    rows = sample_rows(n, [p for (p, _) in x["needles"].values()], count=180)
    tr = torch.from_numpy(rows).to(dev)
    qc = O.qknorm(f(x["q"])[0], f(x["q_gain"]), 1e-6, dt)
    qg = O.grouped_query(qc, Hkv, dt)
    S0h, S1h = f(S0)[0], f(S1)[0]
    for g in range(Hkv):
        assert np.array_equal(S1h[g], O.build_super(S0h[g], F, dt))
    if dt == "f32":
        idx, val, cnt = ops.hier_select(x["q"], x["q_gain"], 1e-6, S0, S1, W, k, F, beam, scale)
        ki, kv, kc_ = (t[0][:, tr].cpu().numpy() for t in (idx, val, cnt))
        oi, ov, oc = O.hier_select(qg, S0h, S1h, F, beam, k, scale, 64, W, pos=rows)
        assert np.array_equal(kc_, oc) and np.array_equal(ki, oi) and np.array_equal(kv, ov)
        return
    idx, val, cnt, scores, sup = ops.hier_select_with_scores(x["q"], x["q_gain"], 1e-6, S0, S1, W, k, F, beam,
                                                             scale)
    torch.cuda.synchronize()
    ki, kv, kc_ = (t[0][:, tr].cpu().numpy() for t in (idx, val, cnt))
    sc = scores[0][:, tr].cpu().numpy()
    sp = sup[0][:, tr].cpu().numpy()
    del scores, sup
    for g in range(Hkv):
        check_hier_rows(qg[g], S0h[g], S1h[g], F, beam, k, scale, W, rows, ki[g], kv[g], kc_[g], sc[g], sp[g])


# ------------------------------------------------ reference-written outputs
def test_fp32_path_matches_reference_outputs(dev):
    """The HIP fp32 path (hba_attention_dense, hba_attention_eval flat and
    hierarchical) against the outputs the reference itself wrote on the same
    seeded inputs (golden_d64: d = 64, 64-key blocks, 4/2 heads, W = 128, k = 3,
    F = 4, beam 2, fp32), within 1e-5."""
    case = MG.CASES["d64"]
    z = np.load(f"{MG.HERE}/golden_d64.npz")
    inp = MG.gen_inputs(case)
    assert np.allclose(MG.checksum(inp["q"]), z["ck_q"])
    c = dict(case["cfg"])
    cfg = hba_amd.HBAConfig(**c)
    n, d = case["n"], c["head_dim"]
    q, k, v = (torch.from_numpy(inp[t]).to(dev) for t in ("q", "k", "v"))
    prm = synth.Params(*(torch.from_numpy(inp[t]).to(dev) for t in ("q_gain", "k_gain", "probes", "proj")))
    cos, sin = hba_amd.rope_tables(n, d, cfg.rope_theta, dev)
    rows = z["rows"]
    out_d, aux = hba_amd.hba_attention_dense(q, k, v, cos, sin, cfg, prm, prm)
    out_e = hba_amd.hba_attention_eval(q, k, v, cos, sin, cfg, prm, prm, None)
    out_h = hba_amd.hba_attention_eval(q, k, v, cos, sin, cfg, prm, prm, None, hier=True)
    torch.cuda.synchronize()
    for got, key in ((out_d, "out_dense"), (out_e, "out_eval"), (out_h, "out_hier")):
        err = np.abs(f(got)[:, rows] - z[key]).max()
        assert err <= 1e-5, (key, err)


# ------------------------------------------- geometry outside the tuned path ----
@pytest.mark.parametrize("Bk,d,Hq,Hkv,n,W,S,k,m", [
    (16, 8, 4, 2, 512, 64, 4, 8, 4),          # the reference's own test geometry (tests/test_qknorm.py:28-35)
    (32, 96, 6, 2, 1024, 128, 8, 6, 2),       # a head dim and block size the tuned kernels do not take
    (64, 64, 14, 2, 8192, 1024, 4, 128, 4),   # k = n / block > 64 (the select-all gate, gates.py:211)
], ids=["block16-d8", "block32-d96", "k128"])
def test_fp32_generic_geometry_vs_oracle(dev, Bk, d, Hq, Hkv, n, W, S, k, m):
    """fp32 forward at geometry outside the tuned kernels (hba_generic.hip
    behind the same entry points): keys bit-exact, summaries within fp32
    rounding of the float64 restatement, the flat selection bit-exact against
    the oracle's declared order on the kernel's own summaries, and the union
    softmax within 1e-5 of the oracle's float64 rows; the eval drop-in gives
    the same output; off the tuned geometry a gradient request runs the
    generic backward (its values: test_gpu_geometry.py against the oracle's
    backward), and bf16 runs on the same kernels (inputs widened)."""
    cfg = hba_amd.HBAConfig(n_heads=Hq, n_kv=Hkv, head_dim=d, window=W, sinks=S, k_blocks=k, slots=m, block=Bk)
    x = synth.layer_inputs(1, n, Hq, Hkv, d, m=m, dtype=torch.float32, device=dev, seed=1, sharp=True)
    prm = synth.Params(x["q_gain"], x["k_gain"], x["probes"], x["proj"])
    cos, sin = hba_amd.rope_tables(n, d, cfg.rope_theta, dev)
    with torch.no_grad():
        r = hba_amd.forward_stages(x["q"], x["k"], x["v"], cos, sin, cfg, prm, prm)
        out_e = hba_amd.hba_attention_eval(x["q"], x["k"], x["v"], cos, sin, cfg, prm, prm)
    torch.cuda.synchronize()
    S0 = f(r["S0"])[0]
    P = O.prepare(f(x["q"])[0], f(x["k"])[0], f(x["v"])[0], f(cos), f(sin), cfg, f(x["probes"]), f(x["proj"]),
                  f(x["q_gain"]), f(x["k_gain"]), 1e-6, "f32", S0=S0)
    assert np.array_equal(f(r["kc"])[0].transpose(1, 0, 2), P.kc)
    assert np.array_equal(f(r["kr"])[0].transpose(1, 0, 2), P.kr)
    assert np.array_equal(f(r["vt"])[0].transpose(2, 0, 1), P.v)
    ref_S0 = O.summarize(P.kc, f(x["probes"]), f(x["proj"]), Bk)
    assert np.abs(S0 - ref_S0).max() <= 2e-5 * max(1.0, np.abs(ref_S0).max())
    kk = min(k, n // Bk)
    o_idx, o_val, o_cnt = O.flat_select(P.qg, P.S0, r["sel_scale"], kk, Bk, W)
    for key, want in (("idx", o_idx), ("val", o_val), ("cnt", o_cnt)):
        assert np.array_equal(r[key][0].cpu().numpy(), want), key
    assert int(o_cnt.max()) > 0
    rows = np.arange(n) if n <= 1024 else np.concatenate([np.arange(0, n, 41), np.arange(n - 64, n)])
    ref = O.attn_rows(P.qc, P.qr, P.kc, P.kr, P.v, o_idx, o_cnt, r["scale"], S, W, Bk, rows)
    assert np.abs(f(r["out"])[0][rows] - ref).max() <= 1e-5
    assert torch.equal(out_e, r["out"])
    if Bk != 64 or d not in (64, 128):   # a gradient request runs the generic fp32 backward
        q = x["q"].clone().requires_grad_(True)
        out_g = hba_amd.hba_attention_eval(q, x["k"], x["v"], cos, sin, cfg, prm, prm)
        assert torch.equal(out_g.detach(), r["out"])
        out_g.sum().backward()
        assert q.grad is not None and bool(torch.isfinite(q.grad).all()) and q.grad.abs().max().item() > 0
    if Bk != 64:   # bf16 off the tuned geometry: the generic kernels on the widened inputs
        xb = {t: x[t].bfloat16() for t in ("q", "k", "v")}
        with torch.no_grad():
            ob = hba_amd.hba_attention_eval(xb["q"], xb["k"], xb["v"], cos, sin, cfg, prm, prm)
            of = hba_amd.hba_attention_eval(xb["q"].float(), xb["k"].float(), xb["v"].float(), cos, sin, cfg, prm,
                                            prm)
        assert ob.dtype == torch.bfloat16 and torch.equal(ob, of.bfloat16())
