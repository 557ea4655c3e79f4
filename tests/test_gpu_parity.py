"""HIP kernels against the oracle, through the C-ABI (torch.library ops).

Bars: block selection bit-exact (indices, values and counts) when the kernel
and the oracle score identical summaries; key preparation and super-summaries
bit-exact; attention outputs within 1e-5 (fp32 inputs) / 2e-2 (bf16 inputs)
of the oracle's float64 union softmax on the same prepared tensors; the
summarizer within fp32 / one-bf16-ulp tolerance of the oracle's float64
restatement.  Sizes are small enough for the oracle to finish in seconds."""
import os

import numpy as np
import pytest
import torch

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


def make(dev, dt, n=2048, B=1, Hq=14, Hkv=2, d=64, m=4, W=512, S=4, k=8, sharp=True, seed=0,
         qknorm=True, needles=False, **cfgkw):
    cfg = hba_amd.HBAConfig(n_heads=Hq, n_kv=Hkv, head_dim=d, slots=m, window=W, sinks=S, k_blocks=k,
                            qknorm=qknorm, **cfgkw)
    x = synth.layer_inputs(B, n, Hq, Hkv, d, m=m, dtype=TDT[dt], device=dev, seed=seed, sharp=sharp,
                           needles=needles, window=W)
    prm = synth.Params(x["q_gain"], x["k_gain"], x["probes"], x["proj"])
    cos, sin = hba_amd.rope_tables(n, d, cfg.rope_theta, dev)
    return cfg, x, prm, cos, sin


def oracle_prep(cfg, x, cos, sin, dt, b, S0):
    return O.prepare(f(x["q"])[b], f(x["k"])[b], f(x["v"])[b], f(cos), f(sin), cfg, f(x["probes"]),
                     f(x["proj"]), f(x["q_gain"]), f(x["k_gain"]), 1e-6, dt, S0=S0)


# ------------------------------------------------------------ key prep -------
@pytest.mark.parametrize("dt", ["f32", "bf16"])
@pytest.mark.parametrize("d", [64, 128])
def test_prep_keys_bit_exact(dev, dt, d):
    cfg, x, prm, cos, sin = make(dev, dt, n=256, d=d, Hq=4, Hkv=2)
    kc, kr, vt = ops.prep_keys(x["k"], x["v"], x["k_gain"], 1e-6, cos, sin)
    torch.cuda.synchronize()
    kc_o = O.qknorm(f(x["k"])[0], f(x["k_gain"]), 1e-6, dt)                 # [n, Hkv, d]
    kr_o = O.apply_rope(kc_o, f(cos), f(sin), dt)
    assert np.array_equal(f(kc)[0].transpose(1, 0, 2), kc_o)
    assert np.array_equal(f(kr)[0].transpose(1, 0, 2), kr_o)
    assert np.array_equal(f(vt)[0], f(x["v"])[0].transpose(1, 2, 0))


def test_prep_keys_without_qknorm_is_passthrough(dev):
    cfg, x, prm, cos, sin = make(dev, "bf16", n=128, Hq=4, Hkv=2)
    kc, kr, vt = ops.prep_keys(x["k"], x["v"], None, 1e-6, cos, sin)
    assert torch.equal(kc[0].transpose(0, 1), x["k"][0])


# ------------------------------------------------------------- summaries -----
@pytest.mark.parametrize("dt", ["f32", "bf16"])
@pytest.mark.parametrize("d,m", [(64, 4), (128, 4), (64, 2)])
def test_summarize_matches_oracle(dev, dt, d, m):
    cfg, x, prm, cos, sin = make(dev, dt, n=512, d=d, m=m, Hq=4, Hkv=2)
    kc, _, _ = ops.prep_keys(x["k"], x["v"], x["k_gain"], 1e-6, cos, sin)
    S0 = ops.summarize(kc, x["probes"], x["proj"])
    ref = O.summarize(f(kc)[0].transpose(1, 0, 2), f(x["probes"]), f(x["proj"]), 64)
    got = f(S0)[0]
    tol = 2e-5 if dt == "f32" else 2 ** -7
    assert np.abs(got - ref).max() <= tol * max(1.0, np.abs(ref).max())


@pytest.mark.parametrize("dt,d,m,n,B,gain", [("bf16", 64, 4, 2048, 1, True), ("bf16", 64, 4, 1000, 2, False),
                                             ("bf16", 128, 4, 1037, 2, True), ("f32", 64, 2, 512, 1, True),
                                             ("f32", 128, 8, 640, 1, False), ("bf16", 64, 1, 64, 1, True)])
def test_prep_keys_summarize_equals_the_two_ops(dev, dt, d, m, n, B, gain):
    """hba_prep_keys_summarize (one launch) against hba_prep_keys then
    hba_summarize, bit for bit on kc, kr, vt and S0: both dtypes, d = 64/128,
    1/2/4/8 slots, with and without the key gains, B = 2, a partial last tile
    (n % 64 != 0: no summary for it) and a sequence of one block."""
    Hq, Hkv = (4, 2) if d == 64 else (8, 4)
    cfg, x, prm, cos, sin = make(dev, dt, n=n, B=B, d=d, m=m, Hq=Hq, Hkv=Hkv, W=64)
    kg = x["k_gain"] if gain else None
    kc, kr, vt = ops.prep_keys(x["k"], x["v"], kg, 1e-6, cos, sin)
    S0 = ops.summarize(kc, x["probes"], x["proj"])
    got = ops.prep_keys_summarize(x["k"], x["v"], kg, 1e-6, cos, sin, x["probes"], x["proj"])
    for name, a, b in zip(("kc", "kr", "vt", "S0"), (kc, kr, vt, S0), got):
        assert a.shape == b.shape and torch.equal(a, b), name


@pytest.mark.parametrize("dt", ["f32", "bf16"])
@pytest.mark.parametrize("nb,F", [(32, 16), (37, 4), (8, 16)])
def test_build_super_bit_exact(dev, dt, nb, F):
    g = torch.Generator().manual_seed(nb)
    S0 = torch.randn(2, 2, nb, 4, 64, generator=g).to(TDT[dt]).to(dev)
    S1 = ops.build_super(S0, F)
    for b in range(2):
        for h in range(2):
            assert np.array_equal(f(S1)[b, h], O.build_super(f(S0)[b, h], F, dt))


# ------------------------------------------------------------- selection -----
SEL_CASES = [
    dict(dt="f32", n=2048, W=512, k=8, d=64, m=4),
    dict(dt="bf16", n=2048, W=512, k=8, d=64, m=4),
    dict(dt="bf16", n=4096, W=1024, k=16, d=64, m=4, needles=True),
    dict(dt="f32", n=1024, W=128, k=16, d=128, m=2, Hq=28, Hkv=4),
    dict(dt="bf16", n=1024, W=256, k=32, d=64, m=8, B=2),
    dict(dt="f32", n=768, W=64, k=64, d=64, m=4),            # select-all (k >= candidates)
    dict(dt="bf16", n=4096, W=512, k=32, d=64, m=4),          # GEMM path, 32-entry lane lists
    dict(dt="bf16", n=2048, W=256, k=16, d=128, m=4, Hq=28, Hkv=4, B=2),   # GEMM path, d = 128
    dict(dt="bf16", n=2048, W=512, k=8, d=64, m=4, qknorm=False),         # routing query without gains
    dict(dt="bf16", n=1088, W=256, k=16, d=64, m=4, Hq=8, Hkv=2),         # G = 4; ragged routed tile
    dict(dt="bf16", n=4096, W=512, k=48, d=64, m=4),          # k > 32: the declared-order kernel in bf16
]


def margin_equal(k_idx, k_cnt, o_scores, kk, rel=1e-5):
    """Kernel selection vs the oracle's declared-order scores o_scores [r, nb]:
    identical sets, except that blocks whose oracle score is within `rel` of
    the k-th score (a near-tie at the top-k boundary) may be swapped."""
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


def uses_mfma(dt, m, k):
    return dt == "bf16" and m == 4 and k <= 32


@pytest.mark.parametrize("case", SEL_CASES, ids=lambda c: "-".join(f"{k}{v}" for k, v in c.items()))
def test_flat_select(dev, case):
    """fp32 (and bf16 with m != 4): bit-exact against the oracle's declared
    order.  bf16 MFMA path: top-k bit-exact on the kernel's own score array,
    scores within fp32 accumulation noise of the oracle's, and the same sets
    up to near-ties at the k boundary."""
    c = dict(case)
    dt = c.pop("dt")
    cfg, x, prm, cos, sin = make(dev, dt, **c)
    n = x["q"].shape[1]
    kk = min(cfg.k_blocks, n // 64)
    r = hba_amd.forward_stages(x["q"], x["k"], x["v"], cos, sin, cfg, prm, prm)
    qg = x["q_gain"] if cfg.qknorm else None
    idx, val, cnt, scores = ops.score_select_with_scores(x["q"], qg, 1e-6, r["S0"], cfg.window,
                                                         kk, r["sel_scale"])
    torch.cuda.synchronize()
    assert torch.equal(idx, r["idx"]) and torch.equal(cnt, r["cnt"])
    S0 = f(r["S0"])
    sc = scores.cpu().numpy()
    for b in range(x["q"].shape[0]):
        P = oracle_prep(cfg, x, cos, sin, dt, b, S0[b])
        o_idx, o_val, o_cnt = O.flat_select(P.qg, P.S0, r["sel_scale"], kk, 64, cfg.window)
        ki, kv, kc_ = idx[b].cpu().numpy(), val[b].cpu().numpy(), cnt[b].cpu().numpy()
        # top-k of the kernel's own scores, by the oracle: bit-exact
        for g in range(cfg.n_kv):
            ti, tv, tc = O.topk(sc[b, g], kk)
            assert np.array_equal(ti, ki[g]) and np.array_equal(tv, kv[g]) and np.array_equal(tc, kc_[g])
        if not uses_mfma(dt, cfg.slots, kk):
            assert np.array_equal(ki, o_idx) and np.array_equal(kv, o_val) and np.array_equal(kc_, o_cnt)
            continue
        for g in range(cfg.n_kv):
            osc = O.block_scores(P.qg[g], P.S0[g], np.arange(n), r["sel_scale"], 64, cfg.window)
            fin = np.isfinite(osc)
            assert np.array_equal(np.isfinite(sc[b, g]), fin)
            assert np.abs(sc[b, g][fin] - osc[fin]).max() <= 2e-6 * max(1.0, np.abs(osc[fin]).max())
            flips = margin_equal(ki[g], kc_[g], osc, kk)
            assert flips <= max(2, n // 1000), flips


@pytest.mark.parametrize("dt", ["f32", "bf16"])
@pytest.mark.parametrize("d,Hq,Hkv,qknorm", [(64, 14, 2, True), (128, 16, 1, True), (64, 4, 4, False),
                                             (128, 28, 4, False)])
def test_route_queries_bit_exact(dev, dt, d, Hq, Hkv, qknorm):
    """hba_route_queries: grouped_query of the QKNorm'd heads (declared order,
    storage roundings) against the oracle, bit for bit."""
    cfg, x, prm, cos, sin = make(dev, dt, n=384, d=d, Hq=Hq, Hkv=Hkv, qknorm=qknorm)
    gain = x["q_gain"] if qknorm else None
    rq = ops.route_queries(x["q"], gain, 1e-6, Hkv)
    torch.cuda.synchronize()
    qc = O.qknorm(f(x["q"])[0], f(x["q_gain"]), 1e-6, dt) if qknorm else f(x["q"])[0]
    want = O.grouped_query(qc, Hkv, dt)                                   # [Hkv, n, d]
    assert np.array_equal(f(rq)[0].transpose(1, 0, 2), want)
    if not qknorm:   # the grouped_query drop-in (summarizer.py:50-54): [B, Hkv, n, d]
        assert np.array_equal(f(hba_amd.grouped_query(x["q"], cfg))[0], want)


@pytest.mark.parametrize("dt,hier", [("bf16", False), ("f32", False), ("bf16", True), ("f32", True)])
def test_selection_on_routed_queries_equals_selection_on_q(dev, dt, hier):
    """The selection kernels on the precomputed routing queries (one head per
    KV group, no gain) pick exactly what they pick on q: idx, val and cnt
    bit-identical, flat and hierarchical."""
    n = 4096
    cfg, x, prm, cos, sin = make(dev, dt, n=n, W=512, k=16, needles=True)
    kc, _, _ = ops.prep_keys(x["k"], x["v"], x["k_gain"], 1e-6, cos, sin)
    S0 = ops.summarize(kc, x["probes"], x["proj"])
    rq = ops.route_queries(x["q"], x["q_gain"], 1e-6, cfg.n_kv)
    scale = hba_amd.union_scale(cfg, 64, n)
    if hier:
        S1 = ops.build_super(S0, 8)
        a = ops.hier_select(x["q"], x["q_gain"], 1e-6, S0, S1, cfg.window, 16, 8, 4, scale)
        b = ops.hier_select(rq, None, 1e-6, S0, S1, cfg.window, 16, 8, 4, scale)
    else:
        a = ops.score_select(x["q"], x["q_gain"], 1e-6, S0, cfg.window, 16, scale)
        b = ops.score_select(rq, None, 1e-6, S0, cfg.window, 16, scale)
    torch.cuda.synchronize()
    for ta, tb in zip(a, b):
        assert torch.equal(ta, tb)


@pytest.mark.parametrize("dt", ["bf16", "f32"])
@pytest.mark.parametrize("pattern", ["lane0", "ties", "zero_q"])
def test_flat_select_adversarial(dev, pattern, dt):
    """Selection on score layouts that stress the tie rule and the bf16 MFMA
    path's first-pass threshold: the best blocks all fall to one of the four
    lanes that scan a query's blocks (blocks 1, 5, 9, ...), massive ties, and
    all-zero scores.  The top-k must equal the top-k (score desc, block asc)
    of the kernel's own score array."""
    torch.manual_seed(3)
    n, Hkv, Hq, d, m, W, kk = 4096, 2, 14, 64, 4, 512, 16
    nb = n // 64
    tdt = torch.bfloat16 if dt == "bf16" else torch.float32
    q = torch.randn(1, n, Hq, d, device=dev).to(tdt)
    if pattern == "zero_q":
        q.zero_()
    gq = torch.full((Hq,), d ** 0.25, device=dev)
    v = torch.randn(d)
    a = torch.ones(nb)
    if pattern == "lane0":
        a[1::4] = 4.0 + torch.arange(a[1::4].numel()) / 64.0      # blocks 1, 5, 9, ... rank above the rest
    elif pattern == "ties":
        a = (torch.arange(nb) % 3).float() + 1.0                    # three values, a third of the blocks each
    S0 = (a[:, None, None] * v[None, None, :]).expand(nb, m, d).contiguous()
    S0 = S0[None, None].expand(1, Hkv, nb, m, d).contiguous().to(tdt).to(dev)
    idx, val, cnt, scores = ops.score_select_with_scores(q, gq, 1e-6, S0, W, kk, 0.125)
    torch.cuda.synchronize()
    sc = scores[0].cpu().numpy()
    ki, kv, kc_ = idx[0].cpu().numpy(), val[0].cpu().numpy(), cnt[0].cpu().numpy()
    for g in range(Hkv):
        ti, tv, tc = O.topk(sc[g], kk)
        assert np.array_equal(ti, ki[g]) and np.array_equal(tv, kv[g]) and np.array_equal(tc, kc_[g])


HIER_CASES = [
    dict(dt="f32", n=4096, W=512, k=8, fanout=4, beam=2),
    dict(dt="bf16", n=4096, W=1024, k=16, fanout=16, beam=2),
    dict(dt="bf16", n=8192, W=1024, k=16, fanout=16, beam=8, needles=True),
    dict(dt="f32", n=2048, W=256, k=16, fanout=8, beam=16, d=128, Hq=28, Hkv=4),
    dict(dt="bf16", n=2048, W=256, k=32, fanout=8, beam=16, d=128, Hq=28, Hkv=4, B=2),   # beam > supers
    dict(dt="bf16", n=4096, W=512, k=8, fanout=4, beam=3, m=2),                          # scalar bf16 path
    dict(dt="bf16", n=6144, W=700, k=12, fanout=5, beam=4),                              # ragged last super
    dict(dt="bf16", n=1024, W=1024, k=16, fanout=16, beam=2),                            # no candidates
    dict(dt="bf16", n=4096, W=512, k=40, fanout=8, beam=6),                              # k > 32: declared order
]


def hier_uses_mfma(dt, m, k, nb, F):
    return uses_mfma(dt, m, k) and (nb + F - 1) // F <= 2048


def check_hier_dumps(qg, S0, S1, F, beam, kk, scale, W, ki, kv, kc_, sc, sup):
    """The bf16 GEMM path of hier_select for one KV head, through the scores
    it ranked: the super set and the child set it scored are exactly the
    oracle's rules, both score arrays agree with the declared-order fp32
    scores to GEMM rounding, and the picks are the oracle's top-k of the
    kernel's own scores (bit-exact)."""
    n, nb = sc.shape
    ns = sup.shape[1]
    beff = min(beam, ns)
    kout = min(kk, beff * F)
    bmax = np.array([O.cand_bmax(i, 64, W) for i in range(n)])
    lo = np.arange(ns) * F
    hi = np.minimum(lo + F - 1, nb - 1)
    valid = (bmax[:, None] >= 1) & (lo[None, :] <= bmax[:, None]) & (hi[None, :] >= 1)
    assert np.array_equal(np.isfinite(sup), valid)
    if valid.any():
        # supers: float64 scores, max over slots
        ex = (qg.astype(np.float64) @ S1.reshape(-1, S1.shape[-1]).T.astype(np.float64))
        ex = ex.reshape(n, ns, -1).max(-1) * scale
        assert np.abs(sup[valid] - ex[valid]).max() <= 2e-6 * max(1.0, np.abs(ex[valid]).max())
    pi, pv, pc = O.topk(sup, beff)
    kept = np.zeros((n, nb), dtype=bool)
    for r in range(n):
        for p in pi[r, : pc[r]]:
            kept[r, p * F: min(nb, p * F + F)] = True
    blk = np.arange(nb)
    cand = (blk[None, :] >= 1) & (blk[None, :] <= bmax[:, None])
    assert np.array_equal(np.isfinite(sc), kept & cand)
    osc = O.block_scores(qg, S0, np.arange(n), scale, 64, W)
    fin = np.isfinite(sc)
    if fin.any():
        assert np.abs(sc[fin] - osc[fin]).max() <= 2e-6 * max(1.0, np.abs(osc[fin]).max())
    ti, tv, tc = O.topk(sc, kout)
    pad = kk - kout
    ti = np.concatenate([ti, np.full((n, pad), -1, np.int32)], 1)
    tv = np.concatenate([tv, np.full((n, pad), -np.inf, np.float32)], 1)
    assert np.array_equal(ti, ki) and np.array_equal(tv, kv) and np.array_equal(tc, kc_)


@pytest.mark.parametrize("case", HIER_CASES, ids=lambda c: "-".join(f"{k}{v}" for k, v in c.items()))
def test_hier_select(dev, case):
    """fp32, and bf16 off the GEMM path: bit-exact against the oracle's
    hier_select.  bf16 on the GEMM path (m == 4, k <= 32): the dump check
    above on the kernel's own super and child scores."""
    c = dict(case)
    dt = c.pop("dt")
    cfg, x, prm, cos, sin = make(dev, dt, **c)
    r = hba_amd.forward_stages(x["q"], x["k"], x["v"], cos, sin, cfg, prm, prm, hier=True)
    torch.cuda.synchronize()
    B, n = x["q"].shape[:2]
    kk = min(cfg.k_blocks, n // 64)
    mfma = hier_uses_mfma(dt, cfg.slots, kk, n // 64, cfg.fanout)
    if mfma:
        idx, val, cnt, scores, sup = ops.hier_select_with_scores(
            x["q"], prm.q.gain, 1e-6, r["S0"], r["S1"], cfg.window, kk, cfg.fanout, cfg.beam, r["sel_scale"])
        torch.cuda.synchronize()
        for t, u in ((idx, r["idx"]), (val, r["val"]), (cnt, r["cnt"])):
            assert torch.equal(t, u)   # the dumps do not change the picks
        sc, sp = scores.cpu().numpy(), sup.cpu().numpy()
    for b in range(B):
        P = oracle_prep(cfg, x, cos, sin, dt, b, f(r["S0"])[b])
        S1 = f(r["S1"])[b]
        for g in range(S1.shape[0]):
            assert np.array_equal(S1[g], O.build_super(P.S0[g], cfg.fanout, dt))
        ki, kv, kc_ = (r[t][b].cpu().numpy() for t in ("idx", "val", "cnt"))
        if not mfma:
            idx, val, cnt = O.hier_select(P.qg, P.S0, S1, cfg.fanout, cfg.beam, kk, r["sel_scale"], 64,
                                          cfg.window)
            assert np.array_equal(kc_, cnt) and np.array_equal(ki, idx) and np.array_equal(kv, val)
            continue
        for g in range(S1.shape[0]):
            check_hier_dumps(P.qg[g], P.S0[g], S1[g], cfg.fanout, cfg.beam, kk, r["sel_scale"], cfg.window,
                             ki[g], kv[g], kc_[g], sc[b, g], sp[b, g])


@pytest.mark.parametrize("pattern", ["ties", "lane0"])
def test_hier_select_adversarial(dev, pattern):
    """bf16 GEMM path of hier_select on tied and lane-aligned block layouts:
    equal super scores must resolve to the lowest super, equal child scores
    to the lowest block."""
    torch.manual_seed(5)
    n, Hkv, Hq, d, m, W, kk, F, beam = 8192, 2, 14, 64, 4, 512, 16, 8, 4
    nb = n // 64
    q = torch.randn(1, n, Hq, d, device=dev).to(torch.bfloat16)
    gq = torch.full((Hq,), d ** 0.25, device=dev)
    v = torch.randn(d)
    if pattern == "lane0":
        a = torch.ones(nb)
        a[1::4] = 4.0 + torch.arange(a[1::4].numel()) / 64.0
    else:
        a = (torch.arange(nb) % 3).float() + 1.0
    S0 = (a[:, None, None] * v[None, None, :]).expand(nb, m, d).contiguous()
    S0 = S0[None, None].expand(1, Hkv, nb, m, d).contiguous().to(torch.bfloat16).to(dev)
    S1 = ops.build_super(S0, F)
    idx, val, cnt, scores, sup = ops.hier_select_with_scores(q, gq, 1e-6, S0, S1, W, kk, F, beam, 0.125)
    torch.cuda.synchronize()
    qg = O.grouped_query(O.qknorm(f(q)[0], f(gq), 1e-6, "bf16"), Hkv, "bf16")
    for g in range(Hkv):
        check_hier_dumps(qg[g], f(S0)[0, g], f(S1)[0, g], F, beam, kk, 0.125, W, idx[0, g].cpu().numpy(),
                         val[0, g].cpu().numpy(), cnt[0, g].cpu().numpy(), scores[0, g].cpu().numpy(),
                         sup[0, g].cpu().numpy())


@pytest.mark.parametrize("dt", ["f32", "bf16"])
@pytest.mark.parametrize("nb,F,beam,kk", [(37, 4, 3, 8), (64, 16, 2, 40), (200, 8, 30, 16), (1000, 16, 8, 16)])
def test_hier_select_drop_in_any_mask(dev, dt, nb, F, beam, kk):
    """hba_amd.hier_select, the reference's hier_select(qn, S0, S1, fanout,
    beam, kk, cand, scale) with an arbitrary candidate mask (hba_hier_select_rows),
    against the oracle's masked form: picks and scores bit-exact in fp32 and
    bf16 (fp32 declared-order scores of the stored values), over ragged last
    supers, beam > ns, kk > beam * fanout, rows without a candidate, an
    all-candidate row and tied summaries; the comparison count as the
    reference returns it."""
    g = torch.Generator().manual_seed(nb + F)
    B, c, m, d = 2, 50, 4, 64
    qn = torch.randn(B, c, d, generator=g).to(TDT[dt]).to(dev)
    S0 = torch.randn(B, nb, m, d, generator=g)
    S0[:, 9] = S0[:, 5]                                   # tied blocks
    S0 = S0.to(TDT[dt]).to(dev)
    S1, ns = hba_amd.build_super(S0, F)
    cand = torch.rand(c, nb, generator=g) < 0.3
    cand[:, 5] = cand[:, 9] = True
    cand[4] = False
    cand[7] = True
    scale = 0.125
    idx, val, ncomp = hba_amd.hier_select(qn, S0, S1, F, beam, kk, cand.to(dev), scale)
    torch.cuda.synchronize()
    assert ncomp == ns + min(beam, ns) * F
    for b in range(B):
        oi, ov, oc = O.hier_select_mask(f(qn[b]), f(S0[b]), f(S1[b]), F, beam, kk, cand.numpy(), scale)
        assert np.array_equal(idx[b].cpu().numpy(), oi), b
        assert np.array_equal(val[b].cpu().numpy(), ov), b
    assert (idx[:, 4] == -1).all()


@pytest.mark.parametrize("n,F,beam,kk,B,dump", [(8192, 8, 4, 16, 1, True), (32768, 16, 8, 16, 2, True),
                                                  (32768, 4, 16, 32, 1, True), (24576, 16, 3, 8, 1, True),
                                                  (131072, 16, 8, 16, 1, False)])
def test_hier_grouped_level2_equals_per_tile(dev, n, F, beam, kk, B, dump):
    """The bf16 descent's second level scored per group of queries (with a
    workspace: each super's children once for the group's queries that kept
    it) and per 64-query tile give the same picks, values and counts, and the
    same super and child score dumps: the same MFMA operands in the same
    order, the same ranking rule.  Cases: fanout 4 / 8 / 16, beam 3 to 16,
    k up to 32, two batches, n not a multiple of the group, 128K (picks
    only: the dump would be 2 GB)."""
    g = torch.Generator().manual_seed(n + F + beam)
    Hkv, Hq, d, m, W = 2, 14, 64, 4, 1024
    nb = n // 64
    q = torch.randn(B, n, Hq, d, generator=g).to(torch.bfloat16).to(dev)
    gq = torch.full((Hq,), d ** 0.25, device=dev)
    S0 = (torch.randn(B, Hkv, nb, m, d, generator=g) * 0.5).to(torch.bfloat16).to(dev)
    S1 = ops.build_super(S0, F)
    assert ops.hier_workspace_bytes(q, S0, kk, F, beam) > 0   # the grouped path applies
    if dump:
        a = ops.hier_select_with_scores(q, gq, 1e-6, S0, S1, W, kk, F, beam, 0.125, grouped=True)
        t = ops.hier_select_with_scores(q, gq, 1e-6, S0, S1, W, kk, F, beam, 0.125, grouped=False)
    else:
        a = ops._hier_select(q, gq, 1e-6, S0, S1, W, kk, F, beam, 0.125, None, None, grouped=True)
        t = ops._hier_select(q, gq, 1e-6, S0, S1, W, kk, F, beam, 0.125, None, None, grouped=False)
    torch.cuda.synchronize()
    for x, y in zip(a, t):
        assert torch.equal(x, y)
    assert int(a[2].max()) == min(kk, min(beam, (nb + F - 1) // F) * F)


def test_hier_select_threshold_overflow(dev):
    """A layout on which the by-super path's threshold admits more children
    than its 64-entry list: child c < 8 of super j scores 255 - 32 c - j
    (times the query's first routing element), child c >= 8 scores 0, so for
    a query with a positive first element the 2 best children per child slot
    put the 16th-best key low and children 0..6 of all 16 kept supers (112)
    clear it; the exact kernel then recomputes those tiles.  Every value is
    exact in bf16 and in the products, so the picks are fixed; beam and
    fanout are the largest that path takes."""
    torch.manual_seed(11)
    n, Hkv, Hq, d, m, W, kk, F, beam = 32768, 2, 14, 64, 4, 1024, 16, 16, 16
    nb = n // 64
    blk = torch.arange(nb)
    a = torch.where(blk % 16 < 8, 255 - 32 * (blk % 16) - blk // 16, torch.zeros_like(blk)).float()
    q = torch.randn(1, n, Hq, d, device=dev).to(torch.bfloat16)
    gq = torch.full((Hq,), d ** 0.25, device=dev)
    S0 = torch.zeros(1, Hkv, nb, m, d)
    S0[..., 0] = a[None, None, :, None]
    S0 = S0.to(torch.bfloat16).to(dev)
    S1 = ops.build_super(S0, F)
    idx, val, cnt, scores, sup = ops.hier_select_with_scores(q, gq, 1e-6, S0, S1, W, kk, F, beam, 0.125)
    torch.cuda.synchronize()
    qg = O.grouped_query(O.qknorm(f(q)[0], f(gq), 1e-6, "bf16"), Hkv, "bf16")
    for g in range(Hkv):
        check_hier_dumps(qg[g], f(S0)[0, g], f(S1)[0, g], F, beam, kk, 0.125, W, idx[0, g].cpu().numpy(),
                         val[0, g].cpu().numpy(), cnt[0, g].cpu().numpy(), scores[0, g].cpu().numpy(),
                         sup[0, g].cpu().numpy())


# ------------------------------------------------------------- attention -----
ATTN_CASES = [
    dict(dt="f32", n=2048, W=512, k=8),
    dict(dt="f32", n=1024, W=256, k=4, d=128, Hq=28, Hkv=4, B=2),
    dict(dt="bf16", n=2048, W=512, k=8),
    dict(dt="bf16", n=4096, W=1024, k=16, needles=True),
    dict(dt="bf16", n=2048, W=512, k=8, d=128, Hq=28, Hkv=4, S=8, B=2),
    dict(dt="bf16", n=1024, W=256, k=4, Hq=4, Hkv=2, S=0),
    dict(dt="bf16", n=512, W=1024, k=16, S=64),                # no candidates, sinks = block
    dict(dt="bf16", n=2048, W=384, k=8, qknorm=False, sharp=False),
    dict(dt="f32", n=2048, W=512, k=8, native_ctx=512, temp_c=0.1),   # temperature active
    dict(dt="bf16", n=1024, W=200, k=6, Hq=16, Hkv=2, content_scale_mode="inv_sqrt_d"),
    dict(dt="bf16", n=1088, W=256, k=16, Hq=8, Hkv=2),        # G = 4: 128-query routed tiles, the last ragged
    dict(dt="bf16", n=2048, W=384, k=12, d=128, Hq=28, Hkv=4, B=2, needles=True),   # d = 128, 48-query tiles
]


@pytest.mark.parametrize("case", ATTN_CASES, ids=lambda c: "-".join(f"{k}{v}" for k, v in c.items()))
def test_attention_matches_oracle(dev, case):
    c = dict(case)
    dt = c.pop("dt")
    cfg, x, prm, cos, sin = make(dev, dt, **c)
    r = hba_amd.forward_stages(x["q"], x["k"], x["v"], cos, sin, cfg, prm, prm)
    torch.cuda.synchronize()
    B, n = x["q"].shape[:2]
    rows = np.unique(np.concatenate([np.arange(0, 72), np.linspace(0, n - 1, 96).astype(int),
                                     np.arange(n - 70, n)]))
    out = f(r["out"])
    for b in range(B):
        P = oracle_prep(cfg, x, cos, sin, dt, b, f(r["S0"])[b])
        kc, kr = f(r["kc"])[b].transpose(1, 0, 2), f(r["kr"])[b].transpose(1, 0, 2)
        ref = O.attn_rows(P.qc, P.qr, kc, kr, P.v, r["idx"][b].cpu().numpy(), r["cnt"][b].cpu().numpy(),
                          r["scale"], cfg.sinks, cfg.window, 64, rows)
        err = np.abs(out[b][rows] - ref).max()
        assert err <= TOL[dt], err
        assert np.isfinite(out[b]).all()


def test_attention_bf16_precision_is_far_inside_the_bar(dev):
    """The bf16 kernel at the benchmark geometry (sharp gains, needles): the
    error against the float64 oracle should be a few bf16 ulps of the output,
    well inside 2e-2 -- a loose pass of the bar is not the target."""
    cfg, x, prm, cos, sin = make(dev, "bf16", n=4096, W=1024, k=16, needles=True)
    r = hba_amd.forward_stages(x["q"], x["k"], x["v"], cos, sin, cfg, prm, prm)
    torch.cuda.synchronize()
    rows = np.linspace(2048, 4095, 64).astype(int)
    P = oracle_prep(cfg, x, cos, sin, "bf16", 0, f(r["S0"])[0])
    ref = O.attn_rows(P.qc, P.qr, P.kc, P.kr, P.v, r["idx"][0].cpu().numpy(), r["cnt"][0].cpu().numpy(),
                      r["scale"], cfg.sinks, cfg.window, 64, rows)
    err = np.abs(f(r["out"])[0][rows] - ref)
    assert err.max() <= 8e-3 and err.mean() <= 1e-3, (err.max(), err.mean())


@pytest.mark.parametrize("dt", ["f32", "bf16"])
def test_end_to_end_eval_and_dense_vs_oracle(dev, dt):
    """The whole wrapper (hba_attention_eval / _dense) against the oracle's
    forward_eval / forward_dense fed the kernel's summaries."""
    cfg, x, prm, cos, sin = make(dev, dt, n=2048, W=512, k=8, native_ctx=1024)
    out_e = hba_amd.hba_attention_eval(x["q"], x["k"], x["v"], cos, sin, cfg, prm, prm, None)
    out_d, aux = hba_amd.hba_attention_dense(x["q"], x["k"], x["v"], cos, sin, cfg, prm, prm)
    S0 = f(ops.summarize(ops.prep_keys(x["k"], x["v"], x["k_gain"], 1e-6, cos, sin)[0], x["probes"],
                         x["proj"]))
    rows = np.linspace(0, 2047, 80).astype(int)
    args = (f(x["q"]), f(x["k"]), f(x["v"]), f(cos), f(sin), cfg, f(x["probes"]), f(x["proj"]),
            f(x["q_gain"]), f(x["k_gain"]), 1e-6, dt)
    ref_e, _ = O.forward_eval(*args, rows=rows, S0=S0)
    ref_d, _ = O.forward_dense(*args, rows=rows, S0=S0)
    assert np.abs(f(out_e)[0][rows] - ref_e[0]).max() <= TOL[dt]
    assert np.abs(f(out_d)[0][rows] - ref_d[0]).max() <= TOL[dt]
    # aux_w = 1 (the default): the summarizer's aux-KL comes back with the output
    qc, kc, su = O.content_qk(f(x["q"]), f(x["k"]), cfg, f(x["q_gain"]), f(x["k_gain"]), 1e-6, 2048, dt)
    aref = O.aux_kl(qc, kc, f(x["probes"]), f(x["proj"]), cfg.n_kv, su, O.route_scale(cfg, 64), 64, cfg.window,
                    S0_scores=S0, dtype=dt)[0]
    assert abs(float(aux) - aref) <= 1e-5 * abs(aref), (float(aux), aref)


def test_strided_views_are_accepted(dev):
    """q/k/v as views into a fused projection output (model.py:121-123 shape)."""
    cfg, x, prm, cos, sin = make(dev, "bf16", n=1024, W=256, k=4)
    B, n, Hq, d = x["q"].shape
    Hkv = x["k"].shape[2]
    big = torch.cat([x["q"].reshape(B, n, -1), x["k"].reshape(B, n, -1), x["v"].reshape(B, n, -1)], -1)
    q = big[..., : Hq * d].view(B, n, Hq, d)
    k = big[..., Hq * d:(Hq + Hkv) * d].view(B, n, Hkv, d)
    v = big[..., (Hq + Hkv) * d:].view(B, n, Hkv, d)
    assert not q.is_contiguous()
    a = hba_amd.hba_attention_eval(q, k, v, cos, sin, cfg, prm, prm, None)
    b = hba_amd.hba_attention_eval(x["q"], x["k"], x["v"], cos, sin, cfg, prm, prm, None)
    assert torch.equal(a, b)


def test_invalid_arguments_raise(dev):
    cfg, x, prm, cos, sin = make(dev, "bf16", n=1024, W=256, k=4)
    with pytest.raises(AssertionError):
        hba_amd.hba_attention_eval(x["q"][:, :1000], x["k"][:, :1000], x["v"][:, :1000], cos, sin, cfg,
                                   prm, prm, None)
    r = hba_amd.forward_stages(x["q"], x["k"], x["v"], cos, sin, cfg, prm, prm)
    with pytest.raises(RuntimeError):                                      # bf16 kernels: at most 128 sinks
        ops.attn_fwd(x["q"], prm.q.gain, prm.k.gain, 1e-6, r["kc"], r["kr"], r["vt"], cos, sin, r["idx"], r["cnt"],
                     129, cfg.window, r["scale"])
    S0 = torch.zeros(1, 2, 16, 4, 64, dtype=torch.bfloat16, device=dev)
    with pytest.raises(RuntimeError):                                      # k > 64
        ops.score_select(x["q"], x["q_gain"], 1e-6, S0, 256, 65, 1 / 64)
    with pytest.raises(ValueError):
        cfg4 = hba_amd.HBAConfig(n_heads=14, n_kv=2, window=256, content_scale_mode="bogus")
        hba_amd.hba_attention_eval(x["q"], x["k"], x["v"], cos, sin, cfg4, prm, prm, None)
    cprm = synth.Params(x["q_gain"].cpu(), x["k_gain"].cpu(), x["probes"].cpu(), x["proj"].cpu())
    with pytest.raises((NotImplementedError, RuntimeError)):               # no CPU path
        hba_amd.hba_attention_eval(x["q"].cpu(), x["k"].cpu(), x["v"].cpu(), cos.cpu(), sin.cpu(), cfg,
                                   cprm, cprm, None)


def test_overlapped_schedule_matches_one_launch(dev):
    """forward_stages(overlap=True) runs the bf16 attention as two launches,
    the window on a second stream while the selection runs, then the sinks
    and routed blocks merged by LSE; the default runs it as one launch after
    the selection (hba_attn_fwd, bit-identical).  The two forms compute the
    same softmax and differ only by the window rows' bf16 rounding before
    the merge (at most 2**-6 apart on these unit-scale values, 1e-4 on
    average), and both are within the bf16 bar of the oracle on sampled rows."""
    cfg, x, prm, cos, sin = make(dev, "bf16", n=4096, W=1024, k=16, needles=True)
    seq = hba_amd.forward_stages(x["q"], x["k"], x["v"], cos, sin, cfg, prm, prm)
    ref = ops.attn_fwd(x["q"], prm.q.gain, prm.k.gain, 1e-6, seq["kc"], seq["kr"], seq["vt"], cos, sin, seq["idx"],
                       seq["cnt"], cfg.sinks, cfg.window, seq["scale"])
    torch.cuda.synchronize()
    assert torch.equal(seq["out"], ref)
    P = O.prepare(f(x["q"])[0], f(x["k"])[0], f(x["v"])[0], f(cos), f(sin), cfg, f(x["probes"]), f(x["proj"]),
                  f(x["q_gain"]), f(x["k_gain"]), 1e-6, "bf16", S0=f(seq["S0"])[0])
    rows = np.unique(np.concatenate([np.arange(0, 70), np.linspace(0, 4095, 120).astype(np.int64),
                                     np.arange(4030, 4096)]))
    idx, cnt = seq["idx"][0].cpu().numpy(), seq["cnt"][0].cpu().numpy()
    dense = O.dense_rows(P.qc, P.qr, P.kc, P.kr, P.v, lambda g, i: idx[g, i, :cnt[g, i]], seq["scale"], cfg.sinks,
                         cfg.window, 64, rows)
    a = f(seq["out"])[0]
    for _ in range(3):   # repeated calls reuse the side stream and the allocator's blocks
        r = hba_amd.forward_stages(x["q"], x["k"], x["v"], cos, sin, cfg, prm, prm, overlap=True)
        torch.cuda.synchronize()
        assert torch.equal(r["idx"], seq["idx"])
        b = f(r["out"])[0]
        dab = np.abs(a - b)
        assert dab.max() <= 2 ** -6 and dab.mean() <= 1e-4, (dab.max(), dab.mean())
        for o in (a, b):
            assert np.abs(o[rows] - dense).max() <= 2e-2


@pytest.mark.parametrize("qknorm,G,k", [(True, 7, 16), (False, 7, 16), (True, 4, 12), (True, 8, 16)])
def test_attention_bf16_is_deterministic(dev, qknorm, G, k):
    """The bf16 union attention gives the same bits on repeated calls (every
    workgroup adds its partials in a fixed order), with the fixed softmax
    shift and with the running maximum (no QKNorm)."""
    cfg, x, prm, cos, sin = make(dev, "bf16", n=4096, W=1024, k=k, Hq=2 * G, Hkv=2, needles=True, qknorm=qknorm,
                                 sharp=qknorm)
    r = hba_amd.forward_stages(x["q"], x["k"], x["v"], cos, sin, cfg, prm, prm, overlap=False)
    qg, kg = (prm.q.gain, prm.k.gain) if qknorm else (None, None)
    outs = [ops.attn_fwd(x["q"], qg, kg, 1e-6, r["kc"], r["kr"], r["vt"], cos, sin, r["idx"], r["cnt"], cfg.sinks,
                         cfg.window, r["scale"]) for _ in range(3)]
    torch.cuda.synchronize()
    assert all(torch.equal(o, r["out"]) for o in outs)
    assert torch.isfinite(outs[0].float()).all()


@pytest.mark.parametrize("dt,qknorm,n", [("bf16", True, 2048), ("bf16", False, 1024), ("f32", True, 512)])
def test_equiv_matches_oracle(dev, dt, qknorm, n):
    """equiv=True (attention.py:330-336, 634-649): dense uniform-RoPE causal
    attention, through the eval and dense drop-ins."""
    cfg, x, prm, cos, sin = make(dev, dt, n=n, qknorm=qknorm)
    out = hba_amd.hba_attention_eval(x["q"], x["k"], x["v"], cos, sin, cfg, prm, prm, None, equiv=True)
    out2, aux = hba_amd.hba_attention_dense(x["q"], x["k"], x["v"], cos, sin, cfg, prm, prm, equiv=True)
    torch.cuda.synchronize()
    assert torch.equal(out, out2) and float(aux) == 0.0
    rows = np.unique(np.concatenate([[0, 1, 2, 63, 64, 65, n // 2, n - 1],
                                     np.random.RandomState(0).randint(0, n, 24)]))
    ref = O.forward_equiv(f(x["q"]), f(x["k"]), f(x["v"]), f(cos), f(sin), cfg, f(x["q_gain"]), f(x["k_gain"]),
                          1e-6, dt, rows)
    err = np.abs(f(out)[:, rows] - ref).max()
    assert err <= TOL[dt], err


@pytest.mark.parametrize("dt", ["f32", "bf16"])
def test_equiv_with_yarn_tables_matches_oracle(dev, dt):
    """The donor+YaRN eval baseline (evals.py:194-197): equiv attention at
    n = 4 x native_ctx with cos/sin built from yarn_theta, against the oracle
    on the same tables (they differ from the native ones)."""
    n = 2048
    cfg, x, prm, cos, sin = make(dev, dt, n=n, native_ctx=512)
    th = hba_amd.yarn_theta(cfg, n)
    assert th > cfg.rope_theta
    cy, sy = hba_amd.rope_tables(n, cfg.head_dim, th, dev)
    assert not torch.equal(cy, cos)
    out = hba_amd.hba_attention_eval(x["q"], x["k"], x["v"], cy, sy, cfg, prm, prm, None, equiv=True)
    torch.cuda.synchronize()
    rows = np.unique(np.concatenate([[0, 1, 63, 64, n // 2, n - 1], np.random.RandomState(1).randint(0, n, 16)]))
    ref = O.forward_equiv(f(x["q"]), f(x["k"]), f(x["v"]), f(cy), f(sy), cfg, f(x["q_gain"]), f(x["k_gain"]),
                          1e-6, dt, rows)
    err = np.abs(f(out)[:, rows] - ref).max()
    assert err <= TOL[dt], err


def test_equiv_rejects_ragged_length(dev):
    cfg, x, prm, cos, sin = make(dev, "bf16", n=128)
    with pytest.raises(ValueError):
        hba_amd.hba_attention_eval(x["q"][:, :100], x["k"][:, :100], x["v"][:, :100], cos[:100], sin[:100], cfg,
                                   prm, prm, None, equiv=True)


def test_kv_append_advance_past_the_tables_appends_nothing(dev):
    """hba_kv_append_advance with a position at or past the RoPE tables
    (n_tab) appends nothing and leaves seq_lens as it is, while the step
    scales are still written; positions inside append and advance."""
    lens = [70, 127]
    cfg, x, prm, cos, sin, cache, kcs, qn = build_cache(dev, "bf16", lens, W=64, k=4, seed=9)
    cache.reserve()
    g = torch.Generator().manual_seed(4)
    kn = torch.randn(2, 2, 64, generator=g).to(torch.bfloat16).to(dev)
    vn = torch.randn(2, 2, 64, generator=g).to(torch.bfloat16).to(dev)
    before = [t_.clone() for t_ in (cache.kc_pages, cache.kr_pages, cache.v_pages, cache.summ_pages)]
    sc = torch.full((2,), -1.0, device=dev)
    tab = cache.scale_table()
    ops.kv_append_advance(kn, vn, x["k_gain"], 1e-6, cos[:100], sin[:100], cache.page_table, cache.seq_lens,
                          cache.kc_pages, cache.kr_pages, cache.v_pages, x["probes"], x["proj"], cache.summ_pages,
                          tab, sc)
    torch.cuda.synchronize()
    # sequence 0 (position 70 < 100) advanced; sequence 1 (position 127 >= 100) did not
    assert cache.seq_lens.cpu().tolist() == [71, 127]
    assert sc[0].item() == tab[71].item() and sc[1].item() == tab[127].item()
    p1 = cache._table[1][127 // 64]
    for a, b_ in zip(before, (cache.kc_pages, cache.kr_pages, cache.v_pages, cache.summ_pages)):
        assert torch.equal(a[p1], b_[p1])
    p0 = cache._table[0][70 // 64]
    assert not torch.equal(before[0][p0], cache.kc_pages[p0])


# ---------------------------------------------------------------- aux-KL -----
def _aux_setup(dev, case_cfg, inp, dt):
    cfg = hba_amd.HBAConfig(**case_cfg, aux_w=1.0)
    T = TDT[dt]
    q, k, v = (torch.from_numpy(inp[x]).to(T).to(dev).requires_grad_(True) for x in ("q", "k", "v"))
    summ = hba_amd.SlotSummarizer(cfg).to(dev)
    qkn = hba_amd.QKNorm(cfg).to(dev)
    with torch.no_grad():
        summ.probes.copy_(torch.from_numpy(inp["probes"]))
        summ.proj.copy_(torch.from_numpy(inp["proj"]))
        qkn.q.gain.copy_(torch.from_numpy(inp["q_gain"]))
        qkn.k.gain.copy_(torch.from_numpy(inp["k_gain"]))
    cos, sin = hba_amd.rope_tables(q.shape[1], cfg.head_dim, cfg.rope_theta, dev)
    return cfg, q, k, v, summ, qkn, cos, sin


def test_aux_kl_matches_reference_golden(dev):
    """The reference's own aux-KL and its gradients into probes and proj
    (golden_aux.npz, written by the reference's hba_attention_dense and
    autograd; d = 64, 64-key blocks, 4/2 heads, n = 1024, W = 128, fp32),
    here from hba_attention_dense / _fused on the GPU; the gradient-isolation
    rule (gates.py:129-167): aux reaches no q/k/v, the output reaches no
    summarizer parameter."""
    import make_golden as MG
    z = np.load(f"{MG.HERE}/golden_aux.npz")
    case = MG.CASES["d64"]
    inp = MG.gen_inputs(case)
    cfg, q, k, v, summ, qkn, cos, sin = _aux_setup(dev, case["cfg"], inp, "f32")
    for fn in (hba_amd.hba_attention_dense, hba_amd.hba_attention_fused):
        summ.zero_grad(set_to_none=True)
        out, aux = fn(q, k, v, cos, sin, cfg, summ, qkn)
        aux.backward()
        torch.cuda.synchronize()
        ga = float(z["d64_aux"])
        assert abs(aux.item() - ga) <= 1e-5 * abs(ga), (aux.item(), ga)
        for p_, key in ((summ.probes, "d64_dprobes"), (summ.proj, "d64_dproj")):
            ref = z[key]
            err = np.abs(f(p_.grad) - ref).max() / np.abs(ref).max()
            assert err <= 1e-4, (key, err)
        assert q.grad is None and k.grad is None and v.grad is None
        summ.zero_grad(set_to_none=True)
        out.sum().backward()
        assert summ.probes.grad is None and summ.proj.grad is None
        assert q.grad is not None and q.grad.abs().max().item() > 0
        q.grad = k.grad = v.grad = None


# (aux relative, gradient relative to its largest element).  Against the
# oracle scoring blocks with the kernels' own summaries, both dtypes measured
# <= 5e-8 (aux) and 1.4e-6 (gradients).  bf16 against the exact (unrounded)
# summaries: bf16 storage of S0 moves the slot argmax of near-tied slots,
# which moved the probe gradients by up to 4.9% and the proj gradients by
# 1.4% (measured), the aux by 1.5e-6.
AUX_TOL = {"f32": (1e-6, 2e-5), "bf16": (1e-6, 2e-5)}
AUX_BF16_EXACT_S0_TOL = (2e-5, 8e-2)


@pytest.mark.parametrize("dt,d,Hq,Hkv,qknorm,B,m", [("f32", 64, 14, 2, True, 2, 4), ("bf16", 64, 14, 2, True, 1, 4),
                                                    ("f32", 128, 28, 4, False, 1, 4), ("bf16", 128, 28, 4, True, 1, 4),
                                                    ("bf16", 64, 8, 2, True, 1, 2), ("f32", 64, 8, 2, False, 1, 8),
                                                    ("f32", 64, 6, 2, True, 1, 3)])
def test_aux_kl_matches_oracle(dev, dt, d, Hq, Hkv, qknorm, B, m):
    """hba_aux_kl at the kernels' geometries (G = 7, d = 64 and 128, qknorm
    on and off, B = 2; 2, 3, 4 and 8 slots: the dS0 products take 16 or 4
    staged entries per thread, or the scalar kernel where 64 % m != 0)
    against the oracle's float64 aux and gradients on the same
    storage-rounded content q/k (n = 2048, W = 512: 1535 queries with
    candidates, up to 23 candidate blocks)."""
    n, W = 2048, 512
    rs = np.random.RandomState(7 + d + B)
    inp = dict(q=rs.standard_normal((B, n, Hq, d)).astype(np.float32),
               k=rs.standard_normal((B, n, Hkv, d)).astype(np.float32),
               v=rs.standard_normal((B, n, Hkv, d)).astype(np.float32),
               probes=(rs.standard_normal((Hkv, m, d)) * d ** -0.5).astype(np.float32),
               proj=(np.eye(d)[None].repeat(Hkv, 0) + rs.standard_normal((Hkv, d, d)) * 0.02).astype(np.float32),
               q_gain=(d ** 0.25 * rs.uniform(0.8, 1.2, Hq)).astype(np.float32),
               k_gain=(d ** 0.25 * rs.uniform(0.8, 1.2, Hkv)).astype(np.float32))
    ccfg = dict(n_heads=Hq, n_kv=Hkv, head_dim=d, window=W, sinks=4, k_blocks=8, slots=m, qknorm=qknorm,
                native_ctx=1024)
    cfg, q, k, v, summ, qkn, cos, sin = _aux_setup(dev, ccfg, inp, dt)
    aux = hba_amd.aux_kl(q, k, v, cos, sin, cfg, summ, qkn)
    aux.backward()
    torch.cuda.synchronize()
    ocfg = O.Cfg(**ccfg)
    qc, kc, su = O.content_qk(f(q), f(k), ocfg, inp["q_gain"], inp["k_gain"], 1e-6, n, dt)
    kch, _, _ = ops.prep_keys(k.detach(), v.detach(), qkn.k.gain if qknorm else None, 1e-6, cos, sin)
    S0k = f(ops.summarize(kch, summ.probes.detach(), summ.proj.detach()))       # the kernels' summaries
    for S0s, (ta, tg) in ((S0k, AUX_TOL[dt]), (None, AUX_BF16_EXACT_S0_TOL if dt == "bf16" else AUX_TOL[dt])):
        ref, dpr, dpj, _ = O.aux_kl(qc, kc, inp["probes"], inp["proj"], Hkv, su, O.route_scale(ocfg, d), 64, W,
                                    S0_scores=S0s, dtype=dt)
        errs = (abs(aux.item() - ref) / abs(ref), np.abs(f(summ.probes.grad) - dpr).max() / np.abs(dpr).max(),
                np.abs(f(summ.proj.grad) - dpj).max() / np.abs(dpj).max())
        print(dt, d, qknorm, B, "kernel S0" if S0s is not None else "exact S0", [f"{e:.2e}" for e in errs])
        assert errs[0] <= ta and errs[1] <= tg and errs[2] <= tg, errs


def test_aux_kl_without_candidates_is_zero(dev):
    """n <= W + 2*64 - 1: no query has a candidate block; aux and its
    gradients are 0 (the reference's graph-free zero, attention.py:382-388)."""
    cfg, x, prm, cos, sin = make(dev, "bf16", n=512, W=512, k=4)
    summ = hba_amd.SlotSummarizer(cfg).to(dev)
    aux = hba_amd.aux_kl(x["q"], x["k"], x["v"], cos, sin, cfg, summ, prm)
    aux.backward()
    assert aux.item() == 0.0
    assert summ.probes.grad.abs().max().item() == 0.0 and summ.proj.grad.abs().max().item() == 0.0


# ------------------------------------------------------------ model layer ----
def test_model_layer_modes_match_cpu_reference(dev):
    """HBAAttention (the attention branch of model.py:118-140: projections,
    QKNorm, the mode switch) on the GPU in fp32 against the same layer on the
    CPU over the oracle's torch restatements: "train" (hba_attention_dense,
    attention.py:306-356) with its output, the gradients of every projection
    weight and bias and of the QKNorm gains under autograd, and the aux-KL
    against the oracle; "eval" / "eval_hier" / "equiv" outputs."""
    import copy

    from oracle import hba_cpu_torch as CT
    cfg = hba_amd.HBAConfig(n_heads=4, n_kv=2, head_dim=64, window=256, sinks=4, k_blocks=4, slots=4,
                            native_ctx=512, fanout=4, beam=2)
    B, n, hidden, d = 1, 1024, 128, 64
    torch.manual_seed(3)
    cpu = hba_amd.HBAAttention(cfg, hidden)
    with torch.no_grad():
        cpu.qknorm.q.gain.copy_(d ** 0.25 * (0.8 + 0.4 * torch.rand(4)))
        cpu.qknorm.k.gain.copy_(d ** 0.25 * (0.8 + 0.4 * torch.rand(2)))
    gpu = copy.deepcopy(cpu).to(dev)
    a = torch.randn(B, n, hidden)
    cos, sin = hba_amd.rope_tables(n, d, cfg.rope_theta, "cpu")
    cd, sd = cos.to(dev), sin.to(dev)
    g = torch.randn(B, n, hidden)
    og, aux = gpu(a.to(dev), cd, sd, mode="train")
    ((og * g.to(dev)).sum() + aux).backward()          # aux reaches only the summarizer
    q = cpu.q_proj(a).view(B, n, 4, d)
    k = cpu.k_proj(a).view(B, n, 2, d)
    v = cpu.v_proj(a).view(B, n, 2, d)
    ref = CT.dense_forward(q, k, v, cos, sin, cfg, cpu.summarizer.probes.detach(), cpu.summarizer.proj.detach(),
                           cpu.qknorm.q.gain, cpu.qknorm.k.gain, 1e-6)
    oc = cpu.o_proj(ref.reshape(B, n, 4 * d))
    (oc * g).sum().backward()
    torch.cuda.synchronize()
    assert (og.cpu() - oc).abs().max().item() <= 1e-4 * oc.abs().max().item()
    for name, pc in cpu.named_parameters():
        if "summarizer" in name:
            continue
        pg = dict(gpu.named_parameters())[name]
        rel = (pg.grad.cpu() - pc.grad).abs().max().item() / pc.grad.abs().max().item()
        assert rel <= 2e-3, (name, rel)
    ocfg = O.Cfg(n_heads=4, n_kv=2, head_dim=64, window=256, sinks=4, k_blocks=4, slots=4, native_ctx=512)
    qc, kc, su = O.content_qk(q.detach().numpy(), k.detach().numpy(), ocfg, f(cpu.qknorm.q.gain),
                              f(cpu.qknorm.k.gain), 1e-6, n, "f32")
    aref, dpr, _, _ = O.aux_kl(qc, kc, f(cpu.summarizer.probes), f(cpu.summarizer.proj), 2, su,
                               O.route_scale(ocfg, d), 64, 256)
    assert abs(aux.item() - aref) <= 1e-5 * abs(aref)
    assert np.abs(f(gpu.summarizer.probes.grad) - dpr).max() <= 1e-4 * np.abs(dpr).max()
    with torch.no_grad():
        x = a.to(dev)
        for mode in ("eval", "eval_hier", "equiv"):
            o, none = gpu(x, cd, sd, mode=mode)
            assert none is None
            qg, kg, vg = (t.view(B, n, -1, d) for t in (gpu.q_proj(x), gpu.k_proj(x), gpu.v_proj(x)))
            direct = hba_amd.hba_attention_eval(qg, kg, vg, cd, sd, cfg, gpu.summarizer, gpu.qknorm, None,
                                                hier=mode == "eval_hier", equiv=mode == "equiv")
            assert torch.equal(o, gpu.o_proj(direct.reshape(B, n, 4 * d))), mode
        rows = np.array([0, 5, 300, 700, n - 1])
        o_eval = gpu(x, cd, sd, mode="eval")[0]
        r_eval = CT.gathered_forward(q.detach(), k.detach(), v.detach(), cos, sin, cfg,
                                     cpu.summarizer.probes.detach(), cpu.summarizer.proj.detach(),
                                     cpu.qknorm.q.gain.detach(), cpu.qknorm.k.gain.detach(), 1e-6)
        r_eval = cpu.o_proj(r_eval.reshape(B, n, 4 * d))
        assert (o_eval.cpu()[:, rows] - r_eval[:, rows]).abs().max().item() <= 1e-4 * r_eval.abs().max().item()
    with pytest.raises(ValueError, match="unknown mode"):
        gpu(x, cd, sd, mode="decode")


# -------------------------------------------------------------- backward -----
# gates.py:247 holds input gradients to 2e-3 relative to their magnitude
# (fp32).  bf16 storage of q/k/v and of the forward's QKNorm/RoPE rows moves
# the recomputed probabilities by about one bf16 ulp.  Measured maxima over
# the bf16 cases below (relative to each gradient's largest magnitude):
# dq 7.7e-3, dk 5.8e-3, dv 4.1e-3; the gain gradients, sums over every row
# and element of a head, 2.7e-2.  The bf16 gates are about twice those.
GRAD_TOL = {"f32": {"dq": 2e-3, "dk": 2e-3, "dv": 2e-3, "gain": 2e-3},
            "bf16": {"dq": 1.5e-2, "dk": 1.2e-2, "dv": 1e-2, "gain": 5.5e-2}}


def check_grads(case, dt, got, ref):
    """Relative max errors of dq, dk, dv (and the gain gradients) against the
    oracle, printed (pytest -s) and held to GRAD_TOL."""
    rel = {name: np.abs(a - b).max() / max(np.abs(b).max(), 1e-6)
           for name, a, b in zip(["dq", "dk", "dv", "dq_gain", "dk_gain"], got, ref)}
    print(case, {k: f"{v:.2e}" for k, v in rel.items()})
    for name, e in rel.items():
        assert e < GRAD_TOL[dt][name.split("_")[-1] if "_" in name else name], (case, name, e)


@pytest.mark.parametrize("dt,qknorm,mode", [("f32", True, "dense"), ("f32", False, "eval"), ("bf16", True, "eval"),
                                            ("bf16", False, "eval"), ("f32", True, "equiv"), ("bf16", True, "hier")])
def test_backward_matches_oracle(dev, dt, qknorm, mode):
    """hba_attn_bwd through autograd of the drop-ins against the oracle's
    float64 backward on the forward's own selection: dq, dk, dv and the
    QKNorm gain gradients."""
    n = 512
    kw = dict(fanout=4, beam=2) if mode == "hier" else {}
    # aux_w = 0: the frozen-summarizer setting, where the reference's aux is a zero too
    cfg, x, prm, cos, sin = make(dev, dt, n=n, W=128, k=4, S=4, qknorm=qknorm, aux_w=0.0, **kw)
    q, k, v = (x[t].clone().requires_grad_(True) for t in ("q", "k", "v"))
    gq = x["q_gain"].clone().requires_grad_(qknorm)
    gk = x["k_gain"].clone().requires_grad_(qknorm)
    qkn = synth.Params(gq, gk, x["probes"], x["proj"])
    if mode == "dense":
        out = hba_amd.hba_attention_dense(q, k, v, cos, sin, cfg, qkn, qkn)[0]
    else:
        out = hba_amd.hba_attention_eval(q, k, v, cos, sin, cfg, qkn, qkn, None, hier=mode == "hier",
                                         equiv=mode == "equiv")
    dout = torch.randn(out.shape, generator=torch.Generator().manual_seed(7)).to(out.dtype).to(dev)
    out.backward(dout)
    torch.cuda.synchronize()
    if mode == "equiv":
        idx = np.zeros((cfg.n_kv, n, 1), dtype=np.int32)
        cnt = np.zeros((cfg.n_kv, n), dtype=np.int32)
        S, W = 0, n
    else:
        with torch.no_grad():
            r = hba_amd.forward_stages(x["q"], x["k"], x["v"], cos, sin, cfg, qkn, qkn, hier=mode == "hier",
                                       dense_route=mode == "dense")
            assert torch.equal(r["out"], out.detach())          # the same forward, the same selection
        idx, cnt = r["idx"][0].cpu().numpy(), r["cnt"][0].cpu().numpy()
        S, W = cfg.sinks, cfg.window
    scale = hba_amd.union_scale(cfg, cfg.head_dim, n)
    ref = O.union_backward(f(x["q"])[0], f(x["k"])[0], f(x["v"])[0], f(cos), f(sin), scale, f(x["q_gain"]),
                           f(x["k_gain"]), 1e-6, idx, cnt, f(dout)[0], S, W, 64, qknorm)
    got = [f(q.grad)[0], f(k.grad)[0], f(v.grad)[0]]
    if qknorm:
        got += [f(gq.grad), f(gk.grad)]
    check_grads(f"{dt}-{qknorm}-{mode}", dt, got, ref)


def test_backward_row_ranges_matches_oracle(dev):
    """bf16 backward at n = 4608: the dk/dv workgroups of the MFMA path each
    take 4096 query rows, so this covers a ragged second range, window rows
    cut at a range edge and needle blocks selected by rows of both ranges."""
    n = 4608
    cfg, x, prm, cos, sin = make(dev, "bf16", n=n, W=512, k=16, S=4, needles=True)
    q, k, v = (x[t].clone().requires_grad_(True) for t in ("q", "k", "v"))
    gq = x["q_gain"].clone().requires_grad_(True)
    gk = x["k_gain"].clone().requires_grad_(True)
    qkn = synth.Params(gq, gk, x["probes"], x["proj"])
    out = hba_amd.hba_attention_eval(q, k, v, cos, sin, cfg, qkn, qkn, None)
    dout = torch.randn(out.shape, generator=torch.Generator().manual_seed(11)).to(out.dtype).to(dev)
    out.backward(dout)
    torch.cuda.synchronize()
    with torch.no_grad():
        r = hba_amd.forward_stages(x["q"], x["k"], x["v"], cos, sin, cfg, qkn, qkn)
        assert torch.equal(r["out"], out.detach())
    idx, cnt = r["idx"][0].cpu().numpy(), r["cnt"][0].cpu().numpy()
    scale = hba_amd.union_scale(cfg, cfg.head_dim, n)
    ref = O.union_backward(f(x["q"])[0], f(x["k"])[0], f(x["v"])[0], f(cos), f(sin), scale, f(x["q_gain"]),
                           f(x["k_gain"]), 1e-6, idx, cnt, f(dout)[0], cfg.sinks, cfg.window, 64, True)
    got = [f(q.grad)[0], f(k.grad)[0], f(v.grad)[0], f(gq.grad), f(gk.grad)]
    check_grads("bf16", "bf16", got, ref)


@pytest.mark.parametrize("Hq,Hkv,k,d", [(8, 2, 4, 64), (10, 2, 8, 64), (16, 1, 4, 64), (7, 1, 4, 128),
                                         (8, 2, 8, 128)])
def test_backward_group_sizes_match_oracle(dev, Hq, Hkv, k, d):
    """bf16 backward with G = 4, 5 and 16 heads per KV head: the MFMA dq
    waves then take 4, 3 (the last wave ragged, n % 3 != 0) and 1 queries;
    and at d = 128 (the donor head size) with G = 7 and 4."""
    n = 512
    cfg, x, prm, cos, sin = make(dev, "bf16", n=n, Hq=Hq, Hkv=Hkv, d=d, W=128, k=k, S=4, needles=True)
    q, k_, v = (x[t].clone().requires_grad_(True) for t in ("q", "k", "v"))
    gq = x["q_gain"].clone().requires_grad_(True)
    gk = x["k_gain"].clone().requires_grad_(True)
    qkn = synth.Params(gq, gk, x["probes"], x["proj"])
    out = hba_amd.hba_attention_eval(q, k_, v, cos, sin, cfg, qkn, qkn, None)
    dout = torch.randn(out.shape, generator=torch.Generator().manual_seed(5)).to(out.dtype).to(dev)
    out.backward(dout)
    torch.cuda.synchronize()
    with torch.no_grad():
        r = hba_amd.forward_stages(x["q"], x["k"], x["v"], cos, sin, cfg, qkn, qkn)
    idx, cnt = r["idx"][0].cpu().numpy(), r["cnt"][0].cpu().numpy()
    scale = hba_amd.union_scale(cfg, cfg.head_dim, n)
    ref = O.union_backward(f(x["q"])[0], f(x["k"])[0], f(x["v"])[0], f(cos), f(sin), scale, f(x["q_gain"]),
                           f(x["k_gain"]), 1e-6, idx, cnt, f(dout)[0], cfg.sinks, cfg.window, 64, True)
    got = [f(q.grad)[0], f(k_.grad)[0], f(v.grad)[0], f(gq.grad), f(gk.grad)]
    check_grads("bf16", "bf16", got, ref)


@pytest.mark.parametrize("case", ["B2", "S0", "S64", "equiv"])
def test_backward_bf16_cases(dev, case):
    """bf16 backward with two batch rows (the per-batch indexing of every
    backward kernel), without sinks (the sink launch skipped), with a full
    64-key sink block, and in equiv mode (W = n: every page staged).  The
    relative errors are printed per gradient (pytest -s)."""
    n, B, S, W, equiv = 512, 1, 4, 128, False
    if case == "B2":
        B = 2
    elif case == "S0":
        S = 0
    elif case == "S64":
        S = 64
    else:
        equiv = True
    cfg, x, prm, cos, sin = make(dev, "bf16", n=n, B=B, W=W, k=4, S=S, needles=True, aux_w=0.0)
    q, k, v = (x[t].clone().requires_grad_(True) for t in ("q", "k", "v"))
    gq = x["q_gain"].clone().requires_grad_(True)
    gk = x["k_gain"].clone().requires_grad_(True)
    qkn = synth.Params(gq, gk, x["probes"], x["proj"])
    out = hba_amd.hba_attention_eval(q, k, v, cos, sin, cfg, qkn, qkn, None, equiv=equiv)
    dout = torch.randn(out.shape, generator=torch.Generator().manual_seed(13)).to(out.dtype).to(dev)
    out.backward(dout)
    torch.cuda.synchronize()
    scale = hba_amd.union_scale(cfg, cfg.head_dim, n)
    if not equiv:
        with torch.no_grad():
            r = hba_amd.forward_stages(x["q"], x["k"], x["v"], cos, sin, cfg, qkn, qkn)
            assert torch.equal(r["out"], out.detach())
    grads = {"dq": 0.0, "dk": 0.0, "dv": 0.0}
    refs = {"dq": 0.0, "dk": 0.0, "dv": 0.0}
    gain_ref = [np.zeros(cfg.n_heads), np.zeros(cfg.n_kv)]
    for b in range(B):
        if equiv:
            idx = np.zeros((cfg.n_kv, n, 1), dtype=np.int32)
            cnt = np.zeros((cfg.n_kv, n), dtype=np.int32)
            Sb, Wb = 0, n
        else:
            idx, cnt = r["idx"][b].cpu().numpy(), r["cnt"][b].cpu().numpy()
            Sb, Wb = S, W
        ref = O.union_backward(f(x["q"])[b], f(x["k"])[b], f(x["v"])[b], f(cos), f(sin), scale, f(x["q_gain"]),
                               f(x["k_gain"]), 1e-6, idx, cnt, f(dout)[b], Sb, Wb, 64, True)
        for name, a, rb in zip(["dq", "dk", "dv"], [f(q.grad)[b], f(k.grad)[b], f(v.grad)[b]], ref[:3]):
            grads[name] = max(grads[name], np.abs(a - rb).max())
            refs[name] = max(refs[name], np.abs(rb).max())
        gain_ref[0] = gain_ref[0] + ref[3]
        gain_ref[1] = gain_ref[1] + ref[4]
    rel = {name: grads[name] / max(refs[name], 1e-6) for name in grads}
    for name, a, rb in (("dq_gain", f(gq.grad), gain_ref[0]), ("dk_gain", f(gk.grad), gain_ref[1])):
        rel[name] = np.abs(a - rb).max() / max(np.abs(rb).max(), 1e-6)
    print(case, {k_: f"{v_:.2e}" for k_, v_ in rel.items()})
    for name, e in rel.items():
        assert e < GRAD_TOL["bf16"][name.split("_")[-1] if "_" in name else name], (case, name, e)


@pytest.mark.parametrize("n", [32768, 65536])
def test_backward_dq_kernels_agree(dev, n):
    """The bf16 query gradient at the benchmarked 32K shape (14/2 heads, d =
    64, W = 1024, k = 16, needles; a 6-slot ring) and at 64K (a 4-slot ring:
    the selection lists take more LDS): the union kernel (64-key blocks
    staged once per 48 queries) against bwd_dq_mfma (HBA_BWD_DQ_KERNEL=pair),
    which the oracle tests pin at small n.  Both compute the same sums in a
    different order and softmax form (fixed shift, its scale folded into the
    bf16 query operand, against a running max), so dq, and dk / dv through
    the LSE and rows they leave, agree to a bf16 ulp or two of each
    gradient's magnitude (dv 6.3e-3 measured at 32K): held to the bf16 gates
    of the oracle tests."""
    cfg, x, prm, cos, sin = make(dev, "bf16", n=n, W=1024, k=16, S=4, needles=True, aux_w=0.0)
    dout = torch.randn((1, n, cfg.n_heads, cfg.head_dim), generator=torch.Generator().manual_seed(3))
    dout = dout.to(torch.bfloat16).to(dev)

    def grads():
        q, k, v = (x[t].clone().requires_grad_(True) for t in ("q", "k", "v"))
        gq = x["q_gain"].clone().requires_grad_(True)
        gk = x["k_gain"].clone().requires_grad_(True)
        qkn = synth.Params(gq, gk, x["probes"], x["proj"])
        out = hba_amd.hba_attention_eval(q, k, v, cos, sin, cfg, qkn, qkn, None)
        out.backward(dout)
        torch.cuda.synchronize()
        return [t.grad.float() for t in (q, k, v, gq, gk)]

    got = grads()
    os.environ["HBA_BWD_DQ_KERNEL"] = "pair"
    try:
        ref = grads()
    finally:
        del os.environ["HBA_BWD_DQ_KERNEL"]
    for name, a, b_ in zip(["dq", "dk", "dv", "dq_gain", "dk_gain"], got, ref):
        assert torch.isfinite(a).all(), name
        rel = ((a - b_).abs().max() / b_.abs().max().clamp_min(1e-6)).item()
        print(n, name, f"{rel:.2e}")
        assert rel < GRAD_TOL["bf16"][name.split("_")[-1] if "_" in name else name], (n, name, rel)


def test_backward_no_grad_inputs_stays_forward_only(dev):
    cfg, x, prm, cos, sin = make(dev, "bf16", n=256, W=64, k=2)
    out = hba_amd.hba_attention_eval(x["q"], x["k"], x["v"], cos, sin, cfg, prm, prm, None)
    assert out.grad_fn is None


def test_causality(dev):
    """gates.py:101-126: randomising tokens after t leaves rows <= t unchanged."""
    cfg, x, prm, cos, sin = make(dev, "bf16", n=2048, W=256, k=8)
    t = 1300
    q2, k2, v2 = x["q"].clone(), x["k"].clone(), x["v"].clone()
    g = torch.Generator().manual_seed(99)
    for z in (q2, k2, v2):
        z[:, t + 1:] = torch.randn(z[:, t + 1:].shape, generator=g).to(z.dtype).to(dev)
    a = hba_amd.hba_attention_eval(x["q"], x["k"], x["v"], cos, sin, cfg, prm, prm, None)
    b = hba_amd.hba_attention_eval(q2, k2, v2, cos, sin, cfg, prm, prm, None)
    assert torch.equal(a[:, : t + 1], b[:, : t + 1])
    assert not torch.equal(a[:, t + 1:], b[:, t + 1:])


# ---------------------------------------------------------------- decode -----
def build_cache(dev, dt, lens, Hq=14, Hkv=2, d=64, m=4, W=1024, S=4, k=16, seed=0, qknorm=True):
    cfg = hba_amd.HBAConfig(n_heads=Hq, n_kv=Hkv, head_dim=d, slots=m, window=W, sinks=S, k_blocks=k,
                            qknorm=qknorm)
    Bd = len(lens)
    L = max(lens)
    x = synth.layer_inputs(Bd, L, Hq, Hkv, d, m=m, dtype=TDT[dt], device=dev, seed=seed, sharp=True)
    prm = synth.Params(x["q_gain"], x["k_gain"] if qknorm else None, x["probes"], x["proj"])
    cos, sin = hba_amd.rope_tables(L + 64, d, cfg.rope_theta, dev)
    cache = hba_amd.PagedKVCache(cfg, Bd, L + 64, TDT[dt], dev)
    cache._free = synth.shuffled_pages(len(cache._free), seed=seed)    # shuffled physical pages
    kcs = []
    for s, Ls in enumerate(lens):
        kc, kr, _ = ops.prep_keys(x["k"][s:s + 1, :Ls], x["v"][s:s + 1, :Ls], x["k_gain"] if qknorm else None,
                                  1e-6, cos, sin)
        kc, kr = kc[0].transpose(0, 1), kr[0].transpose(0, 1)
        cache.load(s, kc, kr, x["v"][s, :Ls], prm)
        kcs.append(kc)
    qn = x["q"][torch.arange(Bd), torch.tensor(lens) - 1]                  # [Bd, Hq, d]
    return cfg, x, prm, cos, sin, cache, kcs, qn


def cache_summaries(cache, s, nfull):
    pt = cache._table[s][:nfull]
    return f(cache.summ_pages[torch.tensor(pt, dtype=torch.long)]).transpose(1, 0, 2, 3)


def _decode_vs_oracle(dev, dt, lens, **kw):
    cfg, x, prm, cos, sin, cache, kcs, qn = build_cache(dev, dt, lens, **kw)
    out, sidx, scnt = hba_amd.hba_decode_step(qn, cache, cfg, prm, cos, sin)
    torch.cuda.synchronize()
    d = cfg.head_dim
    for s, L in enumerate(lens):
        S0s = cache_summaries(cache, s, L // 64)
        scale = hba_amd.union_scale(cfg, d, L)
        ref, (idx, val, cnt) = O.decode_row(f(qn[s]), f(kcs[s]), f(x["v"][s, :L]), f(cos), f(sin), cfg,
                                            S0s, f(x["q_gain"]), 1e-6, dt, scale)
        assert np.array_equal(scnt[s].cpu().numpy(), cnt), s
        for g in range(cfg.n_kv):
            assert list(sidx[s, g, : cnt[g]].cpu().numpy()) == list(idx[g, : cnt[g]]), (s, g)
        assert np.abs(f(out[s]) - ref).max() <= TOL[dt], (s, np.abs(f(out[s]) - ref).max())


def use_decode_kernel(monkeypatch, kern):
    """Pick the bf16 decode kernel (decode_pair_kernel or decode_fused_kernel)
    whatever the batch size, through the library's HBA_DECODE_KERNEL switch."""
    monkeypatch.setenv("HBA_DECODE_KERNEL", kern)


@pytest.mark.parametrize("dt,kern", [("f32", "fused"), ("bf16", "fused"), ("bf16", "pair")])
def test_decode_matches_oracle(dev, dt, kern, monkeypatch):
    use_decode_kernel(monkeypatch, kern)
    _decode_vs_oracle(dev, dt, [1, 3, 70, 1100, 1200, 2500, 2049, 4096, 3333], W=1024, k=16)


@pytest.mark.parametrize("kern", ["fused", "pair"])
@pytest.mark.parametrize("d,k,Hq,Hkv,S", [(128, 16, 28, 4, 8), (64, 40, 14, 2, 4), (64, 64, 8, 1, 0),
                                          (64, 16, 32, 2, 4), (128, 8, 16, 1, 64)])
def test_decode_bf16_shapes(dev, d, k, Hq, Hkv, S, kern, monkeypatch):
    """bf16 decode at d = 128, with more picks than waves (k = 40, 64: each
    wave runs several routed pages), 16 heads per KV head and a full sink
    page, on both bf16 kernels."""
    use_decode_kernel(monkeypatch, kern)
    _decode_vs_oracle(dev, "bf16", [70, 700, 2500, 4096], Hq=Hq, Hkv=Hkv, d=d, S=S, W=512, k=k)


@pytest.mark.parametrize("d,Hq,Hkv", [(64, 32, 2), (128, 16, 1)])
def test_decode_f32_sixteen_heads_per_kv_head(dev, d, Hq, Hkv):
    """The fp32 three-launch decode at 16 query heads per KV head (its
    largest group), against the oracle."""
    _decode_vs_oracle(dev, "f32", [70, 1100, 2500], Hq=Hq, Hkv=Hkv, d=d, S=4, W=512, k=8)


def test_decode_equals_prefill_last_row(dev):
    """The decode step of a length-L sequence equals row L-1 of the prefill
    kernel on the same tokens (bf16, selection identical)."""
    L = 4096
    cfg, x, prm, cos, sin, cache, kcs, qn = build_cache(dev, "bf16", [L], W=1024, k=16, seed=4)
    out, sidx, scnt = hba_amd.hba_decode_step(qn, cache, cfg, prm, cos, sin)
    r = hba_amd.forward_stages(x["q"][:, :L], x["k"][:, :L], x["v"][:, :L], cos[:L], sin[:L], cfg, prm, prm)
    assert torch.equal(sidx[0].sort().values, r["idx"][0, :, L - 1].sort().values)
    assert (out[0].float() - r["out"][0, L - 1].float()).abs().max().item() <= 2e-2


@pytest.mark.parametrize("dt,d", [("bf16", 64), ("f32", 64), ("bf16", 128)])
def test_kv_append_and_page_summaries(dev, dt, d):
    """cache.append (hba_kv_append_advance, one launch): the appended key
    (QKNorm), its rotation and the value bit-exact against the oracle, and
    hba_kv_append writes the same rows; a decode step sees the token; the
    page the token filled gets the oracle's summary, bit-identical to the
    page-list summary kernel's; lengths and step scales move on the device."""
    lens = [127, 60]
    Hq, Hkv = (14, 2) if d == 64 else (28, 4)
    cfg, x, prm, cos, sin, cache, kcs, qn = build_cache(dev, dt, lens, Hq=Hq, Hkv=Hkv, d=d, W=64, k=4, seed=5)
    g = torch.Generator().manual_seed(3)
    kn = torch.randn(2, Hkv, d, generator=g).to(TDT[dt]).to(dev)
    vn = torch.randn(2, Hkv, d, generator=g).to(TDT[dt]).to(dev)
    cache.append(kn, vn, prm, prm, cos, sin)
    torch.cuda.synchronize()
    assert cache.lens == [128, 61]
    kc2, kr2, v2 = (torch.zeros_like(t_) for t_ in (cache.kc_pages, cache.kr_pages, cache.v_pages))
    ops.kv_append(kn, vn, x["k_gain"], 1e-6, cos, sin, cache.page_table, cache.seq_lens, kc2, kr2, v2)
    rows = lambda t_, page, off: t_[page][:, off].unflatten(-1, (64, d))                  # [Hkv, 64, d]
    for s, pos in enumerate([127, 60]):
        page = cache._table[s][pos // 64]
        want = O.qknorm(f(kn)[s], f(x["k_gain"]), 1e-6, dt)
        assert np.array_equal(f(cache.key_rows(page)[:, pos % 64]), want)
        rot = O.apply_rope(want[None], f(cos), f(sin), dt, positions=np.array([pos]))[0]
        assert np.array_equal(f(cache.key_rows(page, rotated=True)[:, pos % 64]), rot)
        assert np.array_equal(f(cache.value_rows(page)[:, pos % 64]), f(vn)[s])
        for a, b, off in ((kc2, cache.kc_pages, cache._koff), (kr2, cache.kr_pages, cache._koff),
                          (v2, cache.v_pages, cache._voff)):
            assert torch.equal(rows(a, page, off)[:, pos % 64], rows(b, page, off)[:, pos % 64]), s
        kcs[s] = torch.cat([kcs[s], torch.from_numpy(want)[None].to(kcs[s])], 0)
    # a decode step after the append sees the appended token (keys, rotation, value)
    qd = torch.randn(2, Hq, d, generator=g).to(TDT[dt]).to(dev)
    out, sidx, scnt = hba_amd.hba_decode_step(qd, cache, cfg, prm, cos, sin)
    for s, L in enumerate(cache.lens):
        vseq = np.concatenate([f(x["v"][s, :L - 1]), f(vn)[s][None]], 0)
        ref, _ = O.decode_row(f(qd[s]), f(kcs[s]), vseq, f(cos), f(sin), cfg, cache_summaries(cache, s, L // 64),
                              f(x["q_gain"]), 1e-6, dt, hba_amd.union_scale(cfg, d, L))
        assert np.abs(f(out[s]) - ref).max() <= TOL[dt], s
    # the page that just filled (sequence 0, tokens 64..127) got its summary
    full = cache._table[0][127 // 64]
    kpage = f(cache.key_rows(full)).transpose(1, 0, 2)                    # [64, Hkv, d]
    sref = O.summarize(kpage, f(x["probes"]), f(x["proj"]), 64)[:, 0]
    assert np.abs(f(cache.summ_pages[full]) - sref).max() <= 2 ** -7 * max(1, np.abs(sref).max())
    # the append's in-launch summary equals the page-list summary kernel's
    again = cache.summ_pages.clone()
    again[full].zero_()
    ops.summarize_pages(cache.kc_pages, torch.tensor([full], dtype=torch.int32), x["probes"], x["proj"], again)
    assert torch.equal(again[full], cache.summ_pages[full])
    # hba_summarize_filled finds the same page from the page table and lengths
    summ2 = torch.zeros_like(cache.summ_pages)
    ops.summarize_filled(cache.kc_pages, cache.page_table, cache.seq_lens, x["probes"], x["proj"], summ2)
    assert torch.equal(summ2[full], cache.summ_pages[full])
    others = [p_ for p_ in range(summ2.shape[0]) if p_ != full]
    assert summ2[others].abs().sum().item() == 0                        # sequence 1 (61 tokens) filled none
    # and the device lengths / step scales moved with the host mirror
    assert cache.seq_lens.cpu().tolist() == [128, 61]
    assert torch.equal(cache._scales, torch.index_select(cache.scale_table(), 0, cache.seq_lens))


@pytest.mark.parametrize("dt,graph,kern", [("bf16", False, "fused"), ("bf16", True, "fused"), ("f32", False, "fused"),
                                            ("bf16", False, "pair"), ("bf16", True, "pair")],
                         ids=["bf16-direct", "bf16-graph", "f32-direct", "bf16-direct-pair", "bf16-graph-pair"])
def test_decode_loop_matches_append_and_step(dev, dt, graph, kern, monkeypatch):
    """DecodeLoop (two launches per token straight through the C-ABI, or both
    captured once as a HIP graph and replayed) against cache.append +
    hba_decode_step on an identical cache, 60 tokens that fill pages of every
    sequence (127 -> 128 at once, 60 -> 64, 2500 -> 2560, the cache's last full
    page): each step's output, selection and counts equal the reference
    path's bit for bit at the same launch size (max_len), and stay within
    the dtype's rounding of the step sized by the longest sequence; the filled
    pages' summaries, the appended rows and the device lengths agree.  Work
    of the other path runs between the replays."""
    use_decode_kernel(monkeypatch, kern)
    lens = [127, 60, 2500]
    kw = dict(W=256, k=8, seed=6)
    cfg, x, prm, cos, sin, ca, kcs, qn = build_cache(dev, dt, lens, **kw)
    _, _, _, _, _, cb, _, _ = build_cache(dev, dt, lens, **kw)
    loop = hba_amd.DecodeLoop(cb, cfg, prm, prm, cos, sin, graph=graph)
    gen = torch.Generator().manual_seed(8)
    B, Hkv, d = len(lens), cfg.n_kv, cfg.head_dim
    T = TDT[dt]
    for t in range(60):
        kn = torch.randn(B, Hkv, d, generator=gen).to(T).to(dev)
        vn = torch.randn(B, Hkv, d, generator=gen).to(T).to(dev)
        qd = torch.randn(B, cfg.n_heads, d, generator=gen).to(T).to(dev)
        ca.append(kn, vn, prm, prm, cos, sin)
        oe, ie, ne = hba_amd.hba_decode_step(qd, ca, cfg, prm, cos, sin, max_len=ca.max_len)
        o2, _, _ = hba_amd.hba_decode_step(qd, ca, cfg, prm, cos, sin)
        og, ig, ng = loop.step(qd, kn, vn)
        torch.cuda.synchronize()
        assert cb.lens == ca.lens, t
        assert torch.equal(ng, ne) and torch.equal(ig, ie), t
        assert torch.equal(og, oe), (t, (og.float() - oe.float()).abs().max().item())
        assert (og.float() - o2.float()).abs().max().item() <= (2 ** -6 if dt == "bf16" else 1e-6), t
    assert torch.equal(cb.seq_lens.cpu(), torch.tensor(ca.lens, dtype=torch.int32))
    assert torch.equal(ca.seq_lens.cpu(), torch.tensor(ca.lens, dtype=torch.int32))
    for s, L in enumerate(ca.lens):
        pa = torch.tensor(ca._table[s][: (L + 63) // 64], dtype=torch.long)
        pb = torch.tensor(cb._table[s][: (L + 63) // 64], dtype=torch.long)
        assert torch.equal(ca.summ_pages[pa[: L // 64]], cb.summ_pages[pb[: L // 64]]), s
        for rows in (lambda c, pg: c.key_rows(pg), lambda c, pg: c.key_rows(pg, rotated=True),
                     lambda c, pg: c.value_rows(pg)):
            assert torch.equal(rows(ca, pa[-2:])[..., : (L - 1) % 64 + 1, :],
                               rows(cb, pb[-2:])[..., : (L - 1) % 64 + 1, :]), s
    with pytest.raises(ValueError, match="at most"):
        cb.lens[0] = cb.max_len
        loop.step(qd, kn, vn)
