"""HIP kernels against the oracle at the benchmarked workloads' full sizes,
through the same entry points the benchmark times:

  donor prefill  B = 2, n = 65536, 28/4 heads, d = 128, 8 sinks, W = 1024,
                 top-16, bf16 (prep_keys, summarize, score_select, attn_fwd):
                 keys bit-exact, the top-k of the kernel's own scores
                 bit-exact, its scores the declared-order fp32 scores up to
                 GEMM rounding, and ~200 sampled rows per batch row of the
                 union attention within 2e-2 of the float64 rows
  donor decode   four append + decode steps per bf16 decode kernel on the
                 64K cache built from that prefill (8 score chunks of 128
                 candidate pages)
  decode 32      the decode workload's own 32 lengths (L ~ U[16384, 32768],
                 seed 0) on both bf16 decode kernels: picks bit-exact,
                 outputs within 2e-2
  hier 128K      hier_select (the timed entry point) gives the picks of
                 hier_select_with_scores (whose scores the 128K selection
                 test checks), on every query; the union attention over
                 those picks on sampled rows within 2e-2
"""
import numpy as np
import pytest
import torch

import oracle.hba_oracle as O

pytestmark = pytest.mark.gpu

hba_amd = pytest.importorskip("hba_amd")
from hba_amd import ops, synth  # noqa: E402

from test_gpu_configs import check_decode, lean_cache, margin_flips, sample_rows  # noqa: E402


@pytest.fixture(scope="module")
def dev():
    if not torch.cuda.is_available():
        pytest.fail("GPU tests need a visible gfx950 device")
    return torch.device("cuda:0")


def f(t):
    return t.detach().float().cpu().numpy()


class RowView:
    """Rows of a [n, H, d] array held only at `rows` (attn_rows indexes its
    query arrays by position)."""

    def __init__(self, sub, rows, n):
        self.sub, self.shape = sub, (n,) + sub.shape[1:]
        self.at = {int(i): r for r, i in enumerate(rows)}

    def __getitem__(self, key):
        i, rest = key[0], key[1:]
        return self.sub[(self.at[int(i)],) + rest]


def check_prefill_rows(q, kc_k, kr_k, v, gq, cos, sin, S0, idx, cnt, scores, out, cfg, scale, rows, W, k):
    """One batch row: keys bit-exact; on `rows` the kernel's picks are the
    top-k of its own scores, those scores the declared-order ones up to GEMM
    rounding and the picks the oracle's up to k-boundary near-ties; the
    union attention within 2e-2 of the float64 rows.  Returns the errors."""
    n, Hq, d = q.shape
    Hkv = kc_k.shape[1]
    qc_r = O.qknorm(q[rows], gq, 1e-6, "bf16")
    qr_r = O.apply_rope(qc_r, cos, sin, "bf16", positions=rows)
    qg_r = O.grouped_query(qc_r, Hkv, "bf16")                         # [Hkv, r, d]
    ki, kcn = idx[:, rows], cnt[:, rows]
    for g in range(Hkv):
        sc = scores[g]                                                # [r, nb] the kernel's own scores
        ti, tv, tc = O.topk(sc, k)
        assert np.array_equal(ti, ki[g]) and np.array_equal(tc, kcn[g]), g
        qfull = np.zeros((n, d), np.float32)
        qfull[rows] = qg_r[g]
        osc = O.block_scores(qfull, S0[g], rows, scale, 64, W)
        fin = np.isfinite(osc)
        assert np.array_equal(np.isfinite(sc), fin)
        assert np.abs(sc[fin] - osc[fin]).max() <= 2e-6 * max(1.0, np.abs(osc[fin]).max())
        assert margin_flips(ki[g], kcn[g], osc, k) <= 2
    ref = O.attn_rows(RowView(qc_r, rows, n), RowView(qr_r, rows, n), kc_k, kr_k, v, idx, cnt, scale,
                      cfg.sinks, W, 64, rows)
    return np.abs(out[rows] - ref)


# ------------------------------------------------------- donor prefill ----
DONOR = dict(B=2, n=65536, Hq=28, Hkv=4, d=128, m=4, S=8, W=1024, k=16)


@pytest.fixture(scope="module")
def donor(dev):
    c = DONOR
    cfg = hba_amd.HBAConfig(n_heads=c["Hq"], n_kv=c["Hkv"], head_dim=c["d"], sinks=c["S"], window=c["W"], block=64,
                            slots=c["m"], k_blocks=c["k"])
    x = synth.layer_inputs(c["B"], c["n"], c["Hq"], c["Hkv"], c["d"], m=c["m"], dtype=torch.bfloat16, device=dev,
                           seed=0, sharp=True, needles=False, window=c["W"])
    prm = synth.Params(x["q_gain"], x["k_gain"], x["probes"], x["proj"])
    cos, sin = hba_amd.rope_tables(c["n"] + 64, c["d"], cfg.rope_theta, dev)
    scale = hba_amd.union_scale(cfg, c["d"], c["n"])
    kc, kr, vt = ops.prep_keys(x["k"], x["v"], prm.k.gain, 1e-6, cos, sin)
    S0 = ops.summarize(kc, prm.probes, prm.proj)
    idx, val, cnt = ops.score_select(x["q"], prm.q.gain, 1e-6, S0, c["W"], c["k"], scale)
    out = ops.attn_fwd(x["q"], prm.q.gain, prm.k.gain, 1e-6, kc, kr, vt, cos, sin, idx, cnt, c["S"], c["W"], scale)
    torch.cuda.synchronize()
    return dict(cfg=cfg, x=x, prm=prm, cos=cos, sin=sin, scale=scale, kc=kc, kr=kr, vt=vt, S0=S0, idx=idx,
                val=val, cnt=cnt, out=out)


def test_donor_prefill_64k_b2_sampled_rows(dev, donor):
    c, D = DONOR, donor
    x, cfg, n = D["x"], D["cfg"], c["n"]
    assert abs(D["scale"] * c["d"] - (1 + 0.1 * np.log(2))) < 1e-6    # tau at 2x native context
    i2, v2, c2, scores = ops.score_select_with_scores(x["q"], D["prm"].q.gain, 1e-6, D["S0"], c["W"], c["k"],
                                                      D["scale"])
    torch.cuda.synchronize()
    assert torch.equal(i2, D["idx"]) and torch.equal(c2, D["cnt"]) and torch.equal(v2, D["val"])
    cos, sin = f(D["cos"]), f(D["sin"])
    gq, gk = f(x["q_gain"]), f(x["k_gain"])
    errs = []
    for b in range(c["B"]):
        rows = sample_rows(n, count=140, seed=b)
        kc_o = O.qknorm(f(x["k"][b]), gk, 1e-6, "bf16")
        kr_o = O.apply_rope(kc_o, cos[:n], sin[:n], "bf16")
        assert np.array_equal(f(D["kc"][b]).transpose(1, 0, 2), kc_o)
        assert np.array_equal(f(D["kr"][b]).transpose(1, 0, 2), kr_o)
        sc = scores[b][:, torch.from_numpy(rows).to(dev)].cpu().numpy()
        err = check_prefill_rows(f(x["q"][b]), kc_o, kr_o, f(x["v"][b]), gq, cos, sin, f(D["S0"][b]),
                                 D["idx"][b].cpu().numpy(), D["cnt"][b].cpu().numpy(), sc, f(D["out"][b]), cfg,
                                 D["scale"], rows, c["W"], c["k"])
        errs.append(err)
    del scores
    err = np.concatenate([e.ravel() for e in errs])
    assert err.max() <= 2e-2, err.max()
    assert err.mean() <= 1e-3, err.mean()


@pytest.mark.parametrize("kern", ["fused", "pair"])
def test_donor_decode_continuation_64k(dev, donor, kern, monkeypatch):
    """Four append + decode steps on the 64K donor cache (L = 65537..65540,
    1007 candidate pages in 8 score chunks): each step against the oracle's
    prefill row L-1 on the cache's own keys and summaries."""
    monkeypatch.setenv("HBA_DECODE_KERNEL", kern)
    c, D = DONOR, donor
    cfg, prm, n = D["cfg"], D["prm"], c["n"]
    cache = hba_amd.PagedKVCache(cfg, c["B"], n + 64, torch.bfloat16, dev)
    cache._free = synth.shuffled_pages(len(cache._free), seed=3)
    kcs, vs = [], []
    for s in range(c["B"]):
        cache.load(s, D["kc"][s].transpose(0, 1), D["kr"][s].transpose(0, 1), D["x"]["v"][s], prm)
        kcs.append(f(D["kc"][s]).transpose(1, 0, 2).copy())
        vs.append(f(D["x"]["v"][s]).copy())
    g = torch.Generator().manual_seed(7)
    gk = f(prm.k.gain)
    for step in range(4):
        kn = torch.randn(c["B"], c["Hkv"], c["d"], generator=g).to(torch.bfloat16).to(dev)
        vn = torch.randn(c["B"], c["Hkv"], c["d"], generator=g).to(torch.bfloat16).to(dev)
        qd = torch.randn(c["B"], c["Hq"], c["d"], generator=g).to(torch.bfloat16).to(dev)
        cache.append(kn, vn, prm, prm, D["cos"], D["sin"])
        out, sidx, scnt = hba_amd.hba_decode_step(qd, cache, cfg, prm, D["cos"], D["sin"])
        torch.cuda.synchronize()
        for s in range(c["B"]):
            kcs[s] = np.concatenate([kcs[s], O.qknorm(f(kn)[s], gk, 1e-6, "bf16")[None]], 0)
            vs[s] = np.concatenate([vs[s], f(vn)[s][None]], 0)
        assert min(int(scnt.min()), 16) == 16
        check_decode(cache, cfg, prm, D["cos"], D["sin"], kcs, vs, qd, "bf16", out, sidx, scnt)


# ------------------------------------------------- decode workload, B = 32 ---
@pytest.mark.parametrize("kern", ["fused", "pair"])
def test_decode_bench_lengths_b32(dev, kern, monkeypatch):
    """The decode workload itself: 32 sequences with the benchmark's lengths
    (synth.decode_lengths(32, 16384, 32768, seed 0)), 14/2 heads, d = 64,
    paged bf16 on a shuffled page table; every sequence's picks bit-exact and
    output within 2e-2 of the oracle's row L-1."""
    monkeypatch.setenv("HBA_DECODE_KERNEL", kern)
    lens = synth.decode_lengths(32, 16384, 32768, seed=0)
    cfg, cache, prm, cos, sin, kcs, vs, g = lean_cache(dev, "bf16", lens)
    qd = torch.randn(len(lens), 14, 64, generator=g).to(torch.bfloat16).to(dev)
    out, sidx, scnt = hba_amd.hba_decode_step(qd, cache, cfg, prm, cos, sin)
    torch.cuda.synchronize()
    check_decode(cache, cfg, prm, cos, sin, kcs, vs, qd, "bf16", out, sidx, scnt)


# ----------------------------------------------- hierarchical at 128K ------
def test_hier_128k_timed_picks_and_attention_rows(dev):
    """The 128K hierarchical workload (n = 131072, 14/2 heads, d = 64, F = 16,
    beam 8, top-16, needles, tau = 1 + 0.1 ln 4): hier_select's picks equal
    hier_select_with_scores's on every query, and the union attention over
    them (attn_fwd, as timed) is within 2e-2 of the float64 rows on sampled
    rows (the last 64, the needle queries and a spread)."""
    n, Hq, Hkv, d, W, k, F, beam, S = 131072, 14, 2, 64, 1024, 16, 16, 8, 4
    cfg = hba_amd.HBAConfig(n_heads=Hq, n_kv=Hkv, head_dim=d, window=W, sinks=S, k_blocks=k, slots=4, fanout=F,
                            beam=beam)
    x = synth.layer_inputs(1, n, Hq, Hkv, d, m=4, dtype=torch.bfloat16, device=dev, seed=0, sharp=True,
                           needles=True, window=W)
    prm = synth.Params(x["q_gain"], x["k_gain"], x["probes"], x["proj"])
    cos, sin = hba_amd.rope_tables(n, d, cfg.rope_theta, dev)
    scale = hba_amd.union_scale(cfg, d, n)
    kc, kr, vt = ops.prep_keys(x["k"], x["v"], prm.k.gain, 1e-6, cos, sin)
    S0 = ops.summarize(kc, prm.probes, prm.proj)
    S1 = ops.build_super(S0, F)
    hi, hv, hc = ops.hier_select(x["q"], prm.q.gain, 1e-6, S0, S1, W, k, F, beam, scale)
    di, dv, dc, scores, sup = ops.hier_select_with_scores(x["q"], prm.q.gain, 1e-6, S0, S1, W, k, F, beam, scale)
    del scores, sup
    torch.cuda.synchronize()
    assert torch.equal(hi, di) and torch.equal(hv, dv) and torch.equal(hc, dc)
    assert int(hc.min()) >= 0 and int(hc[0, :, -1].min()) == k
    out = ops.attn_fwd(x["q"], prm.q.gain, prm.k.gain, 1e-6, kc, kr, vt, cos, sin, hi, hc, S, W, scale)
    torch.cuda.synchronize()
    rows = sample_rows(n, [p for (p, _) in x["needles"].values()], count=120)
    c_, s_ = f(cos), f(sin)
    kc_o = f(kc[0]).transpose(1, 0, 2)
    kr_o = f(kr[0]).transpose(1, 0, 2)
    assert np.array_equal(kc_o, O.qknorm(f(x["k"][0]), f(x["k_gain"]), 1e-6, "bf16"))
    qc_r = O.qknorm(f(x["q"][0])[rows], f(x["q_gain"]), 1e-6, "bf16")
    qr_r = O.apply_rope(qc_r, c_, s_, "bf16", positions=rows)
    ref = O.attn_rows(RowView(qc_r, rows, n), RowView(qr_r, rows, n), kc_o, kr_o, f(x["v"][0]),
                      hi[0].cpu().numpy(), hc[0].cpu().numpy(), scale, S, W, 64, rows)
    err = np.abs(f(out[0])[rows] - ref)
    assert err.max() <= 2e-2, err.max()
    assert err.mean() <= 1e-3, err.mean()
