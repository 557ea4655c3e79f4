"""Geometry the tuned kernels reach only partly, against the oracle:

  sinks > 64    S = 100 / 128 (the fused path's limit, attention.py:452): the
                tuned bf16 kernel stages two sink blocks, and a routed block 1
                counts only its keys from S on; compared with the oracle's
                dense_rows, the reference's union mask (attention.py:342-356),
                which counts a sink key once even when its block is routed
  generic path  geometry off the tuned kernels runs on the generic fp32
                kernels, bf16 inputs widened (forward_stages -> _forward_
                generic): the reference's block-16 test geometry with
                hierarchical selection (tests/test_qknorm.py:28-35, attention.py:
                690-693), beam > 16, k > 64, more than 16 query heads per KV
                head.  Selection bit-exact against the oracle's fp32 selection
                on the same (storage-rounded) inputs, outputs within 1e-5 of
                its float64 rows before the output rounding, and within the
                bf16 bar of the oracle's bf16 emulation.  The backward
                there runs on the generic fp32 kernels (bf16 inputs
                widened), checked against the oracle's float64 backward.
"""
import numpy as np
import pytest
import torch

import oracle.hba_oracle as O

pytestmark = pytest.mark.gpu

hba_amd = pytest.importorskip("hba_amd")
from hba_amd import ops, synth  # noqa: E402


@pytest.fixture(scope="module")
def dev():
    if not torch.cuda.is_available():
        pytest.fail("GPU tests need a visible gfx950 device")
    return torch.device("cuda:0")


def f(t):
    return t.detach().float().cpu().numpy()


def inputs(dev, dt, n, Hq, Hkv, d, m=4, seed=0, sharp=True, needles=False, **cfgkw):
    cfg = hba_amd.HBAConfig(n_heads=Hq, n_kv=Hkv, head_dim=d, slots=m, **cfgkw)
    x = synth.layer_inputs(1, n, Hq, Hkv, d, m=m, dtype=dt, device=dev, seed=seed, sharp=sharp, needles=needles,
                           block=cfg.block, window=cfg.window)
    prm = synth.Params(x["q_gain"], x["k_gain"], x["probes"], x["proj"])
    cos, sin = hba_amd.rope_tables(n, d, cfg.rope_theta, dev)
    return cfg, x, prm, cos, sin


def rows_of(n):
    return np.unique(np.concatenate([np.arange(0, 8), np.linspace(0, n - 1, 80).astype(np.int64),
                                     np.arange(n - 16, n)]))


# ------------------------------------------------------------ sinks > 64 ----
@pytest.mark.parametrize("dt,S,d", [("bf16", 100, 64), ("bf16", 128, 64), ("bf16", 100, 128), ("f32", 100, 64),
                                    ("f32", 200, 64)])
def test_sinks_beyond_one_block_union_mask(dev, dt, S, d):
    """S sinks with S > 64: block 1 is a candidate, and where a query picked
    it, its keys below S count once (as sinks).  The selection is steered so
    that block 1 is picked: its keys lean toward the queries."""
    tdt = torch.bfloat16 if dt == "bf16" else torch.float32
    Hq, Hkv = (14, 2) if d == 64 else (28, 4)
    n, W, k = 2048, 512, 8
    cfg, x, prm, cos, sin = inputs(dev, tdt, n, Hq, Hkv, d, sinks=S, window=W, k_blocks=k)
    # turn block 1's keys toward every KV group's mean query direction
    kk = x["k"].float()
    for g in range(Hkv):
        u = x["q"][0, :, g * (Hq // Hkv):(g + 1) * (Hq // Hkv)].float().mean((0, 1))
        u = u / u.norm()
        kk[0, 64:128, g] = kk[0, 64:128, g].norm(dim=-1, keepdim=True) * u
    x["k"] = kk.to(tdt)
    r = hba_amd.forward_stages(x["q"], x["k"], x["v"], cos, sin, cfg, prm, prm)
    torch.cuda.synchronize()
    idx, cnt = r["idx"][0].cpu().numpy(), r["cnt"][0].cpu().numpy()
    rows = rows_of(n)
    picked1 = sum(int((idx[g, i, :cnt[g, i]] == 1).any()) for g in range(Hkv) for i in rows)
    assert picked1 > len(rows) // 2, picked1          # the case under test occurs
    P = O.prepare(f(x["q"])[0], f(x["k"])[0], f(x["v"])[0], f(cos), f(sin), cfg, f(x["probes"]), f(x["proj"]),
                  f(x["q_gain"]), f(x["k_gain"]), 1e-6, dt, S0=f(r["S0"])[0])
    sel = lambda g, i: idx[g, i, :cnt[g, i]]
    ref = O.dense_rows(P.qc, P.qr, P.kc, P.kr, P.v, sel, r["scale"], S, W, 64, rows)
    err = np.abs(f(r["out"])[0][rows] - ref).max()
    assert err <= (2e-2 if dt == "bf16" else 1e-5), err
    # the eval drop-in gives the same rows
    out_e = hba_amd.hba_attention_eval(x["q"], x["k"], x["v"], cos, sin, cfg, prm, prm)
    assert torch.equal(out_e, r["out"])


# ----------------------------------------------------------- generic path ----
GENERIC = [
    # the reference's test geometry (tests/test_qknorm.py:28-35), flat and hierarchical
    dict(n=512, Hq=4, Hkv=2, d=8, block=16, window=64, sinks=4, k_blocks=8, fanout=4, beam=2, hier=False),
    dict(n=512, Hq=4, Hkv=2, d=8, block=16, window=64, sinks=4, k_blocks=8, fanout=4, beam=2, hier=True),
    # hierarchical off the tuned geometry: block 32, head dim 96
    dict(n=2048, Hq=6, Hkv=2, d=96, block=32, window=128, sinks=8, k_blocks=6, fanout=8, beam=3, hier=True),
    # beam > 16 at the tuned block size
    dict(n=8192, Hq=14, Hkv=2, d=64, block=64, window=1024, sinks=4, k_blocks=16, fanout=4, beam=24, hier=True),
    # k > 64 (the select-all gate sets k = n / block, gates.py:211)
    dict(n=8192, Hq=14, Hkv=2, d=64, block=64, window=1024, sinks=4, k_blocks=128, hier=False),
    # more than 16 query heads per KV head
    dict(n=2048, Hq=34, Hkv=2, d=64, block=64, window=512, sinks=4, k_blocks=8, hier=False),
]


@pytest.mark.parametrize("dt", ["bf16", "f32"])
@pytest.mark.parametrize("case", GENERIC, ids=lambda c: "-".join(f"{k}{v}" for k, v in c.items()))
def test_generic_path_vs_oracle(dev, dt, case):
    c = dict(case)
    hier = c.pop("hier")
    n, Hq, Hkv, d = c.pop("n"), c.pop("Hq"), c.pop("Hkv"), c.pop("d")
    tdt = torch.bfloat16 if dt == "bf16" else torch.float32
    cfg, x, prm, cos, sin = inputs(dev, tdt, n, Hq, Hkv, d, needles=n >= 4096, **c)
    assert not hba_amd.attention._tuned(x["q"], x["k"], cfg, prm, hier) or (dt == "f32" and not hier)
    with torch.no_grad():
        r = hba_amd.forward_stages(x["q"], x["k"], x["v"], cos, sin, cfg, prm, prm, hier=hier)
        out_e = hba_amd.hba_attention_eval(x["q"], x["k"], x["v"], cos, sin, cfg, prm, prm, None, hier=hier)
    torch.cuda.synchronize()
    assert r["out"].dtype == tdt and torch.equal(out_e, r["out"])
    # the oracle in fp32 on the same storage-rounded inputs, on the kernel's summaries
    P = O.prepare(f(x["q"])[0], f(x["k"])[0], f(x["v"])[0], f(cos), f(sin), cfg, f(x["probes"]), f(x["proj"]),
                  f(x["q_gain"]), f(x["k_gain"]), 1e-6, "f32", S0=f(r["S0"])[0])
    rows = rows_of(n)
    oi, ov, oc = O.select(P, cfg, hier=hier, pos=rows, dtype="f32")
    kk = oi.shape[-1]
    gi = r["idx"][0].cpu().numpy()[:, rows, :kk]
    gc = r["cnt"][0].cpu().numpy()[:, rows]
    assert np.array_equal(gc, oc)
    for g in range(Hkv):
        for j in range(len(rows)):
            assert np.array_equal(gi[g, j, :gc[g, j]], oi[g, j, :oc[g, j]]), (g, rows[j])
    assert int(oc.max()) > 0
    I, C = O._scatter_rows(oi, oc, rows, n)
    ref = O.attn_rows(P.qc, P.qr, P.kc, P.kr, P.v, I, C, r["scale"], cfg.sinks, cfg.window, cfg.block, rows)
    err = np.abs(f(r["out"])[0][rows] - ref)
    if dt == "f32":
        assert err.max() <= 1e-5, err.max()
    else:   # one bf16 rounding of the output
        assert (err <= 2 ** -8 * np.maximum(np.abs(ref), 1e-3) + 1e-6).all(), err.max()
        # and the oracle's bf16 emulation, within the bf16 bar
        Pb = O.prepare(f(x["q"])[0], f(x["k"])[0], f(x["v"])[0], f(cos), f(sin), cfg, f(x["probes"]),
                       f(x["proj"]), f(x["q_gain"]), f(x["k_gain"]), 1e-6, "bf16", S0=f(r["S0"])[0])
        refb = O.attn_rows(Pb.qc, Pb.qr, Pb.kc, Pb.kr, Pb.v, I, C, r["scale"], cfg.sinks, cfg.window, cfg.block,
                           rows)
        assert np.abs(f(r["out"])[0][rows] - refb).max() <= 2e-2


# (relative max error of each gradient against the oracle's float64
# backward: fp32 as the tuned fp32 backward's gate; bf16 inputs run the fp32
# kernels on the widened tensors, against float64 from the same bf16 values,
# so only the forward's bf16 operands and output separate them)
GEN_GRAD_TOL = {"f32": 2e-3, "bf16": 1.5e-2}


@pytest.mark.parametrize("dt,n,Hq,Hkv,d,cfgkw,hier", [
    ("f32", 512, 4, 2, 8, dict(block=16, window=64, sinks=4, k_blocks=8), False),     # tests/test_qknorm.py:28-35
    ("bf16", 512, 4, 2, 8, dict(block=16, window=64, sinks=4, k_blocks=8, fanout=4, beam=2), True),
    ("bf16", 1024, 14, 2, 64, dict(block=64, window=256, sinks=100, k_blocks=4), False),  # S > 64: tuned forward
    ("f32", 1024, 6, 2, 96, dict(block=32, window=128, sinks=8, k_blocks=6), False),
    ("f32", 512, 18, 1, 64, dict(block=64, window=128, sinks=4, k_blocks=4), False),     # G = 18
])
def test_generic_backward_matches_oracle(dev, dt, n, Hq, Hkv, d, cfgkw, hier):
    """hba_attn_bwd off the tuned backward's geometry (the fp32 generic
    kernels; bf16 inputs widened) through autograd of hba_attention_eval:
    dq, dk, dv and the QKNorm gain gradients against the oracle's float64
    backward on the forward's own selection -- the reference's block-16 /
    head-dim-8 test geometry (its naive-vs-fused gradient test runs there,
    tests/test_qknorm.py:181-187), hierarchical selection at that geometry,
    100 sinks, d = 96 with 32-key blocks, 18 query heads per KV head."""
    T = torch.float32 if dt == "f32" else torch.bfloat16
    cfg, x, prm, cos, sin = inputs(dev, T, n, Hq, Hkv, d, aux_w=0.0, **cfgkw)
    q, k, v = (x[t].clone().requires_grad_(True) for t in ("q", "k", "v"))
    gq = x["q_gain"].clone().requires_grad_(True)
    gk = x["k_gain"].clone().requires_grad_(True)
    qkn = synth.Params(gq, gk, x["probes"], x["proj"])
    out = hba_amd.hba_attention_eval(q, k, v, cos, sin, cfg, qkn, qkn, None, hier=hier)
    dout = torch.randn(out.shape, generator=torch.Generator().manual_seed(11)).to(out.dtype).to(dev)
    out.backward(dout)
    torch.cuda.synchronize()
    with torch.no_grad():
        r = hba_amd.forward_stages(x["q"], x["k"], x["v"], cos, sin, cfg, qkn, qkn, hier=hier)
        assert torch.equal(r["out"], out.detach())          # the same forward, the same selection
    idx, cnt = r["idx"][0].cpu().numpy(), r["cnt"][0].cpu().numpy()
    scale = hba_amd.union_scale(cfg, d, n)
    ref = O.union_backward(f(x["q"])[0], f(x["k"])[0], f(x["v"])[0], f(cos), f(sin), scale, f(x["q_gain"]),
                           f(x["k_gain"]), 1e-6, idx, cnt, f(dout)[0], cfg.sinks, cfg.window, cfg.block, True)
    got = [f(q.grad)[0], f(k.grad)[0], f(v.grad)[0], f(gq.grad), f(gk.grad)]
    rel = {nm: np.abs(a - b).max() / max(np.abs(b).max(), 1e-6)
           for nm, a, b in zip(["dq", "dk", "dv", "dq_gain", "dk_gain"], got, ref)}
    print(dt, n, Hq, Hkv, d, cfgkw, {kk: f"{e:.2e}" for kk, e in rel.items()})
    for nm, e in rel.items():
        assert e < GEN_GRAD_TOL[dt], (nm, e)


# ------------------------------------------------------ aux-KL, generic ----
@pytest.mark.parametrize("dt,n,Hq,Hkv,d,m,cfgkw", [
    ("f32", 512, 4, 2, 8, 2, dict(block=16, window=64, sinks=2, k_blocks=4)),   # tests/test_qknorm.py:28-35
    ("bf16", 512, 4, 2, 8, 2, dict(block=16, window=64, sinks=2, k_blocks=4)),
    ("f32", 1024, 6, 2, 96, 3, dict(block=32, window=128, sinks=8, k_blocks=6)),
    ("f32", 1024, 18, 1, 64, 4, dict(block=64, window=256, sinks=4, k_blocks=4)),   # G = 18
])
def test_generic_aux_kl_matches_oracle(dev, dt, n, Hq, Hkv, d, m, cfgkw):
    """hba_aux_kl off the tuned geometry (the generic fp32 kernels; bf16
    inputs widened, so compared with the fp32 oracle on the same bf16 values):
    the aux and its gradients into probes and proj against the oracle's
    float64 aux_kl scoring the blocks with the kernels' own summaries -- the
    reference's block-16 / head-dim-8 test geometry with two slots (its tiny
    model trains there with aux_w = 1, tests/test_qknorm.py:28-35, 181-187),
    head dim 96 with 32-key blocks and three slots, 18 query heads per KV
    head; and the dense drop-in returns the same aux with gradients reaching
    only the summarizer."""
    T = torch.float32 if dt == "f32" else torch.bfloat16
    cfg, x, prm, cos, sin = inputs(dev, T, n, Hq, Hkv, d, m=m, native_ctx=1024, **cfgkw)
    summ = hba_amd.SlotSummarizer(cfg).to(dev)
    with torch.no_grad():
        summ.probes.copy_(x["probes"])
        summ.proj.copy_(x["proj"])
    aux = hba_amd.aux_kl(x["q"], x["k"], x["v"], cos, sin, cfg, summ, prm)
    aux.backward()
    torch.cuda.synchronize()
    ocfg = O.Cfg(n_heads=Hq, n_kv=Hkv, head_dim=d, slots=m, qknorm=True, native_ctx=1024, **cfgkw)
    qc, kc, su = O.content_qk(f(x["q"]), f(x["k"]), ocfg, f(x["q_gain"]), f(x["k_gain"]), 1e-6, n, "f32")
    kch, _, _ = ops.prep_keys(x["k"].float(), x["v"].float(), x["k_gain"], 1e-6, cos, sin)
    S0k = f(ops.summarize(kch, summ.probes.detach(), summ.proj.detach(), cfg.block))
    ref, dpr, dpj, _ = O.aux_kl(qc, kc, f(x["probes"]), f(x["proj"]), Hkv, su, O.route_scale(ocfg, d), cfg.block,
                                cfg.window, S0_scores=S0k, dtype="f32")
    errs = (abs(aux.item() - ref) / abs(ref), np.abs(f(summ.probes.grad) - dpr).max() / np.abs(dpr).max(),
            np.abs(f(summ.proj.grad) - dpj).max() / np.abs(dpj).max())
    print(dt, n, Hq, Hkv, d, m, cfgkw, [f"{e:.2e}" for e in errs])
    assert ref > 0 and errs[0] <= 1e-5 and errs[1] <= 1e-4 and errs[2] <= 1e-4, errs
    # the dense drop-in: the same aux, gradients only into the summarizer
    summ.zero_grad(set_to_none=True)
    q = x["q"].clone().requires_grad_(True)
    out, aux2 = hba_amd.hba_attention_dense(q, x["k"], x["v"], cos, sin, cfg, summ, prm)
    assert abs(aux2.item() - aux.item()) <= 1e-6 * abs(aux.item())
    aux2.backward()
    assert q.grad is None and summ.probes.grad is not None and summ.proj.grad is not None
