"""Write golden vectors from the reference implementation (run where the
reference checkout is present; the tests read only the vectors it writes).

It imports the reference's attention/summarizer functions from
/root/reference/src and records, on seeded inputs, the outputs of the functions
that no closed form or invariant pins bit-for-bit:

  SlotSummarizer.summarize          src/hba/summarizer.py:34-42
  route_topk (sel, bsc)             src/hba/attention.py:272-303
  build_super / hier_select         src/hba/attention.py:202-246
  hba_attention_dense (forward)     src/hba/attention.py:306-356
  hba_attention_eval (flat, hier)   src/hba/attention.py:610-713
  QKNorm / _content_qk / rope       src/hba/attention.py:27-44,69-198

Inputs are regenerated from numpy's legacy RandomState (a stream numpy keeps
stable across versions); each fixture stores their checksums so a changed
generator is caught.  Usage:  python tests/golden/make_golden.py
"""
import os
import sys
import tempfile

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
REF_SRC = "/root/reference/src"

CASES = {
    # tiny geometry of the reference's own tests (tests/test_qknorm.py:28-35)
    "tiny_qk": dict(cfg=dict(n_heads=4, n_kv=2, head_dim=8, block=16, window=64, sinks=2,
                             k_blocks=4, slots=2, fanout=4, beam=2, native_ctx=8192,
                             qknorm=True, temp_c=0.1, n_cal=128),
                    B=2, n=256, seed=11, gains="rand", hier_n=1024),
    "tiny_noqk": dict(cfg=dict(n_heads=4, n_kv=2, head_dim=8, block=16, window=64, sinks=2,
                               k_blocks=4, slots=2, fanout=4, beam=2, native_ctx=8192,
                               qknorm=False),
                      B=1, n=256, seed=12, gains="ones", hier_n=1024),
    "tiny_sqrtd": dict(cfg=dict(n_heads=4, n_kv=2, head_dim=8, block=16, window=64, sinks=2,
                                k_blocks=4, slots=2, fanout=4, beam=2, native_ctx=8192,
                                qknorm=True, content_scale_mode="inv_sqrt_d", temp_c=0.0),
                       B=1, n=256, seed=13, gains="rand", hier_n=1024),
    # the kernels' geometry (d=64, Bk=64, m=4) at a small window
    "d64": dict(cfg=dict(n_heads=4, n_kv=2, head_dim=64, block=64, window=128, sinks=4,
                         k_blocks=3, slots=4, fanout=4, beam=2, native_ctx=32768,
                         qknorm=True, temp_c=0.1, n_cal=None),
                B=1, n=1024, seed=14, gains="sharp", hier_n=4096, rows=64),
}


def gen_inputs(case):
    """Seeded inputs of one case (shared with tests/test_oracle_golden.py)."""
    c = case["cfg"]
    B, n = case["B"], case["n"]
    Hq, Hkv, d, m = c["n_heads"], c["n_kv"], c["head_dim"], c["slots"]
    rs = np.random.RandomState(case["seed"])
    q = rs.standard_normal((B, n, Hq, d)).astype(np.float32)
    k = rs.standard_normal((B, n, Hkv, d)).astype(np.float32)
    v = rs.standard_normal((B, n, Hkv, d)).astype(np.float32)
    probes = (rs.standard_normal((Hkv, m, d)) * d ** -0.5).astype(np.float32)
    proj = (np.eye(d)[None].repeat(Hkv, 0) + rs.standard_normal((Hkv, d, d)) * 0.02).astype(np.float32)
    if case["gains"] == "ones":
        qg_, kg_ = np.ones(Hq, np.float32), np.ones(Hkv, np.float32)
    elif case["gains"] == "sharp":
        qg_ = (d ** 0.25 * rs.uniform(0.8, 1.2, Hq)).astype(np.float32)
        kg_ = (d ** 0.25 * rs.uniform(0.8, 1.2, Hkv)).astype(np.float32)
    else:
        qg_ = rs.uniform(0.3, 2.0, Hq).astype(np.float32)
        kg_ = rs.uniform(0.3, 2.0, Hkv).astype(np.float32)
    hn = case["hier_n"]
    nbh = hn // c["block"]
    qg_h = rs.standard_normal((B, 8, d)).astype(np.float32)           # 8 routing queries
    S0_h = rs.standard_normal((B, nbh, m, d)).astype(np.float32)
    pos_h = np.array([hn - 1 - 37 * t for t in range(8)], dtype=np.int64)
    return dict(q=q, k=k, v=v, probes=probes, proj=proj, q_gain=qg_, k_gain=kg_,
                qg_h=qg_h, S0_h=S0_h, pos_h=pos_h)


def checksum(x):
    x = np.ascontiguousarray(x, dtype=np.float32)
    return np.array([float(np.float64(x).sum()), float(np.abs(np.float64(x)).sum())])


def main():
    tmp = tempfile.mkdtemp(prefix="hba-golden-")
    for var in ("HBA_RESULTS_DIR", "HBA_DATA_DIR", "HBA_LOGS_DIR"):
        os.environ[var] = tmp
    sys.path.insert(0, REF_SRC)
    import torch
    from hba.attention import (QKNorm, _content_qk, _route_candidates, build_super,
                               hba_attention_dense, hba_attention_eval, hier_select,
                               rope_tables, route_topk)
    from hba.config import HBAConfig
    from hba.summarizer import SlotSummarizer, grouped_query

    torch.set_num_threads(4)
    for name, case in CASES.items():
        c = case["cfg"]
        cfg = HBAConfig(**c, attn_backend="naive", aux_w=0.0)
        inp = gen_inputs(case)
        B, n = case["B"], case["n"]
        d, Bk, W = c["head_dim"], c["block"], c["window"]
        nb = n // Bk
        q, k, v = (torch.from_numpy(inp[x]) for x in ("q", "k", "v"))
        summ = SlotSummarizer(cfg)
        qkn = QKNorm(cfg)
        with torch.no_grad():
            summ.probes.copy_(torch.from_numpy(inp["probes"]))
            summ.proj.copy_(torch.from_numpy(inp["proj"]))
            qkn.q.gain.copy_(torch.from_numpy(inp["q_gain"]))
            qkn.k.gain.copy_(torch.from_numpy(inp["k_gain"]))
            cos, sin = rope_tables(n, d, cfg.rope_theta, "cpu")
            qc, kc, scale = _content_qk(q, k, cfg, qkn, n)
            S0 = summ.summarize(kc, Bk)                                   # [B,Hkv,nb,m,d]
            cand = _route_candidates(n, W, nb, Bk, "cpu")
            sel, bsc = route_topk(qc, kc, cfg, summ, cand)
            qg = grouped_query(qc, cfg)
            out_dense, _ = hba_attention_dense(q, k, v, cos, sin, cfg, summ, qkn)
            out_eval = hba_attention_eval(q, k, v, cos, sin, cfg, summ, qkn, 2e7)
            out_hier = hba_attention_eval(q, k, v, cos, sin, cfg, summ, qkn, 2e7, hier=True)
            # hier_select on its own, at a longer context (more supers than the beam)
            hn = case["hier_n"]
            nbh = hn // Bk
            S0h = torch.from_numpy(inp["S0_h"])
            qgh = torch.from_numpy(inp["qg_h"])
            posh = torch.from_numpy(inp["pos_h"])
            barr = torch.arange(nbh)
            candh = (barr[None, :] >= 1) & ((barr[None, :] + 1) * Bk <= (posh[:, None] - W + 1))
            S1h, nsh = build_super(S0h, cfg.fanout)
            hsc = 1.0 / d
            hidx, hval, hcomp = hier_select(qgh, S0h, S1h, cfg.fanout, cfg.beam,
                                            min(cfg.k_blocks, nbh), candh, hsc)
            fl = torch.einsum("bcd,bnmd->bcnm", qgh, S0h).amax(-1) * hsc
            fl = fl.masked_fill(~candh[None], float("-inf"))
        rows = case.get("rows")
        keep = (np.arange(n) if rows is None else
                np.unique(np.concatenate([np.linspace(0, n - 1, rows).astype(np.int64),
                                          np.arange(n - 8, n)])))
        rec = dict(
            cos=cos.numpy(), sin=sin.numpy(), scale=np.array(scale, np.float64),
            qc=qc.numpy(), kc=kc.numpy(), qg=qg.numpy(), S0=S0.numpy(),
            sel=sel.numpy(), bsc=bsc.numpy(),
            rows=keep, out_dense=out_dense.numpy()[:, keep], out_eval=out_eval.numpy()[:, keep],
            out_hier=out_hier.numpy()[:, keep],
            S1_h=S1h.numpy(), hier_idx=hidx.numpy(), hier_val=hval.numpy(),
            hier_comp=np.array(hcomp), flat_h=fl.numpy(),
            ck_q=checksum(inp["q"]), ck_k=checksum(inp["k"]), ck_v=checksum(inp["v"]),
            ck_S0h=checksum(inp["S0_h"]))
        if rows is not None:
            rec["ck_cos"] = checksum(rec.pop("cos"))
            rec["ck_sin"] = checksum(rec.pop("sin"))
            rec.pop("qc")
            rec.pop("kc")
            rec.pop("qg")
            rec.pop("bsc")
        path = os.path.join(HERE, f"golden_{name}.npz")
        np.savez_compressed(path, **rec)
        print(f"{name}: wrote {path} ({os.path.getsize(path) / 1024:.0f} KiB) scale={scale:.6g}")


BF16_CASES = {
    # the kernels' geometries: 14/2 heads at d = 64 and the 28/4-head d = 128 shape
    "d64": dict(B=1, n=128, Hq=14, Hkv=2, d=64, seed=21, F=(16, 5), nb=37),
    "d128": dict(B=1, n=32, Hq=28, Hkv=4, d=128, seed=22, F=(16, 3), nb=20),
}


def gen_bf16_inputs(case):
    """Seeded fp32 draws for the bf16 fixture (shared with the tests): q, k,
    gains, S0, and rows that exercise QKNorm's eps clamp (an all-zero row and a
    row far below eps in mean square)."""
    rs = np.random.RandomState(case["seed"])
    B, n, Hq, Hkv, d = case["B"], case["n"], case["Hq"], case["Hkv"], case["d"]
    q = rs.standard_normal((B, n, Hq, d)).astype(np.float32)
    k = rs.standard_normal((B, n, Hkv, d)).astype(np.float32)
    q[0, 5, 3] = 0.0
    q[0, 6, 1] *= 1e-5
    k[0, 7, 1] = 0.0
    k[0, 9, 0] *= 3e-5
    q[0, 10] *= 40.0                                  # large-magnitude rows
    qg_ = (d ** 0.25 * rs.uniform(0.5, 1.5, Hq)).astype(np.float32)
    kg_ = (d ** 0.25 * rs.uniform(0.5, 1.5, Hkv)).astype(np.float32)
    S0 = rs.standard_normal((B, case["nb"], 4, d)).astype(np.float32)
    # far positions: RoPE angles at 128K, where the tables' bf16 rounding matters most
    far = rs.standard_normal((1, 64, Hkv, d)).astype(np.float32)
    return dict(q=q, k=k, q_gain=qg_, k_gain=kg_, S0=S0, far=far)


def round_probe():
    """fp32 values whose bf16 rounding is delicate: halfway ties (both
    parities), values just either side of a tie, the overflow edge, fp32
    subnormals, signed zeros, infinities, NaN, and random magnitudes."""
    rs = np.random.RandomState(23)
    one = np.float32(1.0)
    ulp = np.float32(2.0 ** -7)
    ties = [one + ulp / 2, one + 3 * ulp / 2, -(one + ulp / 2), np.float32(3.0) + np.float32(2.0 ** -7)]
    near = [np.nextafter(t, np.float32(np.inf)) for t in ties] + [np.nextafter(t, np.float32(-np.inf))
                                                                  for t in ties]
    big = [np.float32(3.3895313892515355e38), np.float32(3.3961e38), np.float32(3.4028235e38),
           np.float32(-3.39e38)]
    tiny = [np.float32(1e-40), np.float32(-3e-39), np.float32(1.1754942e-38), np.float32(1e-45)]
    special = [np.float32(0.0), np.float32(-0.0), np.float32(np.inf), np.float32(-np.inf), np.float32(np.nan)]
    rnd = (rs.standard_normal(4096) * np.exp(rs.uniform(-30, 30, 4096))).astype(np.float32)
    return np.concatenate([np.array(ties + near + big + tiny + special, np.float32), rnd])


def bf16_bits(t):
    """Raw bits of a torch bfloat16 tensor as uint16 (the fixture's storage)."""
    import torch
    return t.contiguous().view(torch.int16).numpy().view(np.uint16)


def from_bits(u):
    """uint16 bf16 bits -> float32 values (exact)."""
    return (np.asarray(u, dtype=np.uint32) << 16).view(np.float32)


def main_bf16():
    """Fixture of the reference's bf16 arithmetic (golden_bf16.npz): torch's
    fp32 -> bf16 cast, _HeadRMSNorm on bf16 q/k (attention.py:88-94),
    apply_rope on bf16 tensors (:40-44), grouped_query's bf16 head sum
    (summarizer.py:50-54) and build_super's bf16 sum and divide
    (attention.py:202-214)."""
    tmp = tempfile.mkdtemp(prefix="hba-golden-")
    for var in ("HBA_RESULTS_DIR", "HBA_DATA_DIR", "HBA_LOGS_DIR"):
        os.environ[var] = tmp
    sys.path.insert(0, REF_SRC)
    import torch
    from hba.attention import QKNorm, apply_rope, build_super, rope_tables
    from hba.config import HBAConfig
    from hba.summarizer import grouped_query

    bf = torch.bfloat16
    rec = {}
    probe = round_probe()
    rec["round_in"] = probe
    rec["round_out"] = torch.from_numpy(probe).to(bf).float().numpy()
    for name, case in BF16_CASES.items():
        inp = gen_bf16_inputs(case)
        B, n, Hq, Hkv, d = case["B"], case["n"], case["Hq"], case["Hkv"], case["d"]
        cfg = HBAConfig(n_heads=Hq, n_kv=Hkv, head_dim=d, qknorm=True)
        qkn = QKNorm(cfg)
        with torch.no_grad():
            qkn.q.gain.copy_(torch.from_numpy(inp["q_gain"]))
            qkn.k.gain.copy_(torch.from_numpy(inp["k_gain"]))
            q = torch.from_numpy(inp["q"]).to(bf)
            k = torch.from_numpy(inp["k"]).to(bf)
            qc, kc = qkn.q(q), qkn.k(k)
            cos, sin = rope_tables(n, d, cfg.rope_theta, "cpu")
            qr, kr = apply_rope(qc, cos, sin), apply_rope(kc, cos, sin)
            qg = grouped_query(qc, cfg)
            cf, sf = rope_tables(131072, d, cfg.rope_theta, "cpu")
            far = qkn.k(torch.from_numpy(inp["far"]).to(bf))
            far_r = apply_rope(far, cf[-64:], sf[-64:])
            S0 = torch.from_numpy(inp["S0"]).to(bf)
            for F in case["F"]:
                S1, ns = build_super(S0, F)
                assert S1.dtype == bf
                rec[f"{name}_S1_F{F}"] = bf16_bits(S1)
        for key, t in (("qc", qc), ("kc", kc), ("qr", qr), ("kr", kr), ("qg", qg), ("far_kc", far),
                       ("far_kr", far_r)):
            assert t.dtype == bf, key
            rec[f"{name}_{key}"] = bf16_bits(t)
        rec[f"{name}_far_cos"] = cf[-64:].numpy()
        rec[f"{name}_far_sin"] = sf[-64:].numpy()
        rec[f"{name}_ck_q"] = checksum(inp["q"])
    path = os.path.join(HERE, "golden_bf16.npz")
    np.savez_compressed(path, **rec)
    print(f"bf16: wrote {path} ({os.path.getsize(path) / 1024:.0f} KiB)")


if __name__ == "__main__":
    if "--bf16-only" in sys.argv:
        main_bf16()
    else:
        main()
        main_bf16()
