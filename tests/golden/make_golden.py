"""Write golden vectors from the reference implementation (run in the build
container only; the reference never travels to the GPU box).

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


if __name__ == "__main__":
    main()
