"""Write golden vectors of the reference's summarizer auxiliary loss (run
where the reference checkout is present; the tests read only the vectors).

For the input cases of make_golden.py it runs, in fp32 on the CPU:

  hba_attention_dense(..., aux_w=1) -> aux      src/hba/attention.py:306-389
  aux.backward() -> d aux / d probes, d proj    (autograd of the reference)
  the gradient-isolation rule: d aux / d q,k,v  src/hba/gates.py:129-167
  _teacher_chunk -> the teacher p*             src/hba/attention.py:478-495
  _aux_kl_chunked -> the fused path's aux       src/hba/attention.py:509-549

Usage:  python tests/golden/make_golden_aux.py
"""
import os
import sys
import tempfile

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, HERE)
from make_golden import CASES, REF_SRC, checksum, gen_inputs  # noqa: E402


def main():
    tmp = tempfile.mkdtemp(prefix="hba-golden-")
    for var in ("HBA_RESULTS_DIR", "HBA_DATA_DIR", "HBA_LOGS_DIR"):
        os.environ[var] = tmp
    sys.path.insert(0, REF_SRC)
    import torch
    from hba.attention import (QKNorm, _aux_kl_chunked, _content_qk, _route_candidates, _teacher_chunk,
                               hba_attention_dense, rope_tables, route_topk)
    from hba.config import HBAConfig
    from hba.summarizer import SlotSummarizer

    torch.set_num_threads(4)
    rec = {}
    for name, case in CASES.items():
        c = case["cfg"]
        cfg = HBAConfig(**c, attn_backend="naive", aux_w=1.0)
        inp = gen_inputs(case)
        B, n = case["B"], case["n"]
        d, Bk, W = c["head_dim"], c["block"], c["window"]
        nb = n // Bk
        q, k, v = (torch.from_numpy(inp[x]).requires_grad_(True) for x in ("q", "k", "v"))
        summ = SlotSummarizer(cfg)
        qkn = QKNorm(cfg)
        with torch.no_grad():
            summ.probes.copy_(torch.from_numpy(inp["probes"]))
            summ.proj.copy_(torch.from_numpy(inp["proj"]))
            qkn.q.gain.copy_(torch.from_numpy(inp["q_gain"]))
            qkn.k.gain.copy_(torch.from_numpy(inp["k_gain"]))
        cos, sin = rope_tables(n, d, cfg.rope_theta, "cpu")
        out, aux = hba_attention_dense(q, k, v, cos, sin, cfg, summ, qkn)
        aux.backward()
        g_qkv = max(float(t.grad.abs().max()) if t.grad is not None else 0.0 for t in (q, k, v))
        dprobes, dproj = summ.probes.grad.numpy().copy(), summ.proj.grad.numpy().copy()
        with torch.no_grad():
            qc, kc, scale = _content_qk(q.detach(), k.detach(), cfg, qkn, n)
            cand = _route_candidates(n, W, nb, Bk, "cpu")
            Hkv, G = cfg.n_kv, cfg.G
            qn = qc.view(B, n, Hkv, G, d).permute(0, 2, 3, 1, 4).contiguous()
            kt = kc.permute(0, 2, 3, 1).unsqueeze(2).contiguous()
            pstar = _teacher_chunk(qn, kt, cand, scale, Bk)                    # [B,Hkv,n,nb]
            _, bsc = route_topk(qc, kc, cfg, summ, cand)
            aux_chunked = _aux_kl_chunked(qc, kc, bsc, cand, cfg)
        rec[f"{name}_aux"] = np.array(float(aux), np.float64)
        rec[f"{name}_aux_chunked"] = np.array(float(aux_chunked), np.float64)
        rec[f"{name}_dprobes"] = dprobes
        rec[f"{name}_dproj"] = dproj
        rec[f"{name}_grad_qkv_max"] = np.array(g_qkv, np.float64)
        rec[f"{name}_pstar"] = pstar.numpy() if n <= 256 else pstar.numpy()[:, :, -64:]
        rec[f"{name}_ck_q"] = checksum(inp["q"])
        print(f"{name}: aux={float(aux):.6f} chunked={float(aux_chunked):.6f} |d qkv|={g_qkv} "
              f"|dprobes|={np.abs(dprobes).max():.3e} |dproj|={np.abs(dproj).max():.3e}")
    path = os.path.join(HERE, "golden_aux.npz")
    np.savez_compressed(path, **rec)
    print(f"wrote {path} ({os.path.getsize(path) / 1024:.0f} KiB)")


if __name__ == "__main__":
    main()
