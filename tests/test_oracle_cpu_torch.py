"""The torch CPU restatements the CPU baseline times (oracle/hba_cpu_torch.py)
against the oracle's row-wise float64 forward paths (themselves held to the
reference-written goldens): the same outputs within fp32 accumulation noise,
with and without QKNorm and with the temperature active."""
import numpy as np
import pytest
import torch

import oracle.hba_cpu_torch as T
import oracle.hba_oracle as O


def _inputs(n, Hq, Hkv, d, m, seed, qknorm):
    g = torch.Generator().manual_seed(seed)
    q = torch.randn(1, n, Hq, d, generator=g)
    k = torch.randn(1, n, Hkv, d, generator=g)
    v = torch.randn(1, n, Hkv, d, generator=g)
    probes = torch.randn(Hkv, m, d, generator=g) * d ** -0.5
    proj = torch.eye(d)[None].repeat(Hkv, 1, 1) + torch.randn(Hkv, d, d, generator=g) * 0.02
    qg = (d ** 0.25) * (0.8 + 0.4 * torch.rand(Hq, generator=g))
    kg = (d ** 0.25) * (0.8 + 0.4 * torch.rand(Hkv, generator=g))
    return q, k, v, probes, proj, qg, kg


@pytest.mark.parametrize("qknorm,native_ctx", [(True, 32768), (False, 32768), (True, 256)])
def test_torch_paths_match_oracle(qknorm, native_ctx):
    n, Hq, Hkv, d, m = 512, 4, 2, 64, 4
    cfg = O.Cfg(n_heads=Hq, n_kv=Hkv, head_dim=d, window=128, sinks=4, k_blocks=4, slots=m, qknorm=qknorm,
                native_ctx=native_ctx)
    q, k, v, probes, proj, qg, kg = _inputs(n, Hq, Hkv, d, m, 3, qknorm)
    cos, sin = (torch.from_numpy(t) for t in O.rope_tables(n, d, cfg.rope_theta))
    f = lambda t: t.numpy()
    args = (f(q), f(k), f(v), f(cos), f(sin), cfg, f(probes), f(proj), f(qg), f(kg), 1e-6, "f32")
    rows = np.arange(n)
    ref_d, _ = O.forward_dense(*args, rows=rows)
    ref_e, _ = O.forward_eval(*args, rows=rows)
    out_d = T.dense_forward(q, k, v, cos, sin, cfg, probes, proj, qg, kg, 1e-6)
    out_e = T.gathered_forward(q, k, v, cos, sin, cfg, probes, proj, qg, kg, 1e-6, chunk=96)
    assert np.abs(out_d.numpy() - ref_d).max() <= 1e-4
    assert np.abs(out_e.numpy() - ref_e).max() <= 1e-4
