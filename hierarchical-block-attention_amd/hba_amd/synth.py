"""Seeded synthetic inputs for the benchmark and parity workloads.

  layer_inputs   q/k/v N(0,1) drawn from one seeded generator in the order
                 q, k, v (fp32, then rounded to the storage dtype), the
                 SlotSummarizer's reference init (summarizer.py:25,31-32) from a
                 second generator, QKNorm gains (1, or "sharp" d**0.25 as
                 init_qknorm_gains yields for unit-RMS inputs, model.py:219,250),
                 and optional needle blocks.
  needles        per KV head, 16 distinct candidate blocks whose keys are turned
                 toward the grouped query direction u of one random query in
                 the last 1024 positions with cosine 0.6:
                 k <- |k| (0.6 u + 0.8 unit(k - (k.u) u)).
"""
import math

import numpy as np
import torch


def qknorm_ref(x, gain, eps=1e-6):
    xf = x.float()
    r = xf.pow(2).mean(-1, keepdim=True).clamp_min(eps).sqrt()
    return xf / r * gain.float().view(*([1] * (x.dim() - 2)), -1, 1)


def plant_needles(q, k, n_kv, block, window, nneedle=16, seed=0, q_gain=None):
    """In place on k [B, n, Hkv, d] (fp32).  Returns {(b, g): (p_star, blocks)}."""
    B, n, Hq, d = q.shape
    G = Hq // n_kv
    rng = np.random.RandomState(seed)
    ncand = max(0, (n - 1 - window + 1) // block - 1)
    info = {}
    if ncand < 1:
        return info
    gains = torch.ones(Hq) if q_gain is None else q_gain.float().cpu()
    for b in range(B):
        for g in range(n_kv):
            blocks = rng.choice(np.arange(1, ncand + 1), size=min(nneedle, ncand), replace=False)
            p = int(rng.randint(max(0, n - 1024), n))
            qc = qknorm_ref(q[b, p, g * G:(g + 1) * G].cpu(), gains[g * G:(g + 1) * G])
            u = qc.sum(0)
            u = u / u.norm()
            u = u.to(k.device)
            for blk in blocks:
                kb = k[b, blk * block:(blk + 1) * block, g]                  # [Bk, d]
                nrm = kb.norm(dim=-1, keepdim=True)
                perp = kb - (kb @ u)[:, None] * u[None]
                perp = perp / perp.norm(dim=-1, keepdim=True).clamp_min(1e-12)
                k[b, blk * block:(blk + 1) * block, g] = nrm * (0.6 * u[None] + 0.8 * perp)
            info[(b, g)] = (p, sorted(int(x) for x in blocks))
    return info


def layer_inputs(B, n, Hq, Hkv, d, m=4, dtype=torch.bfloat16, device="cpu", seed=0, sharp=False,
                 needles=False, block=64, window=1024, summ_seed=1):
    g = torch.Generator().manual_seed(seed)
    q = torch.randn(B, n, Hq, d, generator=g)
    k = torch.randn(B, n, Hkv, d, generator=g)
    v = torch.randn(B, n, Hkv, d, generator=g)
    gs = torch.Generator().manual_seed(summ_seed)
    probes = torch.randn(Hkv, m, d, generator=gs) * d ** -0.5
    proj = torch.eye(d).unsqueeze(0).repeat(Hkv, 1, 1) + torch.randn(Hkv, d, d, generator=gs) * 0.02
    gain = d ** 0.25 if sharp else 1.0
    q_gain = torch.full((Hq,), gain)
    k_gain = torch.full((Hkv,), gain)
    info = plant_needles(q, k, Hkv, block, window, seed=seed + 7, q_gain=q_gain) if needles else {}
    to = dict(device=device)
    return dict(q=q.to(dtype).to(**to), k=k.to(dtype).to(**to), v=v.to(dtype).to(**to),
                probes=probes.to(**to), proj=proj.to(**to), q_gain=q_gain.to(**to),
                k_gain=k_gain.to(**to), needles=info)


class Params:
    """Minimal QKNorm / SlotSummarizer stand-ins built from tensors."""

    class _N:
        def __init__(self, gain, eps):
            self.gain = gain
            self.eps = eps

    def __init__(self, q_gain, k_gain, probes, proj, eps=1e-6):
        self.q = Params._N(q_gain, eps)
        self.k = Params._N(k_gain, eps)
        self.probes = probes
        self.proj = proj


def decode_lengths(Bd, lo, hi, seed=0):
    """Per-sequence lengths uniform in [lo, hi] from a seeded generator."""
    g = torch.Generator().manual_seed(seed)
    return torch.randint(lo, hi + 1, (Bd,), generator=g).tolist()


def shuffled_pages(total, seed=0):
    g = torch.Generator().manual_seed(seed)
    return torch.randperm(total, generator=g).tolist()


def ncand(i, block, window):
    lim = i - window + 1
    return 0 if lim < 2 * block else lim // block - 1


def mean_keys(n, S, W, block, k):
    """Mean |union| over queries 0..n-1 (sinks + window + routed keys)."""
    tot = 0
    for i in range(n):
        tot += min(S, i + 1) + max(0, i - max(S, i - W + 1) + 1) + min(k, ncand(i, block, W)) * block
    return tot / n


def attention_flops(B, n, Hq, d, S, W, block, k):
    """Algorithmic attention FLOPs: sum_i sum_h 4 d |U_i|."""
    return 4.0 * d * Hq * B * mean_keys(n, S, W, block, k) * n


def scoring_flops(B, n, Hkv, d, m, block, W):
    tot = sum(ncand(i, block, W) for i in range(n))
    return 2.0 * d * m * tot * Hkv * B


def summarizer_flops(B, n, Hkv, d, m, block):
    return (4.0 * m * block * d + 2.0 * m * d * d) * (n // block) * Hkv * B


def log2_ceil(x):
    return int(math.ceil(math.log2(max(1, x))))
