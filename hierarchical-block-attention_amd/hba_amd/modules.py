"""Parameter holders with the reference's names, shapes and init, so reference
state_dicts load unchanged: QKNorm (src/hba/attention.py:69-120) and
SlotSummarizer (src/hba/summarizer.py:15-42).  Their compute runs in the HIP
kernels; the attention wrappers read `.q.gain`, `.k.gain`, `.eps`,
`.probes` and `.proj` duck-typed, so the reference's own module objects work
as well."""
import torch
import torch.nn as nn

from . import ops


class _HeadRMSNorm(nn.Module):
    """Per-head RMS normalisation with a scalar gain per head (attention.py:69-94)."""

    def __init__(self, n_heads, eps=1e-6):
        super().__init__()
        self.gain = nn.Parameter(torch.ones(n_heads))
        self.eps = eps


class QKNorm(nn.Module):
    """q- and k-side gains of one layer (attention.py:97-120)."""

    def __init__(self, cfg, eps=1e-6):
        super().__init__()
        self.q = _HeadRMSNorm(cfg.n_heads, eps=eps)
        self.k = _HeadRMSNorm(cfg.n_kv, eps=eps)


class SlotSummarizer(nn.Module):
    """m learned probes per KV head attention-pool each block's NoPE keys,
    then a per-head d x d projection (summarizer.py:15-42)."""

    def __init__(self, cfg):
        super().__init__()
        Hkv, dh, m = cfg.n_kv, cfg.head_dim, cfg.slots
        self.m = m
        self.probes = nn.Parameter(torch.randn(Hkv, m, dh) * dh ** -0.5)
        self.proj = nn.Parameter(torch.eye(dh).unsqueeze(0).repeat(Hkv, 1, 1)
                                 + torch.randn(Hkv, dh, dh) * 0.02)

    def summarize_prepared(self, kc_heads):
        """Summaries of QKNorm'd keys in the head-major layout [B, Hkv, n, d]
        -> [B, Hkv, n/64, m, d] (the HIP kernel)."""
        return ops.summarize(kc_heads, self.probes, self.proj)

    def summarize(self, k, Bk):
        """Reference signature: k [B, n, Hkv, d] (already QKNorm'd NoPE keys)
        -> [B, Hkv, nb, m, d]."""
        if Bk != ops.BLOCK:
            raise ValueError(f"block size {Bk} unsupported (kernels use {ops.BLOCK})")
        return ops.summarize(k.transpose(1, 2).contiguous(), self.probes, self.proj)
