"""HBA operator knobs and the shared scale rules.

HBAConfig carries the hot-path fields of the reference config
(src/hba/config.py:105-184) with the same names and defaults, so a reference
HBAConfig object (read duck-typed, as the reference itself does) and this one
are interchangeable as the `cfg` argument of the attention wrappers.
"""
import math
from dataclasses import dataclass
from typing import Optional

import torch


@dataclass
class HBAConfig:
    n_heads: int = 14
    n_kv: int = 2
    head_dim: int = 64
    rope_theta: float = 1_000_000.0
    native_ctx: int = 32768
    block: int = 64
    window: int = 1024
    sinks: int = 4
    k_blocks: int = 16
    slots: int = 4
    fanout: int = 16
    beam: int = 4
    hier_from: int = 32768
    mem_elem_cap: float = 1.0e8
    qknorm: bool = True
    content_scale_mode: str = "inv_d"
    temp_c: float = 0.1
    n_cal: Optional[int] = None
    aux_w: float = 1.0
    attn_backend: str = "hip"

    @property
    def G(self):
        return self.n_heads // self.n_kv


def resolve_backend(cfg):
    """Backend name for the attention call (config.py:187-194).  'hip' and the
    reference's 'fused'/'naive' train backends all map to the HIP kernels:
    the forward, the backward of the attention output through autograd, and
    the aux-KL with its gradient into the summarizer."""
    b = getattr(cfg, "attn_backend", "hip")
    if b in ("hip", "fused", "naive"):
        return "hip"
    raise ValueError(f"unknown attn_backend {b!r}")


def content_scale(cfg, dh):
    """attention.py:123-141"""
    mode = getattr(cfg, "content_scale_mode", "inv_d")
    if mode == "inv_d":
        return 1.0 / dh
    if mode == "inv_sqrt_d":
        return dh ** -0.5
    raise ValueError(f"unknown content_scale_mode {mode!r}")


def log_len_tau(cfg, n):
    """attention.py:144-170: tau = 1 + c * log(max(n / n_cal, 1))."""
    c = getattr(cfg, "temp_c", 0.0)
    if c == 0.0:
        return 1.0
    n_cal = getattr(cfg, "n_cal", None) or cfg.native_ctx
    return 1.0 + c * math.log(max(n / n_cal, 1.0))


def union_scale(cfg, dh, n):
    """The single scale _content_qk returns (attention.py:184-197)."""
    if getattr(cfg, "qknorm", False):
        return content_scale(cfg, dh) * log_len_tau(cfg, n)
    return dh ** -0.5


def route_scale(cfg, dh):
    """route_topk's scale (attention.py:294): no temperature."""
    return content_scale(cfg, dh) if getattr(cfg, "qknorm", False) else dh ** -0.5


def yarn_theta(cfg, n):
    """attention.py:47-53: the RoPE base for the donor+YaRN eval baseline.
    Up to native_ctx it is rope_theta; past it, with s = n / native_ctx,
    NTK-aware rescaling gives rope_theta * s ** (d / (d - 2)), d the head dim
    (the base whose lowest frequency stretches by s)."""
    if n <= cfg.native_ctx:
        return cfg.rope_theta
    d = cfg.head_dim
    return cfg.rope_theta * ((n / cfg.native_ctx) ** (d / (d - 2)))


def rope_tables(n, head_dim, theta, device, dtype=torch.float32):
    """attention.py:27-32 (fp32 cos/sin [n, head_dim]); built with torch on `device`."""
    inv = 1.0 / (theta ** (torch.arange(0, head_dim, 2, device=device).float() / head_dim))
    pos = torch.arange(n, device=device).float()
    fr = torch.outer(pos, inv)
    emb = torch.cat((fr, fr), dim=-1)
    return emb.cos().to(dtype), emb.sin().to(dtype)
