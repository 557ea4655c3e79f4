"""The attention half of a decoder layer as the reference's model runs it
(HBAModel.forward's block_fn, src/hba/model.py:118-140), on the HIP kernels.

  attention_by_mode(q, k, v, cos, sin, cfg, summ, qkn, cap, mode)
      the mode switch of model.py:125-140: "train" -> hba_attention_fused or
      hba_attention_dense (cfg.attn_backend; both are the HIP path here) and
      the aux-KL; "equiv" -> hba_attention_eval(equiv=True); "eval" /
      "eval_hier" -> hba_attention_eval(hier=mode == "eval_hier").
      Returns (out [B, n, Hq, d], aux or None).

  HBAAttention(cfg, hidden)
      q/k/v/o projections (nn.Linear, the donor's Qwen2 layout: biases on
      q, k, v, none on o), the layer's QKNorm and SlotSummarizer, and
      forward(a, cos, sin, mode, cap) -> (o_proj(attention), aux): the
      attention residual branch of one layer, input `a` the layer-normed
      hidden states [B, n, hidden].

The donor model, its embeddings, MLPs and norms, and the training loop stay
outside this package: a model swaps its attention calls for
attention_by_mode (or its attention modules for HBAAttention) and keeps the
rest.
"""
import torch
import torch.nn as nn

from .attention import hba_attention_dense, hba_attention_eval, hba_attention_fused
from .config import resolve_backend
from .modules import QKNorm, SlotSummarizer

MODES = ("train", "equiv", "eval", "eval_hier")


def attention_by_mode(q, k, v, cos, sin, cfg, summ, qkn, cap=None, mode="eval"):
    """model.py:125-140.  aux is None outside "train" (as the reference's
    block_fn leaves it)."""
    if mode not in MODES:
        raise ValueError(f"unknown mode {mode!r}; expected one of {MODES}")
    resolve_backend(cfg)
    if mode == "train":
        fn = hba_attention_fused if getattr(cfg, "attn_backend", "hip") == "fused" else hba_attention_dense
        return fn(q, k, v, cos, sin, cfg, summ, qkn)
    if mode == "equiv":
        return hba_attention_eval(q, k, v, cos, sin, cfg, summ, qkn, cap, equiv=True), None
    return hba_attention_eval(q, k, v, cos, sin, cfg, summ, qkn, cap, hier=(mode == "eval_hier")), None


class HBAAttention(nn.Module):
    """One layer's attention branch: projections around the HBA operator."""

    def __init__(self, cfg, hidden, device=None, dtype=None):
        super().__init__()
        self.cfg = cfg
        Hq, Hkv, dh = cfg.n_heads, cfg.n_kv, cfg.head_dim
        kw = dict(device=device, dtype=dtype)
        self.q_proj = nn.Linear(hidden, Hq * dh, bias=True, **kw)
        self.k_proj = nn.Linear(hidden, Hkv * dh, bias=True, **kw)
        self.v_proj = nn.Linear(hidden, Hkv * dh, bias=True, **kw)
        self.o_proj = nn.Linear(Hq * dh, hidden, bias=False, **kw)
        self.qknorm = QKNorm(cfg).to(device)
        self.summarizer = SlotSummarizer(cfg).to(device)

    def forward(self, a, cos, sin, mode="eval", cap=None):
        cfg = self.cfg
        B, n, _ = a.shape
        Hq, Hkv, dh = cfg.n_heads, cfg.n_kv, cfg.head_dim
        q = self.q_proj(a).view(B, n, Hq, dh)
        k = self.k_proj(a).view(B, n, Hkv, dh)
        v = self.v_proj(a).view(B, n, Hkv, dh)
        o, aux = attention_by_mode(q, k, v, cos, sin, cfg, self.summarizer, self.qknorm, cap, mode)
        return self.o_proj(o.reshape(B, n, Hq * dh)), aux
