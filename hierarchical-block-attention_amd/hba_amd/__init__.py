"""MI355X (gfx950) Hierarchical Block Attention operator.

The forward path of the reference's attention module -- block-summary
scoring, top-k / hierarchical block selection, the union-softmax attention
over sinks, the RoPE window and the selected blocks, and a paged-KV decode
step -- as hand-written HIP kernels behind a C-ABI (include/hba_amd.h), bound
here through ctypes and registered as torch.library ops (namespace `hba`).
"""
from . import ops
from .attention import (aux_kl, build_super, equiv_attention, forward_stages, hba_attention_dense,
                        grouped_query, hba_attention_eval, hba_attention_fused, hier_select, selected_mask)
from .config import (HBAConfig, content_scale, log_len_tau, resolve_backend, rope_tables,
                     route_scale, union_scale, yarn_theta)
from .decode import DecodeLoop, PagedKVCache, hba_decode_step
from .layer import HBAAttention, attention_by_mode
from .modules import QKNorm, SlotSummarizer

__all__ = [
    "ops", "HBAConfig", "resolve_backend", "content_scale", "log_len_tau", "union_scale",
    "route_scale", "rope_tables", "yarn_theta", "QKNorm", "SlotSummarizer", "hba_attention_eval",
    "hba_attention_dense", "hba_attention_fused", "build_super", "hier_select", "grouped_query", "forward_stages",
    "selected_mask", "equiv_attention", "aux_kl", "PagedKVCache", "hba_decode_step", "DecodeLoop", "HBAAttention", "attention_by_mode",
]
