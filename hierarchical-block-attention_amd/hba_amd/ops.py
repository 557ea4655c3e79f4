"""torch.library custom ops over the C-ABI (namespace `hba`).

Every op is registered for the CUDA (ROCm/HIP) dispatch key only and has a
fake (meta) implementation for tracing; CPU tensors raise -- there is no CPU
path.  Kernels run asynchronously on the current HIP stream of the tensors'
device.

    hba::prep_keys        QKNorm(k), RoPE(kc), V^T
    hba::summarize        slot summaries of every 64-key block
    hba::build_super      super-summaries (fanout mean)
    hba::score_select     flat top-k block selection
    hba::hier_select      two-level beam selection
    hba::attn_fwd         union attention forward (prefill)
    hba::attn_bwd         union attention backward (dq, dk, dv, QKNorm gain grads)
    hba::kv_append        paged-cache append (mutates the pages)
    hba::kv_append_advance  the decode loop's append: token, filled-page summary,
                          seq_lens += 1 and the new length's scale, one launch
    hba::summarize_pages  summaries of listed pages (mutates summ_pages)
    hba::summarize_filled summaries of the pages the last append filled (mutates summ_pages)
    hba::decode_fwd       decode step over the paged cache
"""
import ctypes
from typing import Optional, Tuple

import torch
from torch import Tensor

from ._lib import BF16, F32, check, lib, strides3

BLOCK = 64
_DT = {torch.float32: F32, torch.bfloat16: BF16}
_CHECKED = set()


def _code(t):
    if t.dtype not in _DT:
        raise TypeError(f"unsupported dtype {t.dtype}: HBA kernels take float32 or bfloat16")
    return _DT[t.dtype]


def _p(t):
    return None if t is None else ctypes.c_void_p(t.data_ptr())


def _stream(dev):
    return ctypes.c_void_p(torch.cuda.current_stream(dev).cuda_stream)


def _dev(t):
    if t.device.type != "cuda":
        raise RuntimeError("hba ops run on a gfx950 GPU only; got a tensor on " + str(t.device))
    idx = t.device.index if t.device.index is not None else torch.cuda.current_device()
    if idx not in _CHECKED:
        with torch.cuda.device(idx):
            check(lib().hba_device_check(), "hba_device_check")
        _CHECKED.add(idx)
    return t.device


def _f32c(t, dev, n=None, what="tensor"):
    """fp32 contiguous copy/view on `dev` (gains, probes, proj, tables)."""
    if t is None:
        return None
    t = t.detach().to(device=dev, dtype=torch.float32).contiguous()
    if n is not None and t.numel() != n:
        raise ValueError(f"{what}: expected {n} elements, got {t.numel()}")
    return t


def _rows(t, what):
    if t.dim() != 4 or t.stride(3) != 1:
        raise ValueError(f"{what}: expected a [B, n, H, d] view with a contiguous last dim")
    return t


def _tables(cos, sin, n, d, dev):
    if cos.shape[-1] != d or cos.shape[0] < n or sin.shape != cos.shape:
        raise ValueError(f"cos/sin: expected [>= {n}, {d}] tables, got {tuple(cos.shape)}")
    return _f32c(cos, dev), _f32c(sin, dev)


# ------------------------------------------------------------------ prep ----
@torch.library.custom_op("hba::prep_keys", mutates_args=(), device_types="cuda")
def prep_keys(k: Tensor, v: Tensor, k_gain: Optional[Tensor], eps: float, cos: Tensor,
              sin: Tensor) -> Tuple[Tensor, Tensor, Tensor]:
    dev = _dev(k)
    _rows(k, "k")
    _rows(v, "v")
    B, n, Hkv, d = k.shape
    if v.shape != k.shape or v.dtype != k.dtype:
        raise ValueError("v must match k in shape and dtype")
    cos, sin = _tables(cos, sin, n, d, dev)
    kg = _f32c(k_gain, dev, Hkv, "k_gain")
    kc = torch.empty(B, Hkv, n, d, dtype=k.dtype, device=dev)
    kr = torch.empty_like(kc)
    vt = torch.empty(B, Hkv, d, n, dtype=k.dtype, device=dev)
    with torch.cuda.device(dev):
        st = lib().hba_prep_keys(_code(k), _p(k), strides3(k), _p(v), strides3(v), _p(kg), eps,
                                 _p(cos), _p(sin), B, n, Hkv, d, _p(kc), _p(kr), _p(vt), _stream(dev))
    check(st, "hba_prep_keys")
    return kc, kr, vt


@prep_keys.register_fake
def _(k, v, k_gain, eps, cos, sin):
    B, n, Hkv, d = k.shape
    kc = k.new_empty(B, Hkv, n, d)
    return kc, k.new_empty(B, Hkv, n, d), k.new_empty(B, Hkv, d, n)


@torch.library.custom_op("hba::prep_keys_summarize", mutates_args=(), device_types="cuda")
def prep_keys_summarize(k: Tensor, v: Tensor, k_gain: Optional[Tensor], eps: float, cos: Tensor, sin: Tensor,
                        probes: Tensor, proj: Tensor) -> Tuple[Tensor, Tensor, Tensor, Tensor]:
    """prep_keys and summarize (64-key blocks) in one launch: (kc, kr, vt, S0),
    each bit-identical to the two ops'; head dim 64 or 128 only."""
    dev = _dev(k)
    _rows(k, "k")
    _rows(v, "v")
    B, n, Hkv, d = k.shape
    if v.shape != k.shape or v.dtype != k.dtype:
        raise ValueError("v must match k in shape and dtype")
    cos, sin = _tables(cos, sin, n, d, dev)
    kg = _f32c(k_gain, dev, Hkv, "k_gain")
    m = probes.shape[1]
    pr = _f32c(probes, dev, Hkv * m * d, "probes")
    pj = _f32c(proj, dev, Hkv * d * d, "proj")
    kc = torch.empty(B, Hkv, n, d, dtype=k.dtype, device=dev)
    kr = torch.empty_like(kc)
    vt = torch.empty(B, Hkv, d, n, dtype=k.dtype, device=dev)
    S0 = torch.empty(B, Hkv, n // BLOCK, m, d, dtype=k.dtype, device=dev)
    with torch.cuda.device(dev):
        st = lib().hba_prep_keys_summarize(_code(k), _p(k), strides3(k), _p(v), strides3(v), _p(kg), eps,
                                           _p(cos), _p(sin), B, n, Hkv, d, _p(kc), _p(kr), _p(vt), _p(pr),
                                           _p(pj), m, _p(S0), _stream(dev))
    check(st, "hba_prep_keys_summarize")
    return kc, kr, vt, S0


@prep_keys_summarize.register_fake
def _(k, v, k_gain, eps, cos, sin, probes, proj):
    B, n, Hkv, d = k.shape
    return (k.new_empty(B, Hkv, n, d), k.new_empty(B, Hkv, n, d), k.new_empty(B, Hkv, d, n),
            k.new_empty(B, Hkv, n // BLOCK, probes.shape[1], d))


@torch.library.custom_op("hba::summarize", mutates_args=(), device_types="cuda")
def summarize(kc: Tensor, probes: Tensor, proj: Tensor, block: int = 64) -> Tensor:
    dev = _dev(kc)
    B, Hkv, n, d = kc.shape
    if not kc.is_contiguous():
        raise ValueError("kc must be contiguous [B, Hkv, n, d]")
    m = probes.shape[1]
    pr = _f32c(probes, dev, Hkv * m * d, "probes")
    pj = _f32c(proj, dev, Hkv * d * d, "proj")
    out = torch.empty(B, Hkv, n // block, m, d, dtype=kc.dtype, device=dev)
    with torch.cuda.device(dev):
        st = lib().hba_summarize(_code(kc), _p(kc), B, Hkv, n, d, block, _p(pr), _p(pj), m, _p(out),
                                 _stream(dev))
    check(st, "hba_summarize")
    return out


@summarize.register_fake
def _(kc, probes, proj, block=64):
    B, Hkv, n, d = kc.shape
    return kc.new_empty(B, Hkv, n // block, probes.shape[1], d)


@torch.library.custom_op("hba::build_super", mutates_args=(), device_types="cuda")
def build_super(S0: Tensor, fanout: int) -> Tensor:
    dev = _dev(S0)
    S0 = S0.contiguous()
    B, Hkv, nb, m, d = S0.shape
    ns = (nb + fanout - 1) // fanout
    out = torch.empty(B, Hkv, ns, m, d, dtype=S0.dtype, device=dev)
    with torch.cuda.device(dev):
        st = lib().hba_build_super(_code(S0), _p(S0), B, Hkv, nb, m, d, fanout, _p(out), _stream(dev))
    check(st, "hba_build_super")
    return out


@build_super.register_fake
def _(S0, fanout):
    B, Hkv, nb, m, d = S0.shape
    return S0.new_empty(B, Hkv, (nb + fanout - 1) // fanout, m, d)


# ------------------------------------------------------------- selection ----
def _sel_out(q, Hkv, k):
    B, n = q.shape[0], q.shape[1]
    return (torch.empty(B, Hkv, n, k, dtype=torch.int32, device=q.device),
            torch.empty(B, Hkv, n, k, dtype=torch.float32, device=q.device),
            torch.empty(B, Hkv, n, dtype=torch.int32, device=q.device))


@torch.library.custom_op("hba::route_queries", mutates_args=(), device_types="cuda")
def route_queries(q: Tensor, q_gain: Optional[Tensor], eps: float, n_kv: int) -> Tensor:
    """grouped_query (summarizer.py:50-54) of the QKNorm'd queries: [B, n, Hkv, d]
    in q's dtype, a valid one-head-per-group q for score_select / hier_select
    (q_gain None), which then select exactly as on q."""
    dev = _dev(q)
    _rows(q, "q")
    B, n, Hq, d = q.shape
    qg = _f32c(q_gain, dev, Hq, "q_gain")
    out = torch.empty(B, n, n_kv, d, dtype=q.dtype, device=dev)
    with torch.cuda.device(dev):
        st = lib().hba_route_queries(_code(q), _p(q), strides3(q), _p(qg), eps, B, n, Hq, n_kv, d, _p(out),
                                     _stream(dev))
    check(st, "hba_route_queries")
    return out


@route_queries.register_fake
def _(q, q_gain, eps, n_kv):
    B, n, Hq, d = q.shape
    return q.new_empty(B, n, n_kv, d)


@torch.library.custom_op("hba::score_select", mutates_args=(), device_types="cuda")
def score_select(q: Tensor, q_gain: Optional[Tensor], eps: float, S0: Tensor, window: int, k: int,
                 scale: float, block: int = 64) -> Tuple[Tensor, Tensor, Tensor]:
    return _score_select(q, q_gain, eps, S0, window, k, scale, None, block)


def score_select_with_scores(q, q_gain, eps, S0, window, k, scale, block=64):
    """score_select that also returns every ranked candidate's fp32 score
    [B, Hkv, n, nb] (-inf elsewhere): the verification form, not a torch op."""
    B, n = q.shape[0], q.shape[1]
    scores = torch.full((B, S0.shape[1], n, S0.shape[2]), float("-inf"), dtype=torch.float32,
                        device=q.device)
    return (*_score_select(q, q_gain, eps, S0, window, k, scale, scores, block), scores)


def _score_select(q, q_gain, eps, S0, window, k, scale, scores, block=64):
    dev = _dev(q)
    _rows(q, "q")
    B, n, Hq, d = q.shape
    S0 = S0.contiguous()
    Hkv, nb, m = S0.shape[1], S0.shape[2], S0.shape[3]
    if S0.shape[0] != B or S0.shape[4] != d or S0.dtype != q.dtype or nb != n // block:
        raise ValueError(f"S0 {tuple(S0.shape)} does not match q {tuple(q.shape)}")
    qg = _f32c(q_gain, dev, Hq, "q_gain")
    idx, val, cnt = _sel_out(q, Hkv, k)
    with torch.cuda.device(dev):
        st = lib().hba_score_select(_code(q), _p(q), strides3(q), _p(qg), eps, _p(S0), B, n, Hq, Hkv, d,
                                    m, block, window, k, scale, _p(idx), _p(val), _p(cnt), _p(scores),
                                    _stream(dev))
    check(st, "hba_score_select")
    return idx, val, cnt


@score_select.register_fake
def _(q, q_gain, eps, S0, window, k, scale, block=64):
    B, n = q.shape[0], q.shape[1]
    Hkv = S0.shape[1]
    return (q.new_empty(B, Hkv, n, k, dtype=torch.int32), q.new_empty(B, Hkv, n, k, dtype=torch.float32),
            q.new_empty(B, Hkv, n, dtype=torch.int32))


@torch.library.custom_op("hba::hier_select", mutates_args=(), device_types="cuda")
def hier_select(q: Tensor, q_gain: Optional[Tensor], eps: float, S0: Tensor, S1: Tensor, window: int,
                k: int, fanout: int, beam: int, scale: float) -> Tuple[Tensor, Tensor, Tensor]:
    return _hier_select(q, q_gain, eps, S0, S1, window, k, fanout, beam, scale, None, None)


def hier_select_with_scores(q, q_gain, eps, S0, S1, window, k, fanout, beam, scale, grouped=True):
    """hier_select that also returns the fp32 scores it ranked: children of the
    kept supers [B, Hkv, n, nb] and candidate-bearing supers [B, Hkv, n, ns]
    (-inf elsewhere; the super array is filled by the bf16 GEMM path only).
    The verification form, not a torch op.  grouped=False scores the second
    level per 64-query tile (no workspace)."""
    B, n = q.shape[0], q.shape[1]
    Hkv, nb, ns = S0.shape[1], S0.shape[2], S1.shape[2]
    scores = torch.full((B, Hkv, n, nb), float("-inf"), dtype=torch.float32, device=q.device)
    sup = torch.full((B, Hkv, n, ns), float("-inf"), dtype=torch.float32, device=q.device)
    return (*_hier_select(q, q_gain, eps, S0, S1, window, k, fanout, beam, scale, scores, sup, grouped),
            scores, sup)


def hier_workspace_bytes(q, S0, k, fanout, beam):
    """Workspace bytes of the grouped second level (0 where it does not apply)."""
    B, n, Hq, d = q.shape
    Hkv, m = S0.shape[1], S0.shape[3]
    nbytes = ctypes.c_size_t(0)
    check(lib().hba_hier_select_workspace_bytes(_code(q), B, n, Hq, Hkv, d, m, k, fanout, beam,
                                                ctypes.byref(nbytes)), "hba_hier_select_workspace_bytes")
    return int(nbytes.value)


def _hier_select(q, q_gain, eps, S0, S1, window, k, fanout, beam, scale, scores, sup_scores, grouped=True):
    dev = _dev(q)
    _rows(q, "q")
    B, n, Hq, d = q.shape
    S0 = S0.contiguous()
    S1 = S1.contiguous()
    Hkv, nb, m = S0.shape[1], S0.shape[2], S0.shape[3]
    if nb != n // BLOCK or S1.shape[2] != (nb + fanout - 1) // fanout:
        raise ValueError("S0/S1 do not match q and fanout")
    qg = _f32c(q_gain, dev, Hq, "q_gain")
    idx, val, cnt = _sel_out(q, Hkv, k)
    nbytes = hier_workspace_bytes(q, S0, k, fanout, beam) if grouped else 0
    ws = torch.empty(nbytes, dtype=torch.uint8, device=dev) if nbytes else None
    with torch.cuda.device(dev):
        st = lib().hba_hier_select(_code(q), _p(q), strides3(q), _p(qg), eps, _p(S0), _p(S1), B, n, Hq,
                                   Hkv, d, m, BLOCK, window, k, fanout, beam, scale, _p(idx), _p(val),
                                   _p(cnt), _p(scores), _p(sup_scores), _p(ws), nbytes, _stream(dev))
    check(st, "hba_hier_select")
    return idx, val, cnt


@hier_select.register_fake
def _(q, q_gain, eps, S0, S1, window, k, fanout, beam, scale):
    B, n = q.shape[0], q.shape[1]
    Hkv = S0.shape[1]
    return (q.new_empty(B, Hkv, n, k, dtype=torch.int32), q.new_empty(B, Hkv, n, k, dtype=torch.float32),
            q.new_empty(B, Hkv, n, dtype=torch.int32))


@torch.library.custom_op("hba::hier_select_rows", mutates_args=(), device_types="cuda")
def hier_select_rows(qn: Tensor, S0: Tensor, S1: Tensor, fanout: int, beam: int, kk: int, cand: Tensor,
                     scale: float) -> Tuple[Tensor, Tensor]:
    """hier_select (attention.py:217-246) on routing queries qn [B, c, d] with
    a candidate mask cand [c, nb] (any rule): top_idx int64 / top_val fp32
    [B, c, min(kk, min(beam, ns) * fanout)], -1 / -inf past the picks."""
    dev = _dev(qn)
    qn = qn.contiguous()
    S0 = S0.to(qn.dtype).contiguous()
    S1 = S1.to(qn.dtype).contiguous()
    B, c, d = qn.shape
    nb, m = S0.shape[1], S0.shape[2]
    ns = (nb + fanout - 1) // fanout
    if S0.shape[0] != B or S0.shape[3] != d or tuple(S1.shape) != (B, ns, m, d):
        raise ValueError("S0 [B, nb, m, d] / S1 [B, ceil(nb / fanout), m, d] do not match qn [B, c, d]")
    if tuple(cand.shape) != (c, nb):
        raise ValueError(f"cand must be [c, nb] = [{c}, {nb}], got {tuple(cand.shape)}")
    cm = cand.to(device=dev, dtype=torch.uint8).contiguous()
    kke = min(kk, min(beam, ns) * fanout)
    idx = torch.empty(B, c, kke, dtype=torch.int64, device=dev)
    val = torch.empty(B, c, kke, dtype=torch.float32, device=dev)
    with torch.cuda.device(dev):
        st = lib().hba_hier_select_rows(_code(qn), _p(qn), _p(S0), _p(S1), _p(cm), B, c, nb, m, d, fanout, beam,
                                        kk, scale, _p(idx), _p(val), _stream(dev))
    check(st, "hba_hier_select_rows")
    return idx, val


@hier_select_rows.register_fake
def _(qn, S0, S1, fanout, beam, kk, cand, scale):
    B, c = qn.shape[0], qn.shape[1]
    ns = (S0.shape[1] + fanout - 1) // fanout
    kke = min(kk, min(beam, ns) * fanout)
    return (qn.new_empty(B, c, kke, dtype=torch.int64), qn.new_empty(B, c, kke, dtype=torch.float32))


# ------------------------------------------------------------- attention ----
@torch.library.custom_op("hba::attn_fwd", mutates_args=(), device_types="cuda")
def attn_fwd(q: Tensor, q_gain: Optional[Tensor], k_gain: Optional[Tensor], eps: float, kc: Tensor,
             kr: Tensor, vt: Tensor, cos: Tensor, sin: Tensor, idx: Tensor, cnt: Tensor, sinks: int,
             window: int, scale: float, block: int = 64) -> Tensor:
    dev = _dev(q)
    _rows(q, "q")
    B, n, Hq, d = q.shape
    Hkv = kc.shape[1]
    if kc.shape != (B, Hkv, n, d) or kr.shape != kc.shape or vt.shape != (B, Hkv, d, n):
        raise ValueError("kc/kr/vt do not match q")
    if idx.shape[:3] != (B, Hkv, n) or cnt.shape != (B, Hkv, n):
        raise ValueError("idx/cnt do not match q")
    if idx.dtype != torch.int32 or cnt.dtype != torch.int32:
        raise TypeError("idx/cnt must be int32")
    cos, sin = _tables(cos, sin, n, d, dev)
    qg = _f32c(q_gain, dev, Hq, "q_gain")
    kg = _f32c(k_gain, dev, Hkv, "k_gain")
    idx = idx.contiguous()
    cnt = cnt.contiguous()
    out = torch.empty(B, n, Hq, d, dtype=q.dtype, device=dev)
    nbytes = ctypes.c_size_t(0)
    check(lib().hba_attn_fwd_workspace_bytes(_code(q), B, n, Hq, d, ctypes.byref(nbytes)),
          "hba_attn_fwd_workspace_bytes")
    ws = torch.empty(max(int(nbytes.value), 16), dtype=torch.uint8, device=dev)
    with torch.cuda.device(dev):
        st = lib().hba_attn_fwd(_code(q), _p(q), strides3(q), _p(qg), _p(kg), eps, _p(kc.contiguous()),
                                _p(kr.contiguous()), _p(vt.contiguous()), _p(cos), _p(sin), _p(idx),
                                _p(cnt), B, n, Hq, Hkv, d, sinks, window, block, idx.shape[3], scale,
                                _p(ws), int(nbytes.value), _p(out), strides3(out), _stream(dev))
    check(st, "hba_attn_fwd")
    return out


def attn_buffers(q, Hkv):
    """Output and workspace of the two-launch bf16 attention (attn_window_ /
    attn_routed_): out [B, n, Hq, d] in q's dtype and the LSE workspace."""
    dev = _dev(q)
    B, n, Hq, d = q.shape
    nbytes = ctypes.c_size_t(0)
    check(lib().hba_attn_workspace_size(_code(q), B, n, Hq, ctypes.byref(nbytes)), "hba_attn_workspace_size")
    return (torch.empty(B, n, Hq, d, dtype=q.dtype, device=dev),
            torch.empty(max(int(nbytes.value), 16), dtype=torch.uint8, device=dev))


def attn_window_(q, q_gain, k_gain, eps, kr, vt, cos, sin, sinks, window, scale, out, ws):
    """The window launch of the bf16 attention on the current stream: the
    window rows into out, their LSE into ws (hba_attn_window_fwd)."""
    dev = _dev(q)
    _rows(q, "q")
    B, n, Hq, d = q.shape
    Hkv = kr.shape[1]
    if q.dtype != torch.bfloat16:
        raise TypeError("the two-launch attention is bf16 only; use attn_fwd")
    if kr.shape != (B, Hkv, n, d) or vt.shape != (B, Hkv, d, n) or out.shape != q.shape:
        raise ValueError("kr/vt/out do not match q")
    cos, sin = _tables(cos, sin, n, d, dev)
    qg = _f32c(q_gain, dev, Hq, "q_gain")
    kg = _f32c(k_gain, dev, Hkv, "k_gain")
    with torch.cuda.device(dev):
        st = lib().hba_attn_window_fwd(_p(q), strides3(q), _p(qg), _p(kg), eps, _p(kr.contiguous()),
                                       _p(vt.contiguous()), _p(cos), _p(sin), B, n, Hq, Hkv, d, sinks, window,
                                       BLOCK, scale, _p(ws), ws.numel(), _p(out), strides3(out), _stream(dev))
    check(st, "hba_attn_window_fwd")
    return out


def attn_routed_(q, q_gain, k_gain, eps, kc, vt, idx, cnt, sinks, scale, out, ws):
    """The sinks + routed launch of the bf16 attention on the current stream,
    merged into the window rows in out (hba_attn_routed_fwd); must follow
    attn_window_ on the same out and ws."""
    dev = _dev(q)
    _rows(q, "q")
    B, n, Hq, d = q.shape
    Hkv = kc.shape[1]
    if kc.shape != (B, Hkv, n, d) or vt.shape != (B, Hkv, d, n) or out.shape != q.shape:
        raise ValueError("kc/vt/out do not match q")
    if idx.shape[:3] != (B, Hkv, n) or cnt.shape != (B, Hkv, n):
        raise ValueError("idx/cnt do not match q")
    if idx.dtype != torch.int32 or cnt.dtype != torch.int32:
        raise TypeError("idx/cnt must be int32")
    qg = _f32c(q_gain, dev, Hq, "q_gain")
    kg = _f32c(k_gain, dev, Hkv, "k_gain")
    idx = idx.contiguous()
    cnt = cnt.contiguous()
    with torch.cuda.device(dev):
        st = lib().hba_attn_routed_fwd(_p(q), strides3(q), _p(qg), _p(kg), eps, _p(kc.contiguous()),
                                       _p(vt.contiguous()), _p(idx), _p(cnt), B, n, Hq, Hkv, d, sinks, BLOCK,
                                       idx.shape[3], scale, _p(ws), ws.numel(), _p(out), strides3(out),
                                       _stream(dev))
    check(st, "hba_attn_routed_fwd")
    return out


_SIDE = {}


def side_stream(dev):
    """A second stream per device (default priority) for the window launch."""
    key = torch.device(dev).index
    if key not in _SIDE:
        _SIDE[key] = torch.cuda.Stream(device=dev)
    return _SIDE[key]


@attn_fwd.register_fake
def _(q, q_gain, k_gain, eps, kc, kr, vt, cos, sin, idx, cnt, sinks, window, scale, block=64):
    return q.new_empty(q.shape)


# ------------------------------------------------------------- backward ----
@torch.library.custom_op("hba::attn_bwd", mutates_args=(), device_types="cuda")
def attn_bwd(q: Tensor, k: Tensor, v: Tensor, kc: Tensor, kr: Tensor, q_gain: Optional[Tensor],
             k_gain: Optional[Tensor], eps: float, cos: Tensor, sin: Tensor, idx: Tensor, cnt: Tensor,
             out: Tensor, dout: Tensor, sinks: int, window: int, scale: float, block: int = 64
             ) -> Tuple[Tensor, Tensor, Tensor, Tensor, Tensor]:
    """Gradients of the union attention output (hba_attn_bwd): dq, dk, dv in
    q's dtype and the QKNorm gain gradients dq_gain [Hq], dk_gain [Hkv] (fp32;
    zeros without QKNorm), the selection idx/cnt held fixed.  fp32 takes any
    block size and head dim the fp32 forward takes; bf16 64-key blocks and
    head dims 64 / 128."""
    dev = _dev(q)
    B, n, Hq, d = q.shape
    Hkv = k.shape[2]
    if k.shape != (B, n, Hkv, d) or v.shape != k.shape or out.shape != q.shape or dout.shape != q.shape:
        raise ValueError("k/v/out/dout do not match q")
    if kc.shape != (B, Hkv, n, d) or kr.shape != kc.shape:
        raise ValueError("kc/kr do not match q")
    if idx.shape[:3] != (B, Hkv, n) or cnt.shape != (B, Hkv, n):
        raise ValueError("idx/cnt do not match q")
    if idx.dtype != torch.int32 or cnt.dtype != torch.int32:
        raise TypeError("idx/cnt must be int32")
    if not (q.dtype == k.dtype == v.dtype == kc.dtype == kr.dtype == out.dtype == dout.dtype):
        raise TypeError("q, k, v, kc, kr, out and dout must share one dtype")
    cos, sin = _tables(cos, sin, n, d, dev)
    qg = _f32c(q_gain, dev, Hq, "q_gain")
    kg = _f32c(k_gain, dev, Hkv, "k_gain")
    if (qg is None) != (kg is None):
        raise ValueError("q_gain and k_gain are both given (QKNorm) or both None")
    q, k, v, kc, kr, out, dout = (t.contiguous() for t in (q, k, v, kc, kr, out, dout))
    idx = idx.contiguous()
    cnt = cnt.contiguous()
    dq, dk, dv = torch.empty_like(q), torch.empty_like(k), torch.empty_like(v)
    dqg = torch.zeros(Hq, dtype=torch.float32, device=dev)
    dkg = torch.zeros(Hkv, dtype=torch.float32, device=dev)
    nbytes = ctypes.c_size_t(0)
    check(lib().hba_attn_bwd_workspace_bytes(_code(q), B, n, Hq, Hkv, d, ctypes.byref(nbytes)),
          "hba_attn_bwd_workspace_bytes")
    ws = torch.empty(max(int(nbytes.value), 16), dtype=torch.uint8, device=dev)
    with torch.cuda.device(dev):
        st = lib().hba_attn_bwd(_code(q), _p(q), _p(k), _p(v), _p(kc), _p(kr), _p(qg), _p(kg), eps, _p(cos),
                                _p(sin), _p(idx), _p(cnt), _p(out), _p(dout), B, n, Hq, Hkv, d, sinks, window,
                                block, idx.shape[3], scale, _p(ws), int(nbytes.value), _p(dq), _p(dk), _p(dv),
                                _p(dqg), _p(dkg), _stream(dev))
    check(st, "hba_attn_bwd")
    return dq, dk, dv, dqg, dkg


@attn_bwd.register_fake
def _(q, k, v, kc, kr, q_gain, k_gain, eps, cos, sin, idx, cnt, out, dout, sinks, window, scale, block=64):
    return (q.new_empty(q.shape), k.new_empty(k.shape), v.new_empty(v.shape),
            q.new_empty(q.shape[2], dtype=torch.float32), k.new_empty(k.shape[2], dtype=torch.float32))


# ---------------------------------------------------------------- decode ----
@torch.library.custom_op("hba::kv_append", mutates_args=("kc_pages", "kr_pages", "v_pages"),
                         device_types="cuda")
def kv_append(k_new: Tensor, v_new: Tensor, k_gain: Optional[Tensor], eps: float, cos: Tensor, sin: Tensor,
              page_table: Tensor, seq_lens: Tensor, kc_pages: Tensor, kr_pages: Tensor,
              v_pages: Tensor) -> None:
    dev = _dev(k_new)
    Bd, Hkv, d = k_new.shape
    kg = _f32c(k_gain, dev, Hkv, "k_gain")
    cos, sin = _tables(cos, sin, 1, d, dev)
    with torch.cuda.device(dev):
        st = lib().hba_kv_append(_code(k_new), _p(k_new.contiguous()), _p(v_new.contiguous()), _p(kg), eps,
                                 _p(cos), _p(sin), cos.shape[0], _p(page_table), page_table.shape[1],
                                 _p(seq_lens), Bd, Hkv, d, BLOCK, _p(kc_pages), _p(kr_pages), _p(v_pages),
                                 _stream(dev))
    check(st, "hba_kv_append")


@torch.library.custom_op("hba::kv_append_advance", mutates_args=("seq_lens", "kc_pages", "kr_pages", "v_pages",
                                                               "summ_pages", "scales"), device_types="cuda")
def kv_append_advance(k_new: Tensor, v_new: Tensor, k_gain: Optional[Tensor], eps: float, cos: Tensor,
                      sin: Tensor, page_table: Tensor, seq_lens: Tensor, kc_pages: Tensor, kr_pages: Tensor,
                      v_pages: Tensor, probes: Tensor, proj: Tensor, summ_pages: Tensor, scale_tab: Tensor,
                      scales: Tensor) -> None:
    """Append one token per sequence at position seq_lens[s], summarise a page
    it fills, then seq_lens += 1 and scales[s] = scale_tab[seq_lens[s]], all on
    the device (one launch)."""
    dev = _dev(k_new)
    Bd, Hkv, d = k_new.shape
    kg = _f32c(k_gain, dev, Hkv, "k_gain")
    cos, sin = _tables(cos, sin, 1, d, dev)
    m = probes.shape[1]
    pr = _f32c(probes, dev, Hkv * m * d, "probes")
    pj = _f32c(proj, dev, Hkv * d * d, "proj")
    for t, what, dt in ((page_table, "page_table", torch.int32), (seq_lens, "seq_lens", torch.int32),
                        (scale_tab, "scale_tab", torch.float32), (scales, "scales", torch.float32)):
        if t.dtype != dt or not t.is_contiguous() or t.device != dev:
            raise ValueError(f"{what} must be a contiguous {dt} tensor on {dev}")
    if seq_lens.numel() != Bd or scales.numel() != Bd:
        raise ValueError(f"seq_lens and scales must hold {Bd} entries")
    with torch.cuda.device(dev):
        st = lib().hba_kv_append_advance(_code(k_new), _p(k_new.contiguous()), _p(v_new.contiguous()), _p(kg), eps,
                                         _p(cos), _p(sin), cos.shape[0], _p(page_table), page_table.shape[1],
                                         _p(seq_lens), Bd, Hkv, d, BLOCK, _p(kc_pages), _p(kr_pages), _p(v_pages),
                                         _p(pr), _p(pj), m, _p(summ_pages), _p(scale_tab), scale_tab.numel(),
                                         _p(scales), _stream(dev))
    check(st, "hba_kv_append_advance")


@torch.library.custom_op("hba::summarize_pages", mutates_args=("summ_pages",), device_types="cuda")
def summarize_pages(kc_pages: Tensor, pages: Tensor, probes: Tensor, proj: Tensor,
                    summ_pages: Tensor) -> None:
    dev = _dev(kc_pages)
    P, Hkv = kc_pages.shape[:2]
    Bk, d = BLOCK, probes.shape[-1]
    if kc_pages[0, 0].numel() != Bk * d:
        raise ValueError(f"kc_pages: expected {Bk * d} elements per page and KV head")
    m = probes.shape[1]
    pr = _f32c(probes, dev, Hkv * m * d, "probes")
    pj = _f32c(proj, dev, Hkv * d * d, "proj")
    pages = pages.to(device=dev, dtype=torch.int32).contiguous()
    with torch.cuda.device(dev):
        st = lib().hba_summarize_pages(_code(kc_pages), _p(kc_pages), _p(pages), pages.numel(), Hkv, d, Bk,
                                       _p(pr), _p(pj), m, _p(summ_pages), _stream(dev))
    check(st, "hba_summarize_pages")


@torch.library.custom_op("hba::summarize_filled", mutates_args=("summ_pages",), device_types="cuda")
def summarize_filled(kc_pages: Tensor, page_table: Tensor, seq_lens: Tensor, probes: Tensor, proj: Tensor,
                     summ_pages: Tensor) -> None:
    """Summaries of the pages the last append filled (sequences whose
    seq_lens is a positive multiple of 64), found on the device."""
    dev = _dev(kc_pages)
    Hkv = kc_pages.shape[1]
    d = probes.shape[-1]
    if kc_pages[0, 0].numel() != BLOCK * d:
        raise ValueError(f"kc_pages: expected {BLOCK * d} elements per page and KV head")
    for t, what in ((page_table, "page_table"), (seq_lens, "seq_lens")):
        if t.dtype != torch.int32 or not t.is_contiguous() or t.device != dev:
            raise ValueError(f"{what} must be a contiguous int32 tensor on {dev}")
    m = probes.shape[1]
    pr = _f32c(probes, dev, Hkv * m * d, "probes")
    pj = _f32c(proj, dev, Hkv * d * d, "proj")
    with torch.cuda.device(dev):
        st = lib().hba_summarize_filled(_code(kc_pages), _p(kc_pages), _p(page_table), page_table.shape[1],
                                        _p(seq_lens), seq_lens.numel(), Hkv, d, BLOCK, _p(pr), _p(pj), m,
                                        _p(summ_pages), _stream(dev))
    check(st, "hba_summarize_filled")


def aux_kl(q, q_gain, k_gain, eps, kc, S0, probes, proj, window, scale_u, scale_r, want_grad, block=BLOCK):
    """The summarizer auxiliary loss (hba_aux_kl): returns (aux as a 0-d fp32
    tensor, d aux / d probes, d aux / d proj), the gradients None unless
    want_grad.  q [B, n, Hq, d] raw, kc [B, Hkv, n, d], S0 [B, Hkv, n/block,
    m, d].  fp32 takes any block size and head dim the fp32 forward takes;
    bf16 64-key blocks and head dims 64 / 128."""
    dev = _dev(q)
    _rows(q, "q")
    B, n, Hq, d = q.shape
    Hkv, m = S0.shape[1], S0.shape[3]
    kc, S0 = kc.contiguous(), S0.contiguous()
    if kc.shape != (B, Hkv, n, d) or kc.dtype != q.dtype or S0.dtype != q.dtype or S0.shape[2] != n // block:
        raise ValueError(f"kc {tuple(kc.shape)} / S0 {tuple(S0.shape)} do not match q {tuple(q.shape)}")
    qg = _f32c(q_gain, dev, Hq, "q_gain")
    kg = _f32c(k_gain, dev, Hkv, "k_gain")
    pr = _f32c(probes, dev, Hkv * m * d, "probes")
    pj = _f32c(proj, dev, Hkv * d * d, "proj")
    nbytes = ctypes.c_size_t(0)
    check(lib().hba_aux_kl_workspace_size(_code(q), B, n, Hq, Hkv, d, m, block, ctypes.byref(nbytes)),
          "hba_aux_kl_workspace_size")
    ws = torch.empty(max(int(nbytes.value), 1), dtype=torch.uint8, device=dev)
    aux = torch.empty(1, dtype=torch.float32, device=dev)
    dpr = torch.empty(Hkv, m, d, dtype=torch.float32, device=dev) if want_grad else None
    dpj = torch.empty(Hkv, d, d, dtype=torch.float32, device=dev) if want_grad else None
    with torch.cuda.device(dev):
        st = lib().hba_aux_kl(_code(q), _p(q), strides3(q), _p(qg), _p(kg), eps, _p(kc), _p(S0), _p(pr), _p(pj), B,
                              n, Hq, Hkv, d, m, block, window, scale_u, scale_r, _p(ws), ws.numel(), _p(aux),
                              _p(dpr), _p(dpj), _stream(dev))
    check(st, "hba_aux_kl")
    return aux[0], dpr, dpj


def _check_decode_cache(q, kc_pages, kr_pages, v_pages, summ_pages, page_table, seq_lens):
    """The decode step's cache arguments: pages in q's dtype on q's device,
    [P, Hkv, 64 * d] key/value pages and [P, Hkv, m, d] summaries, a
    contiguous int32 page table [Bd, max_pages] and seq_lens [Bd]."""
    dev = q.device
    Bd, Hq, d = q.shape
    P, Hkv = summ_pages.shape[:2]
    for t, what in ((kc_pages, "kc_pages"), (kr_pages, "kr_pages"), (v_pages, "v_pages"),
                    (summ_pages, "summ_pages")):
        if t.dtype != q.dtype or t.device != dev or not t.is_contiguous():
            raise ValueError(f"{what} must be a contiguous {q.dtype} tensor on {dev}")
        if t.shape[:2] != (P, Hkv):
            raise ValueError(f"{what}: expected {P} pages of {Hkv} KV heads, got {list(t.shape[:2])}")
        if t is not summ_pages and t[0, 0].numel() != BLOCK * d:
            raise ValueError(f"{what}: expected {BLOCK * d} elements per page and KV head")
    if summ_pages.dim() != 4 or summ_pages.shape[3] != d:
        raise ValueError(f"summ_pages: expected [pages, {Hkv}, m, {d}]")
    for t, what in ((page_table, "page_table"), (seq_lens, "seq_lens")):
        if t.dtype != torch.int32 or t.device != dev or not t.is_contiguous():
            raise ValueError(f"{what} must be a contiguous int32 tensor on {dev}")
    if page_table.dim() != 2 or page_table.shape[0] != Bd or seq_lens.shape != (Bd,):
        raise ValueError(f"page_table [{Bd}, max_pages] and seq_lens [{Bd}] expected")


def decode_workspace_bytes(Bd, Hq, Hkv, d, k, window, max_len):
    n = ctypes.c_size_t(0)
    check(lib().hba_decode_workspace_size(Bd, Hq, Hkv, d, k, BLOCK, window, max_len, ctypes.byref(n)),
          "hba_decode_workspace_size")
    return int(n.value)


_DECODE_WS = {}   # device index -> the decode workspace (uint8, zero-filled when allocated)


def _decode_workspace(dev, nbytes):
    """The decode step's workspace on `dev`, one per device, grown on demand.
    It is allocated zero-filled: it opens with completion counters that must
    be zero before a step and that every step leaves zero.  Decode steps that
    overlap on one device (two streams) race on it."""
    ws = _DECODE_WS.get(dev.index)
    if ws is None or ws.numel() < nbytes:
        if torch.cuda.is_current_stream_capturing():
            raise RuntimeError("hba decode: the workspace would be allocated under graph capture; run one "
                               "decode step of this size on the device before capturing")
        ws = torch.zeros(nbytes, dtype=torch.uint8, device=dev)
        _DECODE_WS[dev.index] = ws
    return ws


@torch.library.custom_op("hba::decode_fwd", mutates_args=(), device_types="cuda")
def decode_fwd(q: Tensor, q_gain: Optional[Tensor], eps: float, kc_pages: Tensor, kr_pages: Tensor,
               v_pages: Tensor, summ_pages: Tensor, page_table: Tensor, seq_lens: Tensor, cos: Tensor,
               sin: Tensor, scales: Tensor, sinks: int, window: int, k: int,
               max_len: int) -> Tuple[Tensor, Tensor, Tensor]:
    dev = _dev(q)
    Bd, Hq, d = q.shape
    Hkv, m = summ_pages.shape[1], summ_pages.shape[2]
    _check_decode_cache(q, kc_pages, kr_pages, v_pages, summ_pages, page_table, seq_lens)
    cos, sin = _tables(cos, sin, max_len, d, dev)
    qg = _f32c(q_gain, dev, Hq, "q_gain")
    sc = _f32c(scales, dev, Bd, "scales")
    q = q.contiguous()
    out = torch.empty_like(q)
    sel_idx = torch.empty(Bd, Hkv, k, dtype=torch.int32, device=dev)
    sel_cnt = torch.empty(Bd, Hkv, dtype=torch.int32, device=dev)
    nbytes = decode_workspace_bytes(Bd, Hq, Hkv, d, k, window, max_len)
    ws = _decode_workspace(dev, nbytes)
    with torch.cuda.device(dev):
        st = lib().hba_decode_fwd(_code(q), _p(q), _p(qg), eps, _p(kc_pages), _p(kr_pages), _p(v_pages),
                                  _p(summ_pages), _p(page_table), page_table.shape[1], _p(seq_lens), _p(cos),
                                  _p(sin), _p(sc), Bd, Hq, Hkv, d, m, sinks, window, BLOCK, k, max_len, _p(ws),
                                  nbytes, _p(out), _p(sel_idx), _p(sel_cnt), _stream(dev))
    check(st, "hba_decode_fwd")
    return out, sel_idx, sel_cnt


def decode_fwd_noalloc(q, q_gain, eps, kc_pages, kr_pages, v_pages, summ_pages, page_table, seq_lens, cos, sin,
                       scales, sinks, window, k, max_len, out, sel_idx=None, sel_cnt=None):
    """decode_fwd through hba_decode_fwd_noalloc: the step runs in the
    library's fixed per-GPU scratch and allocates nothing; the caller passes
    the outputs (out [Bd, Hq, d] contiguous in q's dtype, optional sel_idx
    int32 [Bd, Hkv, k] and sel_cnt int32 [Bd, Hkv]) and contiguous fp32
    q_gain, cos/sin and scales already on the device.  Calls that overlap on
    one GPU race on the scratch."""
    dev = _dev(q)
    Bd, Hq, d = q.shape
    Hkv, m = summ_pages.shape[1], summ_pages.shape[2]
    for t, what in ((q, "q"), (out, "out"), (cos, "cos"), (sin, "sin"), (scales, "scales")):
        if not t.is_contiguous() or t.device != dev:
            raise ValueError(f"{what} must be a contiguous tensor on {dev}")
    if out.shape != q.shape or out.dtype != q.dtype:
        raise ValueError("out must match q in shape and dtype")
    if cos.dtype != torch.float32 or sin.dtype != torch.float32 or scales.dtype != torch.float32:
        raise TypeError("cos, sin and scales must be float32")
    if q_gain is not None and (q_gain.dtype != torch.float32 or not q_gain.is_contiguous()):
        raise TypeError("q_gain must be a contiguous float32 tensor")
    if cos.shape[0] < max_len or cos.shape[1] != d or sin.shape != cos.shape:
        raise ValueError(f"cos/sin: expected [>= {max_len}, {d}] tables")
    _check_decode_cache(q, kc_pages, kr_pages, v_pages, summ_pages, page_table, seq_lens)
    if scales.shape != (Bd,):
        raise ValueError(f"scales: expected [{Bd}]")
    for t, what, shape in ((sel_idx, "sel_idx", (Bd, Hkv, k)), (sel_cnt, "sel_cnt", (Bd, Hkv))):
        if t is None:
            continue
        if t.dtype != torch.int32 or t.device != dev or not t.is_contiguous() or tuple(t.shape) != shape:
            raise ValueError(f"{what}: expected a contiguous int32 tensor {list(shape)} on {dev}")
    with torch.cuda.device(dev):
        st = lib().hba_decode_fwd_noalloc(_code(q), _p(q), _p(q_gain), eps, _p(kc_pages), _p(kr_pages),
                                          _p(v_pages), _p(summ_pages), _p(page_table), page_table.shape[1],
                                          _p(seq_lens), _p(cos), _p(sin), _p(scales), Bd, Hq, Hkv, d, m, sinks,
                                          window, BLOCK, k, max_len, _p(out), _p(sel_idx), _p(sel_cnt),
                                          _stream(dev))
    check(st, "hba_decode_fwd_noalloc")
    return out


@decode_fwd.register_fake
def _(q, q_gain, eps, kc_pages, kr_pages, v_pages, summ_pages, page_table, seq_lens, cos, sin, scales,
      sinks, window, k, max_len):
    Bd, Hkv = q.shape[0], summ_pages.shape[1]
    return (q.new_empty(q.shape), q.new_empty(Bd, Hkv, k, dtype=torch.int32),
            q.new_empty(Bd, Hkv, dtype=torch.int32))
