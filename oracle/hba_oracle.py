"""CPU oracle for the HBA attention forward path.

TEST INFRASTRUCTURE ONLY.  Only tests/, __graft_entry__.smoke() and bench.py's
cpu_baseline leg import this module, and only to check the kernels' results
(or, for the baseline, as the timed CPU restatement).  The product path
(hierarchical-block-attention_amd/hba_amd) never imports it and has no CPU
fallback.

What it restates (reference file:line):

  rope_tables / rot_half / apply_rope   src/hba/attention.py:27-44
  _HeadRMSNorm / QKNorm                 src/hba/attention.py:69-120   (C, declared order)
  content_scale / log_len_tau           src/hba/attention.py:123-170
  _content_qk                           src/hba/attention.py:173-198
  SlotSummarizer.summarize              src/hba/summarizer.py:34-42
  slot_block_scores / grouped_query     src/hba/summarizer.py:45-54    (C, declared order)
  _route_candidates / masks             src/hba/attention.py:250-269
  route_topk                            src/hba/attention.py:272-303   (C, declared order)
  build_super / hier_select             src/hba/attention.py:202-246   (C, declared order)
  hba_attention_dense (forward)         src/hba/attention.py:306-356   (row-sampled)
  hba_attention_eval (flat and hier)    src/hba/attention.py:610-713   (row-sampled)
  equiv=True (uniform-RoPE causal)      src/hba/attention.py:330-336, 634-649 (row-sampled)
  backward of the union attention       autograd of src/hba/attention.py:306-356 (selection fixed)
  decode step = prefill row L-1         (no reference function; defined from the above)

Arrays are numpy float32 arrays that hold values of the storage dtype
('f32', or 'bf16' values stored exactly in float32).  Storage roundings follow
the reference's tensor dtypes (e.g. QKNorm output cast back to q.dtype,
apply_rope's cos/sin cast to x.dtype and each elementwise op rounded).  The
attention rows themselves are evaluated in float64: that is the mathematics
the reference's three-region softmax fixes, and what the kernels' outputs are
held to (1e-5 for fp32 inputs, 2e-2 for bf16 inputs).

Pinning (each check lives in tests/test_oracle_*.py):
  * golden vectors written from the reference itself (tests/golden/), for
    summarize, route_topk, hier_select, dense and eval outputs;
  * closed forms from the reference's own tests (tests/test_qknorm.py:67-177):
    RMS == gain, content-logit bound, tau closed forms, scale modes;
  * integer closed forms: ncand(n-1) = 495/1007/2031, 2052 keys per deep query,
    hierarchy comparison counts 5.2x/7.9x/10.6x (docs/design.md:79,113);
  * invariants: hier == flat when the beam covers every candidate super,
    select-all eval == masked dense, causality, brute-force loops on tiny
    inputs, and planted mistakes that those checks must catch;
  * equiv rows against torch's scaled_dot_product_attention (a library
    routine, causal, GQA heads expanded) and against the union rows with no
    sinks, a whole-sequence window and no routed blocks;
  * the backward against torch autograd (float64) of a torch restatement of
    the masked dense union softmax, through QKNorm and RoPE.
"""
import ctypes
import math
import os

import numpy as np

from . import build as _build

_LIB = None


def lib():
    """The oracle's C library (built on first use with gcc)."""
    global _LIB
    if _LIB is None:
        path = _build.build()
        L = ctypes.CDLL(path)
        f32p = ctypes.POINTER(ctypes.c_float)
        i32p = ctypes.POINTER(ctypes.c_int32)
        i64p = ctypes.POINTER(ctypes.c_int64)
        c_int, c_i64, c_f = ctypes.c_int, ctypes.c_int64, ctypes.c_float
        L.hba_oracle_round_bf16.argtypes = [f32p, c_i64]
        L.hba_oracle_qknorm.argtypes = [f32p, c_i64, c_int, c_int, f32p, c_f, c_int, f32p]
        L.hba_oracle_group_sum.argtypes = [f32p, c_i64, c_int, c_int, c_int, c_int, f32p]
        L.hba_oracle_cand_bmax.argtypes = [c_i64, c_int, c_int]
        L.hba_oracle_cand_bmax.restype = c_i64
        L.hba_oracle_block_scores.argtypes = [f32p, f32p, i64p, c_i64, c_int, c_int, c_int,
                                              c_f, c_int, c_int, f32p]
        L.hba_oracle_topk.argtypes = [f32p, c_i64, c_int, c_int, i32p, f32p, i32p]
        L.hba_oracle_build_super.argtypes = [f32p, c_int, c_int, c_int, c_int, c_int, f32p]
        L.hba_oracle_hier_select.argtypes = [f32p, f32p, f32p, i64p, c_i64, c_int, c_int, c_int,
                                             c_int, c_int, c_int, c_f, c_int, c_int,
                                             i32p, f32p, i32p]
        L.hba_oracle_hier_select_mask.argtypes = [f32p, f32p, f32p, ctypes.POINTER(ctypes.c_uint8), c_i64,
                                                  c_int, c_int, c_int, c_int, c_int, c_int, c_f,
                                                  i32p, f32p, i32p]
        _LIB = L
    return _LIB


def _p(a, ct=ctypes.c_float):
    return a.ctypes.data_as(ctypes.POINTER(ct))


def _f32(a):
    return np.ascontiguousarray(a, dtype=np.float32)


# --------------------------------------------------------------- dtype emulation
def round_bf16(x):
    """Round to bfloat16 (nearest-even), returned as float32 values."""
    a = np.array(x, dtype=np.float32, copy=True, order="C")
    lib().hba_oracle_round_bf16(_p(a), a.size)
    return a


def to_dtype(x, dtype):
    x = _f32(x)
    return round_bf16(x) if dtype == "bf16" else x.copy()


def _rnd(x, dtype):
    return round_bf16(x) if dtype == "bf16" else _f32(x)


# ------------------------------------------------------------------- config ----
class Cfg:
    """Duck-typed stand-in for the reference HBAConfig (config.py:105-184):
    the fields the forward path reads, with the reference defaults."""

    def __init__(self, **kw):
        d = dict(n_heads=14, n_kv=2, head_dim=64, rope_theta=1_000_000.0, native_ctx=32768,
                 block=64, window=1024, sinks=4, k_blocks=16, slots=4, fanout=16, beam=4,
                 qknorm=True, content_scale_mode="inv_d", temp_c=0.1, n_cal=None)
        d.update(kw)
        self.__dict__.update(d)

    @property
    def G(self):
        return self.n_heads // self.n_kv


def content_scale(cfg, dh):
    """attention.py:123-141"""
    mode = getattr(cfg, "content_scale_mode", "inv_d")
    if mode == "inv_d":
        return 1.0 / dh
    if mode == "inv_sqrt_d":
        return dh ** -0.5
    raise ValueError(f"unknown content_scale_mode {mode!r}")


def log_len_tau(cfg, n):
    """attention.py:144-170"""
    c = getattr(cfg, "temp_c", 0.0)
    if c == 0.0:
        return 1.0
    n_cal = getattr(cfg, "n_cal", None) or cfg.native_ctx
    return 1.0 + c * math.log(max(n / n_cal, 1.0))


def union_scale(cfg, dh, n):
    """The scale _content_qk returns (attention.py:184-197)."""
    if getattr(cfg, "qknorm", False):
        return content_scale(cfg, dh) * log_len_tau(cfg, n)
    return dh ** -0.5


def route_scale(cfg, dh):
    """route_topk's scale: no temperature (attention.py:294)."""
    return content_scale(cfg, dh) if getattr(cfg, "qknorm", False) else dh ** -0.5


# --------------------------------------------------------------------- RoPE ----
def rope_tables(n, d, theta):
    """attention.py:27-32, in float32, evaluated with torch on the CPU in the
    reference's own operation order.  The angle pos * inv carries the last bit
    of inv = 1 / theta^(2i/d) multiplied by the position, so a one-ulp
    difference in the power (numpy's and torch's fp32 pow differ) moves the
    tables by up to 8e-3 at 128K positions; only the reference's expression
    reproduces its tables there (tests/test_oracle_bf16.py)."""
    import torch
    inv = 1.0 / (theta ** (torch.arange(0, d, 2).float() / d))
    pos = torch.arange(n).float()
    fr = torch.outer(pos, inv)
    emb = torch.cat((fr, fr), dim=-1)
    return emb.cos().numpy().astype(np.float32), emb.sin().numpy().astype(np.float32)


def rot_half(x):
    """attention.py:35-37 (NeoX rotate-half)."""
    h = x.shape[-1] // 2
    return np.concatenate([-x[..., h:], x[..., :h]], axis=-1)


def apply_rope(x, cos, sin, dtype, positions=None):
    """attention.py:40-44.  x [..., n, H, d] (n along axis -3); cos/sin cast to
    the storage dtype, each elementwise op rounded to it.  `positions` selects
    table rows when x covers a subset of positions."""
    x = _f32(x)
    c = _rnd(cos if positions is None else cos[positions], dtype)
    s = _rnd(sin if positions is None else sin[positions], dtype)
    c = c[..., :, None, :]
    s = s[..., :, None, :]
    t1 = _rnd(x * c, dtype)
    t2 = _rnd(rot_half(x) * s, dtype)
    return _rnd(t1 + t2, dtype)


# ------------------------------------------------------------------- QKNorm ----
def qknorm(x, gain, eps, dtype):
    """_HeadRMSNorm.forward (attention.py:88-94) in the declared order.
    x [..., H, d] -> same shape, storage dtype."""
    x = _f32(x)
    H, d = x.shape[-2], x.shape[-1]
    g = _f32(gain).reshape(-1)
    assert g.size == H
    y = np.empty_like(x)
    lib().hba_oracle_qknorm(_p(x), x.size // d, d, H, _p(g), float(eps),
                            1 if dtype == "bf16" else 0, _p(y))
    return y


def content_qk(q, k, cfg, q_gain, k_gain, eps, n, dtype):
    """_content_qk (attention.py:173-198): (qc, kc, union scale)."""
    if getattr(cfg, "qknorm", False):
        return qknorm(q, q_gain, eps, dtype), qknorm(k, k_gain, eps, dtype), \
            union_scale(cfg, q.shape[-1], n)
    return _f32(q), _f32(k), q.shape[-1] ** -0.5


def grouped_query(qc, n_kv, dtype):
    """grouped_query (summarizer.py:50-54) for one batch row: qc [n, Hq, d] ->
    [Hkv, n, d], declared order."""
    qc = _f32(qc)
    n, Hq, d = qc.shape
    out = np.empty((n_kv, n, d), dtype=np.float32)
    lib().hba_oracle_group_sum(_p(qc), n, Hq, n_kv, d, 1 if dtype == "bf16" else 0, _p(out))
    return out


# --------------------------------------------------------------- summarizer ----
def init_summarizer(n_kv, m, d, seed=1):
    """SlotSummarizer.__init__ draw order (summarizer.py:25,31-32): probes then
    proj, from one seeded generator.  Returns float32 (probes, proj)."""
    import torch
    g = torch.Generator().manual_seed(seed)
    probes = torch.randn(n_kv, m, d, generator=g) * d ** -0.5
    proj = torch.eye(d).unsqueeze(0).repeat(n_kv, 1, 1) + torch.randn(n_kv, d, d, generator=g) * 0.02
    return probes.numpy().astype(np.float32), proj.numpy().astype(np.float32)


def summarize(kc, probes, proj, Bk):
    """SlotSummarizer.summarize (summarizer.py:34-42) in float64.
    kc [n, Hkv, d] (one batch row) -> [Hkv, nb, m, d] float64."""
    n, Hkv, d = kc.shape
    nb = n // Bk
    kb = kc[: nb * Bk].astype(np.float64).reshape(nb, Bk, Hkv, d)
    pr = probes.astype(np.float64)
    pj = proj.astype(np.float64)
    att = np.einsum("hmd,ckhd->hcmk", pr, kb) * d ** -0.5
    att = att - att.max(-1, keepdims=True)
    att = np.exp(att)
    att = att / att.sum(-1, keepdims=True)
    S = np.einsum("hcmk,ckhd->hcmd", att, kb)
    return np.einsum("hcmd,hde->hcme", S, pj)


def aux_teacher(qc, kc, n_kv, scale, Bk, W):
    """The aux-KL teacher p* (attention.py:375-381; the chunked form
    _teacher_chunk :478-495) in float64.  qc [B, n, Hq, d], kc [B, n, Hkv, d]
    (content q/k) -> [B, Hkv, n, nb]: for each query head, the softmax of its
    content logits (scale) over the keys of candidate blocks, summed per block,
    averaged over the G heads of the KV group and renormalised; rows without a
    candidate block are 0."""
    B, n, Hq, d = qc.shape
    G, nb = Hq // n_kv, n // Bk
    cand = route_candidates(n, W, nb, Bk)
    ckey = np.repeat(cand, Bk, axis=1)                                   # [n, n]
    out = np.zeros((B, n_kv, n, nb))
    for b in range(B):
        for g in range(n_kv):
            kg = kc[b, :, g].astype(np.float64)
            acc = np.zeros((n, nb))
            for h in range(g * G, (g + 1) * G):
                s = (qc[b, :, h].astype(np.float64) @ kg.T) * scale
                s = np.where(ckey, s, -np.inf)
                mx = s.max(-1, keepdims=True)
                e = np.where(ckey, np.exp(s - np.where(np.isfinite(mx), mx, 0.0)), 0.0)
                z = e.sum(-1, keepdims=True)
                w = np.divide(e, z, out=np.zeros_like(e), where=z > 0)
                acc += w.reshape(n, nb, Bk).sum(-1)
            acc /= G
            out[b, g] = acc / np.maximum(acc.sum(-1, keepdims=True), 1e-9)
    return out


def aux_kl(qc, kc, probes, proj, n_kv, scale_u, scale_r, Bk, W, S0_scores=None, dtype="f32"):
    """The summarizer auxiliary loss of hba_attention_dense (attention.py:
    366-389) and its gradients, float64.  qc [B, n, Hq, d], kc [B, n, Hkv, d]
    content q/k; scale_u the union (teacher) scale, scale_r the routing scale.

      bsc = max over slots of (grouped query . summary) * scale_r, -inf off
            the candidates (route_topk, attention.py:272-303)
      aux = -mean over (B, Hkv, queries with a candidate) of
            sum_b p*_b log softmax(bsc)_b   (terms with p*_b = 0 dropped)

    Gradients reach only probes and proj (the routing runs on detached q/k):
    d aux / d bsc_c = (softmax_c * sum_b p*_b - p*_c) / N, the max over slots
    passes it evenly to the tied slots, and the summariser's einsums and
    softmax are differentiated by hand.  S0_scores: summaries [B, Hkv, nb, m, d]
    to score the blocks with instead of the exact ones (a kernel's stored,
    rounded summaries); the summarizer's backward always uses the exact
    forward.  dtype "bf16": the grouped query is rounded to bf16 as
    grouped_query does on bf16 tensors.  Returns (aux, dprobes, dproj, pstar)."""
    B, n, Hq, d = qc.shape
    G, nb = Hq // n_kv, n // Bk
    m = probes.shape[1]
    cand = route_candidates(n, W, nb, Bk)
    vq = cand.any(-1)
    pstar = aux_teacher(qc, kc, n_kv, scale_u, Bk, W)
    pr, pj = probes.astype(np.float64), proj.astype(np.float64)
    qg = np.stack([grouped_query(qc[b], n_kv, dtype) for b in range(B)]).transpose(0, 2, 1, 3).astype(np.float64)
    kb = kc[:, : nb * Bk].astype(np.float64).reshape(B, nb, Bk, n_kv, d)
    logit = np.einsum("hmd,bckhd->bhcmk", pr, kb) * d ** -0.5               # [B,Hkv,nb,m,Bk]
    att = np.exp(logit - logit.max(-1, keepdims=True))
    att /= att.sum(-1, keepdims=True)
    Sp = np.einsum("bhcmk,bckhd->bhcmd", att, kb)                           # pooled
    S0 = np.einsum("bhcmd,hde->bhcme", Sp, pj)
    raw = np.einsum("bihd,bhcmd->bhicm", qg, S0 if S0_scores is None else S0_scores.astype(np.float64))
    mx = raw.max(-1)
    bsc = np.where(cand[None, None], mx * scale_r, -np.inf)
    N = B * n_kv * int(vq.sum())
    if N == 0:
        return 0.0, np.zeros_like(pr), np.zeros_like(pj), pstar
    cm = np.broadcast_to(cand[None, None], bsc.shape)
    fin = np.where(cm, bsc, 0.0)                                            # finite stand-ins off the candidates
    top = np.where(vq[None, None, :, None], fin.max(-1, keepdims=True, initial=-np.inf, where=cm), 0.0)
    z = np.where(cm, np.exp(fin - top), 0.0).sum(-1, keepdims=True)
    lse = top + np.log(np.where(z > 0, z, 1.0))
    soft = np.where(cm, np.exp(fin - lse), 0.0)                             # softmax(bsc)
    pos = (pstar > 0) & cm
    term = np.where(pos, pstar * (fin - lse), 0.0).sum(-1)                  # [B,Hkv,n]
    aux = -term[:, :, vq].sum() / N
    P = np.where(pos, pstar, 0.0).sum(-1, keepdims=True)
    dbsc = np.where(vq[None, None, :, None], soft * P - np.where(pos, pstar, 0.0), 0.0) / N
    ties = raw == mx[..., None]
    draw = (dbsc * scale_r)[..., None] * ties / ties.sum(-1, keepdims=True)   # [B,Hkv,n,nb,m]
    dS0 = np.einsum("bhicm,bihd->bhcmd", draw, qg)
    dproj = np.einsum("bhcmd,bhcme->hde", Sp, dS0)
    dSp = np.einsum("bhcme,hde->bhcmd", dS0, pj)
    datt = np.einsum("bhcmd,bckhd->bhcmk", dSp, kb)
    dlog = att * (datt - (att * datt).sum(-1, keepdims=True))
    dprobes = np.einsum("bhcmk,bckhd->hmd", dlog, kb) * d ** -0.5
    return float(aux), dprobes, dproj, pstar


# ---------------------------------------------------------------- routing -----
def cand_bmax(i, Bk, W):
    """Largest candidate block for query i (0: none). attention.py:250-256"""
    lim = i - W + 1
    return 0 if lim < 2 * Bk else lim // Bk - 1


def ncand(i, Bk, W):
    return max(0, cand_bmax(i, Bk, W))


def route_candidates(n, W, nb, Bk):
    """_route_candidates (attention.py:250-256): bool [n, nb]."""
    i = np.arange(n)[:, None]
    b = np.arange(nb)[None, :]
    return (b >= 1) & ((b + 1) * Bk <= (i - W + 1))


def causal_bucket_masks(n, S, W, nb, Bk):
    """_causal_bucket_masks (attention.py:259-269)."""
    i = np.arange(n)[:, None]
    j = np.arange(n)[None, :]
    return (j < S) & (j <= i), (j >= S) & (j <= i) & (j > i - W), route_candidates(n, W, nb, Bk)


def block_scores(qg_g, S_g, pos, scale, Bk, W):
    """Declared-order masked block scores for one KV head.
    qg_g [n, d]; S_g [nb, m, d]; pos [r] -> [r, nb] float32 (-inf = non-candidate)."""
    qg_g = _f32(qg_g)
    S_g = _f32(S_g)
    pos = np.ascontiguousarray(pos, dtype=np.int64)
    nb, m, d = S_g.shape
    out = np.empty((pos.size, nb), dtype=np.float32)
    lib().hba_oracle_block_scores(_p(qg_g), _p(S_g), _p(pos, ctypes.c_int64), pos.size, nb, m, d,
                                  np.float32(scale), Bk, W, _p(out))
    return out


def topk(scores, kk):
    """Row top-k under (score desc, index asc); -inf never kept."""
    scores = _f32(scores)
    r, nb = scores.shape
    idx = np.empty((r, kk), dtype=np.int32)
    val = np.empty((r, kk), dtype=np.float32)
    cnt = np.empty((r,), dtype=np.int32)
    lib().hba_oracle_topk(_p(scores), r, nb, kk, _p(idx, ctypes.c_int32), _p(val),
                          _p(cnt, ctypes.c_int32))
    return idx, val, cnt


def flat_select(qg, S0, scale, kk, Bk, W, pos=None):
    """Flat routing (route_topk attention.py:295-302 / eval :695-698).
    qg [Hkv, n, d], S0 [Hkv, nb, m, d] -> idx, val [Hkv, r, kk], cnt [Hkv, r]."""
    Hkv, n, d = qg.shape
    pos = np.arange(n) if pos is None else np.asarray(pos)
    res = [topk(block_scores(qg[g], S0[g], pos, scale, Bk, W), kk) for g in range(Hkv)]
    return (np.stack([r[0] for r in res]), np.stack([r[1] for r in res]),
            np.stack([r[2] for r in res]))


def build_super(S0_g, F, dtype):
    """build_super (attention.py:202-214) for one KV head: [nb, m, d] -> [ns, m, d]."""
    S0_g = _f32(S0_g)
    nb, m, d = S0_g.shape
    ns = (nb + F - 1) // F
    out = np.empty((ns, m, d), dtype=np.float32)
    lib().hba_oracle_build_super(_p(S0_g), nb, m, d, F, 1 if dtype == "bf16" else 0, _p(out))
    return out


def hier_select(qg, S0, S1, F, beam, kk, scale, Bk, W, pos=None):
    """hier_select (attention.py:217-246) per KV head.
    qg [Hkv, n, d], S0 [Hkv, nb, m, d], S1 [Hkv, ns, m, d] -> idx, val [Hkv, r, kk], cnt."""
    Hkv, n, d = qg.shape
    nb, m = S0.shape[1], S0.shape[2]
    ns = S1.shape[1]
    assert ns <= 4096 and min(beam, ns) <= 64 and min(beam, ns) * F <= 4096
    pos = np.ascontiguousarray(np.arange(n) if pos is None else pos, dtype=np.int64)
    r = pos.size
    idx = np.empty((Hkv, r, kk), dtype=np.int32)
    val = np.empty((Hkv, r, kk), dtype=np.float32)
    cnt = np.empty((Hkv, r), dtype=np.int32)
    for g in range(Hkv):
        qgg, s0, s1 = _f32(qg[g]), _f32(S0[g]), _f32(S1[g])
        ig, vg, cg = idx[g], val[g], cnt[g]
        lib().hba_oracle_hier_select(_p(qgg), _p(s0), _p(s1), _p(pos, ctypes.c_int64), r, nb, m, d,
                                     F, beam, kk, np.float32(scale), Bk, W,
                                     _p(ig, ctypes.c_int32), _p(vg), _p(cg, ctypes.c_int32))
    return idx, val, cnt


def hier_select_mask(qn, S0, S1, F, beam, kk, cand, scale):
    """hier_select (attention.py:217-246) as the reference states it, with an
    arbitrary candidate mask, for one batch row.  qn [r, d] routing queries,
    S0 [nb, m, d], S1 [ns, m, d], cand bool [r, nb] -> idx, val
    [r, min(kk, min(beam, ns) * F)] (value desc, block asc; -1 / -inf past the
    picks), cnt [r].  Scores: declared-order fp32 dots, slot max, times scale."""
    qn, S0, S1 = _f32(qn), _f32(S0), _f32(S1)
    r, d = qn.shape
    nb, m = S0.shape[0], S0.shape[1]
    ns = S1.shape[0]
    assert ns == (nb + F - 1) // F
    kke = min(kk, min(beam, ns) * F)
    cm = np.ascontiguousarray(cand, dtype=np.uint8)
    assert cm.shape == (r, nb)
    idx = np.empty((r, kke), dtype=np.int32)
    val = np.empty((r, kke), dtype=np.float32)
    cnt = np.empty((r,), dtype=np.int32)
    lib().hba_oracle_hier_select_mask(_p(qn), _p(S0), _p(S1), _p(cm, ctypes.c_uint8), r, nb, m, d, F, beam, kk,
                                      np.float32(scale), _p(idx, ctypes.c_int32), _p(val), _p(cnt, ctypes.c_int32))
    return idx, val, cnt


def hier_comparisons(n, Bk, F, beam):
    """Summary comparisons per query, hierarchical (evals.py:319-320)."""
    ns = math.ceil((n // Bk) / F)
    return ns + min(beam, ns) * F


# -------------------------------------------------------------- attention -----
def attn_rows(qc, qr, kc, kr, v, idx, cnt, scale, S, W, Bk, rows):
    """Union attention rows, float64 (hba_attention_eval attention.py:676-711):
    sinks (NoPE) + RoPE window + the valid routed picks (NoPE), one softmax.
    qc, qr [n, Hq, d]; kc, kr, v [n, Hkv, d]; idx [Hkv, n, kk]; cnt [Hkv, n]
    (indexed by query position).  Returns [len(rows), Hq, d] float64."""
    n, Hq, d = qc.shape
    Hkv = kc.shape[1]
    G = Hq // Hkv
    ar = np.arange(Bk)
    out = np.zeros((len(rows), Hq, d))
    for r, i in enumerate(rows):
        i = int(i)
        js = np.arange(min(S, i + 1))
        jw = np.arange(max(S, i - W + 1), i + 1)
        for g in range(Hkv):
            blocks = idx[g, i, : cnt[g, i]].astype(np.int64)
            jr = (blocks[:, None] * Bk + ar[None, :]).reshape(-1)
            jn = np.concatenate([js, jr])
            Qn = qc[i, g * G:(g + 1) * G].astype(np.float64)
            Qr = qr[i, g * G:(g + 1) * G].astype(np.float64)
            s = np.concatenate([Qn @ kc[jn, g].astype(np.float64).T,
                                Qr @ kr[jw, g].astype(np.float64).T], axis=1) * scale
            vv = v[np.concatenate([jn, jw]), g].astype(np.float64)
            s = s - s.max(1, keepdims=True)
            p = np.exp(s)
            p /= p.sum(1, keepdims=True)
            out[r, g * G:(g + 1) * G] = p @ vv
    return out


def dense_rows(qc, qr, kc, kr, v, sel_blocks, scale, S, W, Bk, rows):
    """hba_attention_dense's masked dense forward (attention.py:342-356), row-
    sampled: full-width NoPE and RoPE score rows, where(window), mask to
    sinks | window | routed(sel), one softmax, @V.  sel_blocks(g, i) -> the
    selected block ids of query i, KV head g.  Returns [len(rows), Hq, d] float64."""
    n, Hq, d = qc.shape
    Hkv = kc.shape[1]
    G = Hq // Hkv
    j = np.arange(n)
    out = np.zeros((len(rows), Hq, d))
    for r, i in enumerate(rows):
        i = int(i)
        m_sink = (j < S) & (j <= i)
        m_win = (j >= S) & (j <= i) & (j > i - W)
        for g in range(Hkv):
            sel = np.zeros(n // Bk + 1, dtype=bool)
            sel[np.asarray(sel_blocks(g, i), dtype=np.int64)] = True
            m_rout = sel[j // Bk]
            keep = m_rout | m_sink | m_win
            Qn = qc[i, g * G:(g + 1) * G].astype(np.float64)
            Qr = qr[i, g * G:(g + 1) * G].astype(np.float64)
            s_nope = Qn @ kc[:, g].astype(np.float64).T * scale
            s_rope = Qr @ kr[:, g].astype(np.float64).T * scale
            sc = np.where(m_win[None], s_rope, s_nope)
            sc = np.where(keep[None], sc, -np.inf)
            sc = sc - sc.max(1, keepdims=True)
            p = np.exp(sc)
            p /= p.sum(1, keepdims=True)
            out[r, g * G:(g + 1) * G] = p @ v[:, g].astype(np.float64)
    return out


# ------------------------------------------------------------ full forward ----
class Prepared:
    """Per-batch-row intermediates of the forward path (storage dtype)."""


def prepare(q, k, v, cos, sin, cfg, probes, proj, q_gain, k_gain, eps, dtype,
            S0=None, dense_route=False):
    """QKNorm, RoPE, summaries and the routing query for q/k/v of ONE batch row
    ([n, H, d] arrays).  S0 may be given (e.g. the kernels' own summaries) so
    selection can be compared on identical inputs."""
    n, Hq, d = q.shape
    Hkv = k.shape[1]
    P = Prepared()
    P.qc, P.kc, P.scale = content_qk(q, k, cfg, q_gain, k_gain, eps, n, dtype)
    P.qr = apply_rope(P.qc, cos[:n], sin[:n], dtype)
    P.kr = apply_rope(P.kc, cos[:n], sin[:n], dtype)
    P.v = _f32(v)
    P.qg = grouped_query(P.qc, Hkv, dtype)
    if S0 is None:
        S0 = _rnd(summarize(P.kc, probes, proj, cfg.block), dtype)
    P.S0 = _f32(S0)
    P.sel_scale = route_scale(cfg, d) if dense_route else P.scale
    return P


def select(P, cfg, hier=False, pos=None, dtype="f32"):
    n = P.qc.shape[0]
    nb = n // cfg.block
    kk = min(cfg.k_blocks, nb)
    if not hier:
        return flat_select(P.qg, P.S0, P.sel_scale, kk, cfg.block, cfg.window, pos)
    S1 = np.stack([build_super(P.S0[g], cfg.fanout, dtype) for g in range(P.S0.shape[0])])
    return hier_select(P.qg, P.S0, S1, cfg.fanout, cfg.beam, kk, P.sel_scale,
                       cfg.block, cfg.window, pos)


def _scatter_rows(idx, cnt, pos, n):
    """Place per-row selections at their query positions ([Hkv, n, kk])."""
    Hkv, r, kk = idx.shape
    I = np.full((Hkv, n, kk), -1, dtype=np.int32)
    C = np.zeros((Hkv, n), dtype=np.int32)
    I[:, pos] = idx
    C[:, pos] = cnt
    return I, C


def forward_eval(q, k, v, cos, sin, cfg, probes, proj, q_gain, k_gain, eps, dtype,
                 hier=False, rows=None, S0=None):
    """hba_attention_eval (attention.py:610-713) for q/k/v [B, n, H, d]; rows
    limits the evaluated query positions.  Returns out [B, r, Hq, d] float64 and
    the selections (idx, val, cnt) per batch row."""
    B, n = q.shape[0], q.shape[1]
    assert n % cfg.block == 0
    rows = np.arange(n) if rows is None else np.asarray(rows)
    outs, sels = [], []
    for b in range(B):
        P = prepare(q[b], k[b], v[b], cos, sin, cfg, probes, proj, q_gain, k_gain, eps, dtype,
                    S0=None if S0 is None else S0[b])
        idx, val, cnt = select(P, cfg, hier=hier, pos=rows, dtype=dtype)
        I, C = _scatter_rows(idx, cnt, rows, n)
        outs.append(attn_rows(P.qc, P.qr, P.kc, P.kr, P.v, I, C, P.scale, cfg.sinks, cfg.window,
                              cfg.block, rows))
        sels.append((idx, val, cnt))
    return np.stack(outs), sels


def forward_dense(q, k, v, cos, sin, cfg, probes, proj, q_gain, k_gain, eps, dtype,
                  rows=None, S0=None):
    """hba_attention_dense forward (attention.py:306-356), row-sampled: selection
    with route_topk's scale (no temperature), masked dense union softmax."""
    B, n = q.shape[0], q.shape[1]
    assert n % cfg.block == 0
    rows = np.arange(n) if rows is None else np.asarray(rows)
    outs, sels = [], []
    for b in range(B):
        P = prepare(q[b], k[b], v[b], cos, sin, cfg, probes, proj, q_gain, k_gain, eps, dtype,
                    S0=None if S0 is None else S0[b], dense_route=True)
        idx, val, cnt = select(P, cfg, hier=False, pos=rows, dtype=dtype)
        rix = {int(i): r for r, i in enumerate(rows)}

        def sel_blocks(g, i, idx=idx, cnt=cnt):
            r = rix[int(i)]
            return idx[g, r, : cnt[g, r]]
        outs.append(dense_rows(P.qc, P.qr, P.kc, P.kr, P.v, sel_blocks, P.scale, cfg.sinks,
                               cfg.window, cfg.block, rows))
        sels.append((idx, val, cnt))
    return np.stack(outs), sels


def equiv_rows(qr, kr, v, scale, rows):
    """Dense uniform-RoPE causal attention rows, float64: the equiv=True branch
    of hba_attention_dense (attention.py:330-336) and hba_attention_eval
    (:634-649).  Query i attends every key j <= i through the rotated q and k,
    one softmax; head h reads KV head h // G.  qr [n, Hq, d]; kr, v [n, Hkv, d].
    Returns [len(rows), Hq, d] float64."""
    n, Hq, d = qr.shape
    G = Hq // kr.shape[1]
    out = np.zeros((len(rows), Hq, d))
    for r, i in enumerate(rows):
        i = int(i)
        for h in range(Hq):
            s = (kr[: i + 1, h // G].astype(np.float64) @ qr[i, h].astype(np.float64)) * scale
            p = np.exp(s - s.max())
            out[r, h] = (p / p.sum()) @ v[: i + 1, h // G].astype(np.float64)
    return out


def forward_equiv(q, k, v, cos, sin, cfg, q_gain, k_gain, eps, dtype, rows=None):
    """hba_attention_eval/dense with equiv=True for q/k/v [B, n, H, d]: the same
    QKNorm and union scale (_content_qk, attention.py:173-198), RoPE on q and k,
    then equiv_rows.  Returns [B, r, Hq, d] float64."""
    B, n = q.shape[0], q.shape[1]
    rows = np.arange(n) if rows is None else np.asarray(rows)
    outs = []
    for b in range(B):
        qc, kc, scale = content_qk(q[b], k[b], cfg, q_gain, k_gain, eps, n, dtype)
        qr = apply_rope(qc, cos[:n], sin[:n], dtype)
        kr = apply_rope(kc, cos[:n], sin[:n], dtype)
        outs.append(equiv_rows(qr, kr, _f32(v[b]), scale, rows))
    return np.stack(outs)


def union_backward(q, k, v, cos, sin, scale, q_gain, k_gain, eps, idx, cnt, dout, S, W, Bk, qknorm=True):
    """Gradients of the union attention output, float64, for ONE batch row
    with the selection fixed (autograd of hba_attention_dense,
    attention.py:306-356; the routing there is on detached q/k, :288-303).
    q [n, Hq, d], k, v [n, Hkv, d] raw; cos/sin [>= n, d]; idx [Hkv, n, kk],
    cnt [Hkv, n]; dout [n, Hq, d].  Returns (dq, dk, dv, dq_gain [Hq],
    dk_gain [Hkv]); the gain gradients are zero without QKNorm.

    With p the union softmax of query row (i, h), D = <dO, O>:
      ds_j = p_j (<dO, v_j> - D) * scale,
      d(q-side) += ds_j y_j, d(y_j) += ds_j x, dv_j += p_j dO
    (x, y: NoPE rows for sinks and routed keys, rotated rows for the window),
    then rope^T(zc, zr) = zc + zr cos + rot^T(zr sin) with rot^T(z) = [z2, -z1],
    then the QKNorm backward dx = g/r y - [ms >= eps] x g <y, x> / (d r^3),
    dg = sum <y, x> / r, r = sqrt(max(mean(x^2), eps))."""
    f = np.float64
    q, k, v, dout = (np.asarray(a, dtype=f) for a in (q, k, v, dout))
    n, Hq, d = q.shape
    Hkv = k.shape[1]
    G = Hq // Hkv
    nb = n // Bk
    kk = idx.shape[2]
    H2 = d // 2

    def norm(x, gain):
        ms = (x * x).mean(-1, keepdims=True)
        r = np.sqrt(np.maximum(ms, eps))
        return x / r * np.asarray(gain, dtype=f)[None, :, None], r, ms

    if qknorm:
        qc, rq, msq = norm(q, q_gain)
        kc, rk, msk = norm(k, k_gain)
    else:
        qc, kc = q, k
    c = np.asarray(cos, dtype=f)[:n, None, :]
    sn = np.asarray(sin, dtype=f)[:n, None, :]

    def rot(x):
        return np.concatenate([-x[..., H2:], x[..., :H2]], -1)

    def rotT(z):
        return np.concatenate([z[..., H2:], -z[..., :H2]], -1)

    qr = qc * c + rot(qc) * sn
    kr = kc * c + rot(kc) * sn
    dqc, dqr = np.zeros_like(qc), np.zeros_like(qc)
    dkc, dkr, dv = np.zeros_like(kc), np.zeros_like(kc), np.zeros_like(v)
    ar = np.arange(Bk)
    for i in range(n):
        js = np.arange(min(S, i + 1))
        jw = np.arange(max(S, i - W + 1), i + 1)
        for g in range(Hkv):
            nc = min(max(int(cnt[g, i]), 0), kk)
            blocks = np.array([b for b in idx[g, i, :nc] if 1 <= b < nb], dtype=np.int64)
            jr = (blocks[:, None] * Bk + ar[None, :]).reshape(-1)
            jr = jr[jr >= S]   # the union: a routed key below S is a sink, counted once (S > Bk)
            jn = np.concatenate([js, jr]).astype(np.int64)
            hs = slice(g * G, (g + 1) * G)
            Qn, Qr = qc[i, hs], qr[i, hs]
            sc = np.concatenate([Qn @ kc[jn, g].T, Qr @ kr[jw, g].T], 1) * scale
            p = np.exp(sc - sc.max(1, keepdims=True))
            p /= p.sum(1, keepdims=True)
            J = np.concatenate([jn, jw])
            Vj = v[J, g]
            dO = dout[i, hs]
            Dv = (dO * (p @ Vj)).sum(1)
            ds = p * (dO @ Vj.T - Dv[:, None]) * scale
            m = len(jn)
            dqc[i, hs] += ds[:, :m] @ kc[jn, g]
            dqr[i, hs] += ds[:, m:] @ kr[jw, g]
            np.add.at(dkc[:, g], jn, ds[:, :m].T @ Qn)
            np.add.at(dkr[:, g], jw, ds[:, m:].T @ Qr)
            np.add.at(dv[:, g], J, p.T @ dO)
    yq = dqc + dqr * c + rotT(dqr * sn)
    yk = dkc + dkr * c + rotT(dkr * sn)

    def normT(x, y, gain, r, ms):
        g_ = np.asarray(gain, dtype=f)[None, :, None]
        yx = (y * x).sum(-1, keepdims=True)
        dx = g_ / r * y - (ms >= eps) * x * g_ * yx / (d * r ** 3)
        return dx, (yx / r).sum(axis=(0, 2))

    if qknorm:
        dq, dgq = normT(q, yq, q_gain, rq, msq)
        dk, dgk = normT(k, yk, k_gain, rk, msk)
    else:
        dq, dgq, dk, dgk = yq, np.zeros(Hq), yk, np.zeros(Hkv)
    return dq, dk, dv, dgq, dgk


def decode_row(q_new, kc_seq, v_seq, cos, sin, cfg, S0_seq, q_gain, eps, dtype, scale):
    """Decode step for one sequence of length L = kc_seq.shape[0]: prefill row
    L-1 of the union attention.  q_new [Hq, d] raw query; kc_seq [L, Hkv, d]
    already-QKNorm'd NoPE keys; S0_seq [Hkv, L//Bk, m, d] page summaries.
    Returns out [Hq, d] float64 and the selection (idx, val, cnt) [Hkv, kk]."""
    L, Hkv, d = kc_seq.shape
    Hq = q_new.shape[0]
    i = L - 1
    if getattr(cfg, "qknorm", False):
        qc = qknorm(q_new[None], q_gain, eps, dtype)[0]
    else:
        qc = _f32(q_new)
    qr = apply_rope(qc[None], cos, sin, dtype, positions=np.array([i]))[0]
    kr = apply_rope(kc_seq, cos[:L], sin[:L], dtype)
    qg = grouped_query(qc[None], Hkv, dtype)[:, 0]                 # [Hkv, d]
    nb = L // cfg.block
    kk = cfg.k_blocks
    idx = np.full((Hkv, kk), -1, dtype=np.int32)
    val = np.full((Hkv, kk), -np.inf, dtype=np.float32)
    cnt = np.zeros((Hkv,), dtype=np.int32)
    for g in range(Hkv):
        qfull = np.zeros((L, d), dtype=np.float32)
        qfull[i] = qg[g]
        if nb > 0:
            sc = block_scores(qfull, S0_seq[g][:nb], np.array([i]), scale, cfg.block, cfg.window)
            a, b_, c = topk(sc, kk)
            idx[g], val[g], cnt[g] = a[0], b_[0], c[0]
    # attn_rows indexes queries by position: give it a one-row view at i
    qc_one = np.broadcast_to(qc[None], (L, Hq, d))
    qr_one = np.broadcast_to(qr[None], (L, Hq, d))
    I = np.broadcast_to(idx[:, None, :], (Hkv, L, kk))
    C = np.broadcast_to(cnt[:, None], (Hkv, L))
    out = attn_rows(qc_one, qr_one, kc_seq, kr, v_seq, I, C, scale, cfg.sinks, cfg.window,
                    cfg.block, [i])[0]
    return out, (idx, val, cnt)
