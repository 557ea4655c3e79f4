"""torch (CPU, fp32) restatements of the reference's two HBA forward paths,
timed by bench.py's cpu_baseline leg.

TEST INFRASTRUCTURE ONLY: the CPU baseline times these; tests/ holds them to
the oracle (tests/test_oracle_cpu_torch.py).  Nothing in the product path
imports this module.

  dense_forward     hba_attention_dense forward, src/hba/attention.py:306-356:
                    QKNorm / scale (:173-198), RoPE (:27-44), route_topk
                    (:272-303, scale without the temperature), full [n, n]
                    NoPE and RoPE score matrices, where(window), the union
                    mask, one softmax, @V
  gathered_forward  hba_attention_eval, src/hba/attention.py:610-713: per KV
                    head, query chunks gather the window, the sinks and the
                    selected blocks and take one softmax over their
                    concatenation
Both take q [B, n, Hq, d], k, v [B, n, Hkv, d], fp32 cos/sin [n, d] and
return out [B, n, Hq, d] (fp32).
"""
import torch

from . import hba_oracle as O


def _qknorm(x, gain, eps):
    xf = x.float()
    r = xf.pow(2).mean(-1, keepdim=True).clamp_min(eps).sqrt()
    return xf / r * gain.float().view(*([1] * (x.dim() - 2)), -1, 1)


def _rope(x, cos, sin):
    h = x.shape[-1] // 2
    rot = torch.cat((-x[..., h:], x[..., :h]), dim=-1)
    return x * cos[None, :, None, :] + rot * sin[None, :, None, :]


def _prepare(q, k, cos, sin, cfg, probes, proj, q_gain, k_gain, eps, dense_route):
    B, n, Hq, d = q.shape
    if cfg.qknorm:
        qc, kc = _qknorm(q, q_gain, eps), _qknorm(k, k_gain, eps)
    else:
        qc, kc = q.float(), k.float()
    scale = O.union_scale(cfg, d, n)
    sel_scale = O.route_scale(cfg, d) if dense_route else scale
    qr, kr = _rope(qc, cos, sin), _rope(kc, cos, sin)
    Hkv, nb, Bk = k.shape[2], n // cfg.block, cfg.block
    # SlotSummarizer.summarize (summarizer.py:34-42)
    kb = kc.view(B, nb, Bk, Hkv, d)
    att = torch.einsum("hmd,bckhd->bhcmk", probes, kb) * d ** -0.5
    S0 = torch.einsum("bhcmd,hde->bhcme", torch.einsum("bhcmk,bckhd->bhcmd", att.softmax(-1), kb), proj)
    qg = qc.view(B, n, Hkv, Hq // Hkv, d).sum(3).transpose(1, 2)        # [B, Hkv, n, d]
    return qc, kc, qr, kr, S0, qg, scale, sel_scale


def _candidates(n, W, Bk, dev):
    i = torch.arange(n, device=dev)[:, None]
    b = torch.arange(n // Bk, device=dev)[None, :]
    return (b >= 1) & ((b + 1) * Bk <= i - W + 1)                        # [n, nb]


def dense_forward(q, k, v, cos, sin, cfg, probes, proj, q_gain, k_gain, eps):
    B, n, Hq, d = q.shape
    Hkv, G, Bk, S, W = k.shape[2], Hq // k.shape[2], cfg.block, cfg.sinks, cfg.window
    kk = min(cfg.k_blocks, n // Bk)
    qc, kc, qr, kr, S0, qg, scale, sel_scale = _prepare(q, k, cos, sin, cfg, probes, proj, q_gain, k_gain,
                                                        eps, True)
    cand = _candidates(n, W, Bk, q.device)
    bsc = torch.einsum("bhid,bhcmd->bhicm", qg, S0).amax(-1) * sel_scale
    bsc = bsc.masked_fill(~cand[None, None], float("-inf"))
    top = bsc.topk(kk, dim=-1)
    sel = torch.zeros_like(bsc, dtype=torch.bool).scatter_(-1, top.indices, True) & cand[None, None]
    i = torch.arange(n)[:, None]
    j = torch.arange(n)[None, :]
    m_sink = (j < S) & (j <= i)
    m_win = (j >= S) & (j <= i) & (j > i - W)
    m_rout = sel.repeat_interleave(G, dim=1).repeat_interleave(Bk, dim=-1)   # [B, Hq, n, n]
    kn = kc.transpose(1, 2).repeat_interleave(G, dim=1)
    krr = kr.transpose(1, 2).repeat_interleave(G, dim=1)
    vv = v.float().transpose(1, 2).repeat_interleave(G, dim=1)
    s_nope = torch.matmul(qc.transpose(1, 2), kn.transpose(-1, -2)) * scale
    s_rope = torch.matmul(qr.transpose(1, 2), krr.transpose(-1, -2)) * scale
    sc = torch.where(m_win[None, None], s_rope, s_nope)
    sc = sc.masked_fill(~(m_rout | (m_sink | m_win)[None, None]), float("-inf"))
    return torch.matmul(sc.softmax(-1), vv).transpose(1, 2)


def gathered_forward(q, k, v, cos, sin, cfg, probes, proj, q_gain, k_gain, eps, chunk=512):
    B, n, Hq, d = q.shape
    Hkv, G, Bk, S, W = k.shape[2], Hq // k.shape[2], cfg.block, cfg.sinks, cfg.window
    nb = n // Bk
    kk = min(cfg.k_blocks, nb)
    qc, kc, qr, kr, S0, qg, scale, _ = _prepare(q, k, cos, sin, cfg, probes, proj, q_gain, k_gain, eps,
                                                False)
    v = v.float()
    out = torch.empty(B, n, Hq, d)
    woff = torch.arange(-W + 1, 1)
    bix = torch.arange(B)[:, None, None]
    for g in range(Hkv):
        kn_g, kr_g, v_g = kc[:, :, g], kr[:, :, g], v[:, :, g]                 # [B, n, d]
        knb, vnb = kn_g.view(B, nb, Bk, d), v_g.view(B, nb, Bk, d)
        for cs in range(0, n, chunk):
            ce = min(n, cs + chunk)
            c = ce - cs
            i = torch.arange(cs, ce)
            cand = (torch.arange(nb)[None, :] >= 1) & ((torch.arange(nb)[None, :] + 1) * Bk <= i[:, None] - W + 1)
            bsc = torch.einsum("bcd,bnmd->bcnm", qg[:, g, cs:ce], S0[:, g]).amax(-1) * scale
            top = bsc.masked_fill(~cand[None], float("-inf")).topk(kk, dim=-1)
            rvalid = (~torch.isinf(top.values))[..., None].expand(B, c, kk, Bk).reshape(B, c, kk * Bk)
            rk = knb[bix, top.indices].reshape(B, c, kk * Bk, d)
            rv = vnb[bix, top.indices].reshape(B, c, kk * Bk, d)
            widx = i[:, None] + woff[None, :]
            wvalid = (widx >= S) & (widx <= i[:, None])
            wflat = widx.clamp(0, n - 1).reshape(-1)
            wk = kr_g[:, wflat].reshape(B, c, W, d)
            wv = v_g[:, wflat].reshape(B, c, W, d)
            svalid = torch.arange(S)[None, :] <= i[:, None]
            for hh in range(G):
                h = g * G + hh
                ssc = torch.einsum("bcd,bsd->bcs", qc[:, cs:ce, h], kn_g[:, :S]) * scale
                wsc = torch.einsum("bcd,bcwd->bcw", qr[:, cs:ce, h], wk) * scale
                rsc = torch.einsum("bcd,bcmd->bcm", qc[:, cs:ce, h], rk) * scale
                allsc = torch.cat([ssc.masked_fill(~svalid[None], float("-inf")),
                                   wsc.masked_fill(~wvalid[None], float("-inf")),
                                   rsc.masked_fill(~rvalid, float("-inf"))], dim=-1)
                wgt = allsc.softmax(-1)
                ws, ww, wr = wgt.split([S, W, kk * Bk], dim=-1)
                out[:, cs:ce, h] = (torch.einsum("bcs,bsd->bcd", ws, v_g[:, :S]) +
                                    torch.einsum("bcw,bcwd->bcd", ww, wv) +
                                    torch.einsum("bcm,bcmd->bcd", wr, rv))
    return out
