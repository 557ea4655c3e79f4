"""Drop-in attention functions with the reference's signatures, backed by the
HIP kernels (forward, and the backward through autograd).

  hba_attention_eval(q, k, v, cos, sin, cfg, summ, qkn, cap, hier=False, equiv=False)
      src/hba/attention.py:610-713 (equiv=True: :634-649)
  hba_attention_dense(q, k, v, cos, sin, cfg, summ, qkn, equiv=False) -> (out, aux)
      src/hba/attention.py:306-389 (equiv=True: :330-336)
  hba_attention_fused(q, k, v, cos, sin, cfg, summ, qkn) -> (out, aux)
      src/hba/attention.py:552-607 (the same math as dense)

Gradients: when grad mode is on and q, k, v or the QKNorm gains require grad,
the output carries an autograd node whose backward is the HIP backward
(ops.attn_bwd): dq, dk, dv and the gain gradients, the selection held fixed
(the reference routes on detached q/k, attention.py:288-303).  aux (the
summarizer's distillation loss, hba_aux_kl) has gradients into the
summarizer's probes and proj only.

Tensors: q [B, n, Hq, d], k, v [B, n, Hkv, d] (token-major views, last dim
contiguous), cos/sin fp32 [n, d] from rope_tables.  `cfg` is read duck-typed
(a reference HBAConfig works), `summ` must expose .probes [Hkv, m, d] and
.proj [Hkv, d, d], `qkn` .q.gain/.k.gain/.q.eps/.k.eps.  The output is a new
tensor of q's shape and dtype; inputs are not modified.  Errors follow the
reference: AssertionError for n % block != 0, ValueError for an unknown
content_scale_mode.  equiv=True is dense causal attention with RoPE on every
query and key; the kernels tile keys in 64s, so it raises ValueError for a
sequence length that is not a multiple of 64.
"""
import torch

from . import ops
from .config import route_scale, union_scale


def _qk(cfg, qkn):
    if getattr(cfg, "qknorm", False):
        return qkn.q.gain, qkn.k.gain, float(qkn.q.eps), float(qkn.k.eps)
    return None, None, 1e-6, 1e-6


def _tuned(q, k, cfg, summ, hier):
    """Whether the tuned kernels take this forward: 64-key blocks, head dim 64
    or 128, k <= 64, 1/2/4/8 slots; in bf16 also at most 16 query heads per KV
    head and S <= 128; hierarchical also beam <= 16, fanout <= 64, G <= 16."""
    B, n, Hq, dh = q.shape
    G = Hq // k.shape[2]
    kk = min(cfg.k_blocks, n // cfg.block)
    ok = cfg.block == ops.BLOCK and dh in (64, 128) and kk <= 64 and summ.probes.shape[1] in (1, 2, 4, 8)
    if q.dtype != torch.float32:
        ok = ok and G <= 16 and cfg.sinks <= 2 * ops.BLOCK
    if hier:
        ok = ok and G <= 16 and cfg.beam <= 16 and cfg.fanout <= 64
    return ok


def _hier_generic(qf, qg, qeps, S0, S1, cfg, kk, scale):
    """Hierarchical selection on the generic kernels (fp32): the routing
    queries (hba_route_queries), then hba_hier_select_rows per KV head with
    the routing candidate mask (attention.py:250-256), in chunks of rows that
    bound the mask.  Returns idx, val [B, Hkv, n, kk] (-1 / -inf past the
    picks) and cnt [B, Hkv, n]."""
    B, n, Hq, d = qf.shape
    Hkv, nb = S0.shape[1], S0.shape[2]
    ns = S1.shape[2]
    keff = min(kk, min(cfg.beam, ns) * cfg.fanout)
    dev = qf.device
    qn = ops.route_queries(qf, qg, qeps, Hkv)
    idx = torch.full((B, Hkv, n, kk), -1, dtype=torch.int32, device=dev)
    val = torch.full((B, Hkv, n, kk), float("-inf"), dtype=torch.float32, device=dev)
    blk = torch.arange(nb, device=dev)
    chunk = max(1, (1 << 26) // max(nb, 1))
    for i0 in range(0, n, chunk):
        i1 = min(n, i0 + chunk)
        i = torch.arange(i0, i1, device=dev)
        cand = (blk[None, :] >= 1) & ((blk[None, :] + 1) * cfg.block <= (i[:, None] - cfg.window + 1))
        for g in range(Hkv):
            ti, tv = ops.hier_select_rows(qn[:, i0:i1, g], S0[:, g], S1[:, g], cfg.fanout, cfg.beam, kk, cand,
                                          scale)
            idx[:, g, i0:i1, :keff] = ti.to(torch.int32)
            val[:, g, i0:i1, :keff] = tv
    cnt = torch.isfinite(val).sum(-1).to(torch.int32)
    return idx, val, cnt


def _forward_generic(q, k, v, cos, sin, cfg, summ, qkn, hier, dense_route):
    """forward_stages off the tuned geometry: every stage on the generic fp32
    kernels (bf16 inputs widened to fp32; the output back in q's dtype) --
    any block size, even head dim <= 256, k, slot count, group size, sink
    count, beam and fanout.  A correctness path, slower than the tuned one."""
    B, n, Hq, dh = q.shape
    qg, kg, qeps, keps = _qk(cfg, qkn)
    qf, kf, vf = q.float(), k.float(), v.float()
    scale = union_scale(cfg, dh, n)
    sel_scale = route_scale(cfg, dh) if dense_route else scale
    r = {"scale": scale, "sel_scale": sel_scale}
    r["kc"], r["kr"], r["vt"] = ops.prep_keys(kf, vf, kg, keps, cos, sin)
    kk = min(cfg.k_blocks, n // cfg.block)
    r["S0"] = ops.summarize(r["kc"], summ.probes, summ.proj, cfg.block)
    if hier:
        r["S1"] = ops.build_super(r["S0"], cfg.fanout)
        r["idx"], r["val"], r["cnt"] = _hier_generic(qf, qg, qeps, r["S0"], r["S1"], cfg, kk, sel_scale)
    else:
        r["idx"], r["val"], r["cnt"] = ops.score_select(qf, qg, qeps, r["S0"], cfg.window, kk, sel_scale,
                                                        cfg.block)
    out = ops.attn_fwd(qf, qg, kg, qeps, r["kc"], r["kr"], r["vt"], cos, sin, r["idx"], r["cnt"], cfg.sinks,
                       cfg.window, scale, cfg.block)
    r["out"] = out.to(q.dtype)
    return r


def forward_stages(q, k, v, cos, sin, cfg, summ, qkn, hier=False, dense_route=False, overlap=False):
    """The forward path stage by stage; returns a dict with every intermediate
    (kc, kr, vt, S0, [S1], idx, val, cnt, out) and the scales used.  Every
    stage runs in sequence on the current stream: the key preparation with
    the block summaries (one launch), the selection, the attention; the bf16 attention is one
    launch over the whole union.  overlap=True (bf16) instead runs the
    attention as two launches, the window on a second stream while the
    selection runs on this one, then the sinks and routed
    blocks merged into it by LSE (the same softmax, with the window rows
    rounded to bf16 once before the merge).  Geometry the tuned kernels do
    not take (_tuned) runs on the generic fp32 kernels (_forward_generic)."""
    B, n, Hq, dh = q.shape
    assert n % cfg.block == 0, (n, cfg.block)
    if not _tuned(q, k, cfg, summ, hier):
        return _forward_generic(q, k, v, cos, sin, cfg, summ, qkn, hier, dense_route)
    qg, kg, qeps, keps = _qk(cfg, qkn)
    scale = union_scale(cfg, dh, n)
    sel_scale = route_scale(cfg, dh) if dense_route else scale
    r = {"scale": scale, "sel_scale": sel_scale}
    # the keys' QKNorm / RoPE / V^T and the block summaries in one launch
    r["kc"], r["kr"], r["vt"], r["S0"] = ops.prep_keys_summarize(k, v, kg, keps, cos, sin, summ.probes,
                                                                 summ.proj)
    kk = min(cfg.k_blocks, n // cfg.block)
    # bf16, overlap: the window launch needs no selection, so it can run on a
    # second stream while the summaries and the selection run on this one
    split = overlap and q.dtype == torch.bfloat16
    if split:
        main = torch.cuda.current_stream(q.device)
        side = ops.side_stream(q.device)
        out, ws = ops.attn_buffers(q, k.shape[2])
        side.wait_stream(main)
        with torch.cuda.stream(side):
            ops.attn_window_(q, qg, kg, qeps, r["kr"], r["vt"], cos, sin, cfg.sinks, cfg.window, scale, out, ws)
        for t in (out, ws, r["kr"], r["vt"]):
            t.record_stream(side)
    if hier:
        r["S1"] = ops.build_super(r["S0"], cfg.fanout)
        r["idx"], r["val"], r["cnt"] = ops.hier_select(q, qg, qeps, r["S0"], r["S1"], cfg.window, kk,
                                                       cfg.fanout, cfg.beam, sel_scale)
    else:
        r["idx"], r["val"], r["cnt"] = ops.score_select(q, qg, qeps, r["S0"], cfg.window, kk, sel_scale,
                                                        cfg.block)
    if split:
        main.wait_stream(side)
        r["out"] = ops.attn_routed_(q, qg, kg, qeps, r["kc"], r["vt"], r["idx"], r["cnt"], cfg.sinks, scale,
                                    out, ws)
    else:
        r["out"] = ops.attn_fwd(q, qg, kg, qeps, r["kc"], r["kr"], r["vt"], cos, sin, r["idx"], r["cnt"],
                                cfg.sinks, cfg.window, scale, cfg.block)
    return r


class _Gains:
    """QKNorm stand-in (.q/.k with .gain and .eps) holding detached gains."""

    class _One:
        def __init__(self, gain, eps):
            self.gain, self.eps = gain, eps

    def __init__(self, qg, kg, qeps, keps):
        self.q, self.k = self._One(qg, qeps), self._One(kg, keps)


class _UnionAttention(torch.autograd.Function):
    """Forward: the HIP forward (forward_stages, or equiv_attention); backward:
    hba_attn_bwd on the saved inputs, prepared keys and selection."""

    @staticmethod
    def forward(ctx, q, k, v, q_gain, k_gain, cos, sin, cfg, summ, qeps, keps, mode):
        qkn = _Gains(None if q_gain is None else q_gain.detach(), None if k_gain is None else k_gain.detach(),
                     qeps, keps)
        B, n, Hq, dh = q.shape
        if mode == "equiv":
            out = equiv_attention(q, k, v, cos, sin, cfg, qkn)
            kc, kr, _ = ops.prep_keys(k, v, qkn.k.gain, keps, cos, sin)
            idx = torch.zeros(B, k.shape[2], n, 1, dtype=torch.int32, device=q.device)
            cnt = torch.zeros(B, k.shape[2], n, dtype=torch.int32, device=q.device)
            S, W = 0, n
        else:
            r = forward_stages(q, k, v, cos, sin, cfg, summ, qkn, hier=mode == "hier",
                               dense_route=mode == "dense")
            out, kc, kr, idx, cnt = r["out"], r["kc"], r["kr"], r["idx"], r["cnt"]
            S, W = cfg.sinks, cfg.window
        ctx.save_for_backward(q, k, v, q_gain, k_gain, cos, sin, kc, kr, idx, cnt, out)
        ctx.meta = (S, W, union_scale(cfg, dh, n), qeps, cfg.block if mode != "equiv" else ops.BLOCK)
        return out

    @staticmethod
    def backward(ctx, dout):
        q, k, v, q_gain, k_gain, cos, sin, kc, kr, idx, cnt, out = ctx.saved_tensors
        S, W, scale, eps, block = ctx.meta
        G = q.shape[2] // k.shape[2]
        # the bf16 kernels take 64-key blocks, head dims 64 / 128, S <= 64,
        # k <= 64 and G <= 16; elsewhere the fp32 kernels run on the widened
        # tensors (any geometry the forward takes) and the gradients are
        # rounded back
        wide = q.dtype != torch.float32 and (block != ops.BLOCK or q.shape[-1] not in (64, 128) or S > ops.BLOCK
                                             or idx.shape[3] > 64 or G > 16)
        if wide:
            f32 = [t.float() for t in (q, k, v, kc, kr, out, dout)]
            dq, dk, dv, dqg, dkg = ops.attn_bwd(f32[0], f32[1], f32[2], f32[3], f32[4], q_gain, k_gain, eps, cos,
                                                sin, idx, cnt, f32[5], f32[6].contiguous(), S, W, scale, block)
            dq, dk, dv = dq.to(q.dtype), dk.to(k.dtype), dv.to(v.dtype)
        else:
            dq, dk, dv, dqg, dkg = ops.attn_bwd(q, k, v, kc, kr, q_gain, k_gain, eps, cos, sin, idx, cnt, out,
                                                dout.contiguous(), S, W, scale, block)
        gq = dqg.to(q_gain.dtype) if q_gain is not None and ctx.needs_input_grad[3] else None
        gk = dkg.to(k_gain.dtype) if k_gain is not None and ctx.needs_input_grad[4] else None
        return dq, dk, dv, gq, gk, None, None, None, None, None, None, None


def _with_grad(q, k, v, cos, sin, cfg, summ, qkn, mode):
    """The output with an autograd node when anything upstream needs a
    gradient; None otherwise (the caller runs the plain forward)."""
    qg, kg, qeps, keps = _qk(cfg, qkn)
    if not torch.is_grad_enabled() or not any(t is not None and t.requires_grad for t in (q, k, v, qg, kg)):
        return None
    if qg is not None and qeps != keps:
        raise NotImplementedError("the backward takes one QKNorm eps for q and k")
    return _UnionAttention.apply(q, k, v, qg, kg, cos, sin, cfg, summ, qeps, keps, mode)


def equiv_attention(q, k, v, cos, sin, cfg, qkn):
    """Dense uniform-RoPE causal attention (the equiv=True branch,
    attention.py:330-336 and :634-649): the same QKNorm and union scale as the
    HBA path, RoPE on every query and key, every key j <= i attended.  It is
    the union kernel with no sinks, a window covering the whole sequence and
    no routed blocks (in bf16, the window launch alone)."""
    B, n, Hq, dh = q.shape
    Hkv = k.shape[2]
    if n % ops.BLOCK:
        raise ValueError(f"equiv attention needs a sequence length that is a multiple of {ops.BLOCK}, got {n}")
    qg, kg, qeps, keps = _qk(cfg, qkn)
    scale = union_scale(cfg, dh, n)
    kc, kr, vt = ops.prep_keys(k, v, kg, keps, cos, sin)
    if q.dtype == torch.bfloat16:
        out, ws = ops.attn_buffers(q, Hkv)
        return ops.attn_window_(q, qg, kg, qeps, kr, vt, cos, sin, 0, n, scale, out, ws)
    idx = torch.zeros(B, Hkv, n, 1, dtype=torch.int32, device=q.device)
    cnt = torch.zeros(B, Hkv, n, dtype=torch.int32, device=q.device)
    return ops.attn_fwd(q, qg, kg, qeps, kc, kr, vt, cos, sin, idx, cnt, 0, n, scale)


def hba_attention_eval(q, k, v, cos, sin, cfg, summ, qkn, cap=None, hier=False, equiv=False):
    """Gathered union attention with flat or hierarchical selection; `cap`
    (the reference's memory cap for its chunk loop) is accepted and unused.
    equiv=True: dense uniform-RoPE causal attention (equiv_attention)."""
    mode = "equiv" if equiv else ("hier" if hier else "eval")
    out = _with_grad(q, k, v, cos, sin, cfg, summ, qkn, mode)
    if out is not None:
        return out
    if equiv:
        return equiv_attention(q, k, v, cos, sin, cfg, qkn)
    return forward_stages(q, k, v, cos, sin, cfg, summ, qkn, hier=hier)["out"]


class _AuxKL(torch.autograd.Function):
    """The summarizer auxiliary loss as an autograd node whose only inputs
    with a gradient are the summarizer's probes and proj (the routing and the
    teacher run on detached q/k: attention.py:288-303, 372-381).  The HIP
    entry point returns the loss and its gradient in one call; backward
    scales the saved gradient."""

    @staticmethod
    def forward(ctx, probes, proj, q, k, v, q_gain, k_gain, cos, sin, cfg, qeps, keps, want):
        B, n, Hq, dh = q.shape
        # the bf16 kernels take 64-key blocks, head dims 64 / 128, at most 8
        # slots and 16 query heads per KV head; elsewhere the fp32 kernels run
        # on the widened inputs
        tuned = (cfg.block == ops.BLOCK and dh in (64, 128) and probes.shape[1] <= 8
                 and Hq // k.shape[2] <= 16)
        if q.dtype != torch.float32 and not tuned:
            q, k, v = q.float(), k.float(), v.float()
        kc, _, _ = ops.prep_keys(k, v, k_gain, keps, cos, sin)
        S0 = ops.summarize(kc, probes.detach(), proj.detach(), cfg.block)
        aux, dpr, dpj = ops.aux_kl(q, q_gain, k_gain, qeps, kc, S0, probes.detach(), proj.detach(), cfg.window,
                                   union_scale(cfg, dh, n), route_scale(cfg, dh), want, cfg.block)
        ctx.save_for_backward(dpr, dpj)
        ctx.dtypes = (probes.dtype, proj.dtype)
        return aux

    @staticmethod
    def backward(ctx, g):
        dpr, dpj = ctx.saved_tensors
        gpr = (g * dpr).to(ctx.dtypes[0]) if dpr is not None and ctx.needs_input_grad[0] else None
        gpj = (g * dpj).to(ctx.dtypes[1]) if dpj is not None and ctx.needs_input_grad[1] else None
        return gpr, gpj, None, None, None, None, None, None, None, None, None, None, None


def aux_kl(q, k, v, cos, sin, cfg, summ, qkn):
    """The aux-KL of the training paths (attention.py:366-389, 509-549): the
    teacher p* (group-averaged content mass of the candidate blocks) against
    log softmax of the summarizer's block scores, a 0-d fp32 tensor whose
    gradient reaches only summ.probes and summ.proj."""
    qg, kg, qeps, keps = _qk(cfg, qkn)
    qg = None if qg is None else qg.detach()
    kg = None if kg is None else kg.detach()
    probes, proj = summ.probes, summ.proj
    want = torch.is_grad_enabled() and (probes.requires_grad or proj.requires_grad)
    return _AuxKL.apply(probes, proj, q.detach(), k.detach(), v.detach(), qg, kg, cos, sin, cfg, qeps, keps, want)


def hba_attention_dense(q, k, v, cos, sin, cfg, summ, qkn, equiv=False):
    """The reference's naive training path: selection with route_topk's
    scale (no temperature), attention with the union scale, and the aux-KL
    (aux_kl) unless cfg.aux_w == 0 (then a zero, as the reference skips its
    teacher, attention.py:363-364).  equiv=True: dense uniform-RoPE causal
    attention (equiv_attention) and aux = 0."""
    out = _with_grad(q, k, v, cos, sin, cfg, summ, qkn, "equiv" if equiv else "dense")
    if out is None:
        if equiv:
            out = equiv_attention(q, k, v, cos, sin, cfg, qkn)
        else:
            out = forward_stages(q, k, v, cos, sin, cfg, summ, qkn, dense_route=True)["out"]
    if equiv or getattr(cfg, "aux_w", 1.0) == 0.0:
        return out, q.new_zeros(())
    return out, aux_kl(q, k, v, cos, sin, cfg, summ, qkn)


def hba_attention_fused(q, k, v, cos, sin, cfg, summ, qkn):
    """The reference's fused training path (the same math as dense: outputs
    agree to rounding, and its chunked teacher gives the same aux)."""
    return hba_attention_dense(q, k, v, cos, sin, cfg, summ, qkn)


def build_super(S0, fanout):
    """attention.py:202-214 for summaries [B, Hkv, nb, m, d] (or [B, nb, m, d]):
    returns (S1, ns) like the reference."""
    squeeze = S0.dim() == 4
    S = S0.unsqueeze(1) if squeeze else S0
    S1 = ops.build_super(S, fanout)
    return (S1.squeeze(1) if squeeze else S1), S1.shape[2]


def grouped_query(qc, cfg):
    """summarizer.py:50-54: the routing query of each KV group, the sum of its
    heads' content queries qc [B, n, Hq, dh] (already QKNorm'd, as the
    reference's callers pass them) in the declared order and qc's storage
    rounding -> [B, Hkv, n, dh]."""
    return ops.route_queries(qc, None, 1e-6, cfg.n_kv).transpose(1, 2)


def hier_select(qn, S0, S1, fanout, beam, kk, cand, scale):
    """attention.py:217-246 with the reference's signature: qn [B, c, dh],
    S0 [B, nb, m, dh], S1 [B, ns, m, dh], cand bool [c, nb].  Returns
    (top_idx [B, c, kk_eff], top_val [B, c, kk_eff], n_comparisons) with
    kk_eff = min(kk, min(beam, ns) * fanout); a pick is valid iff top_val is
    finite (the reference's rule), and an invalid one has index -1.  Scores
    are fp32 (declared order) for fp32 and bf16 inputs alike; ties go to the
    lowest block index."""
    ns = S1.shape[1]
    idx, val = ops.hier_select_rows(qn, S0, S1, int(fanout), int(beam), int(kk), cand, float(scale))
    return idx, val, ns + min(beam, ns) * fanout


def selected_mask(idx, cnt, nb):
    """Boolean selection mask [B, Hkv, n, nb] (route_topk's `sel`) from idx/cnt."""
    B, Hkv, n, kk = idx.shape
    valid = torch.arange(kk, device=idx.device)[None, None, None, :] < cnt[..., None]
    sel = torch.zeros(B, Hkv, n, nb + 1, dtype=torch.bool, device=idx.device)
    sel.scatter_(-1, torch.where(valid, idx.long(), nb), True)
    return sel[..., :nb]
