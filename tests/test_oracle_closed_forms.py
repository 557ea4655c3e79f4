"""The oracle against closed forms, invariants and brute force (CPU only).

Closed forms come from the reference's own tests (tests/test_qknorm.py:67-177)
and published analytic numbers (docs/design.md:79,113; evals.py:319-322).
Brute force = plain Python loops written from the text of the rules in
attention.py, on tiny inputs.  The planted-mistake tests mutate the ORACLE
(never a kernel) and require that some check here catches the mutation."""
import math

import numpy as np
import pytest

import oracle.hba_oracle as O

RS = np.random.RandomState


def tiny_cfg(**kw):
    base = dict(n_heads=4, n_kv=2, head_dim=8, block=16, window=64, sinks=2, k_blocks=4,
                slots=2, fanout=4, beam=2, native_ctx=8192)
    base.update(kw)
    return O.Cfg(**base)


# ----------------------------------------------------------- QKNorm / scale ---
def test_qknorm_rms_equals_gain():
    """tests/test_qknorm.py:67-78"""
    rs = RS(0)
    gain = rs.uniform(0.3, 2.0, 4).astype(np.float32)
    x = (rs.standard_normal((3, 17, 4, 8)) * 5.0 + 2.0).astype(np.float32)
    xn = O.qknorm(x, gain, 1e-6, "f32")
    rms = np.sqrt((xn.astype(np.float64) ** 2).mean(-1))
    assert np.abs(rms - gain[None, None]).max() <= 1e-5


@pytest.mark.parametrize("mag", [1.0, 1e3, 1e6])
def test_content_logit_bounded_by_gain_product(mag):
    """tests/test_qknorm.py:81-99"""
    rs = RS(1)
    cfg = tiny_cfg(qknorm=True, content_scale_mode="inv_d")
    gq, gk = 0.8, 1.3
    q = (rs.standard_normal((5, 4, 8)) * mag).astype(np.float32)
    k = (rs.standard_normal((9, 2, 8)) * mag).astype(np.float32)
    qc = O.qknorm(q, np.full(4, gq, np.float32), 1e-6, "f32").astype(np.float64)
    kc = O.qknorm(k, np.full(2, gk, np.float32), 1e-6, "f32").astype(np.float64)
    logit = np.einsum("ihd,jhd->hij", qc, np.repeat(kc, 2, axis=1)) * O.content_scale(cfg, 8)
    assert np.abs(logit).max() <= gq * gk * (1 + 1e-4)


def test_qknorm_off_is_passthrough_with_legacy_scale():
    """tests/test_qknorm.py:102-111"""
    cfg = tiny_cfg(qknorm=False)
    q = RS(2).standard_normal((5, 4, 8)).astype(np.float32)
    k = RS(3).standard_normal((5, 2, 8)).astype(np.float32)
    qc, kc, scale = O.content_qk(q, k, cfg, None, None, 1e-6, 5, "f32")
    assert np.array_equal(qc, q) and np.array_equal(kc, k)
    assert scale == 8 ** -0.5


def test_content_scale_modes():
    """tests/test_qknorm.py:115-119"""
    assert O.content_scale(tiny_cfg(content_scale_mode="inv_d"), 64) == pytest.approx(1 / 64)
    assert O.content_scale(tiny_cfg(content_scale_mode="inv_sqrt_d"), 64) == pytest.approx(0.125)
    with pytest.raises(ValueError):
        O.content_scale(tiny_cfg(content_scale_mode="bogus"), 64)


def test_log_len_tau_closed_forms():
    """tests/test_qknorm.py:123-177"""
    cfg = tiny_cfg(temp_c=0.1, n_cal=32768)
    assert O.log_len_tau(cfg, 1) == 1.0 and O.log_len_tau(cfg, 4096) == 1.0
    assert O.log_len_tau(cfg, 32768) == 1.0
    assert O.log_len_tau(cfg, 65536) == pytest.approx(1 + 0.1 * math.log(2.0))
    base = O.content_scale(cfg, 8)
    assert O.union_scale(tiny_cfg(qknorm=True, temp_c=0.1, n_cal=32768), 8, 131072) == \
        pytest.approx(base * (1 + 0.1 * math.log(4.0)))
    assert O.log_len_tau(tiny_cfg(temp_c=0.0, n_cal=1), 10 ** 9) == 1.0
    cfg2 = tiny_cfg(temp_c=0.1, n_cal=None, native_ctx=8192)
    assert O.log_len_tau(cfg2, 8192) == 1.0
    assert O.log_len_tau(cfg2, 16384) == pytest.approx(1 + 0.1 * math.log(2.0))
    # gated under qknorm=False
    assert O.union_scale(tiny_cfg(qknorm=False, temp_c=0.5, n_cal=4), 8, 4096) == 8 ** -0.5
    # the benchmark shapes (n_cal = native_ctx = 32768)
    big = O.Cfg()
    assert O.log_len_tau(big, 131072) == pytest.approx(1.138629, abs=1e-6)
    assert O.log_len_tau(big, 65536) == pytest.approx(1.069315, abs=1e-6)


# ------------------------------------------------------------- RoPE ----------
def brute_rope(x, pos, theta):
    """NeoX rotate-half written out: pairs (t, t+d/2) rotated by pos*theta^(-2t/d)."""
    d = x.shape[-1]
    h = d // 2
    out = np.zeros_like(x, dtype=np.float64)
    for t in range(h):
        ang = pos * theta ** (-(2.0 * t) / d)
        c, s = math.cos(ang), math.sin(ang)
        out[..., t] = x[..., t] * c - x[..., t + h] * s
        out[..., t + h] = x[..., t + h] * c + x[..., t] * s
    return out


def _rope_vs_brute():
    rs = RS(4)
    n, d = 40, 8
    x = rs.standard_normal((n, 3, d)).astype(np.float32)
    cos, sin = O.rope_tables(n, d, 1e4)
    y = O.apply_rope(x, cos, sin, "f32")
    worst = max(float(np.abs(y[i] - brute_rope(x[i].astype(np.float64), i, 1e4)).max()) / (1 + i)
                for i in range(n))
    return worst, x, y


def test_rope_matches_rotation_brute_force():
    worst, x, y = _rope_vs_brute()
    assert worst <= 2e-5
    # position 0 is the identity; rotation preserves the norm
    assert np.array_equal(y[0], x[0])
    assert np.allclose(np.linalg.norm(y, axis=-1), np.linalg.norm(x, axis=-1), rtol=1e-5)


# --------------------------------------------------------- routing regions ---
def test_candidate_counts_and_keys_per_query_closed_forms():
    """ncand(n-1) = 495 / 1007 / 2031 (evals.py:302-305 with the default knobs);
    S + W + k*B = 2052 keys for deep queries (docs/design.md:113)."""
    Bk, W, S, k = 64, 1024, 4, 16
    assert [O.ncand(n - 1, Bk, W) for n in (32768, 65536, 131072)] == [495, 1007, 2031]
    i = 32767
    keys = min(S, i + 1) + (i - max(S, i - W + 1) + 1) + min(k, O.ncand(i, Bk, W)) * Bk
    assert keys == 2052
    # the candidate rule against its mask form on a grid
    n, nb = 4096, 64
    cm = O.route_candidates(n, W, nb, Bk)
    for i in range(0, n, 7):
        assert cm[i].sum() == O.ncand(i, Bk, W)
        if cm[i].any():
            assert np.nonzero(cm[i])[0].max() == O.cand_bmax(i, Bk, W)


def test_regions_disjoint_and_cover_union():
    n, S, W, Bk = 512, 2, 64, 16
    ms, mw, cand = O.causal_bucket_masks(n, S, W, n // Bk, Bk)
    rout = np.repeat(cand, Bk, axis=1)
    assert not (ms & mw).any() and not (ms & rout).any() and not (mw & rout).any()
    # routed keys lie strictly before the window start, and never in block 0
    for i in range(n):
        js = np.nonzero(rout[i])[0]
        if js.size:
            assert js.max() < i - W + 1 and js.min() >= Bk


@pytest.mark.parametrize("n,speed", [(32768, 5.2), (65536, 7.9), (131072, 10.6)])
def test_hierarchy_comparison_counts(n, speed):
    """docs/design.md:79: 5.2x / 7.9x / 10.6x (F=16, beam 4)."""
    comps = O.hier_comparisons(n, 64, 16, 4)
    assert round(O.ncand(n - 1, 64, 1024) / comps, 1) == speed


def test_hierarchy_comparisons_beam8_at_128k():
    assert O.hier_comparisons(131072, 64, 16, 8) == 256
    assert round(2031 / 256, 2) == 7.93


# -------------------------------------------------------------- brute force --
def brute_select(qg, S0, scale, kk, Bk, W, i):
    """Top-k from the text of the rule: candidates b>=1, (b+1)*Bk <= i-W+1;
    score = max over slots of q.s times scale; order (score desc, index asc)."""
    nb = S0.shape[0]
    cands = [b for b in range(nb) if b >= 1 and (b + 1) * Bk <= i - W + 1]
    sc = []
    for b in cands:
        best = -math.inf
        for s in range(S0.shape[1]):
            best = max(best, sum(float(qg[t]) * float(S0[b, s, t]) for t in range(qg.size)))
        sc.append((-best * scale, b))
    sc.sort()
    return [b for _, b in sc[:kk]]


def brute_attention_row(qc, qr, kc, kr, v, sel, scale, S, W, Bk, i, h, G):
    g = h // G
    logits, vals = [], []
    for j in range(i + 1):
        in_sink = j < S
        in_win = (j >= S) and (j > i - W)
        in_rout = (j // Bk) in sel
        if in_win:
            logits.append(float(np.dot(qr[i, h].astype(np.float64), kr[j, g])) * scale)
        elif in_sink or in_rout:
            logits.append(float(np.dot(qc[i, h].astype(np.float64), kc[j, g])) * scale)
        else:
            continue
        vals.append(v[j, g].astype(np.float64))
    mx = max(logits)
    w = [math.exp(x - mx) for x in logits]
    tot = sum(w)
    return sum(wi * vi for wi, vi in zip(w, vals)) / tot


def _tiny_problem(seed=5, n=192, qknorm=True):
    cfg = tiny_cfg(qknorm=qknorm, temp_c=0.1, n_cal=64)
    rs = RS(seed)
    q = rs.standard_normal((1, n, 4, 8)).astype(np.float32)
    k = rs.standard_normal((1, n, 2, 8)).astype(np.float32)
    v = rs.standard_normal((1, n, 2, 8)).astype(np.float32)
    pr, pj = O.init_summarizer(2, 2, 8, seed=seed)
    qg = rs.uniform(0.5, 2.0, 4).astype(np.float32)
    kg = rs.uniform(0.5, 2.0, 2).astype(np.float32)
    cos, sin = O.rope_tables(n, 8, 1e6)
    return cfg, q, k, v, pr, pj, qg, kg, cos, sin


def brute_summarize(kc, probes, proj, Bk):
    n, Hkv, d = kc.shape
    nb = n // Bk
    m = probes.shape[1]
    out = np.zeros((Hkv, nb, m, d))
    for h in range(Hkv):
        for c in range(nb):
            kb = kc[c * Bk:(c + 1) * Bk, h].astype(np.float64)
            for s in range(m):
                lg = [float(np.dot(probes[h, s], kb[t])) / math.sqrt(d) for t in range(Bk)]
                mx = max(lg)
                w = [math.exp(x - mx) for x in lg]
                pooled = sum(wi * kb[t] for t, wi in enumerate(w)) / sum(w)
                out[h, c, s] = [sum(pooled[a] * float(proj[h, a, e]) for a in range(d))
                                for e in range(d)]
    return out


def test_summarize_brute_force():
    cfg, q, k, v, pr, pj, qg, kg, cos, sin = _tiny_problem()
    kc = O.qknorm(k[0], kg, 1e-6, "f32")
    assert np.abs(O.summarize(kc, pr, pj, 16) - brute_summarize(kc, pr, pj, 16)).max() < 1e-9


def test_summarize_identity_proj_uniform_probes_is_block_mean():
    kc = RS(6).standard_normal((64, 2, 8)).astype(np.float32)
    S = O.summarize(kc, np.zeros((2, 3, 8), np.float32), np.stack([np.eye(8)] * 2), 16)
    mean = kc.astype(np.float64).reshape(4, 16, 2, 8).mean(1).transpose(1, 0, 2)
    assert np.abs(S - mean[:, :, None, :]).max() < 1e-12


@pytest.mark.parametrize("qknorm", [True, False])
def test_eval_forward_brute_force(qknorm):
    cfg, q, k, v, pr, pj, qg, kg, cos, sin = _tiny_problem(qknorm=qknorm)
    n = q.shape[1]
    rows = [0, 1, 2, 63, 64, 95, 96, 127, 150, 191]
    out, sels = O.forward_eval(q, k, v, cos, sin, cfg, pr, pj, qg, kg, 1e-6, "f32", rows=rows)
    P = O.prepare(q[0], k[0], v[0], cos, sin, cfg, pr, pj, qg, kg, 1e-6, "f32")
    idx, val, cnt = sels[0]
    for r, i in enumerate(rows):
        for g in range(2):
            sel = brute_select(P.qg[g, i], P.S0[g], P.sel_scale, min(cfg.k_blocks, n // 16), 16,
                               cfg.window, i)
            assert list(idx[g, r, : cnt[g, r]]) == sel
        for h in range(4):
            ref = brute_attention_row(P.qc, P.qr, P.kc, P.kr, P.v, set(idx[h // 2, r, :cnt[h // 2, r]]),
                                      P.scale, cfg.sinks, cfg.window, 16, i, h, 2)
            assert np.abs(out[0, r, h] - ref).max() < 1e-12


def test_select_all_eval_equals_dense_and_masked_full_attention():
    """gates.py:193-197,211: with k_blocks >= nb every candidate is selected,
    so the gathered path, the masked dense path and brute-force causal
    attention over sinks|window|all-candidates coincide."""
    cfg, q, k, v, pr, pj, qg, kg, cos, sin = _tiny_problem(n=256)
    cfg.k_blocks = 256 // 16
    rows = np.arange(0, 256, 5)
    oe, _ = O.forward_eval(q, k, v, cos, sin, cfg, pr, pj, qg, kg, 1e-6, "f32", rows=rows)
    od, _ = O.forward_dense(q, k, v, cos, sin, cfg, pr, pj, qg, kg, 1e-6, "f32", rows=rows)
    assert np.abs(oe - od).max() < 1e-12
    P = O.prepare(q[0], k[0], v[0], cos, sin, cfg, pr, pj, qg, kg, 1e-6, "f32")
    for r, i in enumerate(rows[::7]):
        allc = set(range(1, max(0, O.cand_bmax(int(i), 16, cfg.window)) + 1))
        ref = brute_attention_row(P.qc, P.qr, P.kc, P.kr, P.v, allc, P.scale, cfg.sinks,
                                  cfg.window, 16, int(i), 3, 2)
        assert np.abs(oe[0, list(rows).index(i), 3] - ref).max() < 1e-12


def test_hier_equals_flat_when_beam_covers_all_supers():
    cfg, q, k, v, pr, pj, qg, kg, cos, sin = _tiny_problem(n=256)
    cfg.beam = 64
    rows = np.arange(256)
    of, sf = O.forward_eval(q, k, v, cos, sin, cfg, pr, pj, qg, kg, 1e-6, "f32", rows=rows)
    oh, sh = O.forward_eval(q, k, v, cos, sin, cfg, pr, pj, qg, kg, 1e-6, "f32", rows=rows,
                            hier=True)
    assert np.array_equal(sf[0][0], sh[0][0]) and np.array_equal(sf[0][2], sh[0][2])
    assert np.abs(of - oh).max() == 0.0


def test_causality_future_tokens_do_not_change_past_rows():
    """gates.py:101-126"""
    cfg, q, k, v, pr, pj, qg, kg, cos, sin = _tiny_problem(n=256)
    t = 150
    q2, k2, v2 = q.copy(), k.copy(), v.copy()
    rs = RS(9)
    q2[:, t + 1:] = rs.standard_normal(q2[:, t + 1:].shape)
    k2[:, t + 1:] = rs.standard_normal(k2[:, t + 1:].shape)
    v2[:, t + 1:] = rs.standard_normal(v2[:, t + 1:].shape)
    rows = np.arange(0, t + 1)
    o1, _ = O.forward_eval(q, k, v, cos, sin, cfg, pr, pj, qg, kg, 1e-6, "f32", rows=rows)
    o2, _ = O.forward_eval(q2, k2, v2, cos, sin, cfg, pr, pj, qg, kg, 1e-6, "f32", rows=rows)
    assert np.abs(o1 - o2).max() == 0.0


def test_lse_merge_identity():
    """attention.py:559-561: the union softmax equals the LSE merge of region A
    (sinks + routed, NoPE) and region B (window, RoPE)."""
    rs = RS(10)
    sa, sb = rs.standard_normal(37) * 3, rs.standard_normal(21) * 3
    va, vb = rs.standard_normal((37, 5)), rs.standard_normal((21, 5))
    s = np.concatenate([sa, sb])
    p = np.exp(s - s.max())
    full = (p / p.sum()) @ np.concatenate([va, vb])
    lse = lambda x: x.max() + math.log(np.exp(x - x.max()).sum())
    oa = np.exp(sa - lse(sa)) @ va
    ob = np.exp(sb - lse(sb)) @ vb
    la, lb = lse(sa), lse(sb)
    m = max(la, lb)
    merged = (math.exp(la - m) * oa + math.exp(lb - m) * ob) / (math.exp(la - m) + math.exp(lb - m))
    assert np.abs(full - merged).max() < 1e-12


def test_decode_row_equals_prefill_last_row():
    cfg, q, k, v, pr, pj, qg, kg, cos, sin = _tiny_problem(n=192)
    P = O.prepare(q[0], k[0], v[0], cos, sin, cfg, pr, pj, qg, kg, 1e-6, "f32")
    for L in (150, 160, 192):
        out, (idx, val, cnt) = O.decode_row(q[0, L - 1], P.kc[:L], P.v[:L], cos, sin, cfg,
                                            P.S0[:, : L // 16], qg, 1e-6, "f32", P.scale)
        ref, sels = O.forward_eval(q, k, v, cos, sin, cfg, pr, pj, qg, kg, 1e-6, "f32",
                                   rows=[L - 1], S0=P.S0[None])
        assert np.abs(out - ref[0, 0]).max() < 1e-12


# ---------------------------------------------------------- planted mistakes --
def _eval_vs_brute(cfg, q, k, v, pr, pj, qg, kg, cos, sin, rows):
    out, sels = O.forward_eval(q, k, v, cos, sin, cfg, pr, pj, qg, kg, 1e-6, "f32", rows=rows)
    P = O.prepare(q[0], k[0], v[0], cos, sin, cfg, pr, pj, qg, kg, 1e-6, "f32")
    worst = 0.0
    for r, i in enumerate(rows):
        sel = set(brute_select(P.qg[0, i], P.S0[0], P.sel_scale, cfg.k_blocks, 16, cfg.window, i))
        for h in range(2):
            ref = brute_attention_row(P.qc, P.qr, P.kc, P.kr, P.v, sel, P.scale, cfg.sinks,
                                      cfg.window, 16, i, h, 2)
            worst = max(worst, float(np.abs(out[0, r, h] - ref).max()))
    return worst


def test_equiv_rows_match_library_sdpa_and_union_limit():
    """equiv=True (attention.py:330-336, 634-649) is causal attention over the
    rotated q and k.  Checked against torch's scaled_dot_product_attention
    (float64, causal, GQA heads expanded) and against the union rows with no
    sinks, a whole-sequence window and no routed blocks."""
    import torch
    import torch.nn.functional as F
    rs = RS(11)
    n, Hq, Hkv, d = 96, 6, 2, 16
    G = Hq // Hkv
    qr = rs.standard_normal((n, Hq, d)).astype(np.float32)
    kr = rs.standard_normal((n, Hkv, d)).astype(np.float32)
    v = rs.standard_normal((n, Hkv, d)).astype(np.float32)
    scale = 0.31
    rows = np.arange(n)
    got = O.equiv_rows(qr, kr, v, scale, rows)
    Q = torch.from_numpy(qr).double().permute(1, 0, 2)[None]
    K = torch.from_numpy(kr).double().permute(1, 0, 2).repeat_interleave(G, 0)[None]
    V = torch.from_numpy(v).double().permute(1, 0, 2).repeat_interleave(G, 0)[None]
    ref = F.scaled_dot_product_attention(Q, K, V, is_causal=True, scale=scale)[0].permute(1, 0, 2).numpy()
    assert np.abs(got - ref).max() < 1e-12
    idx = np.full((Hkv, n, 1), -1, dtype=np.int32)
    cnt = np.zeros((Hkv, n), dtype=np.int32)
    union = O.attn_rows(qr, qr, kr, kr, v, idx, cnt, scale, 0, n, 16, rows)
    assert np.abs(got - union).max() < 1e-12
    # a dropped causal mask (every key attended) is caught by the library check
    full = F.scaled_dot_product_attention(Q, K, V, is_causal=False, scale=scale)[0].permute(1, 0, 2).numpy()
    assert np.abs(got - full).max() > 1e-3


def test_forward_equiv_applies_qknorm_rope_and_scale():
    """forward_equiv = content_qk (QKNorm, union scale) + RoPE on q and k +
    equiv_rows; without QKNorm the scale is d**-0.5 and q, k pass through."""
    rs = RS(12)
    n, Hq, Hkv, d = 64, 4, 2, 8
    cfg = tiny_cfg(head_dim=d)
    q = rs.standard_normal((1, n, Hq, d)).astype(np.float32)
    k = rs.standard_normal((1, n, Hkv, d)).astype(np.float32)
    v = rs.standard_normal((1, n, Hkv, d)).astype(np.float32)
    cos, sin = O.rope_tables(n, d, 1e6)
    gq = rs.uniform(0.5, 2.0, Hq).astype(np.float32)
    gk = rs.uniform(0.5, 2.0, Hkv).astype(np.float32)
    rows = np.array([0, 5, 31, 63])
    for qk in (True, False):
        cfg.qknorm = qk
        got = O.forward_equiv(q, k, v, cos, sin, cfg, gq, gk, 1e-6, "f32", rows)[0]
        qc = O.qknorm(q[0], gq, 1e-6, "f32") if qk else q[0]
        kc = O.qknorm(k[0], gk, 1e-6, "f32") if qk else k[0]
        scale = O.union_scale(cfg, d, n) if qk else d ** -0.5
        want = O.equiv_rows(O.apply_rope(qc, cos, sin, "f32"), O.apply_rope(kc, cos, sin, "f32"), v[0],
                            scale, rows)
        assert np.abs(got - want).max() < 1e-12


def _torch_union_forward(q, k, v, cos, sin, scale, gq, gk, eps, idx, cnt, S, W, Bk, qknorm):
    """hba_attention_dense's masked dense union softmax (attention.py:306-356)
    in torch float64 with a given selection, for autograd."""
    import torch
    n, Hq, d = q.shape
    Hkv = k.shape[1]
    G = Hq // Hkv

    def norm(x, g):
        return x / (x * x).mean(-1, keepdim=True).clamp_min(eps).sqrt() * g[None, :, None]

    def rope(x):
        c, s = cos[:n, None, :], sin[:n, None, :]
        return x * c + torch.cat([-x[..., d // 2:], x[..., : d // 2]], -1) * s

    qc, kc = (norm(q, gq), norm(k, gk)) if qknorm else (q, k)
    qr, kr = rope(qc), rope(kc)
    i = torch.arange(n)[:, None]
    j = torch.arange(n)[None, :]
    sink = (j < S) & (j <= i)
    win = (j >= S) & (j <= i) & (j > i - W)
    outs = []
    for h in range(Hq):
        g = h // G
        rout = torch.zeros(n, n, dtype=torch.bool)
        for ii in range(n):
            for b in idx[g, ii, : cnt[g, ii]]:
                if 1 <= b < n // Bk:
                    rout[ii, b * Bk:(b + 1) * Bk] = True
        sN = qc[:, h] @ kc[:, g].T * scale
        sR = qr[:, h] @ kr[:, g].T * scale
        sc = torch.where(win, sR, sN).masked_fill(~(sink | win | rout), float("-inf"))
        outs.append(sc.softmax(-1) @ v[:, g])
    return torch.stack(outs, 1)


@pytest.mark.parametrize("qknorm,S", [(True, 2), (False, 2), (True, 20)])
def test_union_backward_matches_torch_autograd(qknorm, S):
    """The oracle backward against torch autograd (float64) of the masked
    dense union softmax through QKNorm and RoPE, on a selection with routed
    blocks, sinks and a window; S = 20 > Bk: routed block 1 holds sink keys,
    which the union counts once."""
    import torch
    rs = RS(21)
    n, Hq, Hkv, d, Bk, W, kk = 128, 4, 2, 8, 16, 32, 3
    q = rs.standard_normal((n, Hq, d)) * 1.5
    k = rs.standard_normal((n, Hkv, d)) * 1.5
    v = rs.standard_normal((n, Hkv, d))
    dout = rs.standard_normal((n, Hq, d))
    gq = rs.uniform(0.5, 2.0, Hq)
    gk = rs.uniform(0.5, 2.0, Hkv)
    cos, sin = O.rope_tables(n, d, 1e4)
    idx = np.full((Hkv, n, kk), -1, dtype=np.int32)
    cnt = np.zeros((Hkv, n), dtype=np.int32)
    for g in range(Hkv):
        for i in range(n):
            bm = O.cand_bmax(i, Bk, W)
            if bm >= 1:
                picks = rs.permutation(np.arange(1, bm + 1))[:kk]
                idx[g, i, : len(picks)] = picks
                cnt[g, i] = len(picks)
    assert cnt.max() == kk
    scale = 0.3
    got = O.union_backward(q, k, v, cos, sin, scale, gq, gk, 1e-6, idx, cnt, dout, S, W, Bk, qknorm)
    T = [torch.tensor(a, dtype=torch.float64, requires_grad=True) for a in (q, k, v, gq, gk)]
    out = _torch_union_forward(*T[:3], torch.tensor(cos, dtype=torch.float64),
                               torch.tensor(sin, dtype=torch.float64), scale, T[3], T[4], 1e-6, idx, cnt, S, W,
                               Bk, qknorm)
    out.backward(torch.tensor(dout))
    for a, t in zip(got, T):
        ref = t.grad.numpy() if t.grad is not None else np.zeros(t.shape)
        assert np.abs(a - ref).max() <= 1e-9 * max(1.0, np.abs(ref).max())


def test_planted_mistakes_are_caught(monkeypatch):
    cfg, q, k, v, pr, pj, qg, kg, cos, sin = _tiny_problem(n=192)
    rows = [1, 40, 100, 150, 191]
    assert _eval_vs_brute(cfg, q, k, v, pr, pj, qg, kg, cos, sin, rows) < 1e-12
    caught = {}
    # (a) rotate-half with the wrong sign
    with monkeypatch.context() as mp:
        mp.setattr(O, "rot_half", lambda x: np.concatenate([x[..., x.shape[-1] // 2:],
                                                            -x[..., :x.shape[-1] // 2]], -1))
        caught["rot_sign"] = _rope_vs_brute()[0] > 1e-3
    # (b) window one token short at its start
    orig_attn = O.attn_rows
    with monkeypatch.context() as mp:
        mp.setattr(O, "attn_rows", lambda *a: orig_attn(*a[:9], a[9] - 1, *a[10:]))
        caught["window_off_by_one"] = _eval_vs_brute(cfg, q, k, v, pr, pj, qg, kg, cos, sin,
                                                     rows) > 1e-6
    # (c) candidate rule one block too late (W passed one short)
    orig_flat = O.flat_select
    with monkeypatch.context() as mp:
        mp.setattr(O, "flat_select", lambda qg_, S0, sc, kk, Bk, W, pos=None:
                   orig_flat(qg_, S0, sc, kk, Bk, W - 16, pos))
        caught["cand_rule"] = _eval_vs_brute(cfg, q, k, v, pr, pj, qg, kg, cos, sin, rows) > 1e-6
    # (d) summarizer projection transposed
    kc = O.qknorm(k[0], kg, 1e-6, "f32")
    caught["proj_T"] = np.abs(O.summarize(kc, pr, pj.transpose(0, 2, 1), 16)
                              - brute_summarize(kc, pr, pj, 16)).max() > 1e-6
    # (e) dropped temperature in the union scale
    cfg_t = tiny_cfg(qknorm=True, temp_c=0.1, n_cal=32768)
    caught["tau_dropped"] = O.union_scale(cfg_t, 8, 131072) != pytest.approx(
        O.content_scale(cfg_t, 8))
    assert all(caught.values()), caught


# ------------------------------------------------ hier_select, any mask -----
def _hier_case(seed, nb=37, m=4, d=16, F=4):
    rng = np.random.default_rng(seed)
    S0 = rng.standard_normal((nb, m, d)).astype(np.float32)
    S1 = O.build_super(S0, F, "f32")
    return rng, S0, S1


def test_hier_select_mask_equals_the_causal_form():
    """On the causal candidate rule the masked hier_select is the row-position
    one (pinned to the reference's hier_select goldens) bit for bit."""
    rng, S0, S1 = _hier_case(1)
    nb, d, F, W, Bk = S0.shape[0], S0.shape[2], 4, 128, 64
    qg = rng.standard_normal((nb * Bk, d)).astype(np.float32)
    pos = np.arange(0, nb * Bk, 29)
    for beam, kk in ((3, 8), (2, 16), (16, 5)):
        i1, v1, c1 = O.hier_select(qg[None], S0[None], S1[None], F, beam, kk, 0.25, Bk, W, pos=pos)
        bmax = np.array([O.cand_bmax(int(i), Bk, W) for i in pos])
        blk = np.arange(nb)
        cand = (blk[None] >= 1) & (blk[None] <= bmax[:, None])
        i2, v2, c2 = O.hier_select_mask(qg[pos], S0, S1, F, beam, kk, cand, 0.25)
        ke = i2.shape[1]
        assert np.array_equal(i1[0][:, :ke], i2) and np.array_equal(v1[0][:, :ke], v2)
        assert np.array_equal(c1[0], c2)


def test_hier_select_mask_with_every_super_expanded_is_the_flat_top_k():
    """beam >= ns expands every super holding a candidate, so the picks are the
    flat top-k of the masked block scores, for any mask (ragged last super)."""
    rng, S0, S1 = _hier_case(2)
    nb, d, F = S0.shape[0], S0.shape[2], 4
    ns = S1.shape[0]
    q = rng.standard_normal((40, d)).astype(np.float32)
    cand = rng.random((40, nb)) < 0.3
    cand[:, 0] = False                                  # block 0 is never a routed candidate
    cand[3] = False                                     # a row with no candidate
    idx, val, cnt = O.hier_select_mask(q, S0, S1, F, ns, 12, cand, 0.5)
    # declared-order scores of blocks 1..nb-1 for rows 0..39 (a window reaching
    # back past the sequence start makes every such block a candidate)
    full = O.block_scores(q, S0, np.arange(40), 0.5, 64, -10 ** 6)
    assert np.isfinite(full[:, 1:]).all()
    ti, tv, tc = O.topk(np.where(cand, full, -np.inf).astype(np.float32), 12)
    fin = np.isfinite(tv)
    assert np.array_equal(cnt, tc) and cnt[3] == 0
    assert np.array_equal(np.where(fin, ti, -1), idx)
    assert np.array_equal(np.where(fin, tv, -np.inf), val)
