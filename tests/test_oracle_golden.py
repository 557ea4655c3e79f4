"""The oracle against golden vectors written from the reference implementation
(tests/golden/make_golden.py).  CPU only.

Tolerances: fp32 reassociation noise (the reference's einsum/reduction orders
are unspecified); selections must agree exactly on these seeded inputs (none of
their k/k+1 gaps is a near-tie), and the declared-order block scores reproduce
the reference's bit for bit where its reduction is sequential."""
import numpy as np
import pytest

import make_golden as MG
import oracle.hba_oracle as O

EPS = 1e-6


def _load(name):
    case = MG.CASES[name]
    z = np.load(f"{MG.HERE}/golden_{name}.npz")
    inp = MG.gen_inputs(case)
    for key, arr in (("ck_q", inp["q"]), ("ck_k", inp["k"]), ("ck_v", inp["v"]),
                     ("ck_S0h", inp["S0_h"])):
        assert np.allclose(MG.checksum(arr), z[key]), f"input generator changed ({key})"
    cfg = O.Cfg(**case["cfg"])
    n, d = case["n"], case["cfg"]["head_dim"]
    if "cos" in z:
        cos, sin = z["cos"], z["sin"]
    else:
        cos, sin = O.rope_tables(n, d, cfg.rope_theta)
        assert np.allclose(MG.checksum(cos), z["ck_cos"], rtol=1e-6)
        assert np.allclose(MG.checksum(sin), z["ck_sin"], rtol=1e-6)
    return case, z, inp, cfg, cos, sin


NAMES = list(MG.CASES)
TINY = [n for n in NAMES if "qc" in np.load(f"{MG.HERE}/golden_{n}.npz")]


@pytest.mark.parametrize("name", TINY)
def test_rope_tables_match_reference(name):
    case, z, inp, cfg, cos, sin = _load(name)
    c2, s2 = O.rope_tables(case["n"], case["cfg"]["head_dim"], cfg.rope_theta)
    assert np.abs(c2 - z["cos"]).max() <= 2e-7 and np.abs(s2 - z["sin"]).max() <= 2e-7


@pytest.mark.parametrize("name", TINY)
def test_qknorm_and_grouped_query_match_reference(name):
    case, z, inp, cfg, cos, sin = _load(name)
    qc, kc, scale = O.content_qk(inp["q"], inp["k"], cfg, inp["q_gain"], inp["k_gain"], EPS,
                                 case["n"], "f32")
    assert scale == float(z["scale"])
    assert np.abs(qc - z["qc"]).max() <= 1e-6 * max(1.0, np.abs(z["qc"]).max())
    assert np.abs(kc - z["kc"]).max() <= 1e-6 * max(1.0, np.abs(z["kc"]).max())
    # grouped_query is a sequential head sum in the reference as well: bit-exact
    for b in range(case["B"]):
        assert np.array_equal(O.grouped_query(z["qc"][b], cfg.n_kv, "f32"), z["qg"][b])


@pytest.mark.parametrize("name", NAMES)
def test_summarize_matches_reference(name):
    case, z, inp, cfg, cos, sin = _load(name)
    for b in range(case["B"]):
        _, kc, _ = O.content_qk(inp["q"][b], inp["k"][b], cfg, inp["q_gain"], inp["k_gain"],
                                EPS, case["n"], "f32")
        S0 = O.summarize(kc, inp["probes"], inp["proj"], cfg.block)
        assert np.abs(S0 - z["S0"][b]).max() <= 2e-6 * max(1.0, np.abs(z["S0"][b]).max())


@pytest.mark.parametrize("name", TINY)
def test_block_scores_bit_exact_vs_reference(name):
    """route_topk's bsc from the reference's own qg/S0: the declared order
    (sequential fp32 FMA over d, max over slots, one multiply by the scale)
    reproduces torch's scores within 1 ulp-scale noise, and exactly at d=8."""
    case, z, inp, cfg, cos, sin = _load(name)
    n = case["n"]
    sc = O.route_scale(cfg, case["cfg"]["head_dim"])
    for b in range(case["B"]):
        for g in range(cfg.n_kv):
            mine = O.block_scores(z["qg"][b, g], z["S0"][b, g], np.arange(n), sc, cfg.block,
                                  cfg.window)
            ref = z["bsc"][b, g]
            fin = np.isfinite(ref)
            assert np.array_equal(np.isfinite(mine), fin)
            assert np.abs(mine[fin] - ref[fin]).max() <= 1e-6 * max(1.0, np.abs(ref[fin]).max())


@pytest.mark.parametrize("name", NAMES)
def test_route_topk_selection_matches_reference(name):
    case, z, inp, cfg, cos, sin = _load(name)
    rows = z["rows"]
    _, sels = O.forward_dense(inp["q"], inp["k"], inp["v"], cos, sin, cfg, inp["probes"],
                              inp["proj"], inp["q_gain"], inp["k_gain"], EPS, "f32", rows=rows)
    for b in range(case["B"]):
        idx, val, cnt = sels[b]
        for g in range(cfg.n_kv):
            for r, i in enumerate(rows):
                mine = set(idx[g, r, : cnt[g, r]].tolist())
                ref = set(np.nonzero(z["sel"][b, g, i])[0].tolist())
                assert mine == ref, (b, g, int(i))


@pytest.mark.parametrize("name", NAMES)
@pytest.mark.parametrize("path", ["dense", "eval", "hier"])
def test_forward_outputs_match_reference(name, path):
    case, z, inp, cfg, cos, sin = _load(name)
    args = (inp["q"], inp["k"], inp["v"], cos, sin, cfg, inp["probes"], inp["proj"],
            inp["q_gain"], inp["k_gain"], EPS, "f32")
    if path == "dense":
        out, _ = O.forward_dense(*args, rows=z["rows"])
    else:
        out, _ = O.forward_eval(*args, rows=z["rows"], hier=(path == "hier"))
    ref = z[f"out_{path}"]
    assert np.abs(out - ref).max() <= 1e-5, np.abs(out - ref).max()


@pytest.mark.parametrize("name", NAMES)
def test_build_super_and_hier_select_match_reference(name):
    case, z, inp, cfg, cos, sin = _load(name)
    hn, d, Bk = case["hier_n"], case["cfg"]["head_dim"], cfg.block
    kk = min(cfg.k_blocks, hn // Bk)
    for b in range(case["B"]):
        S1 = O.build_super(inp["S0_h"][b], cfg.fanout, "f32")
        assert np.array_equal(S1, z["S1_h"][b])                    # sequential sum: bit-exact
        qfull = np.zeros((hn, d), np.float32)
        qfull[inp["pos_h"]] = inp["qg_h"][b]
        idx, val, cnt = O.hier_select(qfull[None], inp["S0_h"][b][None], S1[None], cfg.fanout,
                                      cfg.beam, kk, 1.0 / d, Bk, cfg.window, pos=inp["pos_h"])
        for r in range(len(inp["pos_h"])):
            rv = z["hier_val"][b, r]
            ref = sorted(z["hier_idx"][b, r][np.isfinite(rv)].tolist())
            assert sorted(idx[0, r, : cnt[0, r]].tolist()) == ref
            assert np.allclose(np.sort(val[0, r, : cnt[0, r]]), np.sort(rv[np.isfinite(rv)]),
                               rtol=1e-6, atol=1e-7)
    assert int(z["hier_comp"]) == O.hier_comparisons(hn, Bk, cfg.fanout, cfg.beam)


# ------------------------------------------------------------- aux-KL -------
AUX = np.load(f"{MG.HERE}/golden_aux.npz")


def _aux_oracle(name):
    case = MG.CASES[name]
    inp = MG.gen_inputs(case)
    assert np.allclose(MG.checksum(inp["q"]), AUX[f"{name}_ck_q"]), "input generator changed"
    cfg = O.Cfg(**case["cfg"])
    c = case["cfg"]
    qc, kc, su = O.content_qk(inp["q"], inp["k"], cfg, inp["q_gain"], inp["k_gain"], EPS, case["n"], "f32")
    sr = O.route_scale(cfg, c["head_dim"])
    return O.aux_kl(qc, kc, inp["probes"], inp["proj"], c["n_kv"], su, sr, c["block"], c["window"])


@pytest.mark.parametrize("name", NAMES)
def test_aux_kl_and_its_gradients_match_reference(name):
    """aux (hba_attention_dense, attention.py:366-389) and d aux / d probes,
    d proj from the reference's autograd, fp32; the chunked (fused-path)
    teacher gives the same aux; the reference's aux sends exactly zero
    gradient into q, k, v (gates.py:129-167)."""
    aux, dprobes, dproj, pstar = _aux_oracle(name)
    ga = float(AUX[f"{name}_aux"])
    assert abs(aux - ga) <= 1e-6 * abs(ga)
    assert abs(float(AUX[f"{name}_aux_chunked"]) - ga) <= 1e-6 * abs(ga)
    for got, key in ((dprobes, "dprobes"), (dproj, "dproj")):
        ref = AUX[f"{name}_{key}"]
        assert np.abs(got - ref).max() <= 1e-5 * np.abs(ref).max(), key
    assert float(AUX[f"{name}_grad_qkv_max"]) == 0.0
    gp = AUX[f"{name}_pstar"]
    p = pstar if gp.shape == pstar.shape else pstar[:, :, -gp.shape[2]:]
    rows = np.isfinite(gp).all(-1)                          # the reference's rows without candidates are NaN
    assert rows.any() and np.abs(p[rows] - gp[rows]).max() <= 1e-6
    assert np.all(p[~rows] == 0.0)


def test_aux_kl_is_a_cross_entropy_bounded_by_the_teacher_entropy():
    """aux is a cross-entropy H(p*, softmax(bsc)) >= H(p*): equality needs the
    router to reproduce the teacher, so the oracle's aux sits above the mean
    teacher entropy; and a planted sign error in the teacher renormalisation
    (a mistake the golden check must catch) moves aux off the golden value."""
    name = "d64"
    aux, _, _, pstar = _aux_oracle(name)
    case = MG.CASES[name]
    c = case["cfg"]
    vq = O.route_candidates(case["n"], c["window"], case["n"] // c["block"], c["block"]).any(-1)
    p = pstar[:, :, vq]
    ent = -np.where(p > 0, p * np.log(np.where(p > 0, p, 1.0)), 0.0).sum(-1).mean()
    assert aux > ent > 0
    orig = O.aux_teacher
    try:
        O.aux_teacher = lambda *a: orig(*a) ** 1.01            # a planted mistake
        bad, _, _, _ = _aux_oracle(name)
    finally:
        O.aux_teacher = orig
    assert abs(bad - float(AUX[f"{name}_aux"])) > 1e-4
