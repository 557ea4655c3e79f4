"""The oracle's bf16 emulation against the reference's own bf16 arithmetic
(tests/golden/golden_bf16.npz, written by make_golden.py from the reference
functions run on torch bfloat16 tensors).  CPU only.

Pinned here, bit for bit unless stated:
  round_bf16                 torch's fp32 -> bf16 cast (nearest-even, NaN, inf,
                             overflow edge, subnormals, signed zeros)
  qknorm(..., 'bf16')        _HeadRMSNorm.forward on bf16 q/k (attention.py:88-94):
                             the reference's mean-square reduction order is not
                             specified, so a last-place difference in the fp32
                             RMS may move an output by one bf16 ulp; the bound is
                             one ulp on at most 0.1 % of the elements
  apply_rope(..., 'bf16')    apply_rope on bf16 tensors (:40-44), including
                             positions near 128K
  grouped_query(..., 'bf16') the bf16 head sum (summarizer.py:50-54)
  build_super(..., 'bf16')   the bf16 sum and divide (attention.py:202-214),
                             whole and ragged last supers
"""
import numpy as np
import pytest

import make_golden as MG
import oracle.hba_oracle as O

Z = np.load(f"{MG.HERE}/golden_bf16.npz")
EPS = 1e-6


def bits(x):
    return O.round_bf16(x).view(np.uint32) >> 16


def _case(name):
    case = MG.BF16_CASES[name]
    inp = MG.gen_bf16_inputs(case)
    assert np.allclose(MG.checksum(inp["q"]), Z[f"{name}_ck_q"]), "input generator changed"
    return case, inp


def test_round_bf16_matches_torch_cast():
    got = O.round_bf16(Z["round_in"])
    want = Z["round_out"]
    nan = np.isnan(want)
    assert np.array_equal(np.isnan(got), nan)
    assert np.array_equal(got[~nan].view(np.uint32), want[~nan].view(np.uint32))   # signed zeros too


def test_round_bf16_planted_truncation_is_caught():
    """Truncation instead of nearest-even differs on the probe: the check above
    can fail."""
    trunc = (Z["round_in"].view(np.uint32) & 0xFFFF0000).view(np.float32)
    want = Z["round_out"]
    ok = ~np.isnan(want)
    assert not np.array_equal(trunc[ok].view(np.uint32), want[ok].view(np.uint32))


def _ulps(a, b):
    """Distance in bf16 ulps between two arrays of bf16 values (same sign
    assumed where nonzero)."""
    ia = a.view(np.uint32).astype(np.int64) >> 16
    ib = b.view(np.uint32).astype(np.int64) >> 16
    sa = np.where(ia >= 0x8000, -(ia - 0x8000), ia)
    sb = np.where(ib >= 0x8000, -(ib - 0x8000), ib)
    return np.abs(sa - sb)


@pytest.mark.parametrize("name", list(MG.BF16_CASES))
def test_qknorm_bf16_matches_reference(name):
    case, inp = _case(name)
    q = O.round_bf16(inp["q"])
    k = O.round_bf16(inp["k"])
    for x, gain, key in ((q, inp["q_gain"], "qc"), (k, inp["k_gain"], "kc")):
        got = O.qknorm(x, gain, EPS, "bf16")
        want = MG.from_bits(Z[f"{name}_{key}"])
        u = _ulps(got, want)
        assert u.max() <= 1, (key, u.max())
        assert (u > 0).mean() <= 1e-3, (key, (u > 0).mean())
    # the eps-clamped rows (all zero, and far below eps) are exact
    qc = O.qknorm(q, inp["q_gain"], EPS, "bf16")
    kc = O.qknorm(k, inp["k_gain"], EPS, "bf16")
    qw, kw = MG.from_bits(Z[f"{name}_qc"]), MG.from_bits(Z[f"{name}_kc"])
    for got, want, (t, h) in ((qc, qw, (5, 3)), (qc, qw, (6, 1)), (kc, kw, (7, 1)), (kc, kw, (9, 0))):
        assert np.array_equal(got[0, t, h], want[0, t, h]), (t, h)


@pytest.mark.parametrize("name", list(MG.BF16_CASES))
def test_apply_rope_bf16_matches_reference(name):
    case, inp = _case(name)
    n, d = case["n"], case["d"]
    cos, sin = O.rope_tables(n, d, 1_000_000.0)
    for key in ("q", "k"):
        xc = MG.from_bits(Z[f"{name}_{key}c"])
        got = O.apply_rope(xc, cos, sin, "bf16")
        assert np.array_equal(got, MG.from_bits(Z[f"{name}_{key}r"])), key
    # positions 131008..131071, on the reference's own table rows: the bf16
    # rounding of cos/sin at large angles
    far = MG.from_bits(Z[f"{name}_far_kc"])
    got = O.apply_rope(far, Z[f"{name}_far_cos"], Z[f"{name}_far_sin"], "bf16")
    assert np.array_equal(got, MG.from_bits(Z[f"{name}_far_kr"]))


@pytest.mark.parametrize("d", [64, 128])
def test_rope_tables_match_reference_at_128k(d):
    """rope_tables' rows 131008..131071 equal the reference's bit for bit: the
    angle pos * inv amplifies the last bit of inv, so this pins the power and
    the product order, not just the formula."""
    cf, sf = O.rope_tables(131072, d, 1_000_000.0)
    name = "d64" if d == 64 else "d128"
    assert np.array_equal(cf[-64:], Z[f"{name}_far_cos"])
    assert np.array_equal(sf[-64:], Z[f"{name}_far_sin"])


@pytest.mark.parametrize("name", list(MG.BF16_CASES))
def test_grouped_query_bf16_matches_reference(name):
    case, inp = _case(name)
    qc = MG.from_bits(Z[f"{name}_qc"])
    want = MG.from_bits(Z[f"{name}_qg"])
    for b in range(case["B"]):
        assert np.array_equal(O.grouped_query(qc[b], case["Hkv"], "bf16"), want[b])


@pytest.mark.parametrize("name", list(MG.BF16_CASES))
def test_build_super_bf16_matches_reference(name):
    case, inp = _case(name)
    S0 = O.round_bf16(inp["S0"])
    for F in case["F"]:
        want = MG.from_bits(Z[f"{name}_S1_F{F}"])
        assert case["nb"] % F != 0 or F == 16                 # the cases include ragged last supers
        for b in range(case["B"]):
            assert np.array_equal(O.build_super(S0[b], F, "bf16"), want[b]), F


def test_bf16_planted_mistakes_are_caught():
    """Variants of the bf16 emulation that a plausible mistake would produce
    fail the fixture: apply_rope without the per-op rounding, a head sum
    rounded after every addition, build_super that divides before rounding
    the sum, and QKNorm without the final cast."""
    case, inp = _case("d64")
    n, d = case["n"], case["d"]
    cos, sin = O.rope_tables(n, d, 1_000_000.0)
    kc = MG.from_bits(Z["d64_kc"])
    fused = O.round_bf16(kc * O.round_bf16(cos)[:, None] + O.rot_half(kc) * O.round_bf16(sin)[:, None])
    assert not np.array_equal(fused, MG.from_bits(Z["d64_kr"]))
    qc = MG.from_bits(Z["d64_qc"])[0]
    G = case["Hq"] // case["Hkv"]
    acc = qc[:, 0::G].copy()
    for h in range(1, G):
        acc = O.round_bf16(acc + qc[:, h::G])
    assert not np.array_equal(acc.transpose(1, 0, 2), MG.from_bits(Z["d64_qg"])[0])
    S0 = O.round_bf16(inp["S0"])[0]
    F = 5
    ns = (case["nb"] + F - 1) // F
    early = np.stack([O.round_bf16(S0[p * F:(p + 1) * F].sum(0) / min(F, case["nb"] - p * F))
                      for p in range(ns)])
    assert not np.array_equal(early, MG.from_bits(Z["d64_S1_F5"])[0])
    raw = O.qknorm(O.round_bf16(inp["q"]), inp["q_gain"], EPS, "f32")
    assert not np.array_equal(raw, MG.from_bits(Z["d64_qc"]))
