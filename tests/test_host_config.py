"""Host-side config helpers and checks without a GPU: yarn_theta
(attention.py:47-53), the generic geometry's workspace sizes."""
import math

import pytest
import torch

import hba_amd


@pytest.mark.parametrize("d", [8, 64, 128])
def test_yarn_theta_stretches_the_lowest_frequency_by_the_context_ratio(d):
    """NTK-aware rescaling keeps the highest RoPE frequency (pair 0) and
    divides the lowest (pair d/2 - 1, exponent (d-2)/d) by s = n / native_ctx;
    up to native_ctx the base is unchanged."""
    cfg = hba_amd.HBAConfig(head_dim=d, native_ctx=4096, rope_theta=1e6)
    for n in (1, 4095, 4096):
        assert hba_amd.yarn_theta(cfg, n) == 1e6
    for n in (4097, 8192, 131072):
        s = n / 4096
        th = hba_amd.yarn_theta(cfg, n)
        assert th > 1e6
        low = lambda base: base ** (-(d - 2) / d)
        assert math.isclose(low(th), low(1e6) / s, rel_tol=1e-12), (n, d)
        # the table the eval builds from it: position p of pair 0 is p radians
        cos, sin = hba_amd.rope_tables(8, d, th, "cpu")
        assert torch.allclose(cos[:, 0], torch.cos(torch.arange(8.0)))
        assert torch.allclose(sin[:, d // 2 - 1], torch.sin(torch.arange(8.0) * low(th)), atol=1e-7)


def test_generic_geometry_workspaces_are_sized_on_the_host():
    """The aux-KL and the backward take the reference's block-16 / head-dim-8
    test geometry in fp32 (the generic kernels): their workspace queries
    (host functions, no GPU) accept it and return the sizes of the generic
    layouts -- the aux-KL's qg, teacher LSEs, scores, ties, row terms, dS0,
    pooled rows and d probes partials; the backward's three key-side
    accumulators -- and bf16 at that geometry is refused (the Python side
    widens it to fp32 first)."""
    import ctypes
    from hba_amd import _lib
    L = ctypes.CDLL(_lib.LIB_PATH)
    F32, BF16 = 0, 1
    B, n, Hq, Hkv, d, m, Bk = 2, 512, 4, 2, 8, 2, 16
    nb, G = n // Bk, Hq // Hkv
    up = lambda x: (x + 255) // 256 * 256
    want = (up(B * n * Hkv * d * 4) + up(B * Hkv * n * G * nb * 4) + 2 * up(B * Hkv * n * nb * 4)
            + up(B * Hkv * n * 4) + 3 * up(B * Hkv * nb * m * d * 4))
    got = ctypes.c_size_t(0)
    fn = L.hba_aux_kl_workspace_size
    fn.argtypes = [ctypes.c_int] + [ctypes.c_int64] * 7 + [ctypes.POINTER(ctypes.c_size_t)]
    assert fn(F32, B, n, Hq, Hkv, d, m, Bk, ctypes.byref(got)) == 0
    assert got.value == want
    assert fn(BF16, B, n, Hq, Hkv, d, m, Bk, ctypes.byref(got)) != 0
    bw = L.hba_attn_bwd_workspace_bytes
    bw.argtypes = [ctypes.c_int] + [ctypes.c_int64] * 5 + [ctypes.POINTER(ctypes.c_size_t)]
    assert bw(F32, B, n, Hq, Hkv, d, ctypes.byref(got)) == 0
    assert got.value >= 3 * B * Hkv * n * d * 4
