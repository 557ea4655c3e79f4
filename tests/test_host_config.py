"""Host-side config helpers without a GPU: yarn_theta (attention.py:47-53)."""
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
