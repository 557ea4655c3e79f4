"""Host-side config helpers and checks without a GPU: yarn_theta
(attention.py:47-53), the aux-KL's block-size guard."""
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


def test_aux_kl_refuses_other_block_sizes():
    """The aux-KL kernel scores 64-key blocks: at the reference's block-16
    test geometry it raises instead of training the summarizer on 64-key
    blocks (checked before any tensor is touched, so CPU tensors do)."""
    from hba_amd import attention as A
    cfg = hba_amd.HBAConfig(block=16, head_dim=64, n_heads=4, n_kv=2, window=32, k_blocks=2)
    q = torch.zeros(1, 64, 4, 64)
    k = torch.zeros(1, 64, 2, 64)

    class Summ:
        probes = torch.zeros(2, 4, 64, requires_grad=True)
        proj = torch.zeros(2, 64, 64, requires_grad=True)

    with pytest.raises(NotImplementedError, match="64-key blocks"):
        A.aux_kl(q, k, k, None, None, cfg, Summ(), None)
