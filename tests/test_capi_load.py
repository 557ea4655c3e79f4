"""The C-ABI library loads and exports every entry point include/hba_amd.h
declares (no compute calls: this runs without a GPU)."""
import ctypes
import os
import re

import pytest

import hba_amd
from hba_amd import _lib

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def declared_symbols():
    src = open(os.path.join(ROOT, "include", "hba_amd.h")).read()
    return sorted(set(re.findall(r"^(?:int|const char \*)\s*(hba_\w+)\(", src, flags=re.M)))


def test_every_declared_symbol_is_exported():
    names = declared_symbols()
    assert len(names) >= 13
    L = ctypes.CDLL(_lib.LIB_PATH)
    missing = [n for n in names if not hasattr(L, n)]
    assert not missing, missing


def test_binding_table_covers_the_header():
    assert sorted(_lib.SIGNATURES) == declared_symbols()


def test_static_queries_without_a_gpu():
    L = _lib.lib()
    assert L.hba_abi_version() == 1
    assert L.hba_status_string(0) == b"ok"
    assert L.hba_status_string(-1) == b"invalid argument"
    n = ctypes.c_size_t(0)
    assert L.hba_decode_workspace_size(32, 14, 2, 64, 16, 64, 1024, 32768, ctypes.byref(n)) == 0
    assert n.value > 0
    assert L.hba_decode_workspace_size(32, 14, 2, 64, 16, 32, 1024, 32768, ctypes.byref(n)) == -2


def test_backward_workspace_is_sized_by_dtype_and_kv_heads():
    """bf16 at 32K, 14/2 heads, d = 64: bf16 query rows (2 x n*Hq*d), LSE and
    D (2 x Hq*n fp32), sink accumulators (2*Hkv*64*d fp32), transposed keys
    (2 x Hkv*d*n bf16), dk/dv accumulators (3*Hkv*n*d fp32), the routed-row
    bits (Hkv * n/4096 ranges * n/64 blocks * 4096 bits), each rounded up to
    256 bytes; within the all-dtype bound of hba_attn_bwd_workspace_size."""
    L = _lib.lib()
    B, n, Hq, Hkv, d = 1, 32768, 14, 2, 64
    r = lambda x: (x + 255) // 256 * 256
    want = (2 * r(n * Hq * d * 2) + 2 * r(Hq * n * 4) + r(Hkv * 2 * 64 * d * 4) + 2 * r(Hkv * d * n * 2)
            + r(Hkv * n * 3 * d * 4) + r(Hkv * (n // 4096) * (n // 64) * 4096 // 8))
    got, bound = ctypes.c_size_t(0), ctypes.c_size_t(0)
    assert L.hba_attn_bwd_workspace_bytes(1, B, n, Hq, Hkv, d, ctypes.byref(got)) == 0
    assert got.value == want
    assert L.hba_attn_bwd_workspace_size(B, n, Hq, d, ctypes.byref(bound)) == 0
    assert got.value < bound.value
    f32 = ctypes.c_size_t(0)
    assert L.hba_attn_bwd_workspace_bytes(0, B, n, Hq, Hkv, d, ctypes.byref(f32)) == 0
    assert f32.value == 2 * r(n * Hq * d * 4) + 2 * r(Hq * n * 4) + r(Hkv * 2 * 64 * d * 4) <= bound.value
    assert L.hba_attn_bwd_workspace_bytes(1, B, n, Hq, 3, d, ctypes.byref(got)) == -1   # Hq % Hkv


def test_ops_refuse_cpu_tensors():
    import torch
    q = torch.zeros(1, 64, 2, 64)
    with pytest.raises(NotImplementedError):
        hba_amd.ops.score_select(q, None, 1e-6, torch.zeros(1, 1, 1, 4, 64), 16, 4, 0.1)


def test_argument_checks_run_before_any_launch():
    """Invalid sizes are rejected on the host with no device pointer touched."""
    L = _lib.lib()
    s3 = (ctypes.c_int64 * 3)(0, 0, 0)
    fake = ctypes.c_void_p(16)
    st = L.hba_attn_fwd(1, fake, s3, None, None, 1e-6, fake, fake, fake, fake, fake, fake, fake, 1, 100, 14,
                        2, 64, 4, 1024, 64, 16, 0.1, fake, 1 << 20, fake, s3, None)
    assert st == -1                                    # n % 64 != 0
    st = L.hba_attn_fwd(1, fake, s3, None, None, 1e-6, fake, fake, fake, fake, fake, fake, fake, 1, 128, 14,
                        2, 64, 4, 1024, 64, 16, 0.1, fake, 16, fake, s3, None)
    assert st == -1                                    # workspace smaller than B*n*Hq*d*2
    st = L.hba_attn_window_fwd(fake, s3, None, None, 1e-6, fake, fake, fake, fake, 1, 100, 14, 2, 64, 4, 1024,
                               64, 0.1, fake, 1 << 20, fake, s3, None)
    assert st == -1                                    # n % 64 != 0
    st = L.hba_attn_routed_fwd(fake, s3, None, None, 1e-6, fake, fake, fake, fake, 1, 128, 14, 2, 64, 4, 64, 16,
                               0.1, fake, 16, fake, s3, None)
    assert st == -1                                    # workspace smaller than B*Hq*n*4
    st = L.hba_attn_window_fwd(fake, s3, None, None, 1e-6, fake, fake, fake, fake, 1, 128, 14, 2, 96, 4, 1024,
                               64, 0.1, fake, 1 << 20, fake, s3, None)
    assert st == -2                                    # d = 96 unsupported
    nbytes = ctypes.c_size_t(0)
    assert L.hba_attn_workspace_size(1, 2, 128, 14, ctypes.byref(nbytes)) == 0 and nbytes.value == 2 * 14 * 128 * 4
    assert L.hba_attn_workspace_size(0, 2, 128, 14, ctypes.byref(nbytes)) == 0 and nbytes.value == 0
    assert L.hba_attn_fwd_workspace_bytes(1, 2, 128, 14, 64, ctypes.byref(nbytes)) == 0
    assert nbytes.value == 2 * 128 * 14 * 64 * 2
    assert L.hba_attn_fwd_workspace_bytes(1, 1, 64, 3, 1, ctypes.byref(nbytes)) == 0 and nbytes.value == 512
    assert L.hba_attn_fwd_workspace_bytes(0, 2, 128, 14, 64, ctypes.byref(nbytes)) == 0 and nbytes.value == 0
    assert L.hba_attn_fwd_workspace_bytes(1, 2, 128, 14, 0, ctypes.byref(nbytes)) == -1
    st = L.hba_score_select(1, fake, s3, None, 1e-6, fake, 1, 128, 14, 2, 96, 4, 64, 1024, 16, 0.1,
                            fake, fake, fake, None, None)
    assert st == -2                                    # d = 96 unsupported


def test_training_paths_return_the_aux_kl_and_have_no_cpu_path():
    """hba_attention_dense/fused compute the aux-KL whenever cfg.aux_w != 0
    (attention.py:363-389) on the GPU only: CPU tensors raise before any
    launch, with aux_w = 0 as well (no CPU fallback)."""
    import torch
    from hba_amd import synth
    cfg = hba_amd.HBAConfig(window=64, k_blocks=2)
    q = torch.zeros(1, 128, 14, 64, requires_grad=True)
    k = torch.zeros(1, 128, 2, 64)
    prm = synth.Params(torch.ones(14), torch.ones(2), torch.zeros(2, 4, 64), torch.zeros(2, 64, 64))
    cos = sin = torch.zeros(128, 64)
    for aux_w in (1.0, 0.0):
        cfg.aux_w = aux_w
        for fn in (hba_amd.hba_attention_dense, hba_amd.hba_attention_fused):
            with pytest.raises((RuntimeError, NotImplementedError)):   # the dispatcher's or _dev's refusal
                fn(q, k, k, cos, sin, cfg, prm, prm)
    with pytest.raises((RuntimeError, NotImplementedError)):
        hba_amd.aux_kl(q, k, k, cos, sin, cfg, prm, prm)
