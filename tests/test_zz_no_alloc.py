"""hba_decode_fwd_noalloc (the decode step run in the library's fixed per-GPU
scratch, no allocation) against hba_decode_fwd (caller-provided workspace) on
the same paged cache, through the C-ABI: identical outputs, picks and counts
on two calls in a row, the second with fewer and shorter sequences; a request
larger than the scratch is refused on the host with HBA_ERR_SCRATCH."""
import numpy as np
import pytest
import torch

pytestmark = pytest.mark.gpu

hba_amd = pytest.importorskip("hba_amd")
from hba_amd import _lib, ops, synth  # noqa: E402


@pytest.fixture(scope="module")
def dev():
    if not torch.cuda.is_available():
        pytest.fail("GPU tests need a visible gfx950 device")
    return torch.device("cuda:0")


def _cache(dev, dt, lens, seed, Hq=14, Hkv=2, d=64, m=4, W=1024, S=4, k=16):
    cfg = hba_amd.HBAConfig(n_heads=Hq, n_kv=Hkv, head_dim=d, slots=m, window=W, sinks=S, k_blocks=k)
    g = torch.Generator().manual_seed(seed)
    probes = (torch.randn(Hkv, m, d, generator=g) * d ** -0.5).to(dev)
    proj = (torch.eye(d).unsqueeze(0).repeat(Hkv, 1, 1) + torch.randn(Hkv, d, d, generator=g) * 0.02).to(dev)
    prm = synth.Params(torch.full((Hq,), d ** 0.25, device=dev), torch.full((Hkv,), d ** 0.25, device=dev),
                       probes, proj)
    Lmax = max(lens)
    cos, sin = hba_amd.rope_tables(Lmax, d, cfg.rope_theta, dev)
    cache = hba_amd.PagedKVCache(cfg, len(lens), Lmax, dt, dev)
    cache._free = synth.shuffled_pages(len(cache._free), seed=seed + 5)
    for s, L in enumerate(lens):
        kraw = torch.randn(1, L, Hkv, d, generator=g).to(dt).to(dev)
        vraw = torch.randn(1, L, Hkv, d, generator=g).to(dt).to(dev)
        kc, kr, _ = ops.prep_keys(kraw, vraw, prm.k.gain, 1e-6, cos, sin)
        cache.load(s, kc[0].transpose(0, 1), kr[0].transpose(0, 1), vraw[0], prm)
    q = torch.randn(len(lens), Hq, d, generator=g).to(dt).to(dev)
    return cfg, cache, prm, cos, sin, q


@pytest.mark.parametrize("dt,kern", [(torch.bfloat16, "fused"), (torch.bfloat16, "pair"), (torch.float32, "fused")])
def test_noalloc_decode_equals_decode_on_two_calls(dev, dt, kern, monkeypatch):
    monkeypatch.setenv("HBA_DECODE_KERNEL", kern)   # either bf16 kernel, whatever the batch size
    for lens, seed in (([9000, 4100, 12000, 300, 7777, 20000], 0), ([5000, 130, 2600], 1)):
        cfg, cache, prm, cos, sin, q = _cache(dev, dt, lens, seed)
        scales = cache.scales(cfg)
        max_len = max(cache.lens)
        ref, ridx, rcnt = ops.decode_fwd(q, prm.q.gain, 1e-6, cache.kc_pages, cache.kr_pages, cache.v_pages,
                                         cache.summ_pages, cache.page_table, cache.seq_lens, cos, sin, scales,
                                         cfg.sinks, cfg.window, cfg.k_blocks, max_len)
        out = torch.full_like(q, 7.0)                   # garbage: an entry left unwritten shows
        sidx = torch.full_like(ridx, -7)
        scnt = torch.full_like(rcnt, -7)
        ops.decode_fwd_noalloc(q, prm.q.gain, 1e-6, cache.kc_pages, cache.kr_pages, cache.v_pages,
                               cache.summ_pages, cache.page_table, cache.seq_lens, cos, sin, scales, cfg.sinks,
                               cfg.window, cfg.k_blocks, max_len, out, sidx, scnt)
        torch.cuda.synchronize()
        assert torch.equal(out, ref), (lens, (out.float() - ref.float()).abs().max().item())
        assert torch.equal(sidx, ridx) and torch.equal(scnt, rcnt), lens


def test_noalloc_decode_refuses_requests_beyond_the_scratch(dev):
    """256 sequences of up to 131072 tokens at 28/4 heads, d = 128, k = 64
    need ~350 MB of workspace: refused before any launch."""
    L = _lib.lib()
    need = _lib.ctypes.c_size_t(0)
    assert L.hba_decode_workspace_size(256, 28, 4, 128, 64, 64, 1024, 131072, _lib.ctypes.byref(need)) == 0
    assert need.value > (16 << 20)
    buf = torch.zeros(1 << 16, dtype=torch.bfloat16, device=dev)
    f32 = torch.zeros(1 << 16, dtype=torch.float32, device=dev)
    i32 = torch.zeros(1 << 16, dtype=torch.int32, device=dev)
    p = lambda t: _lib.ctypes.c_void_p(t.data_ptr())
    st = L.hba_decode_fwd_noalloc(1, p(buf), None, 1e-6, p(buf), p(buf), p(buf), p(buf), p(i32), 2048, p(i32),
                                  p(f32), p(f32), p(f32), 256, 28, 4, 128, 4, 8, 1024, 64, 64, 131072, p(buf),
                                  None, None, None)
    assert st == -5
    assert L.hba_status_string(st) == b"request exceeds the fixed scratch of the no-allocation entry point"
    torch.cuda.synchronize()
    assert np.all(buf.cpu().float().numpy() == 0.0)      # nothing was launched
