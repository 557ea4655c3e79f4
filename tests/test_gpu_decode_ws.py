"""The decode step's workspace reused across calls of different shapes.

The one-launch bf16 step counts its workgroups' arrivals in completion
counters at the start of the workspace, which every call leaves zero.  These
tests run calls whose other workspace regions differ (batch sizes, maximum
lengths, fp32 then bf16) on one shared workspace -- the library's no-
allocation scratch and ops.decode_fwd's per-device workspace -- and check each
call against the same call on a freshly zeroed workspace, bit for bit.  A
batch of more (sequence, KV head) pairs than one launch counts runs as
several launches over slices of the batch: checked against the same batch
decoded in two halves."""
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
    return dict(cfg=cfg, cache=cache, prm=prm, cos=cos, sin=sin, q=q, scales=cache.scales(cfg),
                max_len=max(cache.lens), pt=cache.page_table, lens=cache.seq_lens)


def _args(c, q=None, pt=None, lens=None, scales=None):
    cache, cfg = c["cache"], c["cfg"]
    return (c["q"] if q is None else q, c["prm"].q.gain, 1e-6, cache.kc_pages, cache.kr_pages, cache.v_pages,
            cache.summ_pages, c["pt"] if pt is None else pt, c["lens"] if lens is None else lens, c["cos"],
            c["sin"], c["scales"] if scales is None else scales, cfg.sinks, cfg.window, cfg.k_blocks,
            c["max_len"])


def _fresh(c, q=None, pt=None, lens=None, scales=None):
    """The step through the C-ABI on a workspace allocated zero-filled for it."""
    q, qg, eps, kcp, krp, vp, sp, pt, lens, cos, sin, sc, S, W, k, max_len = _args(c, q, pt, lens, scales)
    Bd, Hq, d = q.shape
    Hkv, m = sp.shape[1], sp.shape[2]
    nbytes = ops.decode_workspace_bytes(Bd, Hq, Hkv, d, k, W, max_len)
    ws = torch.zeros(nbytes, dtype=torch.uint8, device=q.device)
    out = torch.full_like(q, 7.0)
    sidx = torch.full((Bd, Hkv, k), -7, dtype=torch.int32, device=q.device)
    scnt = torch.full((Bd, Hkv), -7, dtype=torch.int32, device=q.device)
    p = lambda t: _lib.ctypes.c_void_p(t.data_ptr())
    st = ops.lib().hba_decode_fwd(ops._code(q), p(q), p(qg), eps, p(kcp), p(krp), p(vp), p(sp), p(pt),
                                  pt.shape[1], p(lens), p(cos), p(sin), p(sc), Bd, Hq, Hkv, d, m, S, W, ops.BLOCK,
                                  k, max_len, p(ws), nbytes, p(out), p(sidx), p(scnt),
                                  _lib.ctypes.c_void_p(torch.cuda.current_stream(q.device).cuda_stream))
    ops.check(st, "hba_decode_fwd")
    return out, sidx, scnt


def _noalloc(c):
    q = c["q"]
    Bd, Hkv, k = q.shape[0], c["cache"].summ_pages.shape[1], c["cfg"].k_blocks
    out = torch.full_like(q, 7.0)
    sidx = torch.full((Bd, Hkv, k), -7, dtype=torch.int32, device=q.device)
    scnt = torch.full((Bd, Hkv), -7, dtype=torch.int32, device=q.device)
    ops.decode_fwd_noalloc(*_args(c), out, sidx, scnt)
    return out, sidx, scnt


def _same(a, b, what):
    torch.cuda.synchronize()
    for x, y, name in zip(a, b, ("out", "sel_idx", "sel_cnt")):
        assert torch.equal(x, y), (what, name)


def _lens(count, lo, hi, seed):
    return [int(v) for v in np.random.RandomState(seed).randint(lo, hi + 1, count)]


def test_decode_workspace_reuse_across_batch_sizes(dev, monkeypatch):
    """80 pairs after 32 pairs of longer sequences (whose chunk values lie
    where the larger call's counters would start if the counter region
    grew with the batch), on both shared workspaces."""
    monkeypatch.setenv("HBA_DECODE_KERNEL", "fused")
    a = _cache(dev, torch.bfloat16, _lens(40, 3000, 6000, 1), seed=11)    # 80 pairs
    b = _cache(dev, torch.bfloat16, _lens(16, 12000, 20000, 2), seed=12)  # 32 pairs, 4-5 score chunks
    ra, rb = _fresh(a), _fresh(b)
    _same(_noalloc(b), rb, "noalloc 32 pairs")
    _same(_noalloc(a), ra, "noalloc 80 pairs after 32")
    _same(_noalloc(b), rb, "noalloc 32 pairs after 80")
    for c, r, what in ((a, ra, "decode_fwd 80"), (b, rb, "decode_fwd 32"), (a, ra, "decode_fwd 80 after 32")):
        _same(ops.decode_fwd(*_args(c)), r, what)


def test_decode_workspace_reuse_fp32_then_bf16(dev, monkeypatch):
    """A bf16 call of 80 pairs after an fp32 call of 16 pairs (the fp32
    three-launch layout) on the no-allocation scratch."""
    monkeypatch.setenv("HBA_DECODE_KERNEL", "fused")
    c32 = _cache(dev, torch.float32, _lens(8, 12000, 20000, 3), seed=13)
    a = _cache(dev, torch.bfloat16, _lens(40, 3000, 6000, 4), seed=14)
    r32, ra = _fresh(c32), _fresh(a)
    _same(_noalloc(c32), r32, "noalloc fp32")
    _same(_noalloc(a), ra, "noalloc bf16 after fp32")
    _same(ops.decode_fwd(*_args(c32)), r32, "decode_fwd fp32")
    _same(ops.decode_fwd(*_args(a)), ra, "decode_fwd bf16 after fp32")


def test_decode_batch_beyond_one_launch_of_counters(dev, monkeypatch):
    """2100 sequences x 2 KV heads = 4200 pairs (more than one fused launch
    counts): the same bits as the batch decoded in two halves of 1050.  The
    sequences share the pages of 40 cached ones (page-table rows repeated)."""
    monkeypatch.setenv("HBA_DECODE_KERNEL", "fused")
    a = _cache(dev, torch.bfloat16, _lens(40, 1500, 6000, 5), seed=15)
    Bd = 2100
    rep = torch.arange(Bd, device=dev) % 40
    pt = a["pt"][rep].contiguous()
    lens = a["lens"][rep].contiguous()
    scales = a["scales"][rep].contiguous()
    q = torch.randn(Bd, 14, 64, generator=torch.Generator().manual_seed(16)).to(torch.bfloat16).to(dev)
    whole = _fresh(a, q, pt, lens, scales)
    h = Bd // 2
    halves = [_fresh(a, q[s].contiguous(), pt[s].contiguous(), lens[s].contiguous(), scales[s].contiguous())
              for s in (slice(0, h), slice(h, Bd))]
    joined = tuple(torch.cat([halves[0][i], halves[1][i]]) for i in range(3))
    _same(whole, joined, "4200 pairs vs two launches of 2100")
    # and the first 40 rows equal the cache's own sequences' step
    ra = _fresh(a, q[:40].contiguous())
    _same(tuple(t[:40] for t in whole), ra, "rows 0..39")
