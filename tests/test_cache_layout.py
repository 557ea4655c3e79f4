"""The paged cache's in-page layouts (hba_amd.decode.key_offsets /
value_offsets; the kernels use the same formulas): permutations of the page,
with each 16-byte MFMA operand load of the decode kernel one contiguous 1 KB
run across the 64 lanes of a wave."""
import torch

from hba_amd.decode import key_offsets, value_offsets


def dperm_key(mt, r):
    """Key held by row r of S^T tile mt (the decode kernel's tile order)."""
    return 32 * (mt >> 1) + 8 * (r >> 2) + 4 * (mt & 1) + (r & 3)


def test_offsets_are_permutations():
    for d in (64, 128):
        for off in (key_offsets(d), value_offsets(d)):
            assert off.shape == (64, d)
            assert torch.equal(off.reshape(-1).sort().values, torch.arange(64 * d))


def test_key_operand_loads_are_contiguous():
    for d in (64, 128):
        off = key_offsets(d)
        for mt in range(4):
            for ks in range(d // 32):
                run = []
                for lane in range(64):
                    l16, lg = lane % 16, lane // 16
                    j, t0 = dperm_key(mt, l16), 32 * ks + 8 * lg
                    chunk = off[j, t0:t0 + 8]
                    assert torch.equal(chunk, chunk[0] + torch.arange(8))    # 8 elements, 16 bytes
                    run.append(int(chunk[0]))
                base = ((mt * (d // 32) + ks) * 64) * 8
                assert run == [base + 8 * lane for lane in range(64)]


def test_value_operand_loads_are_contiguous():
    for d in (64, 128):
        off = value_offsets(d)
        for dt in range(d // 16):
            for h in range(2):
                run = []
                for lane in range(64):
                    l16, lg = lane % 16, lane // 16
                    t, j0 = 16 * dt + l16, 32 * h + 8 * lg
                    chunk = off[j0:j0 + 8, t]
                    assert torch.equal(chunk, chunk[0] + torch.arange(8))
                    run.append(int(chunk[0]))
                assert run == [((dt * 2 + h) * 64) * 8 + 8 * lane for lane in range(64)]


def test_scale_table_matches_union_scale():
    """The cache's per-length scale table (gathered by seq_lens on the device)
    holds union_scale(cfg, d, max(L, 1)) rounded to fp32 for every L: it is
    evaluated only past n_cal, where the log-length temperature starts, and the
    closed form 1/d * (1 + c * log(L / n_cal)) fixes a few entries."""
    import math

    import hba_amd
    cfg = hba_amd.HBAConfig(native_ctx=1000, temp_c=0.1)
    c = hba_amd.PagedKVCache(cfg, 2, 3000, torch.bfloat16, "cpu")
    tab = c.scale_table()
    want = torch.tensor([hba_amd.union_scale(cfg, 64, max(L, 1)) for L in range(3001)], dtype=torch.float32)
    assert tab.shape == (3001,) and torch.equal(tab, want)
    for L, v in ((0, 1 / 64), (1, 1 / 64), (1000, 1 / 64), (2000, (1 + 0.1 * math.log(2)) / 64),
                 (3000, (1 + 0.1 * math.log(3)) / 64)):
        assert tab[L].item() == torch.tensor(v, dtype=torch.float32).item(), L
    assert c.scale_table() is tab                                # built once per scale setting
    for other in (hba_amd.HBAConfig(temp_c=0.0), hba_amd.HBAConfig(qknorm=False, head_dim=128)):
        t2 = c.scale_table(other)
        assert torch.equal(t2, torch.full((3001,), hba_amd.union_scale(other, other.head_dim, 5),
                                          dtype=torch.float32))
