"""Paged KV cache and the decode step.

The reference has no decode path or KV cache.  The decode step here is row
L-1 of hba_attention_eval (src/hba/attention.py:610-713) for a sequence of
length L, served from a cache laid out for the operator:

  kc_pages   [P, Hkv, 64*d]  QKNorm'd NoPE keys (normalised once, on append)
  kr_pages   [P, Hkv, 64*d]  the same keys rotated at their own positions
  v_pages    [P, Hkv, 64*d]  values
  summ_pages [P, Hkv, m, d]  slot summaries of full pages
  page_table int32 [batch, max_pages]  logical page -> physical page
  seq_lens   int32 [batch]   tokens in the cache (the current one included)

Within a page (64 tokens of one KV head) keys and values are stored in the
order the decode kernel's MFMA tiles read them, so that each of its operand
loads is one contiguous 1 KB run (key_offsets / value_offsets give the place
of token j, element t; the kernels use the same formulas).  key_rows /
value_rows read pages back as [.., Hkv, 64, d] token rows.

A key's rotation depends only on its own position, so it is applied once, on
append, and the window reads kr directly (the query is rotated in the kernel
with the caller's cos/sin tables).  The second key copy costs 2*d bytes per
token and KV head (bf16).  A page's summary is written when the page fills;
it is read only once the page has left the window.
"""
import torch

from . import ops
from .config import union_scale

PAGE = ops.BLOCK


def key_offsets(d, device=None):
    """Storage offset of key j, element t within a key page, as a [64, d]
    int64 tensor: ((mt * d/32 + ks) * 64 + l16 + 16*lg) * 8 + e with
    mt = 2*(j//32) + (j//4)%2, l16 = 4*((j%32)//8) + j%4, ks = t//32,
    lg = (t%32)//8, e = t%8."""
    j = torch.arange(PAGE, device=device)[:, None]
    t = torch.arange(d, device=device)[None, :]
    mt = 2 * (j // 32) + (j // 4) % 2
    l16 = 4 * ((j % 32) // 8) + j % 4
    return ((mt * (d // 32) + t // 32) * 64 + l16 + 16 * ((t % 32) // 8)) * 8 + t % 8


def value_offsets(d, device=None):
    """Storage offset of token j, element t within a value page, as a
    [64, d] int64 tensor: ((t//16 * 2 + j//32) * 64 + t%16 + 16*((j%32)//8)) * 8
    + j%8."""
    j = torch.arange(PAGE, device=device)[:, None]
    t = torch.arange(d, device=device)[None, :]
    return (((t // 16) * 2 + j // 32) * 64 + t % 16 + 16 * ((j % 32) // 8)) * 8 + j % 8


class PagedKVCache:
    def __init__(self, cfg, batch, max_len, dtype, device, num_pages=None):
        self.cfg = cfg
        self.batch = batch
        self.max_len = max_len
        self.max_pages = (max_len + PAGE - 1) // PAGE
        P = num_pages if num_pages is not None else batch * self.max_pages
        Hkv, d, m = cfg.n_kv, cfg.head_dim, cfg.slots
        self.kc_pages = torch.zeros(P, Hkv, PAGE * d, dtype=dtype, device=device)
        self.kr_pages = torch.zeros(P, Hkv, PAGE * d, dtype=dtype, device=device)
        self.v_pages = torch.zeros(P, Hkv, PAGE * d, dtype=dtype, device=device)
        self._koff = key_offsets(d, device).reshape(-1)
        self._voff = value_offsets(d, device).reshape(-1)
        self.summ_pages = torch.zeros(P, Hkv, m, d, dtype=dtype, device=device)
        self.page_table = torch.zeros(batch, self.max_pages, dtype=torch.int32, device=device)
        self.seq_lens = torch.zeros(batch, dtype=torch.int32, device=device)
        self.lens = [0] * batch
        self._table = [[] for _ in range(batch)]
        self._free = list(range(P - 1, -1, -1))

    def _ensure_pages(self, s, length):
        need = (length + PAGE - 1) // PAGE
        if need > self.max_pages:
            raise ValueError(f"sequence {s}: length {length} exceeds max_len {self.max_len}")
        new = []
        while len(self._table[s]) < need:
            if not self._free:
                raise RuntimeError("paged KV cache is out of pages")
            p = self._free.pop()
            self._table[s].append(p)
            new.append(p)
        return new

    def _sync_table(self):
        rows = [t + [0] * (self.max_pages - len(t)) for t in self._table]
        self.page_table.copy_(torch.tensor(rows, dtype=torch.int32))
        self.seq_lens.copy_(torch.tensor(self.lens, dtype=torch.int32))

    def load(self, s, kc_seq, kr_seq, v_seq, summ):
        """Fill sequence s with already-QKNorm'd keys kc_seq [L, Hkv, d], their
        rotations kr_seq [L, Hkv, d] and values v_seq [L, Hkv, d] (a prefill's
        outputs: hba_prep_keys' kc and kr), and summarise its full pages.
        Setup path: plain tensor copies."""
        L = kc_seq.shape[0]
        self._ensure_pages(s, L)
        pages = torch.tensor(self._table[s], dtype=torch.long, device=self.kc_pages.device)
        npg = (L + PAGE - 1) // PAGE
        pad = npg * PAGE - L
        Hkv, d = kc_seq.shape[1], kc_seq.shape[2]

        def paged(x, off):
            rows = torch.nn.functional.pad(x, (0, 0, 0, 0, 0, pad)).view(npg, PAGE, Hkv, d).transpose(1, 2)
            out = torch.empty(npg, Hkv, PAGE * d, dtype=self.kc_pages.dtype, device=self.kc_pages.device)
            out[:, :, off] = rows.reshape(npg, Hkv, PAGE * d).to(out.dtype)
            return out

        self.kc_pages[pages[:npg]] = paged(kc_seq, self._koff)
        self.kr_pages[pages[:npg]] = paged(kr_seq, self._koff)
        self.v_pages[pages[:npg]] = paged(v_seq, self._voff)
        self.lens[s] = L
        self._sync_table()
        full = pages[: L // PAGE]
        if full.numel():
            ops.summarize_pages(self.kc_pages, full, summ.probes, summ.proj, self.summ_pages)

    def append(self, k_new, v_new, qkn, summ, cos, sin):
        """Append one token per sequence (raw k_new, v_new [batch, Hkv, d]):
        QKNorm, rotation at the token's position and the writes in one kernel;
        summarise the pages that just filled.  cos/sin: fp32 [>= max_len, d]."""
        for s in range(self.batch):
            self._ensure_pages(s, self.lens[s] + 1)
            self.lens[s] += 1
        self._sync_table()
        cfg = self.cfg
        kg = qkn.k.gain if getattr(cfg, "qknorm", False) else None
        keps = float(qkn.k.eps) if kg is not None else 1e-6
        if cos.shape[0] < max(self.lens):
            raise ValueError(f"cos/sin tables cover {cos.shape[0]} positions, need {max(self.lens)}")
        ops.kv_append(k_new, v_new, kg, keps, cos, sin, self.page_table, self.seq_lens, self.kc_pages,
                      self.kr_pages, self.v_pages)
        done = [self._table[s][self.lens[s] // PAGE - 1] for s in range(self.batch)
                if self.lens[s] % PAGE == 0]
        if done:
            ops.summarize_pages(self.kc_pages, torch.tensor(done, dtype=torch.int32), summ.probes,
                                summ.proj, self.summ_pages)

    def key_rows(self, pages, rotated=False):
        """Keys of physical pages (int or index tensor) as token rows
        [..., Hkv, 64, d] (the rotated copy with rotated=True)."""
        src = (self.kr_pages if rotated else self.kc_pages)[pages]
        return src[..., self._koff].unflatten(-1, (PAGE, self.cfg.head_dim))

    def value_rows(self, pages):
        """Values of physical pages as token rows [..., Hkv, 64, d]."""
        return self.v_pages[pages][..., self._voff].unflatten(-1, (PAGE, self.cfg.head_dim))

    def scales(self, cfg=None):
        cfg = cfg or self.cfg
        return torch.tensor([union_scale(cfg, cfg.head_dim, max(L, 1)) for L in self.lens],
                            dtype=torch.float32, device=self.kc_pages.device)


def hba_decode_step(q, cache, cfg, qkn, cos, sin, scales=None):
    """Union attention of each sequence's new query q [batch, Hq, d] (raw;
    QKNorm and RoPE at position L-1 in the kernel) over the cache.  Returns
    (out [batch, Hq, d], selected page ids [batch, Hkv, k], counts [batch, Hkv])."""
    qg = qkn.q.gain if getattr(cfg, "qknorm", False) else None
    qeps = float(qkn.q.eps) if qg is not None else 1e-6
    sc = cache.scales(cfg) if scales is None else scales
    max_len = max(cache.lens)
    return ops.decode_fwd(q, qg, qeps, cache.kc_pages, cache.kr_pages, cache.v_pages, cache.summ_pages,
                          cache.page_table, cache.seq_lens, cos, sin, sc, cfg.sinks, cfg.window, cfg.k_blocks,
                          max_len)
