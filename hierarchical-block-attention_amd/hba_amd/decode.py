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
import math

import torch

from . import ops
from .config import content_scale, union_scale

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
        self._scale_tabs = {}
        self._scales = torch.zeros(batch, dtype=torch.float32, device=device)   # written by append
        self._scales_ok = False          # _scales holds the scales of the current lengths
        self.scale_table()

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
        self._scales_ok = False
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

    def reserve(self, length=None):
        """Allocate every sequence's pages up to `length` tokens (default
        max_len) and write the page table, so that later appends allocate
        nothing (a captured decode loop needs this)."""
        length = self.max_len if length is None else length
        for s in range(self.batch):
            self._ensure_pages(s, length)
        self._sync_table()

    def append(self, k_new, v_new, qkn, summ, cos, sin):
        """Append one token per sequence (raw k_new, v_new [batch, Hkv, d]) in
        one launch: QKNorm, rotation at the token's position, the writes, the
        summaries of a page the token fills, seq_lens += 1 and the new
        lengths' scales, all on the device (page-table entries are written
        only when a page is allocated): no host round trip.  cos/sin: fp32
        [>= max_len, d]."""
        need = max(self.lens) + 1
        if need > self.max_len:
            raise ValueError(f"length {need} exceeds max_len {self.max_len}")
        if cos.shape[0] < need:
            raise ValueError(f"cos/sin tables cover {cos.shape[0]} positions, need {need}")
        for s in range(self.batch):
            first = len(self._table[s])
            for i, p in enumerate(self._ensure_pages(s, self.lens[s] + 1)):
                self.page_table[s, first + i] = p
        cfg = self.cfg
        kg = qkn.k.gain if getattr(cfg, "qknorm", False) else None
        keps = float(qkn.k.eps) if kg is not None else 1e-6
        ops.kv_append_advance(k_new, v_new, kg, keps, cos, sin, self.page_table, self.seq_lens, self.kc_pages,
                              self.kr_pages, self.v_pages, summ.probes, summ.proj, self.summ_pages,
                              self.scale_table(), self._scales)
        self._scales_ok = True
        for s in range(self.batch):
            self.lens[s] += 1

    def key_rows(self, pages, rotated=False):
        """Keys of physical pages (int or index tensor) as token rows
        [..., Hkv, 64, d] (the rotated copy with rotated=True)."""
        src = (self.kr_pages if rotated else self.kc_pages)[pages]
        return src[..., self._koff].unflatten(-1, (PAGE, self.cfg.head_dim))

    def value_rows(self, pages):
        """Values of physical pages as token rows [..., Hkv, 64, d]."""
        return self.v_pages[pages][..., self._voff].unflatten(-1, (PAGE, self.cfg.head_dim))

    def scale_table(self, cfg=None):
        """fp32 [max_len + 1] table on the cache's device: entry L is
        union_scale(cfg, d, max(L, 1)), the scale of a length-L step (the
        same Python float rounded to fp32 as a host-built tensor).  Built once
        per scale setting (the cache's own at construction)."""
        cfg = cfg or self.cfg
        d = cfg.head_dim
        qk, c = bool(getattr(cfg, "qknorm", False)), float(getattr(cfg, "temp_c", 0.0))
        n_cal = (getattr(cfg, "n_cal", None) or getattr(cfg, "native_ctx", None)) if qk and c != 0.0 else None
        key = (qk, getattr(cfg, "content_scale_mode", "inv_d"), c, n_cal, d)
        tab = self._scale_tabs.get(key)
        if tab is None:
            one = union_scale(cfg, d, 1)
            vals = [one] * (self.max_len + 1)
            if n_cal is not None:            # past n_cal: content_scale * (1 + c * log(L / n_cal))
                cs = content_scale(cfg, d)
                first = max(int(n_cal), 1)
                vals[first:] = [cs * (1.0 + c * math.log(max(L / n_cal, 1.0)))
                                for L in range(first, self.max_len + 1)]
            tab = torch.tensor(vals, dtype=torch.float32, device=self.kc_pages.device)
            self._scale_tabs[key] = tab
        return tab

    def scales(self, cfg=None):
        """fp32 [batch] scales of the current lengths: the ones the last
        append wrote, or gathered from the table on the device."""
        if self._scales_ok and (cfg is None or cfg is self.cfg):
            return self._scales
        return torch.index_select(self.scale_table(cfg), 0, self.seq_lens)


def hba_decode_step(q, cache, cfg, qkn, cos, sin, scales=None, max_len=None):
    """Union attention of each sequence's new query q [batch, Hq, d] (raw;
    QKNorm and RoPE at position L-1 in the kernel) over the cache.  Returns
    (out [batch, Hq, d], selected page ids [batch, Hkv, k], counts [batch, Hkv]).
    max_len sizes the step's launch (default: the longest sequence; any
    value >= it gives the same selection and an output within rounding)."""
    qg = qkn.q.gain if getattr(cfg, "qknorm", False) else None
    qeps = float(qkn.q.eps) if qg is not None else 1e-6
    sc = cache.scales(cfg) if scales is None else scales
    if max_len is None:
        max_len = max(cache.lens)
    elif max_len < max(cache.lens):
        raise ValueError(f"max_len {max_len} is below the longest sequence ({max(cache.lens)})")
    return ops.decode_fwd(q, qg, qeps, cache.kc_pages, cache.kr_pages, cache.v_pages, cache.summ_pages,
                          cache.page_table, cache.seq_lens, cos, sin, sc, cfg.sinks, cfg.window, cfg.k_blocks,
                          max_len)


class DecodeLoop:
    """The decode loop over a paged cache, two launches per token: the append
    (hba_kv_append_advance: the new keys and values, the summaries of a page
    they fill, seq_lens += 1 and the step scales) and the step
    (hba_decode_fwd), called straight through the C-ABI with arguments
    prepared once -- or, with graph=True, both captured once as a HIP graph
    and replayed per token.

    The cache's pages are reserved up to max_len and the step is sized for
    max_len, so nothing per token depends on host state; the host keeps the
    cache's length mirror.  out, sel_idx and sel_cnt are static outputs that
    every step overwrites.  In graph mode q, k, v are static input buffers
    (step() copies into them; or write them and call step() with no
    arguments) and replays run on the current stream; eager steps run on the
    current stream of the cache's device."""

    def __init__(self, cache, cfg, qkn, summ, cos, sin, graph=False):
        dev = cache.kc_pages.device
        ops._dev(cache.kc_pages)
        B, Hq, Hkv, d, k = cache.batch, cfg.n_heads, cfg.n_kv, cfg.head_dim, cfg.k_blocks
        dt = cache.kc_pages.dtype
        if cos.shape[0] < cache.max_len or cos.shape[-1] != d or sin.shape != cos.shape:
            raise ValueError(f"cos/sin: expected [>= {cache.max_len}, {d}] tables")
        cache.reserve()
        self.cache, self.cfg, self.dev = cache, cfg, dev
        self._shape_q, self._shape_kv, self._dtype = (B, Hq, d), (B, Hkv, d), dt
        f32 = lambda t: None if t is None else t.detach().to(device=dev, dtype=torch.float32).contiguous()
        qk = getattr(cfg, "qknorm", False)
        qg, kg = (f32(qkn.q.gain), f32(qkn.k.gain)) if qk else (None, None)
        qeps = float(qkn.q.eps) if qk else 1e-6
        keps = float(qkn.k.eps) if qk else 1e-6
        cs, sn = f32(cos), f32(sin)
        probes, proj = f32(summ.probes), f32(summ.proj)
        m = probes.shape[1]
        tab = cache.scale_table(cfg)
        sc = torch.zeros(B, dtype=torch.float32, device=dev)
        self.out = torch.empty(B, Hq, d, dtype=dt, device=dev)
        self.sel_idx = torch.empty(B, Hkv, k, dtype=torch.int32, device=dev)
        self.sel_cnt = torch.empty(B, Hkv, dtype=torch.int32, device=dev)
        nbytes = ops.decode_workspace_bytes(B, Hq, Hkv, d, k, cfg.window, cache.max_len)
        ws = ops._decode_workspace(dev, nbytes)
        self._keep = (qg, kg, cs, sn, probes, proj, tab, sc, ws)      # what the prepared pointers point at
        p = lambda t: None if t is None else t.data_ptr()
        c = cache
        code = ops._code(c.kc_pages)
        self._app = [code, None, None, p(kg), keps, p(cs), p(sn), cs.shape[0], p(c.page_table),
                     c.page_table.shape[1], p(c.seq_lens), B, Hkv, d, PAGE, p(c.kc_pages), p(c.kr_pages),
                     p(c.v_pages), p(probes), p(proj), m, p(c.summ_pages), p(tab), tab.numel(), p(sc), None]
        self._dec = [code, None, p(qg), qeps, p(c.kc_pages), p(c.kr_pages), p(c.v_pages), p(c.summ_pages),
                     p(c.page_table), c.page_table.shape[1], p(c.seq_lens), p(cs), p(sn), p(sc), B, Hq, Hkv, d, m,
                     cfg.sinks, cfg.window, PAGE, k, c.max_len, p(ws), nbytes, p(self.out), p(self.sel_idx),
                     p(self.sel_cnt), None]
        self._lib = ops.lib()
        self.graph = None
        if graph:
            self.q = torch.zeros(self._shape_q, dtype=dt, device=dev)
            self.k = torch.zeros(self._shape_kv, dtype=dt, device=dev)
            self.v = torch.zeros(self._shape_kv, dtype=dt, device=dev)
            self.graph = torch.cuda.CUDAGraph()
            with torch.cuda.device(dev), torch.cuda.graph(self.graph):
                self._launch(self.q, self.k, self.v)

    def _launch(self, q, k, v):
        st = torch.cuda.current_stream(self.dev).cuda_stream
        a = self._app
        a[1], a[2], a[-1] = k.data_ptr(), v.data_ptr(), st
        ops.check(self._lib.hba_kv_append_advance(*a), "hba_kv_append_advance")
        b = self._dec
        b[1], b[-1] = q.data_ptr(), st
        ops.check(self._lib.hba_decode_fwd(*b), "hba_decode_fwd")

    def step(self, q=None, k=None, v=None):
        """Append k, v [batch, Hkv, d] (raw) and decode q [batch, Hq, d] (raw)
        for every sequence.  Returns the static (out, sel_idx, sel_cnt)."""
        c = self.cache
        if max(c.lens) + 1 > c.max_len:
            raise ValueError(f"the cache holds at most {c.max_len} tokens per sequence")
        if self.graph is not None:
            for buf, x in ((self.q, q), (self.k, k), (self.v, v)):
                if x is not None:
                    buf.copy_(x)
            self.graph.replay()
        else:
            for x, shp, what in ((q, self._shape_q, "q"), (k, self._shape_kv, "k"), (v, self._shape_kv, "v")):
                if (x is None or x.shape != shp or x.dtype != self._dtype or x.device != self.dev
                        or not x.is_contiguous()):
                    raise ValueError(f"{what}: expected a contiguous {self._dtype} tensor {shp} on {self.dev}")
            if torch.cuda.current_device() != self.dev.index:
                with torch.cuda.device(self.dev):
                    self._launch(q, k, v)
            else:
                self._launch(q, k, v)
        c._scales_ok = False
        for s in range(c.batch):
            c.lens[s] += 1
        return self.out, self.sel_idx, self.sel_cnt
