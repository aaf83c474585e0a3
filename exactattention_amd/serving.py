"""A serving-loop layer over the certified attention: a paged K/V cache with per-sequence block
tables, chunked prefill, batched decode and speculative tree verification behind one attention
call, every output bit certified (or flagged) by the HIP library.

Reference pattern: the speculative decoding demo drives the reference kernels the same way
(scripts/spec_decode_demo.py:57-73: a prefix cache, draft nodes appended after it, one
verification launch with a tree mask, the accepted path kept); the reference leaves the cache
management to that script. Here the cache lives on the device:

  * K and V pools in NHD pages [num_pages, page_size, Hkv, d] of bf16 bits, pages handed out from a
    free list; block table [max_seqs, max_pages_per_seq] int32, one row per sequence slot;
  * optionally the int8 digit tiles of the prefill path (the KV slice format, exactattn_hip.h
    ea_hip_kv_digits_update), so a prefill chunk or a tree verification reads its K/V tiles
    instead of slicing the whole prefix again. They are re-sliced lazily: an append or a truncation
    only marks the slot's tiles stale from its first changed key, and the stale tiles of every slot
    are re-sliced in one update right before a call that reads the cache (the library says which
    calls do: ea_hip_reads_kv_digits). Decode steps, which read the bf16 cache, slice nothing.

Every call enqueues on torch's current stream and copies its result to the host (the caller sees
(out bits, flags) like the reference's backends).
"""

from __future__ import annotations

import ctypes

import numpy as np

from . import hip
from .formats import ExactAttentionDomainError, ExactAttentionUncertifiedError, alpha_bits_for, alpha_fp32_bits

TILE = 64  # keys per digit tile


class _Stager:
    """Small host-to-device uploads (indices, lengths, offsets) in one asynchronous copy per call
    through a ring of pinned buffers. A host buffer is written again only after the event of its
    last copy has completed, so the host waits only when it runs a whole ring ahead of the GPU.
    The device buffers are reused in stream order: the copy that refills one is enqueued after the
    kernels that read its previous contents."""

    def __init__(self, torch, dev, depth: int = 8, nbytes: int = 1 << 16):
        self.torch, self.dev, self.depth = torch, dev, depth
        self.cuda = dev.type == "cuda"
        self.host, self.devb, self.ev = [None] * depth, [None] * depth, [None] * depth
        self.cap = [0] * depth
        self.nbytes = nbytes
        self.i = 0

    def put(self, *arrays, stream=None):
        """Device tensors holding copies of the numpy arrays (same dtypes and shapes), copied on
        `stream` (a torch stream; torch's current stream by default)."""
        torch = self.torch
        arrays = [np.ascontiguousarray(a) for a in arrays]
        if not self.cuda:
            return [torch.from_numpy(a.copy()) for a in arrays]
        offs, at = [], 0
        for a in arrays:
            offs.append(at)
            at += (a.nbytes + 255) // 256 * 256
        i = self.i
        self.i = (i + 1) % self.depth
        if self.ev[i] is not None:
            self.ev[i].synchronize()
        if self.cap[i] < at:
            self.cap[i] = max(at, self.nbytes)
            self.host[i] = torch.empty(self.cap[i], dtype=torch.uint8, pin_memory=True)
            self.devb[i] = torch.empty(self.cap[i], dtype=torch.uint8, device=self.dev)
        h = self.host[i].numpy()
        for a, o in zip(arrays, offs):
            h[o:o + a.nbytes] = a.view(np.uint8).reshape(-1)
        d = self.devb[i]
        d[:at].copy_(self.host[i][:at], non_blocking=True)
        if self.ev[i] is None:
            self.ev[i] = torch.cuda.Event()
        self.ev[i].record(stream)
        return [d[o:o + a.nbytes].view(_TORCH_DTYPE[a.dtype.str[1:]]).view(a.shape) for a, o in zip(arrays, offs)]


_TORCH_DTYPE = {}


def _torch_dtypes(torch):
    if not _TORCH_DTYPE:
        _TORCH_DTYPE.update({"i4": torch.int32, "i8": torch.int64, "u1": torch.uint8, "i2": torch.int16})
    return _TORCH_DTYPE


class PagedKVCache:
    def __init__(self, num_pages: int, page_size: int, num_kv_heads: int, head_dim: int, max_seqs: int,
                 max_seq_len: int, digits: bool = True, device: str = "cuda"):
        import torch
        if page_size <= 0 or page_size & (page_size - 1):
            raise ValueError("page_size must be a power of two")
        self.torch = torch
        self.dev = torch.device(device)
        self.P, self.Hkv, self.d = page_size, num_kv_heads, head_dim
        self.max_seqs, self.max_seq_len = max_seqs, max_seq_len
        self.max_pages = (max_seq_len + page_size - 1) // page_size
        self.k = torch.zeros((num_pages, page_size, num_kv_heads, head_dim), dtype=torch.int16, device=self.dev)
        self.v = torch.zeros_like(self.k)
        self.block_table = torch.zeros((max_seqs, self.max_pages), dtype=torch.int32, device=self.dev)
        self.bt_host = np.zeros((max_seqs, self.max_pages), dtype=np.int32)
        _torch_dtypes(torch)
        self.stage = _Stager(torch, self.dev)
        self.free = list(range(num_pages))[::-1]
        self.pages = [[] for _ in range(max_seqs)]
        self.length = [0] * max_seqs
        self.live = [False] * max_seqs
        # first key whose digit tile is out of date, per slot (None: every tile is current)
        self.stale = [None] * max_seqs
        self.tiles = (max_seq_len + TILE - 1) // TILE
        self.digits = None
        if digits and head_dim == 128:
            lib = hip.load()
            n = lib.ea_hip_kv_digits_bytes(max_seqs, num_kv_heads, self.tiles)
            self.digit_stride = lib.ea_hip_kv_digits_bytes(1, num_kv_heads, self.tiles)  # bytes per slot
            self.digits = torch.zeros(n, dtype=torch.uint8, device=self.dev)

    # ---- sequence slots
    def add_sequence(self) -> int:
        for s in range(self.max_seqs):
            if not self.live[s]:
                self.live[s], self.length[s], self.pages[s], self.stale[s] = True, 0, [], None
                return s
        raise RuntimeError("no free sequence slot")

    def _check_slots(self, seqs) -> None:
        """Every slot an in-range, live sequence, and each at most once (nothing has changed yet)."""
        live, n, seen = self.live, self.max_seqs, set()
        for s in seqs:
            if not isinstance(s, (int, np.integer)) or not 0 <= s < n:
                raise ValueError(f"sequence slot {s!r} is outside [0, {n})")
            if not live[s]:
                raise ValueError(f"sequence slot {int(s)} holds no live sequence")
            seen.add(int(s))
        if len(seen) != len(seqs):
            raise ValueError("a slot may appear once per batch")

    def drop_sequence(self, s: int) -> None:
        self.free.extend(self.pages[s][::-1])
        self.pages[s], self.length[s], self.live[s], self.stale[s] = [], 0, False, None

    def _digit_base(self, s: int) -> int:
        return self.digits.data_ptr() + s * self.digit_stride

    def _geom1(self, s: int, T: int, Hq: int, seq_len: int) -> dict:
        """Serving geometry of one sequence slot (b = 0) over the shared pools."""
        P, Hkv, d = self.P, self.Hkv, self.d
        return dict(num_seqs=1, num_tokens=T, num_q_heads=Hq, num_kv_heads=Hkv, head_dim=d, head_dim_v=d,
                    q_seq_stride=T * Hq * d, q_tok_stride=Hq * d, q_head_stride=d,
                    o_seq_stride=T * Hq * d, o_tok_stride=Hq * d, o_head_stride=d,
                    k_page_stride=P * Hkv * d, k_slot_stride=Hkv * d, k_head_stride=d,
                    v_page_stride=P * Hkv * d, v_slot_stride=Hkv * d, v_head_stride=d,
                    page_size=P, block_table_stride=self.max_pages, max_seq_len=max(1, seq_len))

    # ---- writes
    def append(self, s: int, k_bits, v_bits) -> None:
        """Append n keys (k_bits, v_bits: (n, Hkv, d) uint16 arrays or int16 device tensors) to slot s;
        the digit tiles they touch are marked stale (flush re-slices them)."""
        self.append_batch([s], [len(k_bits)], k_bits, v_bits)

    def append_batch(self, seqs, counts, k_bits, v_bits) -> None:
        """Append counts[i] keys to slot seqs[i] for every i, the keys flattened in that order
        (k_bits, v_bits: (sum(counts), Hkv, d)); one device scatter for the batch. The digit tiles
        the keys land in are marked stale (flush re-slices them)."""
        plan = self._plan_append(seqs, counts, k_bits, v_bits)
        if plan is not None:
            self._apply_append(plan, self.stage.put(*plan["arrays"]))

    def _plan_append(self, seqs, counts, k_bits, v_bits, checked: bool = False):
        """Host half of an append: checks, page allocation, block-table mirror and lengths. Returns
        None for an empty append, else a plan whose "arrays" the caller uploads (in one staged copy
        with its own arrays appended) and hands, as device tensors in the same order, to
        _apply_append. checked: the caller has run _check_slots on seqs already."""
        torch = self.torch
        k_new = _dev16(torch, k_bits, self.dev)
        v_new = _dev16(torch, v_bits, self.dev)
        counts = [int(n) for n in counts]
        if len(counts) != len(seqs):
            raise ValueError("one count per sequence slot")
        if k_new.shape[0] != sum(counts) or v_new.shape[0] != sum(counts):
            raise ValueError("k/v must hold sum(counts) keys")
        if not checked:
            self._check_slots(seqs)
        if sum(counts) == 0:
            return None
        if all(n == 1 for n in counts):
            return self._plan_one_each(seqs, k_new, v_new)
        return self._plan_general(seqs, counts, k_new, v_new)

    def _plan_general(self, seqs, counts, k_new, v_new):
        """_plan_append after its checks, for any counts (at least one key in all)."""
        sa = np.asarray(seqs, dtype=np.int64)
        cnt = np.asarray(counts, dtype=np.int64)
        L = np.asarray(self.length, dtype=np.int64)[sa]
        if np.any(L + cnt > self.max_seq_len):
            raise ValueError("sequence longer than the cache's max_seq_len")
        have = np.asarray([len(self.pages[s]) for s in seqs], dtype=np.int64)
        need = np.maximum(0, (L + cnt + self.P - 1) // self.P - have)
        if int(need.sum()) > len(self.free):
            raise RuntimeError("out of pages")
        bt_pos, bt_val = [], []  # block-table entries of the new pages
        for i in np.flatnonzero(need):
            s = seqs[i]
            self.pages[s].extend(self.free.pop() for _ in range(int(need[i])))
            self.bt_host[s, :len(self.pages[s])] = self.pages[s]
            for p in range(int(have[i]), len(self.pages[s])):
                bt_pos.append(s * self.max_pages + p)
                bt_val.append(self.pages[s][p])
        b_of = np.repeat(np.arange(len(seqs)), cnt)
        pos = np.arange(int(cnt.sum())) - np.repeat(np.cumsum(cnt) - cnt - L, cnt)
        idx = self.bt_host[sa[b_of], pos // self.P].astype(np.int64) * self.P + pos % self.P
        stale, track = self.stale, self.digits is not None
        for s, a, e in zip(seqs, L.tolist(), (L + cnt).tolist()):
            self.length[s] = e
            if track:
                stale[s] = a if stale[s] is None else min(stale[s], a)
        arrays = [idx]
        if bt_pos:
            arrays += [np.asarray(bt_pos, dtype=np.int64), np.asarray(bt_val, dtype=np.int32)]
        return {"k": k_new.contiguous(), "v": v_new.contiguous(), "grown": bool(bt_pos), "arrays": arrays}

    def _plan_one_each(self, seqs, k_new, v_new):
        """_plan_append for one key per sequence (a decode step), in plain integer arithmetic: the
        same page allocation order and the same plan as the general path."""
        P, length, pages, free = self.P, self.length, self.pages, self.free
        news = 0
        for s in seqs:
            if length[s] + 1 > self.max_seq_len:
                raise ValueError("sequence longer than the cache's max_seq_len")
            news += length[s] // P >= len(pages[s])
        if news > len(free):
            raise RuntimeError("out of pages")
        idx, bt_pos, bt_val = [], [], []
        stale, track = self.stale, self.digits is not None
        for s in seqs:
            L, pg = length[s], pages[s]
            if L // P >= len(pg):  # the key opens a new page
                page = free.pop()
                pg.append(page)
                self.bt_host[s, len(pg) - 1] = page
                bt_pos.append(s * self.max_pages + len(pg) - 1)
                bt_val.append(page)
            idx.append(pg[L // P] * P + L % P)
            length[s] = L + 1
            if track:
                stale[s] = L if stale[s] is None else min(stale[s], L)
        arrays = [np.asarray(idx, dtype=np.int64)]
        if bt_pos:
            arrays += [np.asarray(bt_pos, dtype=np.int64), np.asarray(bt_val, dtype=np.int32)]
        return {"k": k_new.contiguous(), "v": v_new.contiguous(), "grown": bool(bt_pos), "arrays": arrays}

    def _apply_append(self, plan, dev, stream=None) -> None:
        """Device half of an append: the K/V scatter and the new pages' block-table entries, in
        one ea_hip_kv_append launch on `stream` (torch's current stream by default)."""
        self._kv_append(plan["k"], plan["v"], dev[0], int(dev[0].numel()),
                        dev[1] if plan["grown"] else None, dev[2] if plan["grown"] else None,
                        int(dev[1].numel()) if plan["grown"] else 0, stream)

    def _kv_append(self, k_new, v_new, dst, n, bt_pos, bt_val, n_bt, stream=None) -> None:
        if self.dev.type != "cuda":
            # a host-resident cache (bookkeeping without a GPU): plain tensor copies
            H, d = self.Hkv, self.d
            if n_bt:
                self.block_table.view(-1).index_copy_(0, bt_pos, bt_val)
            self.k.view(-1, H, d).index_copy_(0, dst, k_new.reshape(-1, H, d))
            self.v.view(-1, H, d).index_copy_(0, dst, v_new.reshape(-1, H, d))
            return
        rows = self.k.shape[0] * self.P
        hip._check(hip.load().ea_hip_kv_append(
            self.k.data_ptr(), self.v.data_ptr(), rows, self.Hkv * self.d, k_new.data_ptr(), v_new.data_ptr(),
            dst.data_ptr(), n, self.block_table.data_ptr(), self.block_table.numel(),
            None if bt_pos is None else bt_pos.data_ptr(), None if bt_val is None else bt_val.data_ptr(), n_bt,
            stream if stream is not None else hip._stream_ptr(self.torch)), "ea_hip_kv_append")

    def _mark_stale(self, s: int, key: int) -> None:
        if self.digits is not None:
            self.stale[s] = key if self.stale[s] is None else min(self.stale[s], key)

    def truncate(self, s: int, length: int) -> None:
        """Drop the keys at or past `length` (rejected draft nodes); the tile holding the new end is
        sliced again so its digits match the shorter sequence."""
        self._check_slots([s])
        if length < 0 or length > self.length[s]:
            raise ValueError("truncate cannot grow a sequence")
        self.length[s] = length
        keep = (length + self.P - 1) // self.P
        self.free.extend(self.pages[s][keep:][::-1])
        self.pages[s] = self.pages[s][:keep]
        if self.stale[s] is not None and self.stale[s] >= length:
            self.stale[s] = None  # the stale keys are gone
        if length % TILE:
            self._mark_stale(s, length - 1)  # the tile holding the new end: its tail is now empty

    def flush(self, stream=None) -> None:
        """Re-slice the stale digit tiles of every slot (keys stale[s] .. length[s] - 1), in one
        ea_hip_kv_digits_update on `stream` (torch's current stream by default)."""
        if self.digits is None:
            return
        dirty = [(s, a) for s, a in enumerate(self.stale) if a is not None and a < self.length[s]]
        self.stale = [None] * self.max_seqs
        if not dirty:
            return
        kb = np.zeros(self.max_seqs, dtype=np.int32)
        ke = np.zeros(self.max_seqs, dtype=np.int32)
        for s, a in dirty:
            kb[s], ke[s] = a, self.length[s]
        seq_d, kb_d, ke_d = self.stage.put(np.asarray(self.length, dtype=np.int32), kb, ke)
        self._reslice_all(seq_d, kb_d, ke_d, int((ke - kb).max()), stream)

    def _reslice_all(self, seq_d, kb_d, ke_d, span: int, stream=None) -> None:
        """Re-slice keys kb[s]..ke[s]-1 of every slot s (device int32 vectors over all max_seqs
        slots, seq_d their lengths): one update, where slots with an empty range exit at once."""
        torch = self.torch
        lib = hip.load()
        g = self._geom1(0, 1, self.Hkv, max(1, max(self.length)))
        g["num_seqs"] = self.max_seqs
        gc = hip.geometry(g)
        b = hip.Buffers(q=None, k=self.k.data_ptr(), v=self.v.data_ptr(), seq_len=seq_d.data_ptr(), kv_len=None,
                        block_table=self.block_table.data_ptr(), block_table_offset=None, tree_mask=None,
                        tree_base=None, out=None, flags=None)
        st = stream if stream is not None else hip._stream_ptr(torch)
        hip._check(lib.ea_hip_kv_digits_update(ctypes.byref(gc), ctypes.byref(b), kb_d.data_ptr(), ke_d.data_ptr(), span,
                                               ctypes.c_void_p(self.digits.data_ptr()), self.tiles, st),
                   "ea_hip_kv_digits_update")


class ExactAttentionBackend:
    """Certified attention over a PagedKVCache. `alpha` is the base-2 logit scale as an fp32
    value; `alpha_bits=` passes its bit pattern instead."""

    def __init__(self, cache: PagedKVCache, num_q_heads: int, alpha=None, out: str = "bf16", *, alpha_bits=None):
        self.cache, self.Hq, self.out = cache, num_q_heads, out
        self.alpha_bits = alpha_fp32_bits(alpha, alpha_bits)
        self.ws = None
        self._last = None  # the latest launch: its ea_* arguments and the tensors they point at
        self._geoms = {}   # ea_geometry per (B, T): only max_seq_len changes between launches

    def _launch(self, seqs, qd, kvl, tree_mask=None, tree_base=None, digits_slot=None, staged=None, stream=None):
        """Enqueue one ea_hip_attention call over sequences `seqs` on torch's current stream.
        qd: (B, T, Hq, d) int16 device tensor, row (b, t, h) = token t of sequence seqs[b];
        kvl: (B*T,) int32 device tensor of visible prefix lengths; staged: the device seq_len and
        block-table offset vectors of `seqs` when the caller uploaded them already. Returns device
        (out, flags)."""
        c = self.cache
        torch = c.torch
        lib = hip.load()
        B, T, Hq, d = qd.shape
        lens = [c.length[s] for s in seqs]
        gc = self._geoms.get((B, T, Hq))
        if gc is None:
            if len(self._geoms) >= 256:
                self._geoms.clear()  # batch shapes vary without bound in a long run: keep the cache small
            g = c._geom1(seqs[0], T, Hq, 1)
            g["num_seqs"] = B
            gc = self._geoms[(B, T, Hq)] = hip.geometry(g)
        gc.max_seq_len = max(1, max(lens))
        out = torch.empty((B, T, Hq, d), dtype=torch.int32 if self.out == "fp32" else torch.int16, device=c.dev)
        flags = torch.empty(B * T * Hq, dtype=torch.uint8, device=c.dev)
        tm = tb = None
        if staged is not None:
            seq, off = staged[0], staged[1]
        else:
            up = [np.asarray(lens, dtype=np.int32), np.asarray([s * c.max_pages for s in seqs], dtype=np.int64)]
            if tree_mask is not None:
                up += [np.asarray(tree_mask, dtype=np.uint64).view(np.int64).reshape(-1),
                       np.asarray(tree_base, dtype=np.int32)]
            dv = c.stage.put(*up)
            seq, off = dv[0], dv[1]
            if tree_mask is not None:
                tm, tb = dv[2], dv[3]
        o = hip.Options(alpha_bits=self.alpha_bits, out_fp32=int(self.out == "fp32"), splits=0, tier2=1)
        if digits_slot is not None and c.digits is not None:
            o.kv_digits = ctypes.c_void_p(c._digit_base(digits_slot))
            o.kv_digits_tiles = c.tiles
            if staged is not None and len(staged) > 2:
                # slot map: sequence b's tiles live at cache slot seqs[b]
                o.kv_digits = ctypes.c_void_p(c.digits.data_ptr())
                o.kv_digits_slot = staged[2].data_ptr()
            reads = ctypes.c_int32(0)
            hip._check(lib.ea_hip_reads_kv_digits(ctypes.byref(gc), ctypes.byref(o), ctypes.byref(reads)),
                       "ea_hip_reads_kv_digits")
            if reads.value:
                c.flush(stream)  # the stale tiles, re-sliced ahead of the call in stream order
        nb, ns = ctypes.c_size_t(0), ctypes.c_int32(0)
        hip._check(lib.ea_hip_workspace_size(ctypes.byref(gc), ctypes.byref(o), ctypes.byref(nb), ctypes.byref(ns)),
                   "ea_hip_workspace_size")
        if self.ws is None or self.ws.numel() < int(nb.value):
            self.ws = torch.empty(max(int(nb.value), 1 << 20), dtype=torch.uint8, device=c.dev)
        ws = self.ws
        b = hip.Buffers(q=qd.data_ptr(), k=c.k.data_ptr(), v=c.v.data_ptr(), seq_len=seq.data_ptr(),
                        kv_len=kvl.data_ptr(), block_table=c.block_table.data_ptr(), block_table_offset=off.data_ptr(),
                        tree_mask=None if tm is None else tm.data_ptr(), tree_base=None if tb is None else tb.data_ptr(),
                        out=out.data_ptr(), flags=flags.data_ptr())
        st = stream if stream is not None else hip._stream_ptr(torch)
        hip._check(lib.ea_hip_attention(ctypes.byref(gc), ctypes.byref(b), ctypes.byref(o), ws.data_ptr(), int(nb.value),
                                        st), "ea_hip_attention")
        self._last = {"args": (gc, b, o), "keep": (qd, kvl, seq, off, tm, tb, staged), "out": out, "flags": flags,
                      "ret": None}
        return out, flags

    def _exact_tier(self) -> None:
        """The host exact tier on the latest launch (ea_hip_exact_rows): waits for torch's current
        stream and recomputes every row left at flag 1 in place (flag 0, or 2 on a domain error)."""
        c = self.cache
        gc, b, o = self._last["args"]
        hip._check(hip.load().ea_hip_exact_rows(ctypes.byref(gc), ctypes.byref(b), ctypes.byref(o),
                                                hip._stream_ptr(c.torch)), "ea_hip_exact_rows")

    def _run(self, seqs, q, kv_len, tree_mask=None, tree_base=None, digits_slot=None):
        """_launch, then the result on the host: (out bits (B, T, Hq, d), flags); flag 2 raises."""
        c = self.cache
        torch = c.torch
        qd = _dev16(torch, q, c.dev).contiguous()
        (kvl,) = c.stage.put(np.asarray(kv_len, dtype=np.int32).reshape(-1))
        out, flags = self._launch(seqs, qd, kvl, tree_mask, tree_base, digits_slot)
        torch.cuda.current_stream().synchronize()  # the launch stream only, not the whole device
        fl = flags.cpu().numpy()
        if np.any(fl == 1):
            self._exact_tier()
            fl = flags.cpu().numpy()
        res = out.cpu().numpy()
        res = res.view(np.uint32) if self.out == "fp32" else res.view(np.uint16)
        if np.any(fl == 2):
            raise ExactAttentionDomainError("non-finite input or fp32 logit overflow")
        return res, fl

    def forward(self, query, key, value, seqs, query_lens):
        """One attention call per layer over a mixed batch, the way vLLM's attention backends are
        called: `query_lens[i]` new tokens of sequence slot `seqs[i]`, flattened in that order
        (query (num_tokens, Hq, d), key/value (num_tokens, Hkv, d), bf16 or int16 device tensors).
        Their K/V are appended to the cache; token j of sequence i attends the cached prefix and
        tokens 0..j of its chunk (a decode step is a chunk of one token). Enqueued on torch's
        current stream, no host synchronisation: returns device (out (num_tokens, Hq, d) bf16/fp32
        bits, flags (num_tokens, Hq) uint8; 0 certified, 1 not certified by the device tiers (the
        row holds +0), 2 domain error). Call check_flags(flags) before the next forward: it
        finishes flag-1 rows with the host exact tier, in place, and raises on flag 2."""
        c = self.cache
        torch = c.torch
        ql = [int(n) for n in query_lens]
        if len(ql) != len(seqs) or any(n <= 0 for n in ql):
            raise ValueError("query_lens must give a positive token count per sequence")
        c._check_slots(seqs)
        ntok = sum(ql)
        if query.shape[0] != ntok or key.shape[0] != ntok or value.shape[0] != ntok:
            raise ValueError("query/key/value must hold sum(query_lens) tokens")
        if not ql:
            # an empty batch: nothing to append or attend
            Hq, d = query.shape[1], query.shape[2]
            return (torch.empty((0, Hq, d), dtype=torch.int32 if self.out == "fp32" else torch.int16, device=c.dev),
                    torch.empty((0, Hq), dtype=torch.uint8, device=c.dev))
        B, T, Hq, d = len(ql), max(ql), query.shape[1], query.shape[2]
        prefix = [c.length[s] for s in seqs]
        plan = c._plan_append(seqs, ql, key, value, checked=True)
        lens = np.asarray([c.length[s] for s in seqs], dtype=np.int32)
        mine = [lens, np.asarray(seqs, dtype=np.int64) * c.max_pages, np.asarray(seqs, dtype=np.int32)]
        if T > 1:
            start = np.concatenate([[0], np.cumsum(ql)])
            b_of = np.repeat(np.arange(B), ql)
            j_of = np.arange(ntok) - start[b_of]
            kvl_h = np.zeros(B * T, dtype=np.int32)
            kvl_h[b_of * T + j_of] = np.asarray(prefix)[b_of] + j_of + 1
            mine += [kvl_h, (b_of * T + j_of).astype(np.int64)]
        n_app = len(plan["arrays"])
        ts = torch.cuda.current_stream(c.dev)
        st = ctypes.c_void_p(ts.cuda_stream)
        dev = c.stage.put(*plan["arrays"], *mine, stream=ts)
        c._apply_append(plan, dev[:n_app], st)
        staged = (dev[n_app], dev[n_app + 1], dev[n_app + 2])
        # one token per sequence sees the whole sequence: its visible length is the sequence's
        kvl = dev[n_app + 3] if T > 1 else dev[n_app]
        row = dev[n_app + 4] if T > 1 else None
        q16 = query.view(torch.int16) if query.dtype != torch.int16 else query
        if T == 1:
            qd = q16.reshape(B, 1, Hq, d).contiguous()
        else:
            qd = torch.zeros((B * T, Hq, d), dtype=torch.int16, device=c.dev)
            qd.index_copy_(0, row, q16)
            qd = qd.view(B, T, Hq, d)
        slots = list(seqs)
        out, flags = self._launch(slots, qd, kvl, digits_slot=slots[0], staged=staged, stream=st)
        self._last["keep"] += (q16, row)
        if T == 1:
            ret = (out.view(B, Hq, -1), flags.view(B, Hq))
        else:
            ret = (out.view(B * T, Hq, -1).index_select(0, row), flags.view(B * T, Hq).index_select(0, row))
        self._last["ret"] = (ret, row, T)
        return ret

    def check_flags(self, flags) -> None:
        """Synchronise on `flags` (from forward) and make every row usable: rows the device tiers
        left at flag 1 are recomputed by the host exact tier (in the returned out and flags, when
        `flags` is the latest forward's; otherwise ExactAttentionUncertifiedError); flag 2 raises
        ExactAttentionDomainError."""
        if bool((flags == 1).any().item()):
            last = self._last
            if last is None or last["ret"] is None or last["ret"][0][1] is not flags:
                raise ExactAttentionUncertifiedError("flag-1 rows of an earlier forward: call check_flags before "
                                                     "the next forward")
            self._exact_tier()
            (ret_out, ret_flags), row, T = last["ret"]
            if T > 1:
                ret_out.copy_(last["out"].view(-1, *ret_out.shape[1:]).index_select(0, row))
                ret_flags.copy_(last["flags"].view(-1, ret_flags.shape[1]).index_select(0, row))
        if bool((flags == 2).any().item()):
            raise ExactAttentionDomainError("non-finite input or fp32 logit overflow")

    def prefill(self, s: int, q, k, v):
        """Append T tokens' K/V to slot s and attend causally: token t sees the prefix and tokens
        0..t of the chunk. q (T, Hq, d), k/v (T, Hkv, d) bf16 bits. Returns (out (T, Hq, d), flags)."""
        c = self.cache
        L = c.length[s]
        T = q.shape[0]
        c.append(s, k, v)
        kv_len = (L + 1 + np.arange(T)).reshape(1, T)
        res, fl = self._run([s], np.asarray(q)[None], kv_len, digits_slot=s)
        return res[0], fl

    def decode(self, seqs, q, k, v):
        """One new token per sequence: q (B, Hq, d), k/v (B, Hkv, d). Returns (out (B, Hq, d), flags)."""
        c = self.cache
        for i, s in enumerate(seqs):
            c.append(s, np.asarray(k)[i:i + 1] if not hasattr(k, "data_ptr") else k[i:i + 1],
                     np.asarray(v)[i:i + 1] if not hasattr(v, "data_ptr") else v[i:i + 1])
        kv_len = np.array([[c.length[s]] for s in seqs])
        res, fl = self._run(list(seqs), np.asarray(q)[:, None], kv_len)
        return res[:, 0], fl

    def verify_tree(self, s: int, q, k, v, parents):
        """Speculative verification: N <= 64 draft nodes, parents[i] < i (-1: the prefix), appended
        after the prefix; node i attends the prefix and its root-to-node path. q (N, Hq, d), k/v
        (N, Hkv, d). Returns (out (N, Hq, d), flags); keep the accepted path with accept()."""
        c = self.cache
        N = q.shape[0]
        if N > 64:
            raise ValueError("at most 64 draft nodes")
        L = c.length[s]
        c.append(s, k, v)
        mask = np.zeros((1, N), dtype=np.uint64)
        for i in range(N):
            j, m = i, 0
            while j >= 0:
                m |= 1 << j
                j = parents[j]
            mask[0, i] = m
        res, fl = self._run([s], np.asarray(q)[None], np.full((1, N), L), tree_mask=mask, tree_base=[L],
                            digits_slot=s)
        return res[0], fl

    def accept(self, s: int, prefix_len: int, path, k, v) -> None:
        """Keep the accepted draft nodes `path` (node indices in draft order) after the prefix:
        the cache is cut back to the prefix and the path's K/V appended in order."""
        self.cache.truncate(s, prefix_len)
        if len(path):
            idx = np.asarray(path)
            self.cache.append(s, np.asarray(k)[idx], np.asarray(v)[idx])


class DecodeGraph:
    """One decode step of a fixed batch of sequence slots (one new token each), captured once in a
    HIP graph and replayed per step: the block-table update, the K/V scatter into the paged pools
    and the certified attention launch (the decode kernel reads the bf16 cache; the digit tiles the
    new keys land in are only marked stale, for the next call that reads them). Per step the host
    plans the appends (page allocation, scatter slots, lengths) into a pinned buffer, enqueues one
    copy of it and one graph launch on torch's current stream; there is no host synchronisation.

    The caller writes the step's inputs into the static tensors `q` (B, 1, Hq, d), `k` and `v`
    (B, Hkv, d) (int16 views of bf16) before calling step(); the outputs land in `out` and `flags`.
    `max_len` bounds every sequence's length while the graph lives: it sizes the split grid (the
    kernel skips the splits past a sequence's end), so a tight bound keeps the grid dense."""

    RING = 4  # pinned metadata buffers: the host may run this many steps ahead of the GPU

    def __init__(self, backend: "ExactAttentionBackend", seqs, max_len: int | None = None):
        import torch
        from .graph import EVENT_DISABLE_TIMING, HipGraph, hip_rt
        c = backend.cache
        self.be, self.c, self.torch = backend, c, torch
        c._check_slots(seqs)
        self.seqs = np.asarray(seqs, dtype=np.int64)
        B, Hq, Hkv, d = len(seqs), backend.Hq, c.Hkv, c.d
        self.B = B
        self.max_len = int(min(max_len or c.max_seq_len, c.max_seq_len))
        if max(c.length[s] for s in seqs) + 1 > self.max_len:
            raise ValueError("max_len is below a sequence's next length")
        dev = c.dev
        self.q = torch.zeros((B, 1, Hq, d), dtype=torch.int16, device=dev)
        self.k = torch.zeros((B, Hkv, d), dtype=torch.int16, device=dev)
        self.v = torch.zeros((B, Hkv, d), dtype=torch.int16, device=dev)
        fp32 = backend.out == "fp32"
        self.out = torch.empty((B, 1, Hq, d), dtype=torch.int32 if fp32 else torch.int16, device=dev)
        self.flags = torch.empty(B * Hq, dtype=torch.uint8, device=dev)
        # metadata layout (bytes): idx, bt_pos, bt_off (B int64); bt_val, kvl (B int32)
        lay = {}
        at = 0
        for name, n, dt in (("idx", B, np.int64), ("bt_pos", B, np.int64), ("bt_off", B, np.int64),
                            ("bt_val", B, np.int32), ("kvl", B, np.int32)):
            lay[name] = (at, n, dt)
            at += (n * np.dtype(dt).itemsize + 255) // 256 * 256
        self._nbytes = at
        self._host = [torch.zeros(at, dtype=torch.uint8, pin_memory=True) for _ in range(self.RING)]
        # numpy views of each pinned buffer's fields, made once
        self._hv = [{k: h.numpy()[o:o + n * np.dtype(dt).itemsize].view(dt) for k, (o, n, dt) in lay.items()}
                    for h in self._host]
        for hv in self._hv:
            hv["bt_off"][:] = self.seqs * c.max_pages
        self.meta = torch.zeros(at, dtype=torch.uint8, device=dev)
        tdt = {np.int64: torch.int64, np.int32: torch.int32}
        self.dv = {k: self.meta[o:o + n * np.dtype(dt).itemsize].view(tdt[dt]) for k, (o, n, dt) in lay.items()}
        self.h = hip_rt()
        self._ev = []
        for _ in range(self.RING):
            e = ctypes.c_void_p()
            if self.h.hipEventCreateWithFlags(ctypes.byref(e), EVENT_DISABLE_TIMING) != 0:
                raise RuntimeError("hipEventCreateWithFlags")
            self._ev.append(e)
        self._used = [False] * self.RING
        self._ring = 0
        # host mirrors of the batch's lengths and page counts
        self.L = np.asarray([c.length[s] for s in seqs], dtype=np.int64)
        self.npg = np.asarray([len(c.pages[s]) for s in seqs], dtype=np.int64)
        # the attention call's arguments, fixed for the graph's life
        lib = hip.load()
        g = c._geom1(int(self.seqs[0]), 1, Hq, self.max_len)
        g["num_seqs"] = B
        self.gc = hip.geometry(g)
        self.o = hip.Options(alpha_bits=backend.alpha_bits, out_fp32=int(fp32), splits=0, tier2=1)
        nb, ns = ctypes.c_size_t(0), ctypes.c_int32(0)
        hip._check(lib.ea_hip_workspace_size(ctypes.byref(self.gc), ctypes.byref(self.o), ctypes.byref(nb),
                                             ctypes.byref(ns)), "ea_hip_workspace_size")
        self.ws_bytes = int(nb.value)
        self.ws = torch.empty(max(self.ws_bytes, 256), dtype=torch.uint8, device=dev)
        self.bufs = hip.Buffers(q=self.q.data_ptr(), k=c.k.data_ptr(), v=c.v.data_ptr(),
                                seq_len=self.dv["kvl"].data_ptr(), kv_len=self.dv["kvl"].data_ptr(),
                                block_table=c.block_table.data_ptr(), block_table_offset=self.dv["bt_off"].data_ptr(),
                                tree_mask=None, tree_base=None, out=self.out.data_ptr(),
                                flags=self.flags.data_ptr())
        # captured on a side stream (capture records the work without running it); replayed on
        # torch's current stream, right after the step's metadata copy
        self.graph = HipGraph()
        cap = torch.cuda.Stream(device=dev)
        torch.cuda.synchronize()
        with torch.cuda.stream(cap):
            self.graph.capture(cap, lambda: self._enqueue(cap))
        torch.cuda.synchronize()

    def _enqueue(self, stream) -> None:
        c, lib, d = self.c, hip.load(), self.dv
        st = ctypes.c_void_p(stream.cuda_stream)
        c._kv_append(self.k, self.v, d["idx"], self.B, d["bt_pos"], d["bt_val"], self.B, st)
        hip._check(lib.ea_hip_attention(ctypes.byref(self.gc), ctypes.byref(self.bufs), ctypes.byref(self.o),
                                        self.ws.data_ptr(), self.ws_bytes, st), "ea_hip_attention")

    def _plan(self) -> int:
        """Host half of a step: one key per slot appended (pages allocated as needed) into the
        next pinned buffer. Returns the buffer's index."""
        c, seqs, L = self.c, self.seqs, self.L
        if int(L.max()) + 1 > self.max_len:
            raise ValueError("a sequence would pass the graph's max_len")
        pg = L // c.P
        grow = np.flatnonzero(pg >= self.npg)
        if grow.size:
            if grow.size > len(c.free):
                raise RuntimeError("out of pages")
            for i in grow.tolist():
                s = int(seqs[i])
                c.pages[s].append(c.free.pop())
                c.bt_host[s, len(c.pages[s]) - 1] = c.pages[s][-1]
                self.npg[i] += 1
        i = self._ring
        self._ring = (i + 1) % self.RING
        if self._used[i] and self.h.hipEventSynchronize(self._ev[i]) != 0:
            raise RuntimeError("hipEventSynchronize")
        hv = self._hv[i]
        bt_val = c.bt_host[seqs, pg]
        hv["bt_val"][:] = bt_val
        hv["idx"][:] = bt_val.astype(np.int64) * c.P + L % c.P
        hv["bt_pos"][:] = seqs * c.max_pages + pg
        L += 1
        hv["kvl"][:] = L
        for s, n in zip(seqs.tolist(), L.tolist()):
            c.length[s] = n
            c._mark_stale(s, n - 1)  # the digit tiles are re-sliced when a call reads them
        return i

    def step(self):
        """Append the keys in `k`, `v` to every slot and attend with `q`, enqueued on torch's
        current stream. Returns device (out (B, Hq, d), flags (B, Hq))."""
        i = self._plan()
        st = ctypes.c_void_p(self.torch.cuda.current_stream(self.c.dev).cuda_stream)
        if self.h.hipMemcpyAsync(ctypes.c_void_p(self.meta.data_ptr()), ctypes.c_void_p(self._host[i].data_ptr()),
                                 self._nbytes, 1, st) != 0:
            raise RuntimeError("hipMemcpyAsync")
        if self.h.hipEventRecord(self._ev[i], st) != 0:
            raise RuntimeError("hipEventRecord")
        self._used[i] = True
        if self.h.hipGraphLaunch(self.graph.exec, st) != 0:
            raise RuntimeError("hipGraphLaunch")
        return self.out.view(self.B, self.be.Hq, -1), self.flags.view(self.B, self.be.Hq)

    def check_flags(self, flags=None) -> None:
        """After the latest step: flag-1 rows finished by the host exact tier, flag 2 raises."""
        st = ctypes.c_void_p(self.torch.cuda.current_stream(self.c.dev).cuda_stream)
        if bool((self.flags == 1).any().item()):
            hip._check(hip.load().ea_hip_exact_rows(ctypes.byref(self.gc), ctypes.byref(self.bufs),
                                                    ctypes.byref(self.o), st), "ea_hip_exact_rows")
        if bool((self.flags == 2).any().item()):
            raise ExactAttentionDomainError("non-finite input or fp32 logit overflow")

    def close(self) -> None:
        self.graph.close()
        for e in self._ev:
            if e:
                self.h.hipEventDestroy(e)
        self._ev = []


_HF_WS = {}


def hf_attention(module, query, key, value, attention_mask=None, scaling=None, dropout=0.0, **kwargs):
    """ExactAttention as a transformers attention function (register it with
    `transformers.AttentionInterface.register("exact", hf_attention)` or `register_hf()`), the GPU
    drop-in for the reference demo's `exact_attention` (scripts/spec_decode_demo.py:57-73):
    query (B, H, ql, D), key/value (B, Hkv, kl, D) bf16 CUDA tensors holding the whole cache,
    causal with the queries at the end of the key range (query t attends keys 0 .. kl-ql+t);
    `attention_mask` is not read, as in the reference (batches without padding). alpha =
    RN_fp32(scaling / ln 2), scaling defaulting to `module.scaling`. One ea_hip_attention launch
    straight on the tensors' strides (no copies); returns (out (B, ql, H, D) bf16, None). Rows the
    device tiers leave uncertified are finished by the host exact tier (ea_hip_exact_rows); raises
    on non-finite input or fp32 logit overflow, like the reference's kernels (this waits for the
    launch)."""
    import torch
    if dropout:
        raise ValueError("dropout is not part of ExactAttention")
    if kwargs.get("sliding_window"):
        raise ValueError("sliding-window attention is not supported")
    B, H, ql, D = query.shape
    Hkv, kl = key.shape[1], key.shape[2]
    if key.shape != value.shape[:3] + (D,) or key.shape[0] != B or key.shape[3] != D:
        raise ValueError("query/key/value shapes do not match")
    if ql > kl:
        raise ValueError("more queries than keys")
    for t in (query, key, value):
        if t.dtype != torch.bfloat16 or t.device.type != "cuda" or t.stride(3) != 1:
            raise ValueError("query/key/value must be bf16 CUDA tensors with a contiguous last dimension")
    ab = alpha_bits_for(float(scaling if scaling is not None else module.scaling))
    dev = query.device
    out = torch.empty((B, ql, H, D), dtype=torch.bfloat16, device=dev)
    flags = torch.empty(B * ql * H, dtype=torch.uint8, device=dev)
    lens = torch.full((B,), kl, dtype=torch.int32, device=dev)
    kvl = (torch.arange(kl - ql + 1, kl + 1, dtype=torch.int32, device=dev)).repeat(B)
    g = hip.geometry(dict(num_seqs=B, num_tokens=ql, num_q_heads=H, num_kv_heads=Hkv, head_dim=D, head_dim_v=D,
                          q_seq_stride=query.stride(0), q_tok_stride=query.stride(2), q_head_stride=query.stride(1),
                          o_seq_stride=ql * H * D, o_tok_stride=H * D, o_head_stride=D,
                          k_page_stride=key.stride(0), k_slot_stride=key.stride(2), k_head_stride=key.stride(1),
                          v_page_stride=value.stride(0), v_slot_stride=value.stride(2), v_head_stride=value.stride(1),
                          page_size=1, block_table_stride=0, max_seq_len=kl))
    o = hip.Options(alpha_bits=ab, out_fp32=0, splits=0, tier2=1)
    lib = hip.load()
    nb, ns = ctypes.c_size_t(0), ctypes.c_int32(0)
    hip._check(lib.ea_hip_workspace_size(ctypes.byref(g), ctypes.byref(o), ctypes.byref(nb), ctypes.byref(ns)),
               "ea_hip_workspace_size")
    ws = _HF_WS.get(dev)
    if ws is None or ws.numel() < int(nb.value):
        ws = _HF_WS[dev] = torch.empty(max(int(nb.value), 1 << 20), dtype=torch.uint8, device=dev)
    b = hip.Buffers(q=query.data_ptr(), k=key.data_ptr(), v=value.data_ptr(), seq_len=lens.data_ptr(),
                    kv_len=kvl.data_ptr(), block_table=None, block_table_offset=None, tree_mask=None, tree_base=None,
                    out=out.data_ptr(), flags=flags.data_ptr())
    hip._check(lib.ea_hip_attention(ctypes.byref(g), ctypes.byref(b), ctypes.byref(o), ws.data_ptr(), int(nb.value),
                                    hip._stream_ptr(torch)), "ea_hip_attention")
    if bool((flags == 1).any().item()):
        # rows the device tiers left uncertified: the host exact tier, in place
        hip._check(lib.ea_hip_exact_rows(ctypes.byref(g), ctypes.byref(b), ctypes.byref(o), hip._stream_ptr(torch)),
                   "ea_hip_exact_rows")
    if bool((flags == 2).any().item()):
        raise ExactAttentionDomainError("non-finite input or fp32 logit overflow")
    return out, None


def register_hf(name: str = "exact") -> str:
    """Register hf_attention with transformers under `name` (attn_implementation=name)."""
    from transformers import AttentionInterface
    AttentionInterface.register(name, hf_attention)
    return name


def _dev16(torch, x, dev):
    if hasattr(x, "data_ptr"):
        return x.to(dev).view(torch.int16)
    a = np.ascontiguousarray(x)
    if a.dtype == np.uint16:
        a = a.view(np.int16)
    return torch.from_numpy(a).to(dev)
