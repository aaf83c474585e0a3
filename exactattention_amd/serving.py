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
    ea_hip_kv_digits_update), re-sliced for exactly the tiles an append touches, so a prefill
    chunk reads its K/V tiles instead of slicing the whole prefix again.

Every call enqueues on torch's current stream and copies its result to the host (the caller sees
(out bits, flags) like the reference's backends).
"""

from __future__ import annotations

import ctypes

import numpy as np

from . import hip
from .formats import ExactAttentionDomainError, fp32_bits

TILE = 64  # keys per digit tile


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
        self.free = list(range(num_pages))[::-1]
        self.pages = [[] for _ in range(max_seqs)]
        self.length = [0] * max_seqs
        self.live = [False] * max_seqs
        self.tiles = (max_seq_len + TILE - 1) // TILE
        self.digits = None
        if digits and head_dim == 128:
            lib = hip.load()
            n = lib.ea_hip_kv_digits_bytes(max_seqs, num_kv_heads, self.tiles)
            self.digits = torch.zeros(n, dtype=torch.uint8, device=self.dev)

    # ---- sequence slots
    def add_sequence(self) -> int:
        for s in range(self.max_seqs):
            if not self.live[s]:
                self.live[s], self.length[s], self.pages[s] = True, 0, []
                return s
        raise RuntimeError("no free sequence slot")

    def drop_sequence(self, s: int) -> None:
        self.free.extend(self.pages[s][::-1])
        self.pages[s], self.length[s], self.live[s] = [], 0, False

    def _digit_base(self, s: int) -> int:
        return self.digits.data_ptr() + s * self.Hkv * self.tiles * hip.EA_PF_TILE_BYTES

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
        """Append n keys (k_bits, v_bits: (n, Hkv, d) uint16 arrays or int16 device tensors) to slot s,
        then re-slice the digit tiles they touch."""
        self.append_batch([s], [len(k_bits)], k_bits, v_bits)

    def append_batch(self, seqs, counts, k_bits, v_bits) -> None:
        """Append counts[i] keys to slot seqs[i] for every i, the keys flattened in that order
        (k_bits, v_bits: (sum(counts), Hkv, d)); one device scatter for the batch, then one
        digit re-slice over every slot the batch touched."""
        torch = self.torch
        k_new = _dev16(torch, k_bits, self.dev)
        v_new = _dev16(torch, v_bits, self.dev)
        counts = [int(n) for n in counts]
        if k_new.shape[0] != sum(counts) or v_new.shape[0] != sum(counts):
            raise ValueError("k/v must hold sum(counts) keys")
        if len(set(seqs)) != len(seqs):
            raise ValueError("a slot may appear once per batch")
        if sum(counts) == 0:
            return
        need = []
        for s, n in zip(seqs, counts):
            if self.length[s] + n > self.max_seq_len:
                raise ValueError("sequence longer than the cache's max_seq_len")
            need.append(max(0, (self.length[s] + n + self.P - 1) // self.P - len(self.pages[s])))
        if sum(need) > len(self.free):
            raise RuntimeError("out of pages")
        pg, sl, begin, end = [], [], [], []
        for s, n, m in zip(seqs, counts, need):
            L = self.length[s]
            self.pages[s].extend(self.free.pop() for _ in range(m))
            pos = np.arange(L, L + n)
            pg.append(np.asarray(self.pages[s], dtype=np.int64)[pos // self.P])
            sl.append(pos % self.P)
            begin.append(L)
            end.append(L + n)
        for s in seqs:
            self.block_table[s, :len(self.pages[s])] = torch.tensor(self.pages[s], dtype=torch.int32, device=self.dev)
        pg_d = torch.from_numpy(np.concatenate(pg)).to(self.dev)
        sl_d = torch.from_numpy(np.concatenate(sl).astype(np.int64)).to(self.dev)
        self.k[pg_d, sl_d] = k_new
        self.v[pg_d, sl_d] = v_new
        for s, e in zip(seqs, end):
            self.length[s] = e
        self._reslice_slots(list(seqs), begin, end)

    def truncate(self, s: int, length: int) -> None:
        """Drop the keys at or past `length` (rejected draft nodes); the tile holding the new end is
        sliced again so its digits match the shorter sequence."""
        if length > self.length[s]:
            raise ValueError("truncate cannot grow a sequence")
        self.length[s] = length
        keep = (length + self.P - 1) // self.P
        self.free.extend(self.pages[s][keep:][::-1])
        self.pages[s] = self.pages[s][:keep]
        if length % TILE:
            self._reslice(s, length - 1, length)

    def _reslice_slots(self, seqs, begin, end) -> None:
        """Re-slice keys begin[i]..end[i]-1 of slot seqs[i]: one update over all slots, where the
        untouched slots get an empty range (their blocks exit at once)."""
        if self.digits is None:
            return
        torch = self.torch
        lib = hip.load()
        kb = np.zeros(self.max_seqs, dtype=np.int32)
        ke = np.zeros(self.max_seqs, dtype=np.int32)
        kb[list(seqs)] = begin
        ke[list(seqs)] = end
        span = int(max(e - a for a, e in zip(begin, end)))
        if span <= 0:
            return
        g = self._geom1(0, 1, self.Hkv, max(1, max(self.length)))
        g["num_seqs"] = self.max_seqs
        gc = hip.geometry(g)
        seq = torch.tensor(self.length, dtype=torch.int32, device=self.dev)
        kb_d = torch.from_numpy(kb).to(self.dev)
        ke_d = torch.from_numpy(ke).to(self.dev)
        b = hip.Buffers(q=None, k=self.k.data_ptr(), v=self.v.data_ptr(), seq_len=seq.data_ptr(), kv_len=None,
                        block_table=self.block_table.data_ptr(), block_table_offset=None, tree_mask=None,
                        tree_base=None, out=None, flags=None)
        hip._check(lib.ea_hip_kv_digits_update(ctypes.byref(gc), ctypes.byref(b), kb_d.data_ptr(), ke_d.data_ptr(), span,
                                               ctypes.c_void_p(self.digits.data_ptr()), self.tiles,
                                               hip._stream_ptr(torch)), "ea_hip_kv_digits_update")
        self._keep = (seq, kb_d, ke_d)

    def _reslice(self, s: int, a: int, e: int) -> None:
        if self.digits is None or e <= a:
            return
        torch = self.torch
        lib = hip.load()
        g = hip.geometry(self._geom1(s, 1, self.Hkv, self.length[s]))
        seq = torch.tensor([self.length[s]], dtype=torch.int32, device=self.dev)
        off = torch.tensor([s * self.max_pages], dtype=torch.int64, device=self.dev)
        kb = torch.tensor([a], dtype=torch.int32, device=self.dev)
        ke = torch.tensor([e], dtype=torch.int32, device=self.dev)
        b = hip.Buffers(q=None, k=self.k.data_ptr(), v=self.v.data_ptr(), seq_len=seq.data_ptr(), kv_len=None,
                        block_table=self.block_table.data_ptr(), block_table_offset=off.data_ptr(), tree_mask=None,
                        tree_base=None, out=None, flags=None)
        hip._check(lib.ea_hip_kv_digits_update(ctypes.byref(g), ctypes.byref(b), kb.data_ptr(), ke.data_ptr(), e - a,
                                               ctypes.c_void_p(self._digit_base(s)), self.tiles,
                                               hip._stream_ptr(torch)), "ea_hip_kv_digits_update")
        self._keep = (seq, off, kb, ke)  # alive until the stream has run the update


class ExactAttentionBackend:
    """Certified attention over a PagedKVCache. `alpha` is the base-2 logit scale (fp32)."""

    def __init__(self, cache: PagedKVCache, num_q_heads: int, alpha, out: str = "bf16"):
        self.cache, self.Hq, self.out = cache, num_q_heads, out
        self.alpha_bits = alpha if isinstance(alpha, (int, np.integer)) else fp32_bits(alpha)

    def _launch(self, seqs, qd, kvl, tree_mask=None, tree_base=None, digits_slot=None):
        """Enqueue one ea_hip_attention call over sequences `seqs` on torch's current stream.
        qd: (B, T, Hq, d) int16 device tensor, row (b, t, h) = token t of sequence seqs[b];
        kvl: (B*T,) int32 device tensor of visible prefix lengths. Returns device (out, flags)."""
        c = self.cache
        torch = c.torch
        lib = hip.load()
        B, T, Hq, d = qd.shape
        lens = [c.length[s] for s in seqs]
        g = c._geom1(seqs[0], T, Hq, max(lens))
        g["num_seqs"] = B
        gc = hip.geometry(g)
        out = torch.empty((B, T, Hq, d), dtype=torch.int32 if self.out == "fp32" else torch.int16, device=c.dev)
        flags = torch.empty(B * T * Hq, dtype=torch.uint8, device=c.dev)
        seq = torch.tensor(lens, dtype=torch.int32, device=c.dev)
        off = torch.tensor([s * c.max_pages for s in seqs], dtype=torch.int64, device=c.dev)
        tm = None if tree_mask is None else torch.tensor(np.asarray(tree_mask, dtype=np.uint64).view(np.int64).reshape(-1),
                                                         device=c.dev)
        tb = None if tree_base is None else torch.tensor(np.asarray(tree_base, dtype=np.int32), device=c.dev)
        o = hip.Options(alpha_bits=self.alpha_bits, out_fp32=int(self.out == "fp32"), splits=0, tier2=1)
        if digits_slot is not None and c.digits is not None:
            o.kv_digits = ctypes.c_void_p(c._digit_base(digits_slot))
            o.kv_digits_tiles = c.tiles
        nb, ns = ctypes.c_size_t(0), ctypes.c_int32(0)
        hip._check(lib.ea_hip_workspace_size(ctypes.byref(gc), ctypes.byref(o), ctypes.byref(nb), ctypes.byref(ns)),
                   "ea_hip_workspace_size")
        ws = torch.empty(max(int(nb.value), 256), dtype=torch.uint8, device=c.dev)
        b = hip.Buffers(q=qd.data_ptr(), k=c.k.data_ptr(), v=c.v.data_ptr(), seq_len=seq.data_ptr(),
                        kv_len=kvl.data_ptr(), block_table=c.block_table.data_ptr(), block_table_offset=off.data_ptr(),
                        tree_mask=None if tm is None else tm.data_ptr(), tree_base=None if tb is None else tb.data_ptr(),
                        out=out.data_ptr(), flags=flags.data_ptr())
        hip._check(lib.ea_hip_attention(ctypes.byref(gc), ctypes.byref(b), ctypes.byref(o), ws.data_ptr(), int(nb.value),
                                        hip._stream_ptr(torch)), "ea_hip_attention")
        # The caching allocator may hand these buffers to later work on this stream only once the
        # call above has run; keep them referenced until the next launch replaces them.
        self._keep = (seq, off, tm, tb, ws, kvl, qd)
        return out, flags

    def _run(self, seqs, q, kv_len, tree_mask=None, tree_base=None, digits_slot=None):
        """_launch, then the result on the host: (out bits (B, T, Hq, d), flags); flag 2 raises."""
        c = self.cache
        torch = c.torch
        qd = _dev16(torch, q, c.dev).contiguous()
        kvl = torch.tensor(np.asarray(kv_len, dtype=np.int32).reshape(-1), device=c.dev)
        out, flags = self._launch(seqs, qd, kvl, tree_mask, tree_base, digits_slot)
        torch.cuda.synchronize()
        res = out.cpu().numpy()
        res = res.view(np.uint32) if self.out == "fp32" else res.view(np.uint16)
        fl = flags.cpu().numpy()
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
        bits, flags (num_tokens, Hq) uint8; 0 certified, 1 certified by the exact tier, 2 domain
        error — check with check_flags)."""
        c = self.cache
        torch = c.torch
        ql = [int(n) for n in query_lens]
        if len(ql) != len(seqs) or any(n <= 0 for n in ql):
            raise ValueError("query_lens must give a positive token count per sequence")
        ntok = sum(ql)
        if query.shape[0] != ntok or key.shape[0] != ntok or value.shape[0] != ntok:
            raise ValueError("query/key/value must hold sum(query_lens) tokens")
        B, T, Hq, d = len(ql), max(ql), query.shape[1], query.shape[2]
        start = np.concatenate([[0], np.cumsum(ql)])
        prefix = [c.length[s] for s in seqs]
        c.append_batch(seqs, ql, key, value)
        b_of = np.repeat(np.arange(B), ql)
        j_of = np.arange(ntok) - start[b_of]
        row = torch.from_numpy(b_of * T + j_of).to(c.dev)
        kvl_h = np.zeros(B * T, dtype=np.int32)
        kvl_h[b_of * T + j_of] = np.asarray(prefix)[b_of] + j_of + 1
        kvl = torch.from_numpy(kvl_h).to(c.dev)
        q16 = query.view(torch.int16) if query.dtype != torch.int16 else query
        if T == 1:
            qd = q16.reshape(B, 1, Hq, d).contiguous()
        else:
            qd = torch.zeros((B * T, Hq, d), dtype=torch.int16, device=c.dev)
            qd.index_copy_(0, row, q16)
            qd = qd.view(B, T, Hq, d)
        slots = list(seqs)
        contiguous = slots == list(range(slots[0], slots[0] + B))
        out, flags = self._launch(slots, qd, kvl, digits_slot=slots[0] if contiguous else None)
        if T == 1:
            return out.view(B, Hq, -1), flags.view(B, Hq)
        return out.view(B * T, Hq, -1).index_select(0, row), flags.view(B * T, Hq).index_select(0, row)

    @staticmethod
    def check_flags(flags) -> None:
        """Synchronise on `flags` (from forward) and raise on a domain error (flag 2)."""
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
        res, fl = self._run([s], np.asarray(q)[None], np.full((1, N), L), tree_mask=mask, tree_base=[L])
        return res[0], fl

    def accept(self, s: int, prefix_len: int, path, k, v) -> None:
        """Keep the accepted draft nodes `path` (node indices in draft order) after the prefix:
        the cache is cut back to the prefix and the path's K/V appended in order."""
        self.cache.truncate(s, prefix_len)
        if len(path):
            idx = np.asarray(path)
            self.cache.append(s, np.asarray(k)[idx], np.asarray(v)[idx])


def _dev16(torch, x, dev):
    if hasattr(x, "data_ptr"):
        return x.to(dev).view(torch.int16)
    a = np.ascontiguousarray(x)
    if a.dtype == np.uint16:
        a = a.view(np.int16)
    return torch.from_numpy(a).to(dev)
