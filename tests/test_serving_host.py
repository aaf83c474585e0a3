"""Host bookkeeping of exactattention_amd.serving.PagedKVCache on the CPU (no digit cache, no HIP
calls): page allocation from the free list, block tables, batched appends, truncation and slot
reuse, checked by reading each sequence's logical K/V history back through its block table."""

import numpy as np
import pytest

from gen import bf16


def _history(cache, s):
    n = cache.length[s]
    bt = cache.block_table[s].numpy()
    pos = np.arange(n)
    pg, sl = bt[pos // cache.P], pos % cache.P
    k = cache.k.numpy()[pg, sl].view(np.uint16)
    v = cache.v.numpy()[pg, sl].view(np.uint16)
    return k, v


def test_paged_cache_bookkeeping():
    from exactattention_amd.serving import PagedKVCache
    rng = np.random.default_rng(5)
    Hkv, d = 2, 16
    c = PagedKVCache(num_pages=20, page_size=8, num_kv_heads=Hkv, head_dim=d, max_seqs=3, max_seq_len=64,
                     digits=False, device="cpu")
    a, b = c.add_sequence(), c.add_sequence()
    want = {a: [np.zeros((0, Hkv, d), np.uint16)] * 2, b: [np.zeros((0, Hkv, d), np.uint16)] * 2}
    for seqs, counts in (([a], [13]), ([a, b], [3, 17]), ([b, a], [1, 8])):
        n = sum(counts)
        k, v = bf16(rng, (n, Hkv, d)), bf16(rng, (n, Hkv, d))
        c.append_batch(seqs, counts, k, v)
        at = 0
        for s, m in zip(seqs, counts):
            want[s] = [np.concatenate([want[s][0], k[at:at + m]]), np.concatenate([want[s][1], v[at:at + m]])]
            at += m
    for s in (a, b):
        k, v = _history(c, s)
        assert np.array_equal(k, want[s][0]) and np.array_equal(v, want[s][1])
        assert len(c.pages[s]) == -(-c.length[s] // c.P)
    used = len(c.pages[a]) + len(c.pages[b])
    assert len(c.free) == 20 - used
    assert not set(c.pages[a]) & set(c.pages[b])
    # truncation returns whole pages past the new end
    c.truncate(a, 9)
    assert c.length[a] == 9 and len(c.pages[a]) == 2 and len(c.free) == 20 - 2 - len(c.pages[b])
    k, _ = _history(c, a)
    assert np.array_equal(k, want[a][0][:9])
    c.append(a, want[a][0][9:12], want[a][1][9:12])
    assert np.array_equal(_history(c, a)[0], want[a][0][:12])
    # slot reuse starts empty; pages come back to the free list
    c.drop_sequence(b)
    assert c.add_sequence() == b and c.length[b] == 0 and c.pages[b] == []
    assert len(c.free) == 20 - len(c.pages[a])


def test_one_key_appends_plan_like_the_general_path():
    """Decode appends (one key per sequence) take a plain-integer planner; it must leave the same
    plan (scatter rows, new block-table entries) and the same pages, block tables, free list,
    lengths and stale marks as the general planner, including keys that open a new page and slot
    orders that differ from allocation order."""
    from exactattention_amd.serving import PagedKVCache
    rng = np.random.default_rng(8)
    Hkv, d = 2, 16
    k0, v0 = bf16(rng, (14, Hkv, d)), bf16(rng, (14, Hkv, d))

    def fresh():
        c = PagedKVCache(num_pages=40, page_size=4, num_kv_heads=Hkv, head_dim=d, max_seqs=4, max_seq_len=64,
                         digits=False, device="cpu")
        seqs = [c.add_sequence() for _ in range(4)]
        c.append_batch(seqs, [3, 4, 0, 7], k0, v0)
        c.digits = True  # the planners only test for a digit cache: stale marks are kept
        c.stale = [None, 2, None, 5]
        return c

    fast, slow = fresh(), fresh()
    for step in range(7):
        seqs = [3, 0, 2, 1] if step % 2 else [1, 2, 3, 0]
        kd, vd = (fast.torch.from_numpy(bf16(rng, (4, Hkv, d)).view(np.int16)) for _ in range(2))
        a = fast._plan_one_each(seqs, kd, vd)
        b = slow._plan_general(seqs, [1, 1, 1, 1], kd, vd)
        assert a["grown"] == b["grown"] and len(a["arrays"]) == len(b["arrays"]), step
        for x, y in zip(a["arrays"], b["arrays"]):
            assert x.dtype == y.dtype and np.array_equal(x, y), step
        assert fast.pages == slow.pages and fast.free == slow.free, step
        assert np.array_equal(fast.bt_host, slow.bt_host), step
        assert fast.length == slow.length and fast.stale == slow.stale, step
    assert any(len(p) > 2 for p in fast.pages)  # new pages were opened on the way


def test_paged_cache_rejects():
    from exactattention_amd.serving import PagedKVCache
    rng = np.random.default_rng(6)
    with pytest.raises(ValueError):
        PagedKVCache(num_pages=4, page_size=6, num_kv_heads=1, head_dim=8, max_seqs=1, max_seq_len=8,
                     digits=False, device="cpu")
    c = PagedKVCache(num_pages=2, page_size=4, num_kv_heads=1, head_dim=8, max_seqs=2, max_seq_len=12,
                     digits=False, device="cpu")
    s = c.add_sequence()
    with pytest.raises(ValueError):     # past max_seq_len
        c.append(s, bf16(rng, (13, 1, 8)), bf16(rng, (13, 1, 8)))
    with pytest.raises(RuntimeError):   # 3 pages needed, 2 exist
        c.append(s, bf16(rng, (9, 1, 8)), bf16(rng, (9, 1, 8)))
    with pytest.raises(ValueError):     # a slot twice in one batch
        c.append_batch([s, s], [1, 1], bf16(rng, (2, 1, 8)), bf16(rng, (2, 1, 8)))
    with pytest.raises(ValueError):
        c.truncate(s, c.length[s] + 1)
    c.add_sequence()
    with pytest.raises(RuntimeError):
        c.add_sequence()


def test_failed_append_changes_nothing():
    from exactattention_amd.serving import PagedKVCache
    rng = np.random.default_rng(7)
    c = PagedKVCache(num_pages=3, page_size=4, num_kv_heads=1, head_dim=8, max_seqs=2, max_seq_len=16,
                     digits=False, device="cpu")
    a, b = c.add_sequence(), c.add_sequence()
    c.append(a, bf16(rng, (5, 1, 8)), bf16(rng, (5, 1, 8)))
    with pytest.raises(RuntimeError):   # a needs 1 more page, b 1: only 1 left
        c.append_batch([a, b], [4, 1], bf16(rng, (5, 1, 8)), bf16(rng, (5, 1, 8)))
    assert c.length == [5, 0] and len(c.pages[a]) == 2 and c.pages[b] == [] and len(c.free) == 1


def test_alpha_bits_for_scaling():
    """alpha = RN_fp32(scaling / ln 2): the reference's fixture value for Qwen3 heads (scaling
    128^-0.5), mpmath at 200 bits (the reference's method) on seeded scalings, and the closed
    form default_alpha_bits(d) for scaling = 1/sqrt(d) where sqrt(d) is exact."""
    import os
    import mpmath
    from exactattention_amd.formats import alpha_bits_for, default_alpha_bits
    z = np.load(os.path.join(os.path.dirname(__file__), "golden", "qwen3_0.6b_heads.npz"))
    assert alpha_bits_for(128 ** -0.5) == int(z["alpha_0_0"].view(np.uint32)) == int(z["alpha_27_11"].view(np.uint32))
    for d in (1, 4, 16, 64, 256, 1024):
        assert alpha_bits_for(1.0 / np.sqrt(d)) == default_alpha_bits(d)
    rng = np.random.default_rng(9)
    for x in np.concatenate([rng.uniform(0.01, 4.0, 200), 2.0 ** rng.integers(-60, 60, 20)]):
        with mpmath.workprec(200):
            # RN to fp32 decided in mpmath: of the fp32 values around the quotient (irrational, so
            # never a tie), the nearest
            q = mpmath.mpf(float(x)) / mpmath.log(2)
            lo = np.float32(float(q))
            cand = [np.nextafter(lo, np.float32(0)), lo, np.nextafter(lo, np.float32(np.inf))]
            want = min(cand, key=lambda c: abs(mpmath.mpf(float(c)) - q))
        assert alpha_bits_for(float(x)) == int(np.float32(want).view(np.uint32)), x
    with pytest.raises(ValueError):
        alpha_bits_for(0.0)


def test_hf_attention_rejects_before_device_work():
    """serving.hf_attention refuses, before any HIP call, what the certified kernels do not
    define: dropout, sliding windows, non-bf16 or host tensors, mismatched shapes, more queries
    than keys."""
    import torch
    from exactattention_amd.serving import hf_attention

    class M:
        scaling = 128 ** -0.5
    q = torch.zeros((1, 2, 3, 128), dtype=torch.bfloat16)
    k = torch.zeros((1, 1, 5, 128), dtype=torch.bfloat16)
    for kw in ({"dropout": 0.1}, {"sliding_window": 4}):
        with pytest.raises(ValueError):
            hf_attention(M(), q, k, k, None, **kw)
    with pytest.raises(ValueError):            # host tensors
        hf_attention(M(), q, k, k, None)
    with pytest.raises(ValueError):            # fp32 tensors
        hf_attention(M(), q.float(), k.float(), k.float(), None)
    with pytest.raises(ValueError):            # head_dim mismatch
        hf_attention(M(), q, k[..., :64], k[..., :64], None)
    with pytest.raises(ValueError):            # 3 queries, 2 keys
        hf_attention(M(), q, k[:, :, :2], k[:, :, :2], None)


def test_forward_rejects_bad_batches_without_touching_the_cache():
    """ExactAttentionBackend.forward checks the batch description before anything is appended:
    a length list of the wrong size, a zero-token chunk, or tensors that do not hold
    sum(query_lens) tokens raise ValueError and leave the cache as it was."""
    import torch
    from exactattention_amd.serving import ExactAttentionBackend, PagedKVCache
    c = PagedKVCache(num_pages=4, page_size=4, num_kv_heads=1, head_dim=8, max_seqs=2, max_seq_len=16,
                     digits=False, device="cpu")
    be = ExactAttentionBackend(c, 2, alpha_bits=0x3E0293EE)
    a, b = c.add_sequence(), c.add_sequence()
    q, k = torch.zeros((3, 2, 8), dtype=torch.int16), torch.zeros((3, 1, 8), dtype=torch.int16)
    for seqs, lens in (([a, b], [3]), ([a, b], [3, 0]), ([a, b], [1, 1])):
        with pytest.raises(ValueError):
            be.forward(q, k, k, seqs, lens)
    assert c.length == [0, 0] and c.pages == [[], []] and len(c.free) == 4
    # slots out of range (a negative slot would index from the end on the host and read before
    # the block table on the device), dropped, or repeated
    c.drop_sequence(b)
    for seqs, lens in (([-1], [3]), ([2], [3]), ([b], [3]), ([a, a], [2, 1]), ([1.0], [3])):
        with pytest.raises(ValueError):
            be.forward(q, k, k, seqs, lens)
        with pytest.raises(ValueError):
            c.append_batch(seqs, lens, bf16(np.random.default_rng(0), (3, 1, 8)), bf16(np.random.default_rng(0),
                                                                                        (3, 1, 8)))
    with pytest.raises(ValueError):
        c.truncate(b, 0)
    assert c.length == [0, 0] and c.pages == [[], []] and len(c.free) == 4


def test_forward_of_an_empty_batch_returns_empty_results():
    """No sequences (a serving loop with nothing scheduled): empty out and flags, the cache as it
    was, nothing enqueued."""
    import torch
    from exactattention_amd.serving import ExactAttentionBackend, PagedKVCache
    c = PagedKVCache(num_pages=4, page_size=4, num_kv_heads=1, head_dim=8, max_seqs=2, max_seq_len=16,
                     digits=False, device="cpu")
    be = ExactAttentionBackend(c, 2, alpha_bits=0x3E0293EE)
    c.add_sequence()
    z = torch.zeros((0, 2, 8), dtype=torch.int16)
    out, flags = be.forward(z, z[:, :1], z[:, :1], [], [])
    assert out.shape == (0, 2, 8) and out.dtype == torch.int16
    assert flags.shape == (0, 2) and flags.dtype == torch.uint8
    be.check_flags(flags)
    assert c.length == [0, 0] and c.pages == [[], []] and len(c.free) == 4


def test_check_flags_never_passes_flag_one():
    """A flag-1 row (not certified by the device tiers, output +0) is never handed back as valid:
    check_flags finishes the latest forward's rows with the host exact tier, and for any other
    flags tensor raises ExactAttentionUncertifiedError; flag 2 raises ExactAttentionDomainError."""
    import torch
    from exactattention_amd.formats import ExactAttentionDomainError, ExactAttentionUncertifiedError
    from exactattention_amd.serving import ExactAttentionBackend, PagedKVCache
    c = PagedKVCache(num_pages=4, page_size=4, num_kv_heads=1, head_dim=8, max_seqs=2, max_seq_len=16,
                     digits=False, device="cpu")
    be = ExactAttentionBackend(c, 2, alpha_bits=0x3E0293EE)
    be.check_flags(torch.zeros((3, 2), dtype=torch.uint8))
    with pytest.raises(ExactAttentionUncertifiedError):
        be.check_flags(torch.tensor([[0, 1], [0, 0]], dtype=torch.uint8))
    with pytest.raises(ExactAttentionDomainError):
        be.check_flags(torch.tensor([[0, 2]], dtype=torch.uint8))
