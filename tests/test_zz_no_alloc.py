"""GPU: the allocation-free entry point ea_hip_attention_noalloc against ea_hip_attention.

ea_hip_attention_noalloc runs the same step with its workspace in the library's fixed device
array instead of a caller buffer. Called through the C ABI on two problems in a row (the second
smaller, so it reads an array the first one filled), its bits and flags must equal those of
ea_hip_attention with a caller workspace: on the decode, int8 prefill and general kernels, on a
long-context geometry whose workspace fills most of the array, and captured in a HIP graph and
replayed. A geometry whose workspace exceeds the array is refused with -4 before any device work.
"""

import ctypes

import numpy as np
import pytest

from exactattention_amd import problem
from exactattention_amd.formats import default_alpha_bits
from gen import bf16

pytestmark = pytest.mark.gpu


def _problem(rng, B, S, Hq=16, Hkv=8, d=128, page=16):
    q = bf16(rng, (B, 1, Hq, d))
    k = bf16(rng, (B, Hkv, S, d), "outlier")
    v = bf16(rng, (B, Hkv, S, d))
    base = problem.contiguous(q, k, v, np.full((B, 1), S))
    return problem.to_paged(base, page, rng, "NHD")


def _noalloc(lib):
    from exactattention_amd import hip
    f = lib.ea_hip_attention_noalloc
    f.argtypes = [ctypes.POINTER(hip.Geometry), ctypes.POINTER(hip.Buffers), ctypes.POINTER(hip.Options),
                  ctypes.c_void_p]
    f.restype = ctypes.c_int
    return f


def _both_entry_points(prob, ab, kernel="auto", expect_kernel=None):
    """The problem through ea_hip_attention (caller workspace), then through the allocation-free
    entry point with the output poisoned in between: both must give the same bits and flags."""
    import torch
    from exactattention_amd import hip
    noalloc = _noalloc(hip.load())
    dp = hip.DeviceProblem(prob, "bf16", 0, "cuda:0", kernel)
    assert dp.ws_bytes <= (128 << 20), dp.ws_bytes  # EA_NOALLOC_SCRATCH_BYTES
    hip.launch_hip(dp, ab)
    torch.cuda.synchronize()
    want = dp.out.cpu().numpy().copy()
    want_fl = dp.flags.cpu().numpy().copy()
    st = dict(zip(hip.STATS, dp.stats.cpu().numpy().tolist()))
    if expect_kernel:
        assert st[expect_kernel] > 0, st
    dp.out.fill_(0x5A5A)
    dp.flags.fill_(7)
    torch.cuda.synchronize()
    o = hip.options(dp, ab)
    b = dp.buffers()
    rc = noalloc(ctypes.byref(dp._geom_c), ctypes.byref(b), ctypes.byref(o), hip._stream_ptr(torch))
    assert rc == 0
    torch.cuda.synchronize()
    assert not want_fl.any()
    assert np.array_equal(dp.flags.cpu().numpy(), want_fl)
    assert np.array_equal(dp.out.cpu().numpy(), want)
    return dp


def test_noalloc_equals_the_workspace_entry_point(gpu):
    rng = np.random.default_rng(123)
    ab = default_alpha_bits(128)
    for B, S in ((8, 2000), (3, 700)):  # the second call is smaller than the first
        _both_entry_points(_problem(rng, B, S), ab, expect_kernel="decode_kernel_rows")


def test_noalloc_on_the_prefill_and_general_kernels(gpu):
    """A 96-token causal chunk on the int8 prefill kernel, then a d = 64 problem on the general
    split kernel (a smaller workspace over the array the prefill call filled)."""
    rng = np.random.default_rng(124)
    T, S, Hq, Hkv = 96, 300, 4, 2
    q = bf16(rng, (1, T, Hq, 128))
    k, v = bf16(rng, (1, Hkv, S, 128), "outlier"), bf16(rng, (1, Hkv, S, 128))
    kv_len = (S - T + 1 + np.arange(T)).reshape(1, T)
    _both_entry_points(problem.contiguous(q, k, v, kv_len), default_alpha_bits(128),
                       expect_kernel="prefill_kernel_rows")
    q = bf16(rng, (4, 1, 8, 64))
    k, v = bf16(rng, (4, 4, 900, 64), "wide"), bf16(rng, (4, 4, 900, 64))
    _both_entry_points(problem.contiguous(q, k, v, np.full((4, 1), 900)), default_alpha_bits(64))


def test_noalloc_long_context_workspace(gpu):
    """16 ragged sequences planned for 131,072 keys (the long-context bound: 64 KV splits, about
    72 MB of the array's 128 MiB); only the actual lengths are read."""
    rng = np.random.default_rng(125)
    B, S = 16, 1500
    q = bf16(rng, (B, 1, 16, 128))
    k, v = bf16(rng, (B, 8, S, 128), "outlier"), bf16(rng, (B, 8, S, 128))
    lens = rng.integers(1, S + 1, size=B)
    base = problem.to_paged(problem.contiguous(q, k, v, lens.reshape(B, 1)), 64, rng, "NHD")
    # a block table as wide as 131,072 keys; entries past the real pages name page 0
    bt = np.zeros((B, 131072 // 64), np.int32)
    bt[:, :base["block_table"].shape[1]] = base["block_table"]
    prob = problem.paged(base["q"], base["k"], base["v"], bt, lens.reshape(B, 1), lens)
    prob["geom"] = dict(prob["geom"], max_seq_len=131072)
    dp = _both_entry_points(prob, default_alpha_bits(128), expect_kernel="decode_kernel_rows")
    assert dp.ws_bytes > (64 << 20), dp.ws_bytes


def test_noalloc_captured_in_a_graph(gpu):
    """After an eager first call on the device, the allocation-free step is captured in a HIP
    graph (kernel nodes only) and replayed three times with eager work in between: every replay
    gives the eager bits."""
    import torch
    from exactattention_amd import hip
    from exactattention_amd.graph import NODE_KERNEL, HipGraph
    noalloc = _noalloc(hip.load())
    rng = np.random.default_rng(126)
    ab = default_alpha_bits(128)
    dp = _both_entry_points(_problem(rng, 4, 1300), ab)
    want = dp.out.cpu().numpy().copy()
    o = hip.options(dp, ab)
    b = dp.buffers()
    s = torch.cuda.Stream()
    g = HipGraph()
    torch.cuda.synchronize()
    with torch.cuda.stream(s):
        g.capture(s, lambda: hip._check(noalloc(ctypes.byref(dp._geom_c), ctypes.byref(b), ctypes.byref(o),
                                                ctypes.c_void_p(s.cuda_stream)), "ea_hip_attention_noalloc"))
    try:
        assert set(g.node_types()) == {NODE_KERNEL}
        for _ in range(3):
            dp.out.fill_(0x5A5A)
            dp.flags.fill_(7)
            torch.cuda.synchronize()
            g.replay(s)
            s.synchronize()
            assert not dp.flags.cpu().numpy().any()
            assert np.array_equal(dp.out.cpu().numpy(), want)
    finally:
        g.close()


def test_noalloc_refuses_a_workspace_beyond_its_array(gpu):
    import torch
    from exactattention_amd import hip
    lib = hip.load()
    noalloc = _noalloc(lib)
    # a prefill geometry needs far more than the array (q and K/V digit tiles, epoch scratch)
    g = dict(problem.contiguous(np.zeros((1, 4096, 16, 128), np.uint16), np.zeros((1, 8, 4096, 128), np.uint16),
                                np.zeros((1, 8, 4096, 128), np.uint16), np.ones((1, 4096)))["geom"])
    nb, _ = hip.workspace_size(g)
    assert nb > (128 << 20), nb  # EA_NOALLOC_SCRATCH_BYTES
    fake = 4096  # never dereferenced: the call returns before any device work
    b = hip.Buffers(q=fake, k=fake, v=fake, seq_len=fake, kv_len=fake, out=fake, flags=fake)
    o = hip.Options(alpha_bits=default_alpha_bits(128), tier2=1)
    rc = noalloc(ctypes.byref(hip.geometry(g)), ctypes.byref(b), ctypes.byref(o), hip._stream_ptr(torch))
    assert rc == -4
