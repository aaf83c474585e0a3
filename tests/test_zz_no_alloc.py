"""GPU: the allocation-free entry point ea_hip_attention_noalloc against ea_hip_attention.

ea_hip_attention_noalloc runs the same step with its workspace in the library's fixed device
array instead of a caller buffer. Called through the C ABI on two problems in a row (the second
smaller, so it reads an array the first one filled), its bits and flags must equal those of
ea_hip_attention with a caller workspace; a geometry whose workspace exceeds the array is refused
with -4 before any device work.
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


def test_noalloc_equals_the_workspace_entry_point(gpu):
    import torch
    from exactattention_amd import hip
    lib = hip.load()
    noalloc = _noalloc(lib)
    rng = np.random.default_rng(123)
    ab = default_alpha_bits(128)
    for B, S in ((8, 2000), (3, 700)):  # the second call is smaller than the first
        prob = _problem(rng, B, S)
        dp = hip.DeviceProblem(prob, "bf16", 0, "cuda:0")
        hip.launch_hip(dp, ab)
        torch.cuda.synchronize()
        want = dp.out.cpu().numpy().copy()
        want_fl = dp.flags.cpu().numpy().copy()
        dp.out.fill_(0x5A5A)
        dp.flags.fill_(7)
        torch.cuda.synchronize()
        o = hip.options(dp, ab)
        b = dp.buffers()
        rc = noalloc(ctypes.byref(dp._geom_c), ctypes.byref(b), ctypes.byref(o), hip._stream_ptr(torch))
        assert rc == 0
        torch.cuda.synchronize()
        assert not want_fl.any()
        assert np.array_equal(dp.flags.cpu().numpy(), want_fl), (B, S)
        assert np.array_equal(dp.out.cpu().numpy(), want), (B, S)


def test_noalloc_refuses_a_workspace_beyond_its_array(gpu):
    import torch
    from exactattention_amd import hip
    lib = hip.load()
    noalloc = _noalloc(lib)
    # a prefill geometry needs far more than the array (q and K/V digit tiles, epoch scratch)
    g = dict(problem.contiguous(np.zeros((1, 4096, 16, 128), np.uint16), np.zeros((1, 8, 4096, 128), np.uint16),
                                np.zeros((1, 8, 4096, 128), np.uint16), np.ones((1, 4096)))["geom"])
    nb, _ = hip.workspace_size(g)
    assert nb > (64 << 20), nb  # EA_NOALLOC_SCRATCH_BYTES
    fake = 4096  # never dereferenced: the call returns before any device work
    b = hip.Buffers(q=fake, k=fake, v=fake, seq_len=fake, kv_len=fake, out=fake, flags=fake)
    o = hip.Options(alpha_bits=default_alpha_bits(128), tier2=1)
    rc = noalloc(ctypes.byref(hip.geometry(g)), ctypes.byref(b), ctypes.byref(o), hip._stream_ptr(torch))
    assert rc == -4
