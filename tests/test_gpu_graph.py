"""GPU: one certified attention step captured in a HIP graph and replayed.

ea_hip_attention promises an enqueue-only step with fixed grids and no memsets (the reference
runs its step in captured CUDA graphs: scripts/bench_vs_flashinfer.py:79-111, docs/DESIGN.md
D16). The step is captured with hipStreamBeginCapture on a torch stream, its nodes are checked
(kernels only: no memset, memcpy or host node), and the graph is replayed several times with eager
work and synchronisations between the replays; every replay must give the eager step's bits.
"""

import ctypes
import hashlib
import json
import os

import numpy as np
import pytest

from exactattention_amd import configs, problem
from exactattention_amd.formats import default_alpha_bits
from gen import bf16

pytestmark = pytest.mark.gpu
GOLD = os.path.join(os.path.dirname(__file__), "golden")
NODE_KERNEL, NODE_MEMSET = 0, 2


class HipGraph:
    """hipStreamBeginCapture / EndCapture / Instantiate / Launch through libamdhip64."""

    def __init__(self):
        h = ctypes.CDLL("libamdhip64.so")
        P = ctypes.c_void_p
        h.hipStreamBeginCapture.argtypes = [P, ctypes.c_int]
        h.hipStreamEndCapture.argtypes = [P, ctypes.POINTER(P)]
        h.hipGraphGetNodes.argtypes = [P, ctypes.POINTER(P), ctypes.POINTER(ctypes.c_size_t)]
        h.hipGraphNodeGetType.argtypes = [P, ctypes.POINTER(ctypes.c_int)]
        h.hipGraphInstantiate.argtypes = [ctypes.POINTER(P), P, P, P, ctypes.c_size_t]
        h.hipGraphLaunch.argtypes = [P, P]
        h.hipGraphExecDestroy.argtypes = [P]
        h.hipGraphDestroy.argtypes = [P]
        self.h = h
        self.graph = P()
        self.exec = P()

    def capture(self, stream, fn):
        s = ctypes.c_void_p(stream.cuda_stream)
        assert self.h.hipStreamBeginCapture(s, 1) == 0  # thread-local capture mode
        try:
            fn()
        finally:
            rc = self.h.hipStreamEndCapture(s, ctypes.byref(self.graph))
        assert rc == 0
        assert self.h.hipGraphInstantiate(ctypes.byref(self.exec), self.graph, None, None, 0) == 0

    def node_types(self):
        n = ctypes.c_size_t(0)
        assert self.h.hipGraphGetNodes(self.graph, None, ctypes.byref(n)) == 0
        nodes = (ctypes.c_void_p * n.value)()
        assert self.h.hipGraphGetNodes(self.graph, nodes, ctypes.byref(n)) == 0
        types = []
        for i in range(n.value):
            t = ctypes.c_int(-1)
            assert self.h.hipGraphNodeGetType(nodes[i], ctypes.byref(t)) == 0
            types.append(t.value)
        return types

    def replay(self, stream):
        assert self.h.hipGraphLaunch(self.exec, ctypes.c_void_p(stream.cuda_stream)) == 0

    def close(self):
        self.h.hipGraphExecDestroy(self.exec)
        self.h.hipGraphDestroy(self.graph)


def _captured_replays(prob, ab, replays=4, **kw):
    """Eager step, then the captured step replayed `replays` times with eager work between: returns
    (eager out, [replay outs], node types, flags of every replay)."""
    import torch
    from exactattention_amd.hip import DeviceProblem, launch_hip
    dp = DeviceProblem(prob, "bf16", 0, "cuda:0", **kw)
    launch_hip(dp, ab)
    torch.cuda.synchronize()
    eager = dp.out.cpu().numpy().view(np.uint16).copy()
    s = torch.cuda.Stream()
    g = HipGraph()
    with torch.cuda.stream(s):
        g.capture(s, lambda: launch_hip(dp, ab))
    types = g.node_types()
    outs, flags = [], []
    scratch = torch.empty_like(dp.out)
    for i in range(replays):
        dp.out.fill_(0x5A5A)          # eager work between replays: poison the output
        dp.flags.fill_(7)
        scratch.copy_(dp.out)
        torch.cuda.synchronize()
        g.replay(s)
        s.synchronize()
        outs.append(dp.out.cpu().numpy().view(np.uint16).copy())
        flags.append(dp.flags.cpu().numpy().copy())
    g.close()
    return eager, outs, types, flags


def test_c2_step_in_a_graph(gpu):
    p = configs.c2()
    ab = configs.alpha_bits()
    gold = json.load(open(os.path.join(GOLD, "baseline_sha256.json")))["C2"]["sha256"]
    eager, outs, types, flags = _captured_replays(p, ab)
    assert hashlib.sha256(eager.tobytes()).hexdigest() == gold
    assert types and all(t == NODE_KERNEL for t in types), types
    for o, f in zip(outs, flags):
        assert not f.any()
        assert np.array_equal(o, eager)


def test_prefill_step_in_a_graph(gpu):
    """The int8 prefill path (q and K/V slicing, the MFMA kernel, tier 2) captured and replayed."""
    rng = np.random.default_rng(90)
    B, T, Hq, Hkv, d = 1, 130, 4, 2, 128
    q, k, v = bf16(rng, (B, T, Hq, d)), bf16(rng, (B, Hkv, T, d), "outlier"), bf16(rng, (B, Hkv, T, d))
    prob = problem.contiguous(q, k, v, (np.arange(T) + 1).reshape(1, T))
    ab = default_alpha_bits(d)
    from oracle import oracle
    want, _ = oracle.attention_geom(prob, ab)
    eager, outs, types, flags = _captured_replays(prob, ab, kernel="prefill")
    assert np.array_equal(eager, want)
    assert types and all(t == NODE_KERNEL for t in types), types
    for o, f in zip(outs, flags):
        assert not f.any()
        assert np.array_equal(o, want)
