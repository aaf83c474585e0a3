"""GPU: one certified attention step captured in a HIP graph and replayed.

ea_hip_attention promises an enqueue-only step with fixed grids and no memsets (the reference
runs its step in captured CUDA graphs: scripts/bench_vs_flashinfer.py:79-111, docs/DESIGN.md
D16). The step is captured with hipStreamBeginCapture on a torch stream, its nodes are checked
(kernels only: no memset, memcpy or host node), and the graph is replayed several times with eager
work and synchronisations between the replays; every replay must give the eager step's bits.
"""

import hashlib
import json
import os

import numpy as np
import pytest

from exactattention_amd import configs, problem
from exactattention_amd.formats import default_alpha_bits
from exactattention_amd.graph import NODE_KERNEL, HipGraph
from gen import bf16

pytestmark = pytest.mark.gpu
GOLD = os.path.join(os.path.dirname(__file__), "golden")


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


def test_decode_kernel_repeats_back_to_back(gpu):
    """bench.py times the decode kernel alone, relaunched with the captured step's parameters: the
    step holds exactly one such node, every repeat runs the decode kernel (its row counter moves by
    the rows once per launch), and the repeats rewrite the workspace with the same bytes."""
    import sys
    import torch
    sys.path.insert(0, os.path.dirname(os.path.dirname(os.path.abspath(__file__))))
    import bench
    from exactattention_amd.hip import STATS, DeviceProblem, launch_hip
    rng = np.random.default_rng(5)
    B, Hkv, Hq, S, d = 4, 2, 4, 700, 128
    q = bf16(rng, (B, 1, Hq, d), "normal")
    k = bf16(rng, (B, Hkv, S, d), "normal")
    v = bf16(rng, (B, Hkv, S, d), "normal")
    seq = np.array([700, 513, 64, 1])
    prob = problem.to_paged(problem.contiguous(q, k, v, seq.reshape(B, 1), seq_len=seq), 16, rng, "NHD")
    ab = default_alpha_bits(d)
    dp = DeviceProblem(prob, "bf16", 0, "cuda:0")
    launch_hip(dp, ab)
    torch.cuda.synchronize()
    out0 = dp.out.cpu().numpy().copy()
    ws0 = dp.workspace.cpu().numpy().copy()
    st0 = dict(zip(STATS, dp.stats.cpu().numpy().tolist()))
    assert st0["decode_kernel_rows"] == B * Hq
    reps = 3
    ms = bench.back_to_back_ms(dp, ab, 128, reps)
    torch.cuda.synchronize()
    assert ms is not None and ms > 0
    st1 = dict(zip(STATS, dp.stats.cpu().numpy().tolist()))
    # the capture enqueued nothing; reps + 2 decode launches ran
    assert st1["decode_kernel_rows"] - st0["decode_kernel_rows"] == (reps + 2) * B * Hq
    assert st1["rows"] == st0["rows"]
    assert np.array_equal(dp.workspace.cpu().numpy(), ws0)
    assert np.array_equal(dp.out.cpu().numpy(), out0)
