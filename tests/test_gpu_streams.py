"""GPU: the library is stream-ordered and reentrant across streams and host threads.

Two problems with their own device buffers and workspaces (one on the decode kernel, one on the
int8 prefill kernel) are enqueued alternately on two streams with no synchronisation between the
launches, then launched from two host threads each on its own stream; every result must equal the
problem's result run alone (and the oracle's). Streams keep the default priority.
"""

import threading

import numpy as np
import pytest

from exactattention_amd import problem
from exactattention_amd.formats import default_alpha_bits
from gen import bf16

pytestmark = pytest.mark.gpu


def _problems():
    rng = np.random.default_rng(404)
    d = 128
    # decode geometry: 1 token, GQA 2, ragged lengths, paged
    q = bf16(rng, (6, 1, 8, d))
    k = bf16(rng, (6, 4, 700, d))
    v = bf16(rng, (6, 4, 700, d))
    seq = rng.integers(300, 701, size=6)
    dec = problem.to_paged(problem.contiguous(q, k, v, seq.reshape(6, 1), seq_len=seq), 16,
                           np.random.default_rng(1), "NHD")
    # prefill geometry: 96 causal tokens, GQA 2
    T = 96
    q = bf16(rng, (2, T, 4, d), "outlier")
    k = bf16(rng, (2, 2, 300, d))
    v = bf16(rng, (2, 2, 300, d))
    seq = np.array([300, 250])
    kv = np.stack([seq[b] - T + 1 + np.arange(T) for b in range(2)])
    pre = problem.contiguous(q, k, v, kv, seq_len=seq)
    return dec, pre


def test_concurrent_launches_match_solo_runs(gpu):
    import torch
    from exactattention_amd.hip import DeviceProblem, launch_hip
    from oracle import oracle
    ab = default_alpha_bits(128)
    probs = _problems()
    want = [oracle.attention_geom(p, ab)[0] for p in probs]
    dps = [DeviceProblem(p, "bf16", 0, "cuda:0") for p in probs]

    def result(dp):
        return dp.out.cpu().numpy().view(np.uint16).reshape(dp.prob["out_shape"])

    # solo runs
    for dp in dps:
        launch_hip(dp, ab)
    torch.cuda.synchronize()
    solo = [result(dp).copy() for dp in dps]
    # the first runs on the decode kernel, the second on the int8 prefill kernel (stats 9 and 10)
    assert dps[0].stats.cpu().numpy()[9] > 0 and dps[1].stats.cpu().numpy()[10] > 0
    for s_, w_ in zip(solo, want):
        assert np.array_equal(s_, w_)
    # two streams, launches interleaved, no synchronisation between them
    for dp in dps:
        dp.out.zero_()
    streams = [torch.cuda.Stream(), torch.cuda.Stream()]
    torch.cuda.synchronize()
    for _ in range(6):
        for dp, s in zip(dps, streams):
            with torch.cuda.stream(s):
                launch_hip(dp, ab)
    torch.cuda.synchronize()
    for dp, s_ in zip(dps, solo):
        assert np.array_equal(result(dp), s_)
        assert not dp.flags.cpu().numpy().any()
    # two host threads, each launching on its own stream
    for dp in dps:
        dp.out.zero_()
    torch.cuda.synchronize()
    errors = []

    def worker(dp):
        try:
            s = torch.cuda.Stream()
            with torch.cuda.stream(s):
                for _ in range(6):
                    launch_hip(dp, ab)
            s.synchronize()
        except Exception as e:  # reported below
            errors.append(e)

    threads = [threading.Thread(target=worker, args=(dp,)) for dp in dps]
    for t in threads:
        t.start()
    for t in threads:
        t.join(timeout=60)
    assert not errors, errors
    assert not any(t.is_alive() for t in threads)
    torch.cuda.synchronize()
    for dp, s_ in zip(dps, solo):
        assert np.array_equal(result(dp), s_)
