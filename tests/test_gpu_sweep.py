"""GPU parity sweep: seeded random geometries through the public problem path, against the oracle.

Each case draws its own combination of the factors the other GPU tests vary one or two at a time
(every eighth case with long rows of 2,000 to 20,000 keys):
kernel request (auto, decode, prefill, general: an ineligible request falls back, which is part of
what is checked), head dims, GQA group, tokens per sequence, ragged sequence lengths, prefix /
causal / tree masks (tree keys overlapping the prefix and running past seq_len), input kinds, page
size and layout, split count and output format. Every case must return the oracle's bits with
every row certified by the device tiers or the host exact tier (fallback=True), and the sweep as a
whole must have run each of the three tier-1 kernels.
"""

import os

import numpy as np
import pytest

from exactattention_amd import problem
from exactattention_amd.formats import ExactAttentionDomainError, default_alpha_bits
from gen import KINDS, bf16

pytestmark = pytest.mark.gpu

# 1024 cases take about 19 s on an MI355X; EA_SWEEP_CASES=N runs N (20,000 pass in about 350 s:
# run those with pytest -s, which prints every case as it starts), starting at case
# EA_SWEEP_FIRST (default 0), so a longer run can cover indices not run before
NCASES = int(os.environ.get("EA_SWEEP_CASES", "1024"))
FIRST = int(os.environ.get("EA_SWEEP_FIRST", "0"))


def _long_case(i, rng):
    """Every eighth case: long rows (2,000 to 20,000 keys) for a few rows, so that rows span many
    tiles and key splits, and prefill rows pass 256 tiles (epoch folds)."""
    kernel = ["auto", "decode", "prefill", "general"][(i // 8) % 4]
    Hkv = int(rng.choice([1, 2]))
    grp = int(rng.choice([1, 2]))
    T = int(rng.choice([1, 2, 16])) if kernel == "prefill" else int(rng.choice([1, 2]))
    B = int(rng.integers(1, 3))
    S = int(rng.integers(2000, 20001))
    seq = rng.integers(S // 2, S + 1, size=B)
    mode = str(rng.choice(["causal", "prefix", "full"]))
    if mode == "causal":
        kv = np.stack([np.clip(seq[b] - T + 1 + np.arange(T), 0, None) for b in range(B)])
    elif mode == "prefix":
        kv = np.stack([rng.integers(0, seq[b] + 1, size=T) for b in range(B)])
    else:
        kv = np.repeat(seq[:, None], T, axis=1)
    kq, kk, kv_kind = (str(x) for x in rng.choice(KINDS, size=3))
    q = bf16(rng, (B, T, Hkv * grp, 128), kq)
    k = bf16(rng, (B, Hkv, S, 128), kk)
    v = bf16(rng, (B, Hkv, S, 128), kv_kind)
    prob = problem.contiguous(q, k, v, kv, seq_len=seq)
    ps = int(rng.choice([0, 16, 64]))
    if ps:
        prob = problem.to_paged(prob, ps, np.random.default_rng(i), "NHD")
    out = str(rng.choice(["bf16", "fp32"]))
    splits = int(rng.choice([0, 0, 3, 7, 16]))
    desc = (f"case {i} (long rows): kernel={kernel} B={B} T={T} Hq={Hkv * grp} Hkv={Hkv} S={S} seq={seq.tolist()} "
            f"mode={mode} kinds=({kq},{kk},{kv_kind}) page={ps} out={out} splits={splits}")
    return prob, kernel, 128, out, splits, desc


def _case(i):
    rng = np.random.default_rng(90_000 + i)
    if i % 8 == 7:
        return _long_case(i, rng)
    kernel = ["auto", "decode", "prefill", "general"][i % 4]
    full = kernel in ("decode", "prefill") or rng.random() < 0.4
    d = 128 if full else int(rng.choice([8, 16, 40, 64, 96, 120, 128]))
    dv = 128 if full else int(rng.choice([2, 16, 34, 64, 100, 128]))
    Hkv = int(rng.choice([1, 2, 4]))
    grp = int(rng.choice([1, 2, 4, 8]))
    T = int(rng.choice([1, 2, 5, 16, 33, 64, 70])) if kernel == "prefill" else int(rng.choice([1, 1, 2, 3, 7]))
    B = int(rng.integers(1, 4))
    # keep the oracle's work (rows x keys) to a few hundred thousand pairs
    S = int(rng.integers(1, max(2, min(400, 400_000 // max(1, B * T * Hkv * grp)))))
    seq = rng.integers(max(1, S // 3), S + 1, size=B)
    mode = rng.choice(["causal", "prefix", "full", "tree"])
    if mode == "causal":
        kv = np.stack([np.clip(seq[b] - T + 1 + np.arange(T), 0, None) for b in range(B)])
    elif mode == "prefix":
        kv = np.stack([rng.integers(0, seq[b] + 1, size=T) for b in range(B)])
    else:
        kv = np.repeat(seq[:, None], T, axis=1)
    tmask = tbase = None
    if mode == "tree":
        # prefix below tree_base (sometimes past it), random 64-bit masks whose keys may overlap
        # the prefix and run past seq_len
        tbase = np.array([rng.integers(0, seq[b] + 1) for b in range(B)], dtype=np.int32)
        kv = np.stack([np.minimum(tbase[b] + rng.integers(0, 3, size=T), seq[b]) for b in range(B)])
        tmask = rng.integers(0, 1 << 63, size=(B, T), dtype=np.uint64) << np.uint64(1)
        tmask |= rng.integers(0, 2, size=(B, T), dtype=np.uint64)
    kq, kk, kv_kind = (str(x) for x in rng.choice(KINDS, size=3))
    q = bf16(rng, (B, T, Hkv * grp, d), kq)
    k = bf16(rng, (B, Hkv, S, d), kk)
    v = bf16(rng, (B, Hkv, S, dv), kv_kind)
    prob = problem.contiguous(q, k, v, kv, seq_len=seq, tree_mask=tmask, tree_base=tbase)
    ps = int(rng.choice([0, 1, 4, 16, 64]))
    layout = str(rng.choice(["NHD", "HND"]))
    if ps:
        prob = problem.to_paged(prob, ps, np.random.default_rng(i), layout)
    out = str(rng.choice(["bf16", "fp32"]))
    splits = int(rng.choice([0, 0, 1, 2, 3, 5]))
    desc = (f"case {i}: kernel={kernel} B={B} T={T} Hq={Hkv * grp} Hkv={Hkv} d={d} dv={dv} S={S} "
            f"seq={seq.tolist()} mode={mode} kinds=({kq},{kk},{kv_kind}) page={ps}{layout if ps else ''} "
            f"out={out} splits={splits}")
    return prob, kernel, d, out, splits, desc


def test_random_geometries_match_oracle(gpu):
    from exactattention_amd.hip import attention_problem
    from oracle import exact, oracle
    ran = {"decode": 0, "prefill": 0, "general": 0}
    for i in range(FIRST, FIRST + NCASES):
        prob, kernel, d, out, splits, desc = _case(i)
        ab = default_alpha_bits(d)
        try:
            want, _ = oracle.attention_geom(prob, ab, out, acc_bits=128)
        except exact.DomainError:
            want = None
        print(desc, flush=True)
        if want is None:
            with pytest.raises(ExactAttentionDomainError):
                attention_problem(prob, None, out, splits, None, True, True, kernel=kernel, alpha_bits=ab)
            continue
        got, flags, st = attention_problem(prob, None, out, splits, None, True, True, kernel=kernel, alpha_bits=ab)
        assert not np.any(flags), (desc, st)
        assert np.array_equal(got, want), (desc, st)
        if st["decode_kernel_rows"]:
            ran["decode"] += 1
        elif st["prefill_kernel_rows"]:
            ran["prefill"] += 1
        else:
            ran["general"] += 1
    print(f"{NCASES} cases; tier-1 kernels {ran}", flush=True)
    assert min(ran.values()) >= 4, ran
