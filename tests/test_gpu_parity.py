"""GPU parity: the HIP library (through its C ABI) against the CPU oracle, bit for bit.

Every comparison is exact equality of bf16/fp32 bit patterns. The oracle is the C restatement of
the reference's certified CPU kernel plus the Python exact definition for the rows it flags.
"""

import hashlib
import json
import os

import numpy as np
import pytest

from exactattention_amd import configs, problem
from exactattention_amd.formats import default_alpha_bits
from gen import KINDS, bf16

pytestmark = pytest.mark.gpu
GOLD = os.path.join(os.path.dirname(__file__), "golden")


def _run(prob, alpha_bits, out="bf16", splits=0, merge_order=None, **kw):
    """The device tiers only (fallback=False): flags as tier 1 and tier 2 leave them."""
    from exactattention_amd.hip import attention_problem
    return attention_problem(prob, None, out, splits, merge_order, True, False, alpha_bits=alpha_bits, **kw)


def _oracle(prob, alpha_bits, out="bf16"):
    from oracle import oracle
    return oracle.attention_geom(prob, alpha_bits, out)


def _rand_problem(rng, kind, vkind, B, T, Hq, Hkv, S, d, dv, causal=True):
    q = bf16(rng, (B, T, Hq, d), kind)
    k = bf16(rng, (B, Hkv, S, d), kind)
    v = bf16(rng, (B, Hkv, S, dv), vkind)
    seq = rng.integers(max(1, S // 2), S + 1, size=B)
    if causal:
        kv = np.stack([np.clip(seq[b] - T + 1 + np.arange(T), 0, None) for b in range(B)])
    else:
        kv = np.repeat(seq[:, None], T, axis=1)
    return problem.contiguous(q, k, v, kv, seq_len=seq)


# ---------------------------------------------------------------------------------------------
# helper known-answer tests
# ---------------------------------------------------------------------------------------------

def test_weight_kat_matches_oracle(gpu):
    import torch
    from exactattention_amd import hip
    from oracle import exact
    rng = np.random.default_rng(5)
    ts = np.concatenate([rng.uniform(-60, 60, 20000), rng.uniform(-1e-6, 1e-6, 500),
                         np.arange(-40, 40) + rng.uniform(-1e-7, 1e-7, 80), rng.uniform(-1e4, 1e4, 2000),
                         np.float32(2.0) ** rng.uniform(-40, -20, 500) * rng.choice([-1, 1], 500),
                         [0.0, -0.0, 1.0, -1.0, 2.0 ** -25, -(2.0 ** -25), 2.0 ** -26, 0.99999994, 1e9, -1e9]])
    tb = np.float32(ts).view(np.uint32)
    n = tb.size
    dev = {k: torch.zeros(n, dtype=dt, device="cuda") for k, dt in
           (("M", torch.int32), ("E", torch.int64), ("st", torch.int32), ("M2", torch.int32), ("E2", torch.int64),
            ("st2", torch.int32))}
    tt = torch.from_numpy(tb.view(np.int32)).cuda()
    rc = hip.load().ea_hip_kat_weight(n, tt.data_ptr(), *[dev[k].data_ptr() for k in ("M", "E", "st", "M2", "E2", "st2")],
                                      torch.cuda.current_stream().cuda_stream)
    assert rc == 0
    torch.cuda.synchronize()
    h = {k: v.cpu().numpy() for k, v in dev.items()}
    undecided = 0
    for i in range(n):
        tm, te = exact.decode_fp32_bits(int(tb[i]))
        big = abs(float(np.float32(ts[i]))) >= 2 ** 30
        want = exact.exp2_rn(tm, te) if not big else None
        if h["st"][i] == 0:
            assert (int(h["M"][i]), int(h["E"][i])) == want, ts[i]
        else:
            undecided += 1
            assert big or h["st"][i] == 1
        if not big:
            assert h["st2"][i] == 0 and (int(h["M2"][i]), int(h["E2"][i])) == want, ts[i]
    assert undecided <= 12, undecided  # fp64 path leaves ~2^-25 of weights (+ the 2 out-of-range)


def test_round_ratio_kat_matches_oracle(gpu):
    import torch
    from exactattention_amd import hip
    from oracle import oracle
    rng = np.random.default_rng(9)
    cases = []
    for _ in range(4000):
        ab, bb = int(rng.integers(1, 127)), int(rng.integers(1, 127))
        a = int(rng.integers(1, 1 << min(ab, 62))) << max(0, ab - 62)
        b = int(rng.integers(1, 1 << min(bb, 62))) << max(0, bb - 62)
        cases.append((a | int(rng.integers(0, 2)), b, int(rng.integers(-300, 200)), int(rng.integers(0, 2))))
    for fp32 in (0, 1):
        n = len(cases)
        arr = lambda f, dt: torch.from_numpy(np.array([f(c) for c in cases], dtype=dt)).cuda()
        ah = arr(lambda c: c[0] >> 64, np.uint64).view(torch.int64)
        al = arr(lambda c: c[0] & ((1 << 64) - 1), np.uint64).view(torch.int64)
        bh = arr(lambda c: c[1] >> 64, np.uint64).view(torch.int64)
        bl = arr(lambda c: c[1] & ((1 << 64) - 1), np.uint64).view(torch.int64)
        E = arr(lambda c: c[2], np.int32)
        ng = arr(lambda c: c[3], np.int32)
        bits = torch.zeros(n, dtype=torch.int32, device="cuda")
        ov = torch.zeros(n, dtype=torch.int32, device="cuda")
        rc = hip.load().ea_hip_kat_round_ratio(n, ah.data_ptr(), al.data_ptr(), bh.data_ptr(), bl.data_ptr(),
                                               E.data_ptr(), ng.data_ptr(), fp32, bits.data_ptr(), ov.data_ptr(),
                                               torch.cuda.current_stream().cuda_stream)
        assert rc == 0
        torch.cuda.synchronize()
        gb, go = bits.cpu().numpy().view(np.uint32), ov.cpu().numpy()
        for i, (a, b, e, neg) in enumerate(cases):
            wb, wo = oracle.round_ratio_bits(a, b, e, bool(neg), bool(fp32))
            assert bool(go[i]) == wo, (a, b, e, neg, fp32)
            if not wo:
                assert int(gb[i]) == wb, (a, b, e, neg, fp32)


def test_wave_max_dpp_kat(gpu):
    import torch
    from exactattention_amd import hip
    rng = np.random.default_rng(2)
    x = rng.integers(-(1 << 31), (1 << 31) - 1, size=(300, 64), dtype=np.int64).astype(np.int32)
    x[0] = np.iinfo(np.int32).min
    x[1, 37] = np.iinfo(np.int32).max
    x[2] = np.arange(64)[::-1]
    for i in range(3, 67):
        x[i] = -5
        x[i, i - 3] = 7  # the max in each lane position
    xi = torch.from_numpy(x).cuda()
    out = torch.zeros_like(xi)
    assert hip.load().ea_hip_kat_wave_max(x.shape[0], xi.data_ptr(), out.data_ptr(),
                                          torch.cuda.current_stream().cuda_stream) == 0
    torch.cuda.synchronize()
    assert np.array_equal(out.cpu().numpy(), np.repeat(x.max(axis=1, keepdims=True), 64, axis=1))


def test_certify_round_kat(gpu):
    """certify_round on exact points (r = 0) equals RN of the point; with r > 0 it never certifies
    an interval that holds a rounding midpoint."""
    import torch
    from exactattention_amd import hip
    from oracle import exact
    rng = np.random.default_rng(3)
    x = np.concatenate([rng.standard_normal(3000) * np.exp2(rng.uniform(-140, 120, 3000)),
                        np.float32(rng.standard_normal(500)).astype(np.float64)])
    for fp32 in (0, 1):
        p = 24 if fp32 else 8
        # exact midpoints between adjacent values: never certified with r > 0
        r0 = np.zeros_like(x)
        xs = torch.from_numpy(x).cuda()
        rs = torch.from_numpy(r0).cuda()
        bits = torch.zeros(x.size, dtype=torch.int32, device="cuda")
        ok = torch.zeros(x.size, dtype=torch.int32, device="cuda")
        assert hip.load().ea_hip_kat_round(x.size, xs.data_ptr(), rs.data_ptr(), fp32, bits.data_ptr(), ok.data_ptr(),
                                           torch.cuda.current_stream().cuda_stream) == 0
        torch.cuda.synchronize()
        gb, gk = bits.cpu().numpy().view(np.uint32), ok.cpu().numpy()
        fmt = exact.FP32 if fp32 else exact.BF16
        enc = exact.encode_fp32 if fp32 else exact.encode_bf16
        n_ok = 0
        for i, xv in enumerate(x.tolist()):
            num, den = float(xv).as_integer_ratio()
            m, e = exact.round_rational(num, den, fmt)
            want = 0 if m == 0 else enc(m, e)
            if gk[i]:
                n_ok += 1
                assert int(gb[i]) == want, (xv, fp32)
        assert n_ok > 0.9 * x.size


def test_rn32_prod_kat(gpu):
    """The exact logit RN32(am * X * 2^E) (the prefill cold path and tier 2) against the oracle's
    round_dyadic: 128-bit X of every length, both signs, exponents from far below the fp32
    subnormal range to overflow, and products on exact rounding ties."""
    import torch
    from exactattention_amd import hip
    from oracle import exact
    rng = np.random.default_rng(17)
    n = 8000
    am = [int(v) for v in rng.integers(1, 1 << 24, n) * rng.choice([-1, 1], n)]
    X, E = [], []
    for i in range(n):
        bl = int(rng.integers(1, 128))
        x = int(rng.integers(0, 1 << 62)) << 66 | int(rng.integers(0, 1 << 62)) << 4 | int(rng.integers(0, 16))
        x = (x >> (128 - bl)) | (1 << (bl - 1))
        if i % 5 == 0:
            # odd 13-bit factors: a 25-bit odd product is a tie at 24 bits (about half of them)
            am[i] = (int(rng.integers(1 << 11, 1 << 12)) * 2 + 1) * (1 if i % 10 else -1)
            x = (int(rng.integers(1 << 11, 1 << 12)) * 2 + 1) << int(rng.integers(0, 100))
            X.append(x)
            E.append(int(rng.integers(-150, 120)) - (abs(am[i]) * x).bit_length() + 1)
            continue
        X.append(x if rng.random() < 0.5 else -x)
        lead = bl + abs(am[i]).bit_length() - 2
        E.append(int(rng.integers(-200, 140)) - lead)  # floor(log2) from -200 to 139
    xh = np.array([(x >> 64) for x in X], dtype=np.int64)
    xl = np.array([x & ((1 << 64) - 1) for x in X], dtype=np.uint64)
    dev = {k: torch.from_numpy(v).cuda() for k, v in
           (("am", np.array(am, dtype=np.int32)), ("xh", xh), ("xl", xl.view(np.int64)), ("E", np.array(E, dtype=np.int32)))}
    bits = torch.zeros(n, dtype=torch.int32, device="cuda")
    st = torch.zeros(n, dtype=torch.int32, device="cuda")
    assert hip.load().ea_hip_kat_rn32_prod(n, dev["am"].data_ptr(), dev["xh"].data_ptr(), dev["xl"].data_ptr(),
                                           dev["E"].data_ptr(), bits.data_ptr(), st.data_ptr(),
                                           torch.cuda.current_stream().cuda_stream) == 0
    torch.cuda.synchronize()
    gb, gs = bits.cpu().numpy().view(np.uint32), st.cpu().numpy()
    kinds = {"normal": 0, "subnormal": 0, "zero": 0, "overflow": 0}
    for i in range(n):
        try:
            m, e = exact.round_dyadic(am[i] * X[i], E[i], exact.FP32)
        except exact.DomainError:
            assert gs[i] == 2, (am[i], X[i], E[i])
            kinds["overflow"] += 1
            continue
        assert gs[i] == 0, (am[i], X[i], E[i])
        want = 0 if m == 0 else exact.encode_fp32(m, e)
        got = int(gb[i]) & (0x7FFFFFFF if m == 0 else 0xFFFFFFFF)  # the sign of a zero is not part of it
        assert got == want, (am[i], X[i], E[i], hex(got), hex(want))
        kinds["zero" if m == 0 else ("subnormal" if (want & 0x7F800000) == 0 else "normal")] += 1
    assert min(kinds.values()) > 20, kinds


def test_certify_round_intervals(gpu):
    """certify_round on intervals [x - r, x + r] with r > 0, through both its normal-range fast
    path and the general path (subnormal and zero-region magnitudes, ends near 2^127, intervals
    on a rounding midpoint): whenever it certifies, both ends round (exactly, as rationals) to the
    bits it returned, so every point of the interval does."""
    import torch
    from fractions import Fraction
    from exactattention_amd import hip
    from oracle import exact
    rng = np.random.default_rng(11)
    n = 6000
    for fp32 in (0, 1):
        p = 24 if fp32 else 8
        fmt = exact.FP32 if fp32 else exact.BF16
        enc = exact.encode_fp32 if fp32 else exact.encode_bf16
        x = rng.standard_normal(n) * np.exp2(rng.uniform(-150, 128, n))
        r = np.abs(x) * np.exp2(rng.uniform(-60, -p + 1, n))
        r[::7] = 0.0
        # points just off a midpoint between two format values
        mids = np.float32(rng.standard_normal(n // 6) * np.exp2(rng.uniform(-130, 120, n // 6))).astype(np.float64)
        ulp = np.exp2(np.floor(np.log2(np.abs(mids))) - (p - 1))
        mids = mids + 0.5 * ulp * np.sign(mids) + rng.uniform(-4, 4, mids.size) * np.abs(mids) * 2.0 ** -52
        x[: mids.size] = mids
        r[: mids.size] = np.abs(mids) * 2.0 ** -55
        xs, rs = torch.from_numpy(x).cuda(), torch.from_numpy(r).cuda()
        bits = torch.zeros(n, dtype=torch.int32, device="cuda")
        ok = torch.zeros(n, dtype=torch.int32, device="cuda")
        assert hip.load().ea_hip_kat_round(n, xs.data_ptr(), rs.data_ptr(), fp32, bits.data_ptr(), ok.data_ptr(),
                                           torch.cuda.current_stream().cuda_stream) == 0
        torch.cuda.synchronize()
        gb, gk = bits.cpu().numpy().view(np.uint32), ok.cpu().numpy()

        def rn(v):
            m, e = exact.round_rational(v.numerator, v.denominator, fmt)
            return 0 if m == 0 else enc(m, e)

        n_ok = 0
        for i in range(n):
            if not gk[i]:
                continue
            n_ok += 1
            lo, hi = Fraction(float(x[i])) - Fraction(float(r[i])), Fraction(float(x[i])) + Fraction(float(r[i]))
            assert rn(lo) == rn(hi) == int(gb[i]), (float(x[i]), float(r[i]), fp32)
        assert n_ok > 0.5 * n, n_ok


# ---------------------------------------------------------------------------------------------
# rows against the oracle
# ---------------------------------------------------------------------------------------------

@pytest.mark.parametrize("kind", KINDS)
@pytest.mark.parametrize("vkind", ["normal", "wide", "dupes"])
def test_random_rows_match_oracle(gpu, kind, vkind):
    rng = np.random.default_rng(hash((kind, vkind)) % (1 << 32))
    prob = _rand_problem(rng, kind, vkind, B=2, T=3, Hq=4, Hkv=2, S=150, d=64, dv=64)
    ab = default_alpha_bits(64)
    want, _ = _oracle(prob, ab)
    got, flags, st = _run(prob, ab, splits=3)
    assert not np.any(flags == 1), (flags, st)
    assert np.array_equal(got, want)


@pytest.mark.parametrize("out", ["bf16", "fp32"])
def test_d128_rows_match_oracle_and_split_invariance(gpu, out):
    rng = np.random.default_rng(11)
    prob = _rand_problem(rng, "normal", "normal", B=3, T=2, Hq=4, Hkv=2, S=700, d=128, dv=128)
    ab = default_alpha_bits(128)
    want, _ = _oracle(prob, ab, out)
    for splits in (1, 2, 3, 7, 11):
        got, flags, st = _run(prob, ab, out, splits=splits, merge_order=list(range(64))[::-1])
        assert not np.any(flags), (splits, st)
        assert np.array_equal(got, want), splits


@pytest.mark.parametrize("kernel", ["decode", "general"])
def test_more_than_64_splits(gpu, kernel):
    """Split counts past one wave's 64 lanes (the combine takes them in slabs of 64): 71 and 141
    splits of 64 keys, ragged lengths, bf16 and fp32, with and without a caller's merge order,
    against the oracle and against 4 splits."""
    rng = np.random.default_rng(77)
    B, T, Hq, Hkv, d = 3, 1, 4, 2, 128
    seq = np.array([9000, 5003, 1])
    q = bf16(rng, (B, T, Hq, d))
    k = bf16(rng, (B, Hkv, 9000, d), "outlier")
    v = bf16(rng, (B, Hkv, 9000, d))
    prob = problem.contiguous(q, k, v, seq.reshape(B, 1), seq_len=seq)
    ab = default_alpha_bits(d)
    for out in ("bf16", "fp32"):
        want, _ = _oracle(prob, ab, out)
        ref, flags, _ = _run(prob, ab, out, splits=4, kernel=kernel)
        assert not np.any(flags) and np.array_equal(ref, want), out
        for splits, order in ((1000, None), (80, list(range(200))[::-1])):
            got, flags, st = _run(prob, ab, out, splits=splits, merge_order=order, kernel=kernel)
            assert st["nsplit"] > 64, st
            assert not np.any(flags), (out, splits, st)
            assert np.array_equal(got, want), (out, splits, st["nsplit"])


@pytest.mark.parametrize("kernel", ["decode", "prefill", "general"])
def test_batch_equals_separate_launches(gpu, kernel):
    """One launch over a ragged batch gives each sequence the bits and flags it gets launched
    alone (batch composition never changes bits; the reference's segments-versus-separate-launches
    check, tests/test_triton.py:314-361)."""
    rng = np.random.default_rng(hash(("batch", kernel)) % (1 << 32))
    B, Hq, Hkv, S, d = 3, 4, 2, 260, 128
    T = 24 if kernel == "prefill" else 2
    q = bf16(rng, (B, T, Hq, d), "outlier")
    k = bf16(rng, (B, Hkv, S, d), "normal")
    v = bf16(rng, (B, Hkv, S, d), "wide")
    seq = np.array([260, 97, 181])
    kv = np.stack([np.clip(seq[b] - T + 1 + np.arange(T), 0, None) for b in range(B)])
    ab = default_alpha_bits(d)
    batch = problem.to_paged(problem.contiguous(q, k, v, kv, seq_len=seq), 16, np.random.default_rng(9), "NHD")
    got, flags, st = _run(batch, ab, kernel=kernel)
    want, _ = _oracle(batch, ab)
    assert np.array_equal(got, want) and not np.any(flags), st
    key = {"decode": "decode_kernel_rows", "prefill": "prefill_kernel_rows"}.get(kernel)
    if key:
        assert st[key] == _rows(batch), st
    rows = T * Hq
    for b in range(B):
        one = problem.contiguous(q[b:b + 1], k[b:b + 1, :, :seq[b]], v[b:b + 1, :, :seq[b]], kv[b:b + 1],
                                 seq_len=seq[b:b + 1])
        alone, fl1, _ = _run(one, ab, kernel=kernel)
        assert np.array_equal(got[b], alone[0]), b
        assert np.array_equal(flags[b * rows:(b + 1) * rows], fl1), b


def test_paged_layouts_and_page_sizes_same_bits(gpu):
    rng = np.random.default_rng(12)
    base = _rand_problem(rng, "outlier", "normal", B=3, T=1, Hq=8, Hkv=4, S=333, d=128, dv=128, causal=False)
    ab = default_alpha_bits(128)
    want, _ = _oracle(base, ab)
    for ps in (1, 16, 64):
        for layout in ("NHD", "HND"):
            p = problem.to_paged(base, ps, np.random.default_rng(ps), layout)
            got, flags, _ = _run(p, ab, splits=4)
            assert not np.any(flags)
            assert np.array_equal(got, want), (ps, layout)


def test_tree_rows_equal_sequential_decode(gpu):
    """Each draft node's row equals decoding its root-to-node path after the prefix."""
    rng = np.random.default_rng(21)
    B, P, N, Hq, Hkv, d = 2, 300, 9, 4, 2, 128
    parents = [configs.draft_tree(rng, N) for _ in range(B)]
    q = bf16(rng, (B, N, Hq, d))
    k = bf16(rng, (B, Hkv, P + N, d))
    v = bf16(rng, (B, Hkv, P + N, d))
    mask = np.array([[sum(1 << a for a in configs.path_of(parents[b], i)) for i in range(N)] for b in range(B)],
                    dtype=np.uint64)
    tree = problem.contiguous(q, k, v, np.full((B, N), P), tree_mask=mask, tree_base=np.full(B, P))
    ab = default_alpha_bits(d)
    got, flags, _ = _run(tree, ab, splits=3)
    assert not np.any(flags)
    for b in range(B):
        for i in range(N):
            path = configs.path_of(parents[b], i)
            idx = np.concatenate([np.arange(P), P + np.array(path)])
            seq = problem.contiguous(q[b:b + 1, i:i + 1], k[b:b + 1][:, :, idx], v[b:b + 1][:, :, idx],
                                     np.array([[len(idx)]]))
            s_out, s_fl, _ = _run(seq, ab, splits=2)
            assert not np.any(s_fl)
            assert np.array_equal(got[b, i], s_out[0, 0]), (b, i)


def test_nonfinite_flags_exactly_the_rows_that_see_them(gpu):
    rng = np.random.default_rng(4)
    prob = _rand_problem(rng, "normal", "normal", B=1, T=8, Hq=2, Hkv=1, S=64, d=64, dv=64)
    prob["seq_len"][:] = 64
    prob["kv_len"][:] = 57 + np.arange(8)
    prob["k"][0, 0, 60, 3] = 0x7FC0   # NaN key at position 60
    prob["v"][0, 0, 62, 1] = 0x7F80   # inf value at position 62
    ab = default_alpha_bits(64)
    got, flags, _ = _run(prob, ab)
    kvl = prob["kv_len"]
    for t in range(8):
        for h in range(2):
            r = t * 2 + h
            assert flags[r] == (2 if kvl[t] > 60 else 0), (t, h, flags)


def test_fixture_sha256(gpu):
    """The reference's published SHA-256 of all 2x2048 causal rows of two real Qwen3-0.6B heads
    (fixtures/expected_sha256.json), computed by the HIP path."""
    z = np.load(os.path.join(GOLD, "qwen3_0.6b_heads.npz"))
    exp = json.load(open(os.path.join(GOLD, "expected_sha256.json")))
    for key, info in exp["heads"].items():
        q, k, v = z[f"q_{key}"], z[f"k_{key}"], z[f"v_{key}"]
        ab = int(np.asarray(z[f"alpha_{key}"], dtype=np.float32).view(np.uint32))
        L = q.shape[0]
        prob = problem.contiguous(q.reshape(1, L, 1, -1), k.reshape(1, 1, L, -1), v.reshape(1, 1, L, -1),
                                  (np.arange(L) + 1).reshape(1, L))
        got, flags, st = _run(prob, ab, splits=8)
        assert not np.any(flags), st
        assert hashlib.sha256(got.reshape(L, -1).tobytes()).hexdigest() == info["sha256"], key


# ---------------------------------------------------------------------------------------------
# the d = 128 decode kernel (one wave per segment row block and split)
# ---------------------------------------------------------------------------------------------

@pytest.mark.parametrize("kind", KINDS)
@pytest.mark.parametrize("vkind", ["normal", "wide", "dupes"])
def test_decode_kernel_kinds_match_oracle(gpu, kind, vkind):
    rng = np.random.default_rng(hash(("dec", kind, vkind)) % (1 << 32))
    prob = _rand_problem(rng, kind, vkind, B=2, T=1, Hq=4, Hkv=2, S=300, d=128, dv=128, causal=False)
    ab = default_alpha_bits(128)
    want, _ = _oracle(prob, ab)
    for splits in (1, 3):
        got, flags, st = _run(prob, ab, splits=splits)
        assert st["decode_kernel_rows"] == prob["q"].shape[0] * prob["q"].shape[2], st
        assert not np.any(flags == 1), (splits, flags, st)
        assert np.array_equal(got, want), (splits, st)


@pytest.mark.parametrize("hq,hkv,T", [(4, 4, 1), (8, 2, 1), (4, 2, 2), (2, 1, 3), (16, 8, 1)])
@pytest.mark.parametrize("ps", [0, 4, 16, 64])
def test_decode_kernel_shapes_pages_ragged(gpu, hq, hkv, T, ps):
    """Row blocks of 1, 2 and 4 rows (and a partial one), contiguous and paged caches of page
    size 4, 16 and 64 (NHD), sequence lengths around the 64-key tile edges."""
    rng = np.random.default_rng(1000 * hq + 100 * hkv + 10 * T + ps)
    B, d = 6, 128
    seq = np.array([1, 63, 64, 65, 129, 200])
    q = bf16(rng, (B, T, hq, d))
    k = bf16(rng, (B, hkv, 200, d))
    v = bf16(rng, (B, hkv, 200, d))
    kv = np.stack([np.clip(seq[b] - T + 1 + np.arange(T), 1, None) for b in range(B)])
    prob = problem.contiguous(q, k, v, kv, seq_len=seq)
    if ps:
        prob = problem.to_paged(prob, ps, np.random.default_rng(ps), "NHD")
    ab = default_alpha_bits(d)
    want, _ = _oracle(prob, ab)
    for splits in (1, 2):
        got, flags, st = _run(prob, ab, splits=splits)
        assert st["decode_kernel_rows"] > 0, st
        assert not np.any(flags), (splits, st)
        assert np.array_equal(got, want), (splits, st)


def test_decode_kernel_nonfinite_flags_exactly_the_rows_that_see_them(gpu):
    rng = np.random.default_rng(44)
    prob = _rand_problem(rng, "normal", "normal", B=1, T=8, Hq=2, Hkv=1, S=200, d=128, dv=128)
    prob["seq_len"][:] = 200
    prob["kv_len"][:] = 125 + 10 * np.arange(8)
    prob["k"][0, 0, 140, 3] = 0x7FC0   # NaN key at position 140
    prob["v"][0, 0, 162, 100] = 0xFF80  # -inf value at position 162
    ab = default_alpha_bits(128)
    got, flags, st = _run(prob, ab)
    assert st["decode_kernel_rows"] > 0, st
    kvl = prob["kv_len"]
    clean = {**prob, "k": prob["k"].copy(), "v": prob["v"].copy()}
    clean["k"][0, 0, 140, 3] = 0
    clean["v"][0, 0, 162, 100] = 0
    want, _ = _oracle(clean, ab)  # rows that do not see the non-finite keys are unaffected
    for t in range(8):
        for h in range(2):
            r = t * 2 + h
            assert flags[r] == (2 if kvl[t] > 140 else 0), (t, h, flags)
            if kvl[t] <= 140:
                assert np.array_equal(got[0, t, h], want[0, t, h]), (t, h)


@pytest.mark.parametrize("splits", [1, 2, 4])
def test_decode_kernel_converts_q_rows_itself(gpu, splits):
    """On the uniform grid the decode kernel converts its blocks' q rows (no prep launch): a NaN q
    row alone in the last, partial 2-row block of a segment (3 rows per segment), a -inf element
    in the first row of another block, and a q row of zeros, with 1, 2 and 4 splits writing the
    same converted rows. Exactly the non-finite rows are flag 2 and every other row equals the
    oracle; the clean q on the same geometry then leaves no flag."""
    rng = np.random.default_rng(4242 + splits)
    B, T, H, S = 2, 3, 2, 300
    prob = _rand_problem(rng, "normal", "normal", B=B, T=T, Hq=H, Hkv=H, S=S, d=128, dv=128)
    prob["q"][0, 2, 1, 7] = 0x7FC0     # NaN: segment (0, 1), row 2 (the partial block's only row)
    prob["q"][1, 0, 0, 100] = 0xFF80   # -inf: segment (1, 0), row 0
    prob["q"][1, 1, 1, :] = 0          # zeros: uniform weights
    bad = {(0, 2, 1), (1, 0, 0)}
    clean = {**prob, "q": prob["q"].copy()}
    for b, t, h in bad:
        clean["q"][b, t, h, :] = 0
    ab = default_alpha_bits(128)
    want, _ = _oracle(clean, ab)
    got, flags, st = _run(prob, ab, splits=splits)
    assert st["decode_kernel_rows"] > 0 and st["decode_equal_share_steps"] == 0, st
    fl = flags.reshape(B, T, H)
    for b in range(B):
        for t in range(T):
            for h in range(H):
                if (b, t, h) in bad:
                    assert fl[b, t, h] == 2, (b, t, h, flags)
                else:
                    assert fl[b, t, h] == 0, (b, t, h, flags)
                    assert np.array_equal(got[b, t, h], want[b, t, h]), (b, t, h)
    # the clean problem on the same geometry: no flag survives from the previous q rows
    got2, flags2, _ = _run(clean, ab, splits=splits)
    assert not np.any(flags2)
    assert np.array_equal(got2, want)


@pytest.mark.parametrize("B,S", [(64, 600), (16, 2048), (32, 1100)])
def test_decode_lead_wave_splits(gpu, B, S):
    """Uniform decode grids of exactly one round of resident blocks (MI355X: 1,024 = 512 units x
    2 splits, 128 x 8, 256 x 4): the first wave's splits take weighted key ranges, so units see
    1, 2 or no lead splits and cut their keys differently; ragged lengths leave some splits short
    or empty. Bits equal the oracle, every row certified."""
    rng = np.random.default_rng(7000 + B)
    prob = _rand_problem(rng, "normal", "normal", B=B, T=1, Hq=16, Hkv=8, S=S, d=128, dv=128, causal=False)
    prob["seq_len"][:] = rng.integers(S // 3, S + 1, size=B)
    prob["seq_len"][0] = S
    prob["kv_len"][:] = prob["seq_len"]  # one token per sequence
    ab = default_alpha_bits(128)
    want, _ = _oracle(prob, ab)
    got, flags, st = _run(prob, ab)
    assert st["decode_kernel_rows"] > 0 and st["decode_equal_share_steps"] == 0, st
    assert not np.any(flags), st
    assert np.array_equal(got, want)


@pytest.mark.parametrize("seed", range(401, 409))
def test_decode_lead_wave_random_grids(gpu, seed):
    """Seeded random uniform decode grids of exactly 1,024 blocks (the weighted first wave on
    MI355X): GQA group 1-4 (2-row blocks, several per segment, the XCD permutation when the
    segment count is a multiple of 8), 1-2 tokens, ragged lengths, contiguous or paged NHD caches.
    Bits equal the oracle and a one-split run, every row certified."""
    rng = np.random.default_rng(seed)
    while True:
        Hkv = int(rng.choice([1, 2, 4, 8]))
        grp = int(rng.choice([1, 2, 4]))
        T = int(rng.choice([1, 2]))
        B = int(rng.choice([4, 8, 16, 32, 64]))
        nrb = (T * grp + 1) // 2
        items = B * Hkv * nrb
        if items in (64, 128, 256, 512) and B * T * Hkv * grp <= 2048:
            break
    ns = 1024 // items
    S = ns * 64 * int(rng.integers(4, 9))
    prob = _rand_problem(rng, "normal", "normal", B=B, T=T, Hq=Hkv * grp, Hkv=Hkv, S=S, d=128, dv=128)
    prob["seq_len"][0] = S
    prob["kv_len"][:] = np.clip(prob["seq_len"][:, None] - T + 1 + np.arange(T), 1, None).reshape(prob["kv_len"].shape)
    if rng.random() < 0.5:
        prob = problem.to_paged(prob, int(rng.choice([16, 64])), np.random.default_rng(seed), "NHD")
    ab = default_alpha_bits(128)
    want, _ = _oracle(prob, ab)
    got, flags, st = _run(prob, ab)
    assert st["decode_kernel_rows"] > 0 and st["decode_equal_share_steps"] == 0, (seed, st)
    assert st["nsplit"] == ns, (seed, ns, st)
    assert not np.any(flags), (seed, st)
    assert np.array_equal(got, want), seed
    got1, _, _ = _run(prob, ab, splits=1)
    assert np.array_equal(got1, want), seed


# ---------------------------------------------------------------------------------------------
# the int8-MFMA prefill kernel (32 rows per block, balanced radix-256 digits)
# ---------------------------------------------------------------------------------------------

def _rows(prob):
    return prob["q"].shape[0] * prob["q"].shape[1] * prob["q"].shape[2]


@pytest.mark.parametrize("kind", KINDS)
@pytest.mark.parametrize("vkind", ["normal", "wide", "dupes"])
def test_prefill_kernel_kinds_match_oracle(gpu, kind, vkind):
    rng = np.random.default_rng(hash(("pf", kind, vkind)) % (1 << 32))
    prob = _rand_problem(rng, kind, vkind, B=2, T=40, Hq=4, Hkv=2, S=150, d=128, dv=128)
    ab = default_alpha_bits(128)
    want, _ = _oracle(prob, ab)
    got, flags, st = _run(prob, ab, kernel="prefill")
    assert st["prefill_kernel_rows"] == _rows(prob), st
    assert not np.any(flags == 1), st
    assert np.array_equal(got, want), st


@pytest.mark.parametrize("out", ["bf16", "fp32"])
def test_prefill_causal_matches_oracle_and_decode(gpu, out):
    """A causal prefill of 200 tokens (no forcing: T >= 64 selects the kernel) equals the oracle,
    and each token's row equals a single-token decode over the same keys."""
    rng = np.random.default_rng(31)
    B, T, Hq, Hkv, d = 1, 200, 4, 2, 128
    q = bf16(rng, (B, T, Hq, d))
    k = bf16(rng, (B, Hkv, T, d))
    v = bf16(rng, (B, Hkv, T, d))
    prob = problem.contiguous(q, k, v, (np.arange(T) + 1).reshape(1, T))
    ab = default_alpha_bits(d)
    want, _ = _oracle(prob, ab, out)
    got, flags, st = _run(prob, ab, out)
    assert st["prefill_kernel_rows"] == _rows(prob), st
    assert not np.any(flags), st
    assert np.array_equal(got, want), st
    # token-by-token decode (decode kernel) over the same keys
    dec = problem.contiguous(q.transpose(1, 0, 2, 3), np.repeat(k, T, axis=0), np.repeat(v, T, axis=0),
                             (np.arange(T) + 1).reshape(T, 1))
    got_d, fl_d, st_d = _run(dec, ab, out)
    assert st_d["prefill_kernel_rows"] == 0 and not np.any(fl_d)
    assert np.array_equal(got_d.reshape(got.shape[1:]), got[0])


def test_prefill_paged_gqa_ragged(gpu):
    """Paged NHD cache (page 16), GQA 4, ragged sequence lengths (partial 64-row blocks and
    partial 64-key tiles), rows whose prefix is empty."""
    rng = np.random.default_rng(32)
    B, T, Hq, Hkv, d = 3, 37, 8, 2, 128
    seq = np.array([37, 90, 130])
    q = bf16(rng, (B, T, Hq, d))
    k = bf16(rng, (B, Hkv, 130, d))
    v = bf16(rng, (B, Hkv, 130, d))
    kv = np.stack([np.clip(seq[b] - T + 1 + np.arange(T), 0, None) for b in range(B)])
    kv[0, :3] = 0
    base = problem.contiguous(q, k, v, kv, seq_len=seq)
    prob = problem.to_paged(base, 16, np.random.default_rng(3), "NHD")
    ab = default_alpha_bits(d)
    want, _ = _oracle(base, ab)
    got, flags, st = _run(prob, ab, kernel="prefill")
    assert st["prefill_kernel_rows"] == _rows(prob), st
    assert not np.any(flags), st
    assert np.array_equal(got, want)


def test_prefill_tree_masks_equal_decode(gpu):
    """Speculative-tree rows (prefix + 64-bit draft mask) through the prefill kernel give the same
    bits as the decode path on the same problem."""
    rng = np.random.default_rng(22)
    B, P, N, Hq, Hkv, d = 2, 150, 12, 4, 2, 128
    parents = [configs.draft_tree(rng, N) for _ in range(B)]
    q = bf16(rng, (B, N, Hq, d))
    k = bf16(rng, (B, Hkv, P + N, d))
    v = bf16(rng, (B, Hkv, P + N, d))
    mask = np.array([[sum(1 << a for a in configs.path_of(parents[b], i)) for i in range(N)] for b in range(B)],
                    dtype=np.uint64)
    tree = problem.contiguous(q, k, v, np.full((B, N), P), tree_mask=mask, tree_base=np.full(B, P))
    ab = default_alpha_bits(d)
    want, fl_d, st_d = _run(tree, ab, splits=2)
    assert st_d["prefill_kernel_rows"] == 0 and not np.any(fl_d), st_d
    got, flags, st = _run(tree, ab, kernel="prefill")
    assert st["prefill_kernel_rows"] == _rows(tree), st
    assert not np.any(flags), st
    assert np.array_equal(got, want)


def test_prefill_four_wave_block_matches_oracle(gpu):
    """The 4-wave prefill block (ea_options.prefill_waves = 4) gives the oracle's bits, like the
    default 8-wave block."""
    rng = np.random.default_rng(23)
    prob = _rand_problem(rng, "normal", "normal", B=2, T=70, Hq=4, Hkv=2, S=300, d=128, dv=128)
    ab = default_alpha_bits(128)
    want, _ = _oracle(prob, ab)
    got8, fl8, st8 = _run(prob, ab, kernel="prefill")
    got4, fl4, st4 = _run(prob, ab, kernel="prefill", prefill_waves=4)
    for got, fl, st in ((got8, fl8, st8), (got4, fl4, st4)):
        assert st["prefill_kernel_rows"] == _rows(prob), st
        assert not np.any(fl == 1), st
        assert np.array_equal(got, want), st


@pytest.mark.parametrize("splits", [2, 3, 5])
def test_prefill_key_splits_match_oracle(gpu, splits):
    """The int8 prefill kernel with its key range cut into 2, 3 and 5 splits (partials merged and
    rounded by ea_pf_combine): the oracle's bits, as with one split; ragged causal rows, so some
    splits of a row block hold no visible key, and wide values whose bases differ per split."""
    rng = np.random.default_rng(70 + splits)
    prob = _rand_problem(rng, "outlier", "wide", B=2, T=40, Hq=4, Hkv=2, S=700, d=128, dv=128)
    ab = default_alpha_bits(128)
    want, _ = _oracle(prob, ab)
    one, fl1, st1 = _run(prob, ab, splits=1, kernel="prefill")
    got, flags, st = _run(prob, ab, splits=splits, kernel="prefill")
    assert st["nsplit"] >= 2 and st1["nsplit"] == 1, (st, st1)  # 11 tiles: 2, 3 and 4 splits
    assert st["prefill_kernel_rows"] == _rows(prob), st
    assert not np.any(flags == 1) and not np.any(fl1 == 1), (st, st1)
    assert np.array_equal(one, want)
    assert np.array_equal(got, want)


def test_prefill_rows_longer_than_256_tiles(gpu):
    """Rows that see 16,837 to 16,900 keys (more than 256 tiles of 64): the per-lane epoch sums
    fold at least once on age alone, and the rows still equal the oracle."""
    rng = np.random.default_rng(77)
    B, T, Hq, Hkv, d, S = 1, 64, 2, 1, 128, 16900
    q = bf16(rng, (B, T, Hq, d))
    k = bf16(rng, (B, Hkv, S, d))
    v = bf16(rng, (B, Hkv, S, d))
    prob = problem.contiguous(q, k, v, (S - T + 1 + np.arange(T)).reshape(1, T))
    ab = default_alpha_bits(d)
    want, _ = _oracle(prob, ab)
    got, flags, st = _run(prob, ab)
    assert st["prefill_kernel_rows"] == _rows(prob), st
    assert st["prefill_epoch_folds"] > 0, st
    assert not np.any(flags), st
    assert np.array_equal(got, want)


# ---------------------------------------------------------------------------------------------
# the digit-tile cache (the KV slice format kept across steps: ea_hip_kv_digits_update)
# ---------------------------------------------------------------------------------------------

def _kv_digits_problem(rng, paged_cache):
    B, T, Hq, Hkv, d, S = 2, 70, 4, 2, 128, 300
    q = bf16(rng, (B, T, Hq, d))
    k = bf16(rng, (B, Hkv, S, d), "wide")
    v = bf16(rng, (B, Hkv, S, d), "outlier")
    seq = np.array([300, 251])
    kv = np.stack([np.clip(seq[b] - T + 1 + np.arange(T), 0, None) for b in range(B)])
    base = problem.contiguous(q, k, v, kv, seq_len=seq)
    return problem.to_paged(base, 16, np.random.default_rng(5), "NHD") if paged_cache else base


@pytest.mark.parametrize("paged_cache", [False, True])
def test_kv_digits_appends_equal_one_update(gpu, paged_cache):
    """Slicing a cache in appended chunks (seq_len growing with each append, so partly filled tiles
    are sliced again) leaves the same bytes as one update over every key."""
    import torch
    from exactattention_amd.hip import DeviceProblem, KVDigits
    prob = _kv_digits_problem(np.random.default_rng(61), paged_cache)
    dp = DeviceProblem(prob, "bf16", 0, "cuda:0")
    seq = prob["seq_len"].copy()
    tiles = (int(seq.max()) + 63) // 64
    one = KVDigits(dp, tiles)
    zeros = torch.zeros(2, dtype=torch.int32, device="cuda")
    one.update(dp, zeros, torch.from_numpy(seq.astype(np.int32)).cuda(), int(seq.max()))
    chunked = KVDigits(dp, tiles)
    bounds = [0, 100, 170, 229, 300]
    for a, e in zip(bounds[:-1], bounds[1:]):
        cur = np.minimum(seq, e).astype(np.int32)
        dp.t["seq_len"].copy_(torch.from_numpy(cur))
        kb = torch.from_numpy(np.minimum(seq, a).astype(np.int32)).cuda()
        chunked.update(dp, kb, dp.t["seq_len"].clone(), e - a)
    torch.cuda.synchronize()
    assert torch.equal(one.buf, chunked.buf)


@pytest.mark.parametrize("paged_cache", [False, True])
def test_prefill_reads_kv_digits_cache(gpu, paged_cache):
    """The prefill kernel reading the caller's digit cache gives the bits it gives when it slices
    K/V itself, and the oracle's."""
    import torch
    from exactattention_amd.hip import DeviceProblem, KVDigits, STATS, launch_hip
    prob = _kv_digits_problem(np.random.default_rng(62), paged_cache)
    ab = default_alpha_bits(128)
    want, _ = _oracle(prob, ab)
    plain, fl, st = _run(prob, ab, kernel="prefill")
    assert st["prefill_kernel_rows"] == _rows(prob) and not np.any(fl), st
    assert np.array_equal(plain, want)
    dp = DeviceProblem(prob, "bf16", 0, "cuda:0", kernel="prefill")
    cache = KVDigits(dp, (int(prob["seq_len"].max()) + 63) // 64)
    cache.update(dp, torch.zeros(2, dtype=torch.int32, device="cuda"), dp.t["seq_len"].clone(),
                 int(prob["seq_len"].max()))
    launch_hip(dp, ab, kv_digits=cache)
    torch.cuda.synchronize()
    got = dp.out.cpu().numpy().view(np.uint16)
    st2 = dict(zip(STATS, dp.stats.cpu().numpy().tolist()))
    assert st2["prefill_kernel_rows"] == _rows(prob), st2
    assert not np.any(dp.flags.cpu().numpy())
    assert np.array_equal(got, want)


def test_chunked_prefill_from_the_cache_equals_full_prefill(gpu):
    """A 192-token prefill served as three 64-token chunks: each chunk appends its keys to the
    digit cache (only the new tiles are sliced) and attends through the cache; every row equals the
    one-shot causal prefill's."""
    import torch
    from exactattention_amd.hip import DeviceProblem, KVDigits, launch_hip
    rng = np.random.default_rng(63)
    B, T, Hq, Hkv, d = 1, 192, 4, 2, 128
    q = bf16(rng, (B, T, Hq, d))
    k = bf16(rng, (B, Hkv, T, d))
    v = bf16(rng, (B, Hkv, T, d))
    ab = default_alpha_bits(d)
    full = problem.contiguous(q, k, v, (np.arange(T) + 1).reshape(1, T))
    want, fl, st = _run(full, ab)
    assert st["prefill_kernel_rows"] == _rows(full) and not np.any(fl), st
    # the cache lives beside a problem that holds the whole K/V; seq_len grows with each chunk
    host = DeviceProblem(full, "bf16", 0, "cuda:0")
    cache = KVDigits(host, T // 64)
    for c in range(3):
        a, e = 64 * c, 64 * c + 64
        host.t["seq_len"].fill_(e)
        cache.update(host, torch.full((1,), a, dtype=torch.int32, device="cuda"),
                     torch.full((1,), e, dtype=torch.int32, device="cuda"), 64)
        chunk = problem.contiguous(q[:, a:e], k, v, (np.arange(a, e) + 1).reshape(1, 64), seq_len=np.array([e]))
        dp = DeviceProblem(chunk, "bf16", 0, "cuda:0")
        launch_hip(dp, ab, kv_digits=cache)
        torch.cuda.synchronize()
        got = dp.out.cpu().numpy().view(np.uint16)
        assert not np.any(dp.flags.cpu().numpy()), c
        assert np.array_equal(got[0], want[0, a:e]), c


def test_prefill_nonfinite_flags_exactly_the_rows_that_see_them(gpu):
    rng = np.random.default_rng(45)
    T = 80
    prob = _rand_problem(rng, "normal", "normal", B=1, T=T, Hq=2, Hkv=1, S=T, d=128, dv=128)
    prob["seq_len"][:] = T
    prob["kv_len"][:] = np.arange(T) + 1
    prob["k"][0, 0, 50, 3] = 0x7FC0   # NaN key at position 50
    prob["v"][0, 0, 70, 100] = 0xFF80  # -inf value at position 70
    prob["q"][0, 10, 1, 5] = 0x7F80    # inf in one query row
    ab = default_alpha_bits(128)
    got, flags, st = _run(prob, ab, kernel="prefill")
    clean = {**prob, "k": prob["k"].copy(), "v": prob["v"].copy(), "q": prob["q"].copy()}
    clean["k"][0, 0, 50, 3] = 0
    clean["v"][0, 0, 70, 100] = 0
    clean["q"][0, 10, 1, 5] = 0
    want, _ = _oracle(clean, ab)
    for t in range(T):
        for h in range(2):
            bad = t >= 50 or (t == 10 and h == 1)
            assert flags[t * 2 + h] == (2 if bad else 0), (t, h)
            if not bad:
                assert np.array_equal(got[0, t, h], want[0, t, h]), (t, h)


def test_prefill_c3_golden_hash(gpu):
    """BASELINE config C3 at full size (4096 tokens, 16/8 heads): the committed oracle hash."""
    p = configs.c3()
    ab = configs.alpha_bits()
    got, flags, st = _run(p, ab)
    gold = json.load(open(os.path.join(GOLD, "baseline_sha256.json")))["C3"]["sha256"]
    assert st["prefill_kernel_rows"] == _rows(p), st
    assert not np.any(flags), st
    assert hashlib.sha256(got.tobytes()).hexdigest() == gold, st


@pytest.fixture(scope="module")
def c4_problem():
    return configs.c4()


@pytest.mark.parametrize("name,kernel,splits", [("C1", "auto", 0), ("C2", "auto", 0), ("C2", "auto", 1),
                                                 ("C2", "auto", 8), ("C4", "auto", 0), ("C4", "decode", 0)],
                         ids=["C1", "C2", "C2-splits1", "C2-splits8", "C4", "C4-decode-kernel"])
def test_config_golden_hash(gpu, request, name, kernel, splits):
    """BASELINE configs C1, C2 and C4 at full size against the committed hashes (the oracle's and
    the reference C++ kernel's bits). C2 also at 1 and 8 KV splits (BASELINE: the bits must not
    depend on the split count). C4 (16-node draft trees, GQA 2: 32 rows per sequence and KV head)
    runs on the int8 prefill kernel by default and on the decode kernel when the prefill kernel is
    switched off; both give the golden bits. No row may need more than the device tiers."""
    p = request.getfixturevalue("c4_problem") if name == "C4" else configs.CONFIGS[name]()
    got, flags, st = _run(p, configs.alpha_bits(), splits=splits, kernel=kernel)
    gold = json.load(open(os.path.join(GOLD, "baseline_sha256.json")))[name]["sha256"]
    assert not flags.any() and st["uncertified"] == 0, st
    if splits:
        assert st["nsplit"] == splits, st
    assert hashlib.sha256(got.tobytes()).hexdigest() == gold, st
    if name == "C4":
        assert st["prefill_kernel_rows"] == (_rows(p) if kernel == "auto" else 0), st


@pytest.fixture(scope="module")
def c5_problem(request):
    """BASELINE config C5 (16 sequences of 8K-131K keys, outlier channels): about 4.5 GB of K/V
    generated from its seed on the host, once for the module. Generation prints its progress (the
    seeded draws take a minute or two)."""
    import time
    capman = request.config.pluginmanager.getplugin("capturemanager")
    t0 = time.time()
    with capman.global_and_fixture_disabled():
        print(f"\n[c5] generating BASELINE C5 inputs (seed 1005) ...", flush=True)
    p = configs.c5()
    with capman.global_and_fixture_disabled():
        print(f"[c5] generated in {time.time() - t0:.0f} s", flush=True)
    return p


@pytest.mark.parametrize("page", [16, 64])
def test_c5_golden_hash_page_sizes(gpu, request, page):
    """BASELINE config C5 at full size, the cache in pages of 16 and of 64 keys: both give the
    committed golden bits (the reference C++ kernel's), and no row needs more than tier 1."""
    import time
    p = request.getfixturevalue("c5_problem")
    capman = request.config.pluginmanager.getplugin("capturemanager")
    if page != 16:
        t0 = time.time()
        p = configs.c5_repage(p, page)
        with capman.global_and_fixture_disabled():
            print(f"\n[c5] repaged to {page} in {time.time() - t0:.0f} s", flush=True)
    got, flags, st = _run(p, configs.alpha_bits())
    gold = json.load(open(os.path.join(GOLD, "baseline_sha256.json")))["C5"]["sha256"]
    assert not flags.any() and st["tier1_flagged"] == 0, st
    assert hashlib.sha256(got.tobytes()).hexdigest() == gold, (page, st)


def test_prefill_c3_back_to_back(gpu):
    """C3 launched 12 times in a row with no host synchronisation between steps: the kernel's
    pipeline (tile DMA into LDS overlapping the MFMA work) must give the same certified rows in
    every step, so no row may leave the prefill kernel uncertified and the last output still
    carries the golden hash."""
    import torch
    from exactattention_amd.hip import STATS, DeviceProblem, launch_hip
    p = configs.c3()
    ab = configs.alpha_bits()
    gold = json.load(open(os.path.join(GOLD, "baseline_sha256.json")))["C3"]["sha256"]
    dp = DeviceProblem(p, "bf16", 0, "cuda:0")
    steps = 12
    for _ in range(steps):
        launch_hip(dp, ab)
    torch.cuda.synchronize()
    st = dict(zip(STATS, dp.stats.cpu().numpy().tolist()))
    out = dp.out.cpu().numpy().view(np.uint16)
    assert st["prefill_kernel_rows"] == steps * _rows(p), st
    assert st["tier1_flagged"] == 0 and st["uncertified_final"] == 0, st
    assert hashlib.sha256(out.tobytes()).hexdigest() == gold, st


def _zero_length_problems(kernel):
    """A batch holding sequences with no keys at all (seq_len 0) beside a 5-key and a multi-tile
    sequence, contiguous and in NHD / HND pages of 16; T = 64 causal tokens for the prefill kernel,
    one decode token otherwise."""
    rng = np.random.default_rng(404)
    T = 64 if kernel == "prefill" else 1
    B, Hkv, grp, S, d = 4, 2, 2, 300, 128
    seq = np.array([0, 5, 300, 0])
    kv = np.stack([np.clip(seq[b] - T + 1 + np.arange(T), 0, None) for b in range(B)])
    q = bf16(rng, (B, T, Hkv * grp, d), "normal")
    k = bf16(rng, (B, Hkv, S, d), "normal")
    v = bf16(rng, (B, Hkv, S, d), "normal")
    base = problem.contiguous(q, k, v, kv, seq_len=seq)
    return [("contiguous", base)] + [(lay, problem.to_paged(base, 16, np.random.default_rng(405), lay))
                                     for lay in ("NHD", "HND")]


@pytest.mark.parametrize("kernel", ["decode", "prefill", "general"])
def test_sequences_of_length_zero(gpu, kernel):
    """Rows of a sequence with seq_len 0 see an empty set: +0 with flag 0, as the oracle gives;
    every other row of the batch stays exact, at the automatic split count and at 3 splits."""
    ab = default_alpha_bits(128)
    for name, prob in _zero_length_problems(kernel):
        want, _ = _oracle(prob, ab)
        assert not want[[0, 3]].any()
        for splits in (0, 3):
            got, flags, st = _run(prob, ab, "bf16", splits, kernel=kernel)
            assert not flags.any(), (name, splits, st)
            assert np.array_equal(got, want), (name, splits)
            if kernel != "general":
                assert st[f"{kernel}_kernel_rows"] > 0, (name, splits, st)


@pytest.mark.parametrize("case", ["many_small_units", "ragged_long"])
def test_decode_equal_share_plan(gpu, case):
    """The decode kernel's equal-share plan (taken when the uniform split grid would need more
    than one round of resident blocks): with 1,040 short units every block's share reaches several
    units (the piece loop), and with a few long ragged sequences shares cut units at arbitrary
    tiles. Bits equal the oracle's row by row and the same problem at one fixed split count."""
    rng = np.random.default_rng(77 if case == "many_small_units" else 78)
    ab = default_alpha_bits(128)
    if case == "many_small_units":
        B, S, Hq, Hkv, page = 130, 700, 16, 8, 16
        lens = rng.integers(0, S + 1, size=B)
        lens[:3] = [0, 1, S]
    else:
        B, S, Hq, Hkv, page = 5, 24000, 16, 8, 64
        lens = rng.integers(2000, S + 1, size=B)
    q = bf16(rng, (B, 1, Hq, 128))
    k = bf16(rng, (B, Hkv, S, 128), "outlier")
    v = bf16(rng, (B, Hkv, S, 128))
    base = problem.contiguous(q, k, v, lens.reshape(B, 1), seq_len=lens)
    prob = problem.to_paged(base, page, rng, "NHD")
    got, flags, st = _run(prob, ab)
    assert st["decode_kernel_rows"] > 0 and st["decode_equal_share_steps"] == 1, st
    want, _ = _oracle(prob, ab)
    assert not flags.any()
    assert np.array_equal(got, want)
    # one step with a split count the caller fixes (uniform splits when it fits one round)
    got2, flags2, st2 = _run(prob, ab, splits=1)
    assert np.array_equal(got2, want) and not flags2.any()


@pytest.mark.parametrize("case", ["uniform", "equal_share"])
def test_decode_xcd_placement(gpu, case):
    """GQA 4 decode (2-row blocks, 2 units per segment, segments a multiple of 8): the decode
    kernel places a segment's row blocks on one XCD, on the uniform split grid and, with more
    units than an eighth of the equal-share plan's blocks, by a permutation of the shares. The
    work moves between workgroups only: bits equal the general split kernel's on the same problem
    (ragged lengths, paged NHD) and, on the uniform case, the oracle's."""
    rng = np.random.default_rng(91 if case == "uniform" else 92)
    ab = default_alpha_bits(128)
    if case == "uniform":
        B, S, page = 4, 1500, 16          # 32 segments x 2 row blocks, uniform splits
    else:
        B, S, page = 16, 9500, 64         # 128 segments x 2 row blocks, 8 splits: equal-share plan
    Hq, Hkv = 32, 8
    lens = rng.integers(S // 3, S + 1, size=B)
    q = bf16(rng, (B, 1, Hq, 128))
    k = bf16(rng, (B, Hkv, S, 128), "outlier")
    v = bf16(rng, (B, Hkv, S, 128))
    base = problem.contiguous(q, k, v, lens.reshape(B, 1), seq_len=lens)
    prob = problem.to_paged(base, page, rng, "NHD")
    got, flags, st = _run(prob, ab)
    assert st["decode_kernel_rows"] > 0 and not flags.any(), st
    assert st["decode_equal_share_steps"] == (1 if case == "equal_share" else 0), st
    ref, flags2, st2 = _run(prob, ab, kernel="general")
    assert st2["decode_kernel_rows"] == 0 and not flags2.any()
    assert np.array_equal(got, ref)
    if case == "uniform":
        want, _ = _oracle(prob, ab)
        assert np.array_equal(got, want)


@pytest.mark.parametrize("seed", [301, 302, 303, 304, 305, 306])
def test_decode_placement_random_many_segments(gpu, seed):
    """Seeded geometries with 128-256 segments (8 KV heads) and 2-8 row blocks per segment, ragged
    lengths, pages of 16 or 64 keys, 1 or 2 tokens: the decode kernel, its row blocks placed by
    XCD on the uniform grid or the equal-share plan (whichever the step takes), gives the general
    split kernel's bits, every row certified."""
    rng = np.random.default_rng(seed)
    ab = default_alpha_bits(128)
    Hkv = 8
    grp = int(rng.choice([2, 4, 8]))
    T = int(rng.choice([1, 2]))
    B = int(rng.choice([16, 24, 32]))
    S = int(rng.integers(1500, 9001))
    lens = rng.integers(S // 4, S + 1, size=B)
    kv = np.stack([np.clip(lens[b] - T + 1 + np.arange(T), 0, None) for b in range(B)])
    q = bf16(rng, (B, T, Hkv * grp, 128))
    k = bf16(rng, (B, Hkv, S, 128), str(rng.choice(["normal", "outlier", "wide"])))
    v = bf16(rng, (B, Hkv, S, 128))
    base = problem.contiguous(q, k, v, kv, seq_len=lens)
    prob = problem.to_paged(base, int(rng.choice([16, 64])), rng, "NHD")
    got, flags, st = _run(prob, ab)
    desc = f"seed {seed}: B={B} T={T} grp={grp} S={S} {st}"
    assert st["decode_kernel_rows"] > 0 and not flags.any(), desc
    ref, flags2, st2 = _run(prob, ab, kernel="general")
    assert not flags2.any(), desc
    assert np.array_equal(got, ref), desc
