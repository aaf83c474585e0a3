"""Pins the CPU oracle before anything is compared with it.

Each check is chosen so a plausible mistake (a dropped term, a wrong sign or index, a wrong
rounding direction) fails it: closed forms (numpy's IEEE conversions, Fractions), independent
high-precision evaluations (mpmath 1.3.0 at 400 bits), exact integer brackets, the reference's
published SHA-256 of two real heads, the reference's own C++ kernel built from its source, and
invariants the definition fixes (split/tile/order invariance, tree = sequential decode).
"""

import hashlib
import json
import math
import os
from fractions import Fraction

import numpy as np
import pytest
from hypothesis import given, strategies as st

from gen import KINDS, bf16
from oracle import exact, oracle

GOLD = os.path.join(os.path.dirname(__file__), "golden")
A32 = exact.default_alpha_bits(32)
A64 = exact.default_alpha_bits(64)
A128 = exact.default_alpha_bits(128)


def f32(bits):
    return float(np.array([bits], dtype=np.uint32).view(np.float32)[0])


def bf2f(bits):
    return (np.asarray(bits, dtype=np.uint16).astype(np.uint32) << 16).view(np.float32)


# ---------------------------------------------------------------------------------------------
# formats (reference tests/test_formats.py)
# ---------------------------------------------------------------------------------------------

@pytest.mark.parametrize("seed", range(3))
def test_round_rational_matches_numpy_fp32(seed):
    rng = np.random.default_rng(seed)
    xs = np.exp2(rng.uniform(-160, 130, 3000)) * rng.choice([-1.0, 1.0], 3000)
    ties = np.float32(rng.standard_normal(600)).astype(np.float64)
    ties = ties + np.spacing(np.float32(ties)).astype(np.float64) / 2  # exact midpoints
    for x in np.concatenate([xs, ties]).tolist():
        num, den = float(x).as_integer_ratio()
        with np.errstate(over="ignore"):
            want = np.float32(x)
        if math.isinf(want):
            with pytest.raises(exact.DomainError):
                exact.round_rational(num, den, exact.FP32)
            continue
        m, e = exact.round_rational(num, den, exact.FP32)
        assert math.ldexp(m, e) == float(want), x
        assert (exact.encode_fp32(m, e) if m else 0) == (int(np.float32(want).view(np.uint32)) & (0x7FFFFFFF if want == 0 else 0xFFFFFFFF))


@pytest.mark.parametrize("seed", range(2))
def test_round_rational_bf16_matches_bit_trick(seed):
    from exactattention_amd.formats import float_to_bf16_bits
    rng = np.random.default_rng(seed)
    xs = np.float32(rng.standard_normal(4000) * np.exp2(rng.uniform(-135, 100, 4000)))
    bits = float_to_bf16_bits(xs)
    for x, b in zip(xs.tolist(), bits.tolist()):
        num, den = float(x).as_integer_ratio()
        m, e = exact.round_rational(num, den, exact.BF16)
        if m == 0:
            assert b & 0x7FFF == 0
        else:
            assert exact.encode_bf16(m, e) == b


def test_ties_to_even_and_decode():
    assert math.ldexp(*exact.round_dyadic(3, -1, exact.FP32)) == 1.5
    assert math.ldexp(*exact.round_dyadic((1 << 24) + 1, 0, exact.FP32)) == float(1 << 24)
    assert math.ldexp(*exact.round_dyadic((1 << 24) + 3, 0, exact.FP32)) == float((1 << 24) + 4)
    rng = np.random.default_rng(0)
    for x in np.float32(rng.standard_normal(500) * np.exp2(rng.uniform(-149, 127, 500))).tolist():
        assert math.ldexp(*exact.decode_fp32_bits(int(np.float32(x).view(np.uint32)))) == x
    for b in (0x7F80, 0x7FC0, 0xFF80):
        with pytest.raises(exact.DomainError):
            exact.decode_bf16(b)


# ---------------------------------------------------------------------------------------------
# exp2 weights (reference tests/test_exp2.py)
# ---------------------------------------------------------------------------------------------

def _rn24_mpmath(t: float):
    from mpmath import mp, mpf, power
    with mp.workprec(400):
        n = math.floor(t)
        q = int(mp.floor(power(2, mpf(t) - n) * 2 ** 23 + mpf("0.5")))
    e = n - 23
    if q == 1 << 24:
        q >>= 1
        e += 1
    return q, e


def test_ln2_enclosure_brackets_ln2():
    from mpmath import mp, log
    for W in (64, 126, 200):
        lo, hi = exact.ln2_enclosure(W)
        with mp.workprec(W + 80):
            x = log(2) * mp.mpf(2) ** W
            assert lo <= x <= hi and hi - lo < W  # about one unit per series term
    lo, hi = oracle.ln2_126()  # the C oracle's own constant
    plo, phi = exact.ln2_enclosure(126)
    assert lo <= phi and plo <= hi and hi - lo < 64


def test_integer_t_is_exact_power_of_two():
    for n in (-200, -1, 0, 1, 5, 127, 300):
        assert exact.exp2_rn(n, 0) == (1 << 23, n - 23)


@pytest.mark.parametrize("seed", range(2))
def test_exp2_matches_mpmath(seed):
    rng = np.random.default_rng(seed)
    for t in np.float32(np.concatenate([rng.uniform(-80, 80, 300), rng.uniform(-1e-5, 1e-5, 50)])).tolist():
        tm, te = exact.decode_fp32_bits(int(np.float32(t).view(np.uint32)))
        assert exact.exp2_rn(tm, te) == _rn24_mpmath(t), t


@pytest.mark.parametrize("seed", range(2))
def test_c_oracle_weights_match_python(seed):
    rng = np.random.default_rng(100 + seed)
    ts = np.float32(np.concatenate([rng.uniform(-60, 60, 3000), rng.uniform(-1e-6, 1e-6, 300),
                                    np.arange(-40, 40) + rng.uniform(-1e-7, 1e-7, 80),
                                    rng.uniform(-1e4, 1e4, 500), [2.0 ** -25, -(2.0 ** -25), 2.0 ** -24]]))
    for t in ts.tolist():
        b = int(np.float32(t).view(np.uint32))
        got = oracle.weight(b)
        assert got == exact.exp2_rn(*exact.decode_fp32_bits(b)), t


def test_default_alpha():
    from exactattention_amd.formats import default_alpha_bits
    assert f32(A128) == float(np.float32(np.log2(np.e) / np.sqrt(128)))
    for d in (16, 32, 64, 80, 96, 128, 256):
        assert exact.default_alpha_bits(d) == default_alpha_bits(d), d
        from mpmath import mp, log, sqrt, mpf
        with mp.workprec(200):
            v = 1 / (log(2) * sqrt(mpf(d)))
            m, e = mp.mpf(v).man_exp
        assert exact.encode_fp32(*exact.round_dyadic(int(m), int(e), exact.FP32)) == exact.default_alpha_bits(d)


def test_c_oracle_logit_is_exact_rounding():
    rng = np.random.default_rng(17)
    for kind in KINDS:
        q = bf16(rng, 64, kind)
        for _ in range(40):
            k = bf16(rng, 64, kind)
            qd = [exact.decode_bf16(x) for x in q.tolist()]
            kd = [exact.decode_bf16(x) for x in k.tolist()]
            am, ae = exact.decode_fp32_bits(A64)
            tm, te = exact.logit(am, ae, exact.exact_dot(qd, kd))
            assert oracle.logit_bits(q, k, A64) == (exact.encode_fp32(tm, te) if tm else 0)


def test_round_ratio_matches_python():
    rng = np.random.default_rng(4)
    for _ in range(3000):
        ab, bb = int(rng.integers(1, 128)), int(rng.integers(1, 128))
        a = (int(rng.integers(1, 1 << min(ab, 62))) << max(0, ab - 62)) | int(rng.integers(0, 2))
        b = int(rng.integers(1, 1 << min(bb, 62))) << max(0, bb - 62)
        E = int(rng.integers(-320, 200))
        neg = bool(rng.integers(0, 2))
        for fmt, is32 in ((exact.FP32, True), (exact.BF16, False)):
            bits, ov = oracle.round_ratio_bits(a, b, E, neg, is32)
            num, den = (a << E, b) if E >= 0 else (a, b << -E)
            try:
                m, e = exact.round_rational(-num if neg else num, den, fmt)
                assert not ov
                want = 0 if m == 0 else (exact.encode_fp32(m, e) if is32 else exact.encode_bf16(m, e))
                assert bits == want, (a, b, E, neg, is32)
            except exact.DomainError:
                assert ov


# ---------------------------------------------------------------------------------------------
# the definition's closed forms (reference tests/test_reference.py)
# ---------------------------------------------------------------------------------------------

def test_single_key_returns_value_exactly():
    rng = np.random.default_rng(0)
    q, k, v = bf16(rng, 64), bf16(rng, (1, 64)), bf16(rng, (1, 64))
    assert np.array_equal(exact.attention_row(q, k, v, A64), v[0])
    res, fl = oracle.attention_csr(q.reshape(1, -1), k, v, A64)
    assert np.array_equal(res[0], v[0])


def test_identical_keys_average_values():
    rng = np.random.default_rng(1)
    q = bf16(rng, 32)
    k = np.repeat(bf16(rng, (1, 32)), 4, axis=0)
    v = bf16(rng, (4, 32))
    want = np.float32(bf2f(v).astype(np.float64).mean(axis=0)).view(np.uint32)
    assert np.array_equal(exact.attention_row(q, k, v, A32, "fp32"), want)
    res, _ = oracle.attention_csr(q.reshape(1, -1), k, v, A32, out="fp32")
    assert np.array_equal(res[0], want)


def test_zero_query_gives_rn_of_mean():
    rng = np.random.default_rng(2)
    q = np.zeros(64, np.uint16)
    k, v = bf16(rng, (7, 64)), bf16(rng, (7, 16))
    vf = bf2f(v).astype(np.float64)
    for out in ("bf16", "fp32"):
        got = exact.attention_row(q, k, v, A64, out)
        num, den = Fraction(0), 7
        for c in range(16):
            m, e = exact.round_rational(*(Fraction(sum(Fraction(x) for x in vf[:, c])) / 7).as_integer_ratio(),
                                        exact.BF16 if out == "bf16" else exact.FP32)
            want = 0 if m == 0 else (exact.encode_bf16(m, e) if out == "bf16" else exact.encode_fp32(m, e))
            assert int(got[c]) == want


def test_empty_set_and_nan():
    rng = np.random.default_rng(2)
    q = bf16(rng, 16)
    assert np.array_equal(exact.attention_row(q, np.zeros((0, 16), np.uint16), np.zeros((0, 8), np.uint16),
                                              exact.default_alpha_bits(16)), np.zeros(8, np.uint16))
    k = bf16(rng, (3, 16))
    k[1, 2] = 0x7FC0
    with pytest.raises(exact.DomainError):
        exact.attention_row(q, k, bf16(rng, (3, 16)), exact.default_alpha_bits(16))
    with pytest.raises(exact.DomainError):
        oracle.attention_csr(q.reshape(1, -1), k, bf16(rng, (3, 16)), exact.default_alpha_bits(16))


def test_bf16_out_is_nearest_to_exact_ratio():
    rng = np.random.default_rng(7)
    q, k, v = bf16(rng, 16), bf16(rng, (40, 16)), bf16(rng, (40, 8))
    tr = exact.trace_row(q, k, v, exact.default_alpha_bits(16))
    Zm, Ze = tr["Z"]
    for c, (Nm, Ne) in enumerate(tr["N"]):
        ratio = Fraction(Nm) * Fraction(2) ** Ne / (Fraction(Zm) * Fraction(2) ** Ze)
        got = Fraction(float(bf2f(tr["out"][c])))
        for nb in (int(tr["out"][c]) + 1, int(tr["out"][c]) - 1):
            if nb & 0x7FFF == 0x7F80 or nb < 0:
                continue
            assert abs(got - ratio) <= abs(Fraction(float(bf2f(nb))) - ratio)


@pytest.mark.parametrize("seed", range(2))
def test_accuracy_against_float64(seed):
    rng = np.random.default_rng(seed)
    d, n = 64, 96
    q, k, v = bf16(rng, d), bf16(rng, (n, d)), bf16(rng, (n, d))
    qf, kf, vf = (bf2f(x).astype(np.float64) for x in (q, k, v))
    s = kf @ qf * f32(A64)
    p = np.exp2(s - s.max())
    ref = (p @ vf) / p.sum()
    out32 = exact.attention_row(q, k, v, A64, "fp32").view(np.float32).astype(np.float64)
    assert np.max(np.abs(out32 - ref)) <= np.abs(vf).max() * 2.0 ** -18


def test_pv_fully_lost_channel_kat():
    """docs/DESIGN.md:997-998 (reference): channel 0 = 1 and channel 1 = 2^-40 on every key gives
    channel 1 = bf16 0x2b80."""
    rng = np.random.default_rng(3)
    n, d = 50, 64
    q, k = bf16(rng, d), bf16(rng, (n, d))
    v = np.zeros((n, 4), np.uint16)
    v[:, 0] = 0x3F80
    v[:, 1] = 0x2B80  # 2^-40
    assert int(exact.attention_row(q, k, v, A64)[1]) == 0x2B80
    res, _ = oracle.attention_csr(q.reshape(1, -1), k, v, A64)
    assert int(res[0, 1]) == 0x2B80 and int(res[0, 0]) == 0x3F80


# ---------------------------------------------------------------------------------------------
# the C oracle against the Python definition, the reference build and the published hashes
# ---------------------------------------------------------------------------------------------

@given(seed=st.integers(0, 2**32 - 1), kind=st.sampled_from(KINDS), vkind=st.sampled_from(["normal", "wide", "dupes"]),
       n=st.integers(1, 120), splits=st.integers(1, 7), tile=st.sampled_from([1, 7, 64]),
       acc=st.sampled_from([64, 128]), out=st.sampled_from(["bf16", "fp32"]))
def test_c_oracle_certified_rows_equal_definition(seed, kind, vkind, n, splits, tile, acc, out):
    rng = np.random.default_rng(seed)
    d, dv = 32, 16
    Q, K, V = bf16(rng, (2, d), kind), bf16(rng, (n, d), kind), bf16(rng, (n, dv), vkind)
    res, flags, _ = oracle.raw_csr(Q, K, V, A32, out=out, acc_bits=acc, tile=tile, splits=splits, order_seed=seed)
    for r in range(2):
        if flags[r] == 0:
            assert np.array_equal(res[r], exact.attention_row(Q[r], K, V, A32, out))


def test_schedule_invariance_many_schedules():
    rng = np.random.default_rng(11)
    d, dv, n = 128, 64, 700
    Q, K, V = bf16(rng, (6, d), "outlier"), bf16(rng, (n, d), "outlier"), bf16(rng, (n, dv))
    base, flags, _ = oracle.raw_csr(Q, K, V, A128)
    assert not flags.any()
    for splits in (2, 3, 7, 16, 64):
        for tile in (1, 5, 64, 256):
            for acc in (64, 128):
                got, fl, _ = oracle.raw_csr(Q, K, V, A128, acc_bits=acc, tile=tile, splits=splits,
                                            order_seed=splits * 1000 + tile)
                assert not fl.any() and np.array_equal(got, base)
    for r in range(2):
        assert np.array_equal(base[r], exact.attention_row(Q[r], K, V, A128))


def test_tree_mask_equals_sequential_decode():
    rng = np.random.default_rng(5)
    d, dv, P, T = 64, 32, 300, 15
    parent = [-1] + [int(rng.integers(0, i)) for i in range(1, T)]
    Kp, Vp = bf16(rng, (P, d)), bf16(rng, (P, dv))
    Kt, Vt, Qt = bf16(rng, (T, d)), bf16(rng, (T, dv)), bf16(rng, (T, d))
    K, V = np.concatenate([Kp, Kt]), np.concatenate([Vp, Vt])
    rows = []
    for i in range(T):
        path, x = [], i
        while x != -1:
            path.append(P + x)
            x = parent[x]
        rows.append(np.concatenate([np.arange(P), np.array(path)]))
    row_ptr = np.concatenate([[0], np.cumsum([len(r) for r in rows])]).astype(np.int64)
    tree, flags = oracle.attention_csr(Qt, K, V, A64, row_ptr, np.concatenate(rows), splits=4)
    for i in range(T):
        seq_idx = np.sort(rows[i])
        seq, _ = oracle.attention_csr(Qt[i:i + 1], K[seq_idx], V[seq_idx], A64, splits=1, tile=128)
        assert np.array_equal(tree[i], seq[0])
        assert np.array_equal(tree[i], exact.attention_row(Qt[i], K[seq_idx], V[seq_idx], A64))


@pytest.mark.skipif(not oracle.ref_available(), reason="reference checkout not built into oracle/_ref")
@pytest.mark.parametrize("kind", KINDS)
def test_c_oracle_agrees_with_reference_build(kind):
    rng = np.random.default_rng(31)
    d, dv, n = 64, 32, 400
    Q, K, V = bf16(rng, (8, d), kind), bf16(rng, (n, d), kind), bf16(rng, (n, dv), "normal")
    for splits, tile in ((1, 64), (5, 16)):
        mine, f1, _ = oracle.raw_csr(Q, K, V, A64, splits=splits, tile=tile)
        ref, f2, _ = oracle.raw_csr(Q, K, V, A64, splits=splits, tile=tile, reference=True)
        both = (f1 == 0) & (f2 == 0)
        assert np.array_equal(mine[both], ref[both])
        # whatever the reference certifies, the oracle reproduces exactly
        full, _ = oracle.attention_csr(Q, K, V, A64, splits=splits, tile=tile)
        assert np.array_equal(full[f2 == 0], ref[f2 == 0])


def test_fixture_sha256_via_oracle():
    z = np.load(os.path.join(GOLD, "qwen3_0.6b_heads.npz"))
    exp = json.load(open(os.path.join(GOLD, "expected_sha256.json")))
    for key, info in exp["heads"].items():
        q, k, v = z[f"q_{key}"], z[f"k_{key}"], z[f"v_{key}"]
        ab = int(np.asarray(z[f"alpha_{key}"], dtype=np.float32).view(np.uint32))
        rp, ki = oracle.csr_from_kv_len(np.arange(1, q.shape[0] + 1))
        out, flags = oracle.attention_csr(q, k, v, ab, rp, ki, splits=8, tile=64)
        assert hashlib.sha256(out.tobytes()).hexdigest() == info["sha256"], key
        if key == "0_0":  # spot rows against the Python definition
            for pos in (0, 1, 17, 300, 2047):
                assert np.array_equal(out[pos], exact.attention_row(q[pos], k[:pos + 1], v[:pos + 1], ab))


def test_planted_mistake_is_caught():
    """A wrong exponent in one weight (the kind of slip the windows could hide) changes the bits:
    the Python definition with a perturbed weight disagrees with the C oracle."""
    rng = np.random.default_rng(8)
    q, k, v = bf16(rng, 32), bf16(rng, (20, 32)), bf16(rng, (20, 8))
    tr = exact.trace_row(q, k, v, A32)
    good = tr["out"]
    res, _ = oracle.attention_csr(q.reshape(1, -1), k, v, A32)
    assert np.array_equal(res[0], good)
    w = list(tr["w"])
    w[3] = (w[3][0], w[3][1] + 1)  # planted: one weight doubled
    wmin = min(e for _, e in w)
    Z = sum(m << (e - wmin) for m, e in w)
    vd = [[exact.decode_bf16(x) for x in row] for row in v.tolist()]
    differs = False
    for c in range(8):
        terms = [(w[j][0] * vd[j][c][0], w[j][1] + vd[j][c][1]) for j in range(20) if vd[j][c][0]]
        base = min(e for _, e in terms)
        Nc = sum(m << (e - base) for m, e in terms)
        sh = base - wmin
        m, e = exact.round_rational(*((Nc << sh, Z) if sh >= 0 else (Nc, Z << -sh)), exact.BF16)
        differs |= (0 if m == 0 else exact.encode_bf16(m, e)) != int(good[c])
    assert differs
