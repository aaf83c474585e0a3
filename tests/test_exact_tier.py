"""The library's host exact tier (ea_exact_row, ea_round_ratio, trace_row) against the oracle, on
the CPU: these entry points run host code only, so they are checked here row by row, including
the adversarial rows the device tiers cannot certify (cancellation in a numerator, weights far
apart, the fully-lost V channel). The argument checks of the reference-compatible drop-in
ea_attention_hip are also exercised here: each bad call returns before any device work."""

import ctypes

import numpy as np
import pytest

from exactattention_amd.formats import ExactAttentionDomainError, float_to_bf16_bits
from gen import KINDS, bf16


def _hip():
    from exactattention_amd import hip
    if not hip.available():
        pytest.skip("libexactattn_hip.so not built (run __graft_entry__.build())")
    hip.load()
    return hip


def _oracle_row(q, k, v, ab, out="bf16"):
    from oracle import exact
    return exact.attention_row(q, k, v, ab, out)


@pytest.mark.parametrize("kind", KINDS)
@pytest.mark.parametrize("out", ["bf16", "fp32"])
def test_exact_row_matches_oracle(kind, out):
    hip = _hip()
    from oracle import exact
    rng = np.random.default_rng(abs(hash((kind, out))) % (1 << 32))
    for d, dv in ((64, 32), (128, 128), (8, 2)):
        ab = exact.default_alpha_bits(d)
        for vkind in ("normal", "wide", "dupes", "subnormal"):
            n = int(rng.integers(0, 48))
            q, k, v = bf16(rng, (d,), kind), bf16(rng, (n, d), kind), bf16(rng, (n, dv), vkind)
            got, tb, wm, we = hip.exact_row(q, k, v, ab, out, trace=True)
            tr = exact.trace_row(q, k, v, ab, out)
            assert np.array_equal(got, tr["out"]), (d, vkind, n)
            assert [(int(a), int(b)) for a, b in zip(wm, we)] == tr["w"]
            assert [int(x) for x in tb] == [exact.encode_fp32(*t) if t[0] else 0 for t in tr["t"]]


def _rows_with(d=8):
    q = np.zeros(d, np.uint16)
    q[0] = 0x3F80  # 1.0
    return q


def test_exact_row_cancellation_rows():
    """Two equal weights carry v = +1 and -1 and a third key is 2^-k lighter: the numerator is the
    light key's term alone, far below the window of any fixed-width tier."""
    hip = _hip()
    from oracle import exact
    q = _rows_with()
    for light in (-100.0, -30.0, -5.0, 0.5):
        k = np.zeros((3, 8), np.uint16)
        k[0, 0] = k[1, 0] = 0x3F80
        k[2, 0] = float_to_bf16_bits(np.array([light]))[0]
        v = np.zeros((3, 2), np.uint16)
        v[:, 0] = [0x3F80, 0xBF80, 0x3F80]
        v[:, 1] = 0x3F80
        for ab in (exact.default_alpha_bits(8), 0x3F800000, 0x41200000):
            for out in ("bf16", "fp32"):
                assert np.array_equal(hip.exact_row(q, k, v, ab, out), exact.attention_row(q, k, v, ab, out)), \
                    (light, hex(ab), out)


def test_exact_row_fully_lost_v_channel():
    """V channel 1 is 2^-40 of channel 0 on every key (the reference's D24 case): output channel 1
    is 2^-40 exactly, bf16 0x2B80."""
    hip = _hip()
    from oracle import exact
    rng = np.random.default_rng(5)
    d, dv, n = 64, 32, 40
    q = float_to_bf16_bits(rng.standard_normal(d))
    k = float_to_bf16_bits(rng.standard_normal((n, d)))
    vv = rng.standard_normal((n, dv))
    vv[:, 0], vv[:, 1] = 1.0, 2.0 ** -40
    v = float_to_bf16_bits(vv)
    got = hip.exact_row(q, k, v, exact.default_alpha_bits(d))
    assert got[1] == 0x2B80 and got[0] == 0x3F80
    assert np.array_equal(got, exact.attention_row(q, k, v, exact.default_alpha_bits(d)))


def test_exact_row_closed_forms_and_errors():
    hip = _hip()
    from oracle import exact
    rng = np.random.default_rng(8)
    d, ab = 16, exact.default_alpha_bits(16)
    q = bf16(rng, (d,))
    # empty key set: +0 everywhere
    assert not hip.exact_row(q, np.zeros((0, d), np.uint16), np.zeros((0, 4), np.uint16), ab).any()
    # one key: v exactly; identical keys: RN of the mean of v
    k1, v1 = bf16(rng, (1, d)), bf16(rng, (1, 4))
    assert np.array_equal(hip.exact_row(q, k1, v1, ab), v1[0])
    kk = np.repeat(k1, 4, axis=0)
    vv = float_to_bf16_bits(np.array([[1.0], [2.0], [4.0], [8.0]]))
    assert hip.exact_row(q, kk, vv, ab)[0] == float_to_bf16_bits(np.array([3.75]))[0]
    # NaN in a key, inf in a value, fp32 logit overflow: domain errors
    bad = k1.copy()
    bad[0, 3] = 0x7FC0
    with pytest.raises(ExactAttentionDomainError):
        hip.exact_row(q, bad, v1, ab)
    badv = v1.copy()
    badv[0, 0] = 0xFF80
    with pytest.raises(ExactAttentionDomainError):
        hip.exact_row(q, k1, badv, ab)
    big = np.zeros(d, np.uint16)
    big[0] = 0x7F00  # 2^127
    with pytest.raises(ExactAttentionDomainError):
        hip.exact_row(big, big.reshape(1, d), v1, 0x3F800000)


def test_exact_row_huge_logits():
    """Logits of any fp32 size: integer t far beyond the int32 range (weights 2^(2^21) and
    beyond), negative alpha, and subnormal logits, against the oracle's Python integers."""
    hip = _hip()
    from oracle import exact
    rng = np.random.default_rng(9)
    for trial in range(30):
        n, d = int(rng.integers(1, 6)), 16
        q, k, v = bf16(rng, (d,), "wide"), bf16(rng, (n, d), "wide"), bf16(rng, (n, 4), "wide")
        ab = int(np.float32(rng.choice([1e-30, 1e-3, 0.127, -0.5, 3.0, 1e4, 1e12])).view(np.uint32))
        try:
            want = exact.attention_row(q, k, v, ab)
        except exact.DomainError:
            continue
        assert np.array_equal(hip.exact_row(q, k, v, ab), want), trial


def test_exact_row_logits_near_the_fp32_limit():
    """Logits t = RN32(alpha s) of 1.5 * 2^127, whose weight exponents t - 23 pass the 128-bit
    range: keys with one such logit have equal weights (N / Z is the exact mean of v, as the oracle
    computes with Python integers), and two distinct logits that large lie at least 2^76 apart,
    past the exponent-spread limit, so the row is refused as the reference refuses it."""
    hip = _hip()
    from oracle import exact
    rng = np.random.default_rng(11)
    q = np.zeros(8, np.uint16)
    q[0] = 0x5D80                        # 2^60
    k = np.zeros((3, 8), np.uint16)
    k[:, 0] = 0x5D80                     # s = 2^120 for every key
    v = bf16(rng, (3, 5))
    ab = int(np.float32(192.0).view(np.uint32))  # t = 1.5 * 2^127
    for out in ("bf16", "fp32"):
        want = exact.attention_row(q, k, v, ab, out)
        assert np.array_equal(hip.exact_row(q, k, v, ab, out), want), out
    k2 = k.copy()
    k2[1, 0] = 0x5D81                    # a second, larger logit
    with pytest.raises(ExactAttentionDomainError):
        hip.exact_row(q, k2, v, ab)
    with pytest.raises(exact.DomainError):
        exact.attention_row(q, k2, v, ab)
    # one such logit beside t = 0: 2^t overwhelms the other weight, but its exponent does not fit
    # 128 bits (a wrapped exponent would make it the lightest key and return the other key's v)
    k3 = k.copy()
    k3[1, 0] = 0
    with pytest.raises(ExactAttentionDomainError):
        hip.exact_row(q, k3, v, ab)
    with pytest.raises(exact.DomainError):
        exact.attention_row(q, k3, v, ab)


def test_exact_row_spread_beyond_the_reference_limit():
    """Weights 2^(2^21) apart. When the rounding is decided without the lightest key (its term
    cannot move the quotient off +0) the tier returns the bits; where the reference's exact sums
    would need the whole 2^21-bit spread it refuses with a domain error, as the reference does
    (src/exactattn/reference.py:124-125)."""
    hip = _hip()
    q = _rows_with()
    k = np.zeros((3, 8), np.uint16)
    k[0, 0] = k[1, 0] = 0x4A00  # 2^21: t = 2^21 at alpha = 1
    v = np.zeros((3, 2), np.uint16)
    v[:, 0] = [0x3F80, 0xBF80, 0x3F80]
    v[:, 1] = 0x3F80
    got = hip.exact_row(q, k, v, 0x3F800000)
    assert got[0] == 0 and got[1] == 0x3F80  # N_0 = 1 against Z ~ 2^(2^21 + 1): +0
    # the numerator's only term is the light key's, and the quotient is about 2^-(2^21): +0 too;
    # with v channel 0 of the heavy keys zero, N_0 / Z is that tiny value exactly
    v2 = v.copy()
    v2[:2, 0] = 0
    assert hip.exact_row(q, k, v2, 0x3F800000)[0] == 0


def test_round_ratio_matches_oracle():
    """ea_round_ratio, the reference's test hook with its signature (float result, int* overflow),
    against the oracle on random 128-bit cases, ties, subnormals and overflow."""
    hip = _hip()
    lib = hip.load()
    from oracle import oracle
    rng = np.random.default_rng(12)
    cases = []
    for _ in range(3000):
        ab, bb = int(rng.integers(1, 127)), int(rng.integers(1, 127))
        a = int(rng.integers(1, 1 << min(ab, 62))) << max(0, ab - 62)
        b = int(rng.integers(1, 1 << min(bb, 62))) << max(0, bb - 62)
        cases.append((a | int(rng.integers(0, 2)), b, int(rng.integers(-320, 220)), int(rng.integers(0, 2))))
    cases += [((1 << 24) + 1, 1, 0, 0), ((1 << 24) + 3, 1, 0, 0), (3, 2, -150, 0), (1, 1, 128, 0), (1, 3, -140, 1)]
    M = (1 << 64) - 1
    for fp32 in (0, 1):
        for a, b, e, neg in cases:
            ov = ctypes.c_int(0)
            f = lib.ea_round_ratio(a >> 64, a & M, b >> 64, b & M, e, neg, fp32, ctypes.byref(ov))
            wb, wo = oracle.round_ratio_bits(a, b, e, bool(neg), bool(fp32))
            assert bool(ov.value) == wo, (a, b, e, neg, fp32)
            if not wo:
                got = int(np.float32(f).view(np.uint32))
                want = wb if fp32 else wb << 16
                assert got == want, (a, b, e, neg, fp32)


def test_trace_row_matches_oracle():
    import exactattention_amd as ea
    _hip()
    from oracle import exact
    rng = np.random.default_rng(14)
    for kind in ("normal", "wide"):
        q, k, v = bf16(rng, (64,), kind), bf16(rng, (20, 64), kind), bf16(rng, (20, 16), "wide")
        tr = ea.trace_row(q, k, v, ea.default_alpha(64))
        o = exact.trace_row(q, k, v, exact.default_alpha_bits(64))
        assert tr.s == o["s"] and tr.w == o["w"] and tr.Z == o["Z"] and tr.N == o["N"]
        assert np.array_equal(tr.out, o["out"])
        assert [int(np.float32(t).view(np.uint32)) for t in tr.t] == \
            [exact.encode_fp32(*t) if t[0] else 0 for t in o["t"]]


def test_drop_in_validates_like_the_reference():
    """ea_attention_hip bound with the reference's argtypes (src/exactattn/cpu.py:35-38) returns
    the reference's codes before any device work: -1 for tile <= 0, splits <= 0, a head size out
    of range or a key index outside [0, nkeys); -2 for acc_bits other than 64 and 128; -3 for a
    non-finite alpha."""
    hip = _hip()
    lib = hip.load()
    q = np.zeros((2, 8), np.uint16)
    k = np.zeros((4, 8), np.uint16)
    rp = np.array([0, 2, 4], np.int64)
    ki = np.array([0, 1, 2, 3], np.int64)
    res = np.zeros((2, 8), np.uint16)
    fl = np.zeros(2, np.uint8)
    st = np.zeros(3, np.int64)

    def call(d=8, dv=8, alpha=0.125, tile=64, splits=2, acc=64, key_idx=ki):
        return lib.ea_attention_hip(q.ctypes.data, 2, d, k.ctypes.data, k.ctypes.data, 4, dv, ctypes.c_float(alpha),
                                    rp.ctypes.data, key_idx.ctypes.data, 0, acc, tile, splits, 0, 1, res.ctypes.data,
                                    fl.ctypes.data, st.ctypes.data)

    assert call(tile=0) == -1
    assert call(splits=0) == -1
    assert call(d=0) == -1 and call(dv=0) == -1 and call(d=256) == -1
    assert call(acc=32) == -2 and call(acc=96) == -2
    assert call(alpha=float("nan")) == -3 and call(alpha=float("inf")) == -3
    assert call(key_idx=np.array([0, 1, 2, 4], np.int64)) == -1
    assert call(key_idx=np.array([0, -1, 2, 3], np.int64)) == -1
    assert not st.any()


@pytest.mark.parametrize("gap_log2", [33, 38, 39])
@pytest.mark.parametrize("out", ["bf16", "fp32"])
def test_exact_row_weights_2_to_the_2_to_the_gap_apart(gap_log2, out):
    """q = e_0, key 0 with k_0 = 2^gap, key 1 with k = 0, alpha = 1: the weights are 2^(2^gap)
    and 1. N_c / Z is v_0c within a relative 2^-(2^gap), so it rounds to v_0c, and channels where
    v_0c = 0 hold v_1c 2^-(2^gap), which rounds to +0. The tier decides both without building
    operands of 2^gap bits (it once asked for them and aborted with bad_alloc). trace_row refuses
    the row, as the reference does for any spread past 2^20."""
    hip = _hip()
    import exactattention_amd as ea
    rng = np.random.default_rng(gap_log2)
    d, dv = 16, 8
    q = np.zeros(d, np.uint16)
    q[0] = 0x3F80                                    # 1.0
    k = np.zeros((2, d), np.uint16)
    k[0, 0] = (127 + gap_log2) << 7                  # 2^gap
    v = bf16(rng, (2, dv))
    v[v == 0] = 0x3F80
    v[v == 0x8000] = 0x3F80
    v[0, 3] = 0                                      # a channel the heavy key does not reach
    v[0, 5] = 0x8000                                 # -0 from the heavy key: the result is +0
    got = hip.exact_row(q, k, v, 0x3F800000, out)
    want = v[0].astype(np.uint32) << 16 if out == "fp32" else v[0].copy()
    want[3] = want[5] = 0
    assert np.array_equal(got, want)
    with pytest.raises(ExactAttentionDomainError):
        ea.trace_row(q, k, v, 1.0, out)


def test_round_ratio_far_outside_the_range():
    """ea_round_ratio with exponents far below and above every format: +0 and an overflow flag,
    decided without shifting operands by E."""
    hip = _hip()
    lib = hip.load()
    lib.ea_round_ratio.restype = ctypes.c_float
    lib.ea_round_ratio.argtypes = [ctypes.c_uint64] * 4 + [ctypes.c_int, ctypes.c_int, ctypes.c_int,
                                                           ctypes.POINTER(ctypes.c_int)]
    ov = ctypes.c_int(-1)
    for E in (-(1 << 30), -(1 << 31), -400, -300):
        r = lib.ea_round_ratio(0, 3, 0, 1, E, 0, 1, ctypes.byref(ov))
        assert r == 0.0 and ov.value == 0, E
    for E in ((1 << 30), (1 << 31) - 1, 5000, 200):
        r = lib.ea_round_ratio(0, 3, 0, 1, E, 0, 1, ctypes.byref(ov))
        assert ov.value == 1, E
    # near the boundaries the exact rounding still runs: 3 * 2^-151 rounds to 2^-149 (fp32), and
    # 2^-151 is below half the smallest subnormal, so +0
    r = lib.ea_round_ratio(0, 3, 0, 1, -151, 0, 1, ctypes.byref(ov))
    assert np.float32(r).view(np.uint32) == 1 and ov.value == 0
    r = lib.ea_round_ratio(0, 1, 0, 1, -151, 0, 1, ctypes.byref(ov))
    assert r == 0.0 and ov.value == 0


def test_trace_row_of_equal_logits_past_2_to_the_62():
    """Equal logits t = 1.5 * 2^127 (weights 2^t, exponents past the library's +-2^62 trace
    range): trace_row's weights and Z carry the exact exponent t - 23, as the reference's
    RowTrace does, and the output is the mean of v."""
    hip = _hip()
    import exactattention_amd as ea
    from oracle import exact
    rng = np.random.default_rng(13)
    q = np.zeros(8, np.uint16)
    q[0] = 0x5D80                        # 2^60
    k = np.zeros((3, 8), np.uint16)
    k[:, 0] = 0x5D80                     # s = 2^120 for every key
    v = bf16(rng, (3, 5))
    tr = ea.trace_row(q, k, v, 192.0)    # t = 1.5 * 2^127
    t = 1.5 * 2.0 ** 127
    assert tr.t == [t] * 3
    assert tr.w == [(1 << 23, int(t) - 23)] * 3
    assert tr.Z == (3 << 23, int(t) - 23)
    assert np.array_equal(tr.out, exact.attention_row(q, k, v, int(np.float32(192.0).view(np.uint32))))
