"""The library's exact quotient rounding (exactattention_amd/csrc/ea_quotient.h: rn_quotient,
cmp_quotient, certify_quotient, fmt_bits), the final rounding of the device tier 2, built for the
host from the same header and checked against exact rationals on the CPU.

certify_quotient must decide exactly what the definition asks (SPEC: both ends of the interval
of N / Z round to one pattern, zeros canonical, no overflow): it rounds one end and tests the
other against that result's rounding boundary, so it is compared with the oracle's RN of both
ends (oracle/exact.py round_rational) on random intervals and on intervals whose ends sit exactly
on midpoints (ties to even either way), on the quarter-quantum midpoint at the bottom of a
binade, at half the smallest subnormal, across zero and at the overflow threshold."""

import ctypes
import os
import subprocess
import tempfile
from fractions import Fraction

import numpy as np
import pytest

from oracle import exact

HERE = os.path.dirname(os.path.abspath(__file__))
FMT = {0: (8, -133, 127), 1: (24, -149, 127)}
M64 = (1 << 64) - 1


@pytest.fixture(scope="module")
def lib():
    out = os.path.join(tempfile.mkdtemp(prefix="ea_quot_"), "libquot.so")
    src = os.path.join(HERE, "native", "quotient_harness.cpp")
    subprocess.run(["g++", "-O2", "-std=c++17", "-shared", "-fPIC", "-o", out, src], check=True)
    L = ctypes.CDLL(out)
    L.h_rn_quotient.argtypes = [ctypes.c_uint64] * 4 + [ctypes.c_int64, ctypes.c_int,
                                                        ctypes.POINTER(ctypes.c_uint32), ctypes.POINTER(ctypes.c_int32)]
    L.h_certify_quotient.argtypes = [ctypes.POINTER(ctypes.c_int64), ctypes.c_int, ctypes.POINTER(ctypes.c_uint32)]
    L.h_fmt_bits.argtypes = [ctypes.c_uint32, ctypes.c_int, ctypes.c_int, ctypes.c_int]
    L.h_fmt_bits.restype = ctypes.c_uint32
    return L


def _rn(x: Fraction, fp32: int):
    """Oracle RN of a rational: (bits, overflow)."""
    try:
        m, e = exact.round_rational(x.numerator, x.denominator, FMT[fp32])
    except exact.DomainError:
        return None, True
    enc = exact.encode_fp32 if fp32 else exact.encode_bf16
    return (enc(m, e) if m else 0), False


def _want(Nlo, Nhi, Zlo, Zhi, sh, fp32):
    scale = Fraction(2) ** sh
    ends = [Fraction(n, z) * scale for n in (Nlo, Nhi) for z in (Zlo, Zhi)]
    lo, hi = min(ends), max(ends)
    bl, ol = _rn(lo, fp32)
    bh, oh = _rn(hi, fp32)
    if ol or oh or bl != bh:
        return False, None
    return True, bl


def _words(x: int):
    return [(x >> 64) if x >= 0 else -((-x - 1 >> 64) + 1), x & M64]


def _certify(lib, Nlo, Nhi, Zlo, Zhi, sh, fp32):
    v = (ctypes.c_int64 * 9)()
    vals = _words(Nlo) + _words(Nhi) + _words(Zlo) + _words(Zhi) + [sh]
    for i, x in enumerate(vals):
        v[i] = ctypes.c_int64(x if x < (1 << 63) else x - (1 << 64)).value
    bits = ctypes.c_uint32(0)
    ok = lib.h_certify_quotient(v, fp32, ctypes.byref(bits))
    return bool(ok), int(bits.value)


def _check(lib, Nlo, Nhi, Zlo, Zhi, sh, fp32):
    ok, bits = _certify(lib, Nlo, Nhi, Zlo, Zhi, sh, fp32)
    wok, wbits = _want(Nlo, Nhi, Zlo, Zhi, sh, fp32)
    assert ok == wok, (Nlo, Nhi, Zlo, Zhi, sh, fp32)
    if ok:
        assert bits == wbits, (Nlo, Nhi, Zlo, Zhi, sh, fp32, hex(bits), hex(wbits))
    return ok


def test_rn_quotient_matches_rationals(lib):
    rng = np.random.default_rng(31)
    Q, qe = ctypes.c_uint32(0), ctypes.c_int32(0)
    for i in range(6000):
        a = int(rng.integers(1, 1 << 62)) << int(rng.integers(0, 65))
        b = int(rng.integers(1, 1 << 62)) << int(rng.integers(0, 65))
        if i % 7 == 0:
            a = b * int(rng.integers(1, 1 << 20)) + int(rng.integers(-2, 3)) * (b >> 1)
            a = max(a, 1)
        a, b = a & ((1 << 127) - 1) or 1, b & ((1 << 127) - 1) or 1
        sh = int(rng.integers(-300, 250))
        for fp32 in (0, 1):
            st = lib.h_rn_quotient(a >> 64, a & M64, b >> 64, b & M64, sh, fp32, ctypes.byref(Q), ctypes.byref(qe))
            bits, ov = _rn(Fraction(a, b) * Fraction(2) ** sh, fp32)
            assert st == (1 if ov else 0), (a, b, sh, fp32)
            if not ov:
                assert lib.h_fmt_bits(Q.value, qe.value, 0, fp32) == bits, (a, b, sh, fp32)
    # far outside the range: zero and overflow without any shift by sh
    for sh, want in ((-(1 << 40), 0), (-5000, 0), (5000, 1), (1 << 40, 1)):
        assert lib.h_rn_quotient(0, 3, 0, 1, sh, 1, ctypes.byref(Q), ctypes.byref(qe)) == want


def test_fmt_bits_known_patterns(lib):
    assert lib.h_fmt_bits(0, -149, 1, 1) == 0                 # zero is +0
    assert lib.h_fmt_bits(1, -149, 0, 1) == 1                 # smallest fp32 subnormal
    assert lib.h_fmt_bits(1 << 23, -23, 0, 1) == 0x3F800000   # 1.0
    assert lib.h_fmt_bits(1 << 23, -23, 1, 1) == 0xBF800000
    assert lib.h_fmt_bits((1 << 24) - 1, 104, 0, 1) == 0x7F7FFFFF
    assert lib.h_fmt_bits(1 << 7, -7, 0, 0) == 0x3F80         # bf16 1.0
    assert lib.h_fmt_bits(1, -133, 1, 0) == 0x8001            # -smallest bf16 subnormal
    assert lib.h_fmt_bits(255, 120, 0, 0) == 0x7F7F           # bf16 max


def test_certify_random_intervals(lib):
    rng = np.random.default_rng(32)
    decided = 0
    for i in range(5000):
        zb = int(rng.integers(24, 126))
        Zlo = int(rng.integers(1 << (zb - 1), 1 << zb, dtype=np.uint64) if zb <= 64 else
                  (int(rng.integers(1 << 40, 1 << 62)) << (zb - 62)))
        Zhi = Zlo + int(rng.integers(0, 1 << int(rng.integers(0, 40))))
        nb = int(rng.integers(1, 126))
        N = int(rng.integers(1, 1 << min(nb, 62))) << max(0, nb - 62)
        N = -N if rng.random() < 0.4 else N
        width = int(rng.integers(0, 1 << int(rng.integers(0, 50))))
        Nlo, Nhi = (N - width, N) if rng.random() < 0.5 else (N, N + width)
        if rng.random() < 0.1:
            Nlo, Nhi = -abs(width) - 1, abs(width) + 1   # across zero
        Nlo = max(Nlo, -(1 << 126))
        Nhi = min(Nhi, (1 << 126))
        sh = int(rng.integers(-260, 140)) - (nb - zb)
        for fp32 in (0, 1):
            decided += _check(lib, Nlo, Nhi, Zlo, min(Zhi, (1 << 126)), sh, fp32)
    assert decided > 2000, decided


def _midpoint_cases(fp32: int, seed: int, count: int):
    """Intervals whose ends sit exactly on the midpoint above or below a result (or one unit
    past it), for even and odd significands, positive and negative, normal and subnormal, the
    quarter-quantum midpoint below a binade's first significand, and the largest finite value."""
    p, qmin, _ = FMT[fp32]
    rng = np.random.default_rng(seed)
    for i in range(count):
        Z = int(rng.integers(1 << 20, 1 << 60)) << int(rng.integers(0, 60))
        kind = i % 4
        if kind == 0:
            Q, qe = int(rng.integers(1 << (p - 1), 1 << p)), int(rng.integers(qmin, 100))
        elif kind == 1:
            Q, qe = 1 << (p - 1), int(rng.integers(qmin + 1, 100))   # bottom of a binade
        elif kind == 2:
            Q, qe = int(rng.integers(0, 1 << (p - 1))), qmin          # subnormal or zero
        else:
            Q, qe = (1 << p) - 1, 127 - (p - 1)                       # the largest finite value
        # midpoints as multiples of 2^(qe - 2): upper 4Q + 2, lower 4Q - 2 (4Q - 1 at a binade's bottom)
        bottom = Q == 1 << (p - 1) and qe > qmin
        for mult in (4 * Q + 2, (4 * Q - 1) if bottom else (4 * Q - 2), 4 * Q):
            if mult <= 0:
                continue
            N = mult * Z
            for sgn in (1, -1):
                for a, b in ((N, N), (N - 1, N), (N, N + 1), (N - 1, N + 1), (N - Z, N), (N, N + Z)):
                    lo, hi = (a, b) if sgn > 0 else (-b, -a)
                    if abs(lo) >= 1 << 126 or abs(hi) >= 1 << 126:
                        continue
                    for zl, zh in ((Z, Z), (Z - 1, Z), (Z, Z + 1)):
                        yield lo, hi, zl, zh, qe - 2


@pytest.mark.parametrize("fp32", [0, 1])
def test_certify_at_rounding_midpoints(lib, fp32):
    cases = 0
    for c in _midpoint_cases(fp32, 33 + fp32, 600):
        _check(lib, *c, fp32)
        cases += 1
    assert cases > 10000


@pytest.mark.gpu
@pytest.mark.parametrize("fp32", [0, 1])
def test_device_certify_quotient_kat(gpu, fp32):
    """The device build of certify_quotient (ea_hip_kat_certify_quotient) decides the midpoint
    cases exactly as the definition does."""
    import torch
    from exactattention_amd import hip
    cases = list(_midpoint_cases(fp32, 35 + fp32, 200))
    rows = []
    for lo, hi, zl, zh, sh in cases:
        rows.append(_words(lo) + _words(hi) + _words(zl) + _words(zh) + [sh])
    arr = np.array([[x if x < (1 << 63) else x - (1 << 64) for x in r] for r in rows], dtype=np.int64)
    dev = torch.from_numpy(arr).cuda()
    bits = torch.zeros(len(cases), dtype=torch.int32, device="cuda")
    ok = torch.zeros(len(cases), dtype=torch.int32, device="cuda")
    rc = hip.load().ea_hip_kat_certify_quotient(len(cases), dev.data_ptr(), fp32, bits.data_ptr(), ok.data_ptr(),
                                                torch.cuda.current_stream().cuda_stream)
    assert rc == 0
    torch.cuda.synchronize()
    gb, go = bits.cpu().numpy().view(np.uint32), ok.cpu().numpy()
    for i, c in enumerate(cases):
        wok, wbits = _want(*c, fp32)
        assert bool(go[i]) == wok, c
        if wok:
            assert int(gb[i]) == wbits, c


@pytest.mark.parametrize("fp32", [0, 1])
def test_certify_around_zero_and_the_smallest_subnormal(lib, fp32):
    p, qmin, _ = FMT[fp32]
    Z = 3 << 70
    half = Fraction(2) ** (qmin - 1)
    for num in (Z, Z - 1, Z + 1, 3 * Z, 3 * Z - 1, 3 * Z + 1):   # about 2^(qmin-1) and 3 * 2^(qmin-1)
        sh = qmin - 1
        for lo, hi in ((num, num), (-num, num), (-num, 0), (0, num), (-num, -num), (-1, 1), (0, 0)):
            _check(lib, lo, hi, Z, Z, sh, fp32)
            _check(lib, lo, hi, Z - 5, Z + 5, sh, fp32)
    assert half > 0
