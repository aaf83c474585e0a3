"""CPU oracle, part 1: the ExactAttention definition restated with Python integers.

TEST INFRASTRUCTURE ONLY. Nothing in the product package may import this module; only
`tests/`, `__graft_entry__.smoke()` and the `cpu_baseline` leg of `bench.py` use it, and only
as the checker.

Every value is an exact dyadic (m, e) = m * 2**e or an exact rational. No hardware floating
point is used for anything that decides a result bit. Each function cites the reference
file:line whose behaviour it restates (paths relative to the reference checkout).

The weight oracle does not use mpmath: it encloses 2**f with integer Taylor series and an
integer enclosure of ln 2, doubling the working precision until the enclosure decides the
rounding (Ziv's strategy; the reference does the same with mpmath intervals,
src/exactattn/exp2.py:48-78).
"""

from __future__ import annotations

from functools import lru_cache

import numpy as np


class DomainError(ValueError):
    """Input outside the spec's domain (docs/SPEC.md:57-65): NaN/inf, or an fp32 overflow of
    a logit. Mirrors src/exactattn/formats.py:16-17."""


# (p, qmin, emax) per docs/SPEC.md:12-21 and src/exactattn/formats.py:34-36.
BF16 = (8, -133, 127)
FP32 = (24, -149, 127)
FP24 = (24, None, None)

# src/exactattn/reference.py:30: the reference refuses exponent spreads past 2**20.
MAX_EXPONENT_SPREAD = 1 << 20


# ---------------------------------------------------------------------------
# Rounding (src/exactattn/formats.py:39-100)
# ---------------------------------------------------------------------------

def round_rational(num: int, den: int, fmt) -> tuple[int, int]:
    """RN-even of num/den into fmt=(p, qmin, emax). Returns (m, e), |m| < 2**p; zero is (0, 0).

    Follows src/exactattn/formats.py:39-85: floor(log2), quantum exponent with the subnormal
    clamp, round half to even, carry into the next binade, and overflow as a DomainError."""
    p, qmin, emax = fmt
    if den == 0:
        raise ZeroDivisionError("round_rational: zero denominator")
    if den < 0:
        num, den = -num, -den
    if num == 0:
        return (0, 0)
    sign = -1 if num < 0 else 1
    a = -num if num < 0 else num
    k = a.bit_length() - den.bit_length()
    if k >= 0:
        if a < (den << k):
            k -= 1
    elif (a << -k) < den:
        k -= 1
    qe = k - (p - 1)
    if qmin is not None and qe < qmin:
        qe = qmin
    if qe >= 0:
        n, d = a, den << qe
    else:
        n, d = a << -qe, den
    q, r = divmod(n, d)
    if 2 * r > d or (2 * r == d and (q & 1)):
        q += 1
    if q == (1 << p):
        q >>= 1
        qe += 1
    if emax is not None:
        # largest finite: (2**p - 1) * 2**(emax - p + 1)
        if qe + q.bit_length() - 1 > emax:
            raise DomainError("overflow")
    return (sign * q, qe)


def round_dyadic(m: int, e: int, fmt) -> tuple[int, int]:
    """RN of the exact dyadic m * 2**e (src/exactattn/formats.py:88-92)."""
    if e >= 0:
        return round_rational(m << e, 1, fmt)
    return round_rational(m, 1 << -e, fmt)


# ---------------------------------------------------------------------------
# Bit patterns (src/exactattn/formats.py:107-153)
# ---------------------------------------------------------------------------

def decode_bf16(bits: int) -> tuple[int, int]:
    """bf16 bits -> (m, e) (src/exactattn/formats.py:107-117)."""
    bits = int(bits) & 0xFFFF
    sign = -1 if bits & 0x8000 else 1
    ex = (bits >> 7) & 0xFF
    fr = bits & 0x7F
    if ex == 0xFF:
        raise DomainError("bf16 NaN or infinity in input")
    if ex == 0:
        return (sign * fr, -133)
    return (sign * (fr | 0x80), ex - 134)


def decode_fp32_bits(bits: int) -> tuple[int, int]:
    """fp32 bits -> (m, e) (src/exactattn/formats.py:120-130)."""
    bits = int(bits) & 0xFFFFFFFF
    sign = -1 if bits & 0x80000000 else 1
    ex = (bits >> 23) & 0xFF
    fr = bits & 0x7FFFFF
    if ex == 0xFF:
        raise DomainError("fp32 NaN or infinity in input")
    if ex == 0:
        return (sign * fr, -149)
    return (sign * (fr | 0x800000), ex - 150)


def fp32_bits(x) -> int:
    return int(np.asarray(x, dtype=np.float32).view(np.uint32))


def _encode(m: int, e: int, p: int, qmin: int, ebits: int) -> int:
    """Bits of the representable value m * 2**e in a binary format with precision p, min
    quantum qmin and ebits exponent bits. Built from integers only."""
    if m == 0:
        return 0
    sign = 1 if m < 0 else 0
    a = -m if m < 0 else m
    # normalise to p bits where possible
    while a < (1 << (p - 1)) and e > qmin:
        a <<= 1
        e -= 1
    while a >= (1 << p):
        assert a & 1 == 0
        a >>= 1
        e += 1
    if a < (1 << (p - 1)):
        assert e == qmin
        field = 0
        frac = a
    else:
        field = e - qmin + 1
        frac = a - (1 << (p - 1))
    assert 0 < field < (1 << ebits) - 1 or field == 0
    return (sign << (p - 1 + ebits)) | (field << (p - 1)) | frac


def encode_bf16(m: int, e: int) -> int:
    return _encode(m, e, 8, -133, 8)


def encode_fp32(m: int, e: int) -> int:
    return _encode(m, e, 24, -149, 8)


# ---------------------------------------------------------------------------
# ln 2 and exp2 enclosures (own integer method; replaces the mpmath interval oracle of
# src/exactattn/exp2.py:48-78 and the constants of :137-152)
# ---------------------------------------------------------------------------

@lru_cache(maxsize=None)
def ln2_enclosure(W: int) -> tuple[int, int]:
    """(lo, hi) with lo <= ln(2) * 2**W <= hi, from ln 2 = 2 atanh(1/3) = sum 2/((2k+1) 3**(2k+1)).

    Each term is floored for lo and ceiled for hi; the tail after K terms is below
    2 * 2**W / 3**(2K+1) * 9/8, which hi adds (rounded up)."""
    lo = hi = 0
    k = 0
    scale = 1 << W
    while True:
        den = (2 * k + 1) * 3 ** (2 * k + 1)
        t_lo = (2 * scale) // den
        lo += t_lo
        hi += -((-2 * scale) // den)
        k += 1
        if t_lo == 0:
            break
    tail = -((-2 * scale * 9) // (8 * 3 ** (2 * k + 1))) + 1
    return lo, hi + tail


def _exp_enclosure(x_lo: int, x_hi: int, W: int) -> tuple[int, int]:
    """Enclose exp(x) * 2**W for x in [x_lo, x_hi] * 2**-W with 0 <= x_lo <= x_hi < 2**W.

    Lower end: Taylor terms of x_lo, each floored, truncated (all terms positive). Upper end:
    terms of x_hi ceiled, plus the tail bound 2 * next term (x < 1 makes the tail ratio < 1/2)."""
    one = 1 << W
    lo = 0
    t = one
    n = 0
    while t:
        lo += t
        n += 1
        t = (t * x_lo) // (n << W)
    hi = 0
    t = one
    n = 0
    while True:
        hi += t
        n += 1
        t = -((-t * x_hi) // (n << W))
        if t <= 1 and n > 3:
            hi += 2 * t + 2
            break
    return lo, hi


def exp2_rn(t_m: int, t_e: int, p: int = 24) -> tuple[int, int]:
    """RN_p(2**t) with unbounded exponent for the exact dyadic t = t_m * 2**t_e.

    Returns (M, E), 2**(p-1) <= M < 2**p. Same contract as src/exactattn/exp2.py:48-78: integer t
    is an exact power of two; otherwise 2**f (f = t - floor t) is irrational (docs/SPEC.md:69-80)
    so an enclosure that rounds the same at both ends decides the result."""
    if t_e >= 0:
        return (1 << (p - 1), (t_m << t_e) - (p - 1))
    k = -t_e
    n = t_m >> k                      # floor(t)
    a = t_m - (n << k)                # f = a / 2**k, 0 <= a < 2**k
    if a == 0:
        return (1 << (p - 1), n - (p - 1))
    W = 96
    while True:
        L_lo, L_hi = ln2_enclosure(W)
        x_lo = (a * L_lo) >> k
        x_hi = -((-a * L_hi) >> k)
        y_lo, y_hi = _exp_enclosure(x_lo, x_hi, W)
        # M = round(2**f * 2**(p-1)); value y * 2**-W * 2**(p-1)
        sh = W - (p - 1)
        q_lo = (y_lo + (1 << (sh - 1))) >> sh
        q_hi = (y_hi + (1 << (sh - 1))) >> sh
        if q_lo == q_hi:
            q, e = q_lo, n - (p - 1)
            if q == (1 << p):
                q >>= 1
                e += 1
            return (q, e)
        W *= 2
        if W > 1 << 16:
            raise RuntimeError("exp2 enclosure did not converge")


def default_alpha_bits(d: int) -> int:
    """fp32 bits of RN_fp32(log2(e) / sqrt(d)) = RN(1 / (ln 2 * sqrt(d)))
    (src/exactattn/reference.py:164-173), from integer enclosures of ln 2 and sqrt(d)."""
    import math
    W = 80
    while True:
        L_lo, L_hi = ln2_enclosure(W)
        s = math.isqrt(d << (2 * W))
        s_lo, s_hi = s, (s if s * s == d << (2 * W) else s + 1)
        one = 1 << (2 * W)
        lo = round_rational(one, L_hi * s_hi, FP32)
        hi = round_rational(one, L_lo * s_lo, FP32)
        if lo == hi:
            return encode_fp32(*lo)
        W *= 2


# ---------------------------------------------------------------------------
# The definition (src/exactattn/reference.py:47-161)
# ---------------------------------------------------------------------------

def exact_dot(q, k) -> tuple[int, int]:
    """Exact sum_i q_i k_i of decoded bf16 lists [(m, e)] (src/exactattn/reference.py:47-61)."""
    terms = [(qm * km, qe + ke) for (qm, qe), (km, ke) in zip(q, k) if qm and km]
    if not terms:
        return (0, 0)
    emin = min(e for _, e in terms)
    if max(e for _, e in terms) - emin > MAX_EXPONENT_SPREAD:
        raise DomainError("score exponent spread exceeds reference limit")
    return (sum(m << (e - emin) for m, e in terms), emin)


def logit(am: int, ae: int, s: tuple[int, int]) -> tuple[int, int]:
    """t = RN_fp32(alpha * s) as an exact dyadic (src/exactattn/reference.py:74-79)."""
    sm, se = s
    if sm == 0 or am == 0:
        return (0, 0)
    return round_dyadic(am * sm, ae + se, FP32)


def trace_row(q_bits, k_bits, v_bits, alpha_bits: int, out: str = "bf16") -> dict:
    """Every intermediate of one row (src/exactattn/reference.py:82-143).

    q_bits (d,), k_bits (n, d), v_bits (n, dv) bf16 bit patterns; alpha as fp32 bits.
    Returns dict with s, t, w (dyadics), Z, N and out (uint16 bf16 or uint32 fp32 bits)."""
    if out not in ("bf16", "fp32"):
        raise ValueError("out must be 'bf16' or 'fp32'")
    fmt = BF16 if out == "bf16" else FP32
    enc = encode_bf16 if out == "bf16" else encode_fp32
    q_bits = np.asarray(q_bits, dtype=np.uint16).reshape(-1)
    d = q_bits.shape[0]
    k_bits = np.asarray(k_bits, dtype=np.uint16).reshape(-1, d)
    v_bits = np.asarray(v_bits, dtype=np.uint16)
    n = k_bits.shape[0]
    dv = v_bits.shape[-1]
    v_bits = v_bits.reshape(n, dv)
    am, ae = decode_fp32_bits(alpha_bits)
    q = [decode_bf16(b) for b in q_bits.tolist()]
    K = [[decode_bf16(b) for b in row] for row in k_bits.tolist()]
    V = [[decode_bf16(b) for b in row] for row in v_bits.tolist()]
    s = [exact_dot(q, kj) for kj in K]
    t = [logit(am, ae, sj) for sj in s]
    w = [exp2_rn(tm, te) for tm, te in t]
    res = np.zeros(dv, dtype=np.uint16 if out == "bf16" else np.uint32)
    if n == 0:
        return dict(s=s, t=t, w=w, Z=(0, 0), N=[(0, 0)] * dv, out=res)
    wE = [e for _, e in w]
    wmin = min(wE)
    if max(wE) - wmin > MAX_EXPONENT_SPREAD:
        raise DomainError("weight exponent spread exceeds reference limit")
    Z = sum(m << (e - wmin) for m, e in w)
    N = []
    for c in range(dv):
        terms = [(w[j][0] * V[j][c][0], w[j][1] + V[j][c][1]) for j in range(n)]
        terms = [(m, e) for m, e in terms if m]
        if not terms:
            N.append((0, 0))
            continue
        base = min(e for _, e in terms)
        Nc = sum(m << (e - base) for m, e in terms)
        N.append((Nc, base))
        sh = base - wmin
        num, den = (Nc << sh, Z) if sh >= 0 else (Nc, Z << -sh)
        om, oe = round_rational(num, den, fmt)
        res[c] = 0 if om == 0 else enc(om, oe)
    return dict(s=s, t=t, w=w, Z=(Z, wmin), N=N, out=res)


def attention_row(q_bits, k_bits, v_bits, alpha_bits: int, out: str = "bf16") -> np.ndarray:
    """src/exactattn/reference.py:146-147."""
    return trace_row(q_bits, k_bits, v_bits, alpha_bits, out)["out"]


def attention(q_bits, k_bits, v_bits, alpha_bits: int, mask=None, out: str = "bf16") -> np.ndarray:
    """Batched form (src/exactattn/reference.py:150-161): q (r, d), k (n, d), v (n, dv),
    mask (r, n) bool or None. Returns (r, dv) uint16 (bf16) or uint32 (fp32 bits)."""
    q_bits = np.asarray(q_bits, dtype=np.uint16)
    k_bits = np.asarray(k_bits, dtype=np.uint16)
    v_bits = np.asarray(v_bits, dtype=np.uint16)
    r, dv = q_bits.shape[0], v_bits.shape[1]
    res = np.zeros((r, dv), dtype=np.uint16 if out == "bf16" else np.uint32)
    for i in range(r):
        sel = np.arange(k_bits.shape[0]) if mask is None else np.flatnonzero(mask[i])
        res[i] = attention_row(q_bits[i], k_bits[sel], v_bits[sel], alpha_bits, out)
    return res
