"""bf16/fp32 bit-pattern helpers of the public API (src/exactattn/formats.py:16-17,160-181 and
src/exactattn/reference.py:164-173 of the reference): input generation and the default scale.
None of these sits on the attention path itself."""

from __future__ import annotations

import math
from functools import lru_cache

import numpy as np


class ExactAttentionDomainError(ValueError):
    """An input is outside the definition's domain: NaN/inf, or an fp32-overflowing logit
    (mirrors src/exactattn/formats.py:16-17)."""


class ExactAttentionUncertifiedError(RuntimeError):
    """A row that no device tier could certify. The library never substitutes a CPU result."""


def float_to_bf16_bits(x) -> np.ndarray:
    """RN-even conversion of float32-castable values to bf16 bit patterns (uint16), through float32
    (src/exactattn/formats.py:160-176). For generating inputs only."""
    f = np.asarray(x, dtype=np.float32)
    if not np.all(np.isfinite(f)):
        raise ExactAttentionDomainError("non-finite value")
    u = f.view(np.uint32)
    # finite patterns are <= 0xFF7FFFFF, so adding at most 0x8000 cannot wrap 32 bits
    out = ((u + (np.uint32(0x7FFF) + ((u >> np.uint32(16)) & np.uint32(1)))) >> np.uint32(16)).astype(np.uint16)
    if np.any((out & 0x7F80) == 0x7F80):
        raise ExactAttentionDomainError("bf16 overflow when generating input")
    return out


def bf16_bits_to_float32(bits) -> np.ndarray:
    """src/exactattn/formats.py:179-181."""
    return (np.asarray(bits, dtype=np.uint16).astype(np.uint32) << 16).view(np.float32)


def fp32_bits(x) -> int:
    return int(np.asarray(x, dtype=np.float32).view(np.uint32))


def alpha_fp32_bits(alpha=None, alpha_bits=None) -> int:
    """The fp32 bit pattern of a logit scale. `alpha` is a value of any type numpy converts to
    float32 (an int 1 or True is 1.0, as src/exactattn/formats.py:120-130 decodes it); a raw
    pattern is taken only through `alpha_bits`. NaN or infinity raises
    ExactAttentionDomainError, as the reference's decode_fp32 does."""
    if alpha_bits is not None:
        if alpha is not None:
            raise ValueError("give alpha or alpha_bits, not both")
        if isinstance(alpha_bits, (bool, np.bool_)) or not isinstance(alpha_bits, (int, np.integer)):
            raise TypeError("alpha_bits must be an integer fp32 bit pattern")
        bits = int(alpha_bits)
        if not 0 <= bits < 1 << 32:
            raise ValueError("alpha_bits must lie in [0, 2^32)")
    elif alpha is None:
        raise TypeError("alpha is required")
    else:
        a = np.asarray(alpha, dtype=np.float32)
        if a.size != 1:
            raise ValueError("alpha must be a scalar")
        bits = int(a.reshape(()).view(np.uint32))
    if (bits >> 23) & 0xFF == 0xFF:
        raise ExactAttentionDomainError("fp32 NaN or infinity in input")
    return bits


def _ln2_interval(W: int) -> tuple[int, int]:
    # ln 2 = 2 atanh(1/3) = sum_k 2 / ((2k+1) 3^(2k+1)), both ends enclosed at scale 2^W
    lo = hi = 0
    k = 0
    one = 1 << W
    while True:
        den = (2 * k + 1) * 3 ** (2 * k + 1)
        t = (2 * one) // den
        lo += t
        hi += -((-2 * one) // den)
        k += 1
        if t == 0:
            return lo, hi + 2


def _rn32_ratio(num: int, den: int) -> int:
    """fp32 bits of RN-even(num/den) for num, den > 0 (normal range)."""
    k = num.bit_length() - den.bit_length()
    if (num << max(0, -k)) < (den << max(0, k)):
        k -= 1
    qe = k - 23
    n, d = (num, den << qe) if qe >= 0 else (num << -qe, den)
    q, r = divmod(n, d)
    if 2 * r > d or (2 * r == d and q & 1):
        q += 1
    if q == 1 << 24:
        q >>= 1
        qe += 1
    return ((qe + 23 + 127) << 23) | (q - (1 << 23))


@lru_cache(maxsize=None)
def default_alpha_bits(d: int) -> int:
    """fp32 bits of RN_fp32(log2(e) / sqrt(d)) = RN(1 / (ln 2 sqrt d)), decided by integer
    enclosures with doubling precision (src/exactattn/reference.py:164-173 uses mpmath)."""
    W = 80
    while True:
        L_lo, L_hi = _ln2_interval(W)
        s = math.isqrt(d << (2 * W))
        s_hi = s if s * s == (d << (2 * W)) else s + 1
        lo = _rn32_ratio(1 << (2 * W), L_hi * s_hi)
        hi = _rn32_ratio(1 << (2 * W), L_lo * s)
        if lo == hi:
            return lo
        W *= 2


@lru_cache(maxsize=None)
def alpha_bits_for(scaling: float) -> int:
    """fp32 bits of RN_fp32(scaling / ln 2) for a positive float64 logit scale (an attention
    module's `scaling`), decided by integer enclosures of ln 2 with doubling precision
    (scripts/validate_model.py:35-40 rounds an mpmath quotient at 200 bits)."""
    scaling = float(scaling)
    if not (scaling > 0.0 and math.isfinite(scaling)):
        raise ValueError("scaling must be positive and finite")
    m, e = math.frexp(scaling)
    M, E = int(m * (1 << 53)), e - 53          # scaling = M * 2^E exactly
    W = 80
    while True:
        L_lo, L_hi = _ln2_interval(W)          # L_lo / 2^W <= ln 2 <= L_hi / 2^W
        sh = E + W                             # scaling / ln 2 = M 2^(E+W) / L
        num = M << sh if sh >= 0 else M
        scale = 1 if sh >= 0 else 1 << -sh
        lo = _rn32_ratio(num, L_hi * scale)
        hi = _rn32_ratio(num, L_lo * scale)
        if lo == hi:
            if not 0 < (lo >> 23) < 255:
                raise ValueError("scaling / ln 2 is outside the normal fp32 range")
            return lo
        W *= 2


def default_alpha(d: int) -> np.float32:
    return np.array([default_alpha_bits(d)], dtype=np.uint32).view(np.float32)[0]
