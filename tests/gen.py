"""Seeded bf16 test inputs for the parity tests.

Each kind stresses a different part of the certified path:
  normal     N(0, 1): typical activations
  wide       magnitudes spread over 48 binades (2^-40 .. 2^8) with random signs: wide score
             windows, weights far apart, elements rounded at slicing
  outlier    a quiet background (sigma 0.05) with 2% of entries replaced by 30-sigma spikes: the
             shape of real attention inputs with outlier channels
  dupes      a palette of seven values (0, +-1/2, +-1, +-2): exact ties and exact cancellation
  subnormal  values around 2^-130, most of them bf16 subnormals
The distribution parameters follow the kinds the reference's tests use; the generators are this
repository's own.
"""

from __future__ import annotations

import numpy as np

from exactattention_amd.formats import float_to_bf16_bits

_PALETTE = np.array([0.0, 0.5, -0.5, 1.0, -1.0, 2.0, -2.0])


def _normal(rng, shape, scale):
    return scale * rng.standard_normal(shape)


def _wide(rng, shape, scale):
    # integer binade plus a uniform position inside it: every binade in range equally likely
    binade = rng.integers(-40, 8, size=shape)
    frac = rng.random(shape)
    sign = np.where(rng.random(shape) < 0.5, -1.0, 1.0)
    return sign * np.ldexp(1.0 + frac, binade)


def _outlier(rng, shape, scale):
    quiet = 0.05 * scale * rng.standard_normal(shape)
    spikes = 30.0 * scale * rng.standard_normal(shape)
    return np.where(rng.random(shape) < 0.02, spikes, quiet)


def _dupes(rng, shape, scale):
    return scale * _PALETTE[rng.integers(0, _PALETTE.size, size=shape)]


def _subnormal(rng, shape, scale):
    return np.ldexp(rng.standard_normal(shape), -130)


GENERATORS = {"normal": _normal, "wide": _wide, "outlier": _outlier, "dupes": _dupes, "subnormal": _subnormal}
KINDS = list(GENERATORS)


def bf16(rng: np.random.Generator, shape, kind: str = "normal", scale: float = 1.0) -> np.ndarray:
    """uint16 bf16 bit patterns of the given kind and shape (RN-even from float64 via float32)."""
    try:
        make = GENERATORS[kind]
    except KeyError:
        raise ValueError(f"unknown kind {kind!r}; one of {KINDS}") from None
    return float_to_bf16_bits(make(rng, shape, scale))
