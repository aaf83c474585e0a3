"""Random bf16 test inputs: typical, wide-range and adversarial kinds (the kinds of the
reference's tests/gen.py:10-35)."""

from __future__ import annotations

import numpy as np

from exactattention_amd.formats import float_to_bf16_bits


def bf16(rng: np.random.Generator, shape, kind: str = "normal", scale: float = 1.0) -> np.ndarray:
    if kind == "normal":
        x = rng.standard_normal(shape) * scale
    elif kind == "wide":  # log-uniform magnitudes 2^-40 .. 2^8, random signs
        x = np.exp2(rng.uniform(-40, 8, size=shape)) * rng.choice([-1.0, 1.0], size=shape)
    elif kind == "outlier":  # small values with 2% large spikes
        x = rng.standard_normal(shape) * 0.05 * scale
        x = np.where(rng.random(shape) < 0.02, rng.standard_normal(shape) * 30 * scale, x)
    elif kind == "dupes":  # few distinct values: ties and exact cancellation
        x = rng.choice(np.array([-2.0, -1.0, -0.5, 0.0, 0.5, 1.0, 2.0]) * scale, size=shape)
    elif kind == "subnormal":
        x = rng.standard_normal(shape) * 2.0 ** -130
    else:
        raise ValueError(kind)
    return float_to_bf16_bits(x)


KINDS = ["normal", "wide", "outlier", "dupes", "subnormal"]
