"""Deterministic expert rows for the tier tests (the host server on the CPU,
the request ring and the Store on the GPU).

Each (layer, expert, name) gets its own bytes from a seeded generator: fp8
e4m3 values with the exponent field drawn from a skewed distribution like a
block-quantised weight row's (so the codec builds a real code, not a
constant row), sign and mantissa uniform. Two rows never agree by accident,
so a row that lands in the wrong place or a stale row is always caught.
"""

from __future__ import annotations

import numpy as np

# Exponent-field probabilities (fields 6..14) of an N(0, 0.02) row quantised
# with a per-block amax / 448 scale: the mode sits at 13.
_EXP_FIELDS = np.arange(6, 15)
_EXP_P = np.array([1, 2, 4, 9, 20, 45, 95, 180, 90], np.float64)
_EXP_P /= _EXP_P.sum()


def expert_row(layer: int, expert: int, name: int, nbytes: int) -> np.ndarray:
    """uint8[nbytes] of expert `expert`, weight `name` (0: w13, 1: w2), layer `layer`."""
    rng = np.random.default_rng([7, layer, expert, name, nbytes])
    exp = rng.choice(_EXP_FIELDS, size=nbytes, p=_EXP_P).astype(np.uint8)
    return (exp << 3) | (rng.integers(0, 256, nbytes, dtype=np.uint8) & 0x87)
