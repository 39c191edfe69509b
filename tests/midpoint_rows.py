"""Rotated rows whose STRATA scale lands exactly on an fp16 rounding midpoint.

strata_quantize (STRATA_KV.py:1158-1168) stores s = fp16(float32(step) * rms), rms the float32
square root of the row's mean square.  Each row built here has one nonzero coordinate v, chosen so
that under correctly rounded float32 arithmetic (numpy's, torch's) float32(step * rms) is exactly
the midpoint of two adjacent fp16 values: the stored scale is then decided by the round-half-even
rule, and a square root one ulp off moves the product off the midpoint and, about half the time,
to the other fp16 neighbour.  A tie of this kind decided the one distortion-table element that once
differed (a scale one fp16 ulp low from a hardware square root that was not correctly rounded).
"""
from __future__ import annotations

import numpy as np


def _nudge(x: np.float32, k: int) -> np.float32:
    """x moved by k ulps (positive finite x)."""
    return np.array([np.int64(np.float32(x).view(np.uint32)) + k], dtype=np.int64).astype(np.uint32).view(np.float32)[0]


def midpoint_rows(bits: int, count: int, seed: int, step: float, d: int = 128) -> np.ndarray:
    """(count, d) float32 rows: coordinate (i * 37) % d holds v, the rest are 0."""
    st = np.float64(np.float32(step))
    rng = np.random.default_rng(seed)
    rows = np.zeros((count, d), np.float32)
    made = 0
    while made < count:
        e = int(rng.integers(-5, 4))
        m16 = int(rng.integers(0, 1024))
        h = 2.0 ** e * (1 + m16 / 1024)
        mid = np.float32(h + 2.0 ** e / 2048)                     # exact: 12 significant bits
        r0 = np.float32(np.float64(mid) / st)
        found = None
        for k in range(-4, 5):
            r = _nudge(r0, k)
            if np.float32(st * np.float64(r)) != mid:             # product of two floats: exact in float64
                continue
            if any(np.float32(st * np.float64(_nudge(r, u))) == mid for u in (-1, 1)):
                continue                                           # a root one ulp off must leave the tie
            ms0 = np.float32(np.float64(r) ** 2)
            for j in range(-3, 4):
                ms = _nudge(ms0, j)
                if np.sqrt(ms) != r:                               # numpy's float32 root is correctly rounded
                    continue
                v0 = np.float32(np.sqrt(np.float64(ms) * d))
                for t in range(-3, 4):
                    v = _nudge(v0, t)
                    if np.float32(np.float64(v) ** 2 / d) == ms:
                        found = v
                        break
                if found is not None:
                    break
            if found is not None:
                break
        if found is None:
            continue
        rows[made, (made * 37) % d] = found if rng.integers(0, 2) else -found
        made += 1
    return rows
