"""STRATA codec and tier decode (numpy restatement).

TEST INFRASTRUCTURE ONLY (see ``oracle/__init__.py``).

Reference (STRATA_KV.py):
  * ``rotation_matrix(d, key)``   1110-1128: R = H_d / sqrt(d) * diag(s), H_d the Sylvester Hadamard
                                  matrix, s in {-1, +1}^d drawn by
                                  ``np.random.default_rng([42, crc32("rotation"), crc32(key)])
                                  .choice([-1.0, 1.0], d)`` (_rng, 306-307); key "strata" (1517)
  * ``uniform_step(bits)``        1132-1155: golden-section search of the MSE-optimal mid-rise
                                  uniform quantiser step of N(0, 1) on a 360001-point grid
  * ``strata_quantize(Y, bits)``  1158-1168: s = max(fp16(step * rms(y)), 2^-24) per vector,
                                  c = clamp(round(y / s + (2^b - 1) / 2)), y_hat = (c - half) s
  * ``pack_planar`` / ``unpack_planar`` 1171-1189
  * compression of one side       1546-1548: mu = fp16(mean over tokens), Y = (X - mu) R^T
  * ``tier_reference`` + merge    1751-1795 (StrataState.attend)

Fixed arithmetic order (what the GPU kernels compute, restated here so both agree bit for bit):
  * sums over tokens (mu) and over channels (rms) are accumulated in float64, then rounded to
    float32 once (the reference's torch fp32 reductions agree to float32 rounding);
  * the rotation is the fast Walsh-Hadamard transform of (x - mu) * s in float32, butterfly
    stages h = 1, 2, 4, ..., d/2, then a float32 multiply by float32(1/sqrt(d)); it equals the
    reference's dense (X - mu) @ R.T up to float32 rounding.

Pinning (tests/test_oracle_strata.py, tests/test_golden.py): golden vectors written by the
reference's own functions (tests/golden/strata_codec.npz): uniform_step floats for 1..8 bits
bit-equal, the rotation signs for d = 64, 128 equal, and one side's compression on seeded fp32
rows -- fp16 means bit-equal, the FWHT rows within 1e-6 of the reference's dense product, codes
and scales at 2, 4 and 8 bits bit-equal on the reference's rows and end to end (the float64 sums
and the FWHT order give the reference's codes on these rows: no mismatch in 73,728); also
rotation orthogonality (1e-6; the reference's own check is 1e-5 at 1918), the reference's KAT
UNIFORM_1960 (1912), strata_quantize by hand KATs and a nearest-level brute force, planar packing
by KAT bytes and round trips, and the tier decode by the reference's identity "decode over the
strata == attention over the reconstructions mu + y_hat R" (1e-4 at 1983-1985) against
chunked_attention.
"""
from __future__ import annotations

import math
import zlib
from functools import lru_cache

import numpy as np

from .kivi import as_stored


def rotation_signs(d: int, key: str = "strata") -> np.ndarray:
    """The sign vector s of rotation_matrix(d, key) (STRATA_KV.py:1119-1124, 306-307)."""
    g = np.random.default_rng([42, zlib.crc32(b"rotation"), zlib.crc32(key.encode())])
    return g.choice([-1.0, 1.0], d)


def rotation_matrix(d: int, key: str = "strata") -> np.ndarray:
    """R = H_d / sqrt(d) * s[None, :] as float32 (d a power of two), STRATA_KV.py:1118-1124."""
    Hm = np.array([[1.0]])
    while Hm.shape[0] < d:
        Hm = np.block([[Hm, Hm], [Hm, -Hm]])
    return (Hm / math.sqrt(d) * rotation_signs(d, key)[None, :]).astype(np.float32)


def fwht_rotate(x: np.ndarray, signs: np.ndarray) -> np.ndarray:
    """y = x R^T for R = H diag(s) / sqrt(d), in the kernels' float32 order: FWHT of x * s
    (stages h = 1, 2, ..., d/2; pairs (a, b) -> (a + b, a - b)), then * float32(1/sqrt(d))."""
    y = (x.astype(np.float32) * signs.astype(np.float32)).copy()
    d = y.shape[-1]
    h = 1
    while h < d:
        y = y.reshape(*y.shape[:-1], d // (2 * h), 2, h)
        a, b = y[..., 0, :].copy(), y[..., 1, :].copy()
        y[..., 0, :] = a + b
        y[..., 1, :] = a - b
        y = y.reshape(*y.shape[:-3], d)
        h *= 2
    return (y * np.float32(1.0 / math.sqrt(d))).astype(np.float32)


def fwht_unrotate(y: np.ndarray, signs: np.ndarray) -> np.ndarray:
    """x = y R (the inverse rotation): FWHT of y in the same stage order, * float32(1/sqrt(d)),
    then * s."""
    return (fwht_rotate(y, np.ones_like(signs)) * signs.astype(np.float32)).astype(np.float32)


@lru_cache(maxsize=None)
def uniform_step(bits: int):
    """(step, mse) of the MSE-optimal mid-rise uniform quantiser of N(0, 1), STRATA_KV.py:1132-1155."""
    x = np.linspace(-9.0, 9.0, 360001)
    w = np.exp(-0.5 * x * x)
    w /= w.sum()
    half = (2 ** bits - 1) / 2.0

    def mse(step):
        c = np.clip(np.round(x / step + half), 0, 2 ** bits - 1)
        return float((w * (x - (c - half) * step) ** 2).sum())
    lo, hi = 1e-4, 4.0
    g = (math.sqrt(5) - 1) / 2
    for _ in range(200):
        a, b = hi - g * (hi - lo), lo + g * (hi - lo)
        lo, hi = (lo, b) if mse(a) < mse(b) else (a, hi)
    step = 0.5 * (lo + hi)
    return step, mse(step)


def strata_quantize(Y: np.ndarray, bits: int, step: float):
    """Per-vector code of rotated vectors Y (..., d), STRATA_KV.py:1158-1168, in the kernels' order:
    rms = sqrt(float32(sum64(y^2) / d)); s = max(fp16(float32(step) * rms), 2^-24);
    c = clamp(rint(y / s + half)).  Returns (codes uint8, s float32 (...), y_hat float32)."""
    Y = Y.astype(np.float32)
    half = np.float32((2 ** bits - 1) / 2.0)
    ms = np.float32((Y.astype(np.float64) ** 2).sum(-1) / Y.shape[-1])
    rms = np.sqrt(ms).astype(np.float32)
    s = np.maximum(as_stored((np.float32(step) * rms).astype(np.float32)), np.float32(2.0 ** -24))
    c = np.clip(np.rint(Y / s[..., None] + half), 0, 2 ** bits - 1)
    return c.astype(np.uint8), s.astype(np.float32), ((c - half) * s[..., None]).astype(np.float32)


def strata_center_rotate(X: np.ndarray, signs: np.ndarray):
    """One side of STRATA_KV.py:1546-1547 for vectors X (BH, n, d): mu = fp16(float32(sum64 / n)) per
    channel over all n coded tokens, Y = (X - mu) R^T.  Returns (mu (BH, d) float32, Y float32)."""
    X = X.astype(np.float32)
    mu = as_stored(np.float32(X.astype(np.float64).sum(1) / X.shape[1]).astype(np.float32))
    return mu, fwht_rotate(X - mu[:, None, :], signs)


def strata_encode(X: np.ndarray, bits: int, signs: np.ndarray, step: float):
    """strata_center_rotate then strata_quantize of every token at one width.
    Returns (mu (BH, d), codes, s, y_hat, Y)."""
    mu, Y = strata_center_rotate(X, signs)
    c, s, yh = strata_quantize(Y, bits, step)
    return mu, c, s, yh, Y


def pack_planar(codes: np.ndarray, bits: int) -> np.ndarray:
    """(..., d) -> (..., d*bits/8): byte i holds coordinate p*d/P + i in bits [p*bits, (p+1)*bits),
    P = 8/bits (STRATA_KV.py:1171-1182)."""
    P = 8 // bits
    d = codes.shape[-1]
    c = codes.astype(np.int64).reshape(*codes.shape[:-1], P, d // P)
    shifts = (np.arange(P) * bits)[:, None]
    return (c << shifts).sum(-2).astype(np.uint8)


def unpack_planar(packed: np.ndarray, bits: int) -> np.ndarray:
    """Inverse of pack_planar (STRATA_KV.py:1185-1189)."""
    P = 8 // bits
    x = packed.astype(np.int64)
    return np.concatenate([(x >> (p * bits)) & (2 ** bits - 1) for p in range(P)], -1)


def tier_partials(qr: np.ndarray, qb: np.ndarray, codes_k: np.ndarray, ks: np.ndarray, codes_v: np.ndarray,
                  vs: np.ndarray, bits: int):
    """tier_reference (STRATA_KV.py:1751-1760) in float64: qr (Hkv, rows, d) rotated scaled query,
    qb (Hkv, rows); codes (Hkv, n, d), scales (Hkv, n).  Returns m, l (Hkv, rows), acc (Hkv, rows, d)
    in the rotated value basis (natural-exponent softmax partials)."""
    half = (2 ** bits - 1) / 2.0
    kh = (codes_k.astype(np.float64) - half) * ks.astype(np.float64)[..., None]
    vh = (codes_v.astype(np.float64) - half) * vs.astype(np.float64)[..., None]
    s = np.einsum("hrd,hnd->hrn", qr.astype(np.float64), kh) + qb.astype(np.float64)[..., None]
    m = s.max(-1)
    e = np.exp(s - m[..., None])
    return m, e.sum(-1), np.einsum("hrn,hnd->hrd", e, vh)


def strata_attend(q: np.ndarray, scaling: float, k_exact: np.ndarray, v_exact: np.ndarray, tiers, mu_k: np.ndarray,
                  mu_v: np.ndarray, R: np.ndarray) -> np.ndarray:
    """StrataState.attend (STRATA_KV.py:1762-1795) in float64 for one sequence: q (1, Hq, Tq, d),
    exact rows (Hkv, e, d) all visible, tiers = [(bits, codes_k, ks, codes_v, vs)] with codes
    (Hkv, n, d) and scales (Hkv, n), mu_k / mu_v (Hkv, d), R (d, d).  Returns (1, Tq, Hq, d)."""
    _, Hq, Tq, d = q.shape
    Hkv = k_exact.shape[0]
    rep = Hq // Hkv
    qg = q.reshape(Hkv, rep * Tq, d).astype(np.float64)
    R = R.astype(np.float64)
    if k_exact.shape[1]:
        s_ex = np.einsum("hrd,hnd->hrn", qg, k_exact.astype(np.float64)) * scaling
        m_e = s_ex.max(-1)
        e_ex = np.exp(s_ex - m_e[..., None])
        l_e = e_ex.sum(-1)
        o = np.einsum("hrn,hnd->hrd", e_ex, v_exact.astype(np.float64))
    else:                                   # no exact rows: an empty partial
        m_e = np.full(qg.shape[:2], -np.inf)
        l_e = np.zeros(qg.shape[:2])
        o = np.zeros(qg.shape)
    if tiers:
        qr = (qg @ R.T) * scaling
        qb = np.einsum("hrd,hd->hr", qg, mu_k.astype(np.float64)) * scaling
        parts = [tier_partials(qr, qb, ck, ks, cv, vs, b) for b, ck, ks, cv, vs in tiers]
        M = np.maximum(m_e, np.max([p[0] for p in parts], 0))
        we = np.exp(m_e - M)
        acc = sum(np.exp(p[0] - M)[..., None] * p[2] for p in parts)
        wl = sum(np.exp(p[0] - M) * p[1] for p in parts)
        o = (we[..., None] * o + acc @ R + wl[..., None] * mu_v.astype(np.float64)[:, None, :]) \
            / (we * l_e + wl)[..., None]
    else:
        o = o / l_e[..., None]
    return o.reshape(1, Hq, Tq, d).transpose(0, 2, 1, 3)
