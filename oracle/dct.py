"""Blockwise token-axis DCT coding of K/V and decode over it (numpy restatement).

TEST INFRASTRUCTURE ONLY (see ``oracle/__init__.py``).

The reference has no DCT (no DCT transform appears in its sources); the build defines the contract, following the
reference's own conventions where it has them:
  * per (KV head, channel, 64-token block): orthonormal DCT-II along tokens,
    C[k, n] = a_k cos(pi (2n + 1) k / 128), a_0 = sqrt(1/64), a_k = sqrt(2/64); keep k = 0..15;
  * the 16 kept coefficients of each (block, channel) are quantised with symmetric absmax
    (absmax_quant, STRATA_KV.py:549-554): s = max(fp16(max|X| / 7), 2^-24), codes
    clamp(round(X / s), -7, 7), stored offset-binary (+7) in 4 bits as TILT_KV.py:2621-2625 does;
  * decode = attention over the reconstructions x_n = sum_k C[k, n] s (code_k - 7) (plus exact
    rows), i.e. chunked_attention (STRATA_KV.py:641-675) over them.

Fixed arithmetic order of the encoder (the GPU kernel computes exactly this): C in float32
(float32 of the float64 closed form); X_k = sum over n = 0..63 in increasing n of
float32(C[k, n] * x_n), each product and each partial sum rounded to float32 (no fused
multiply-add); s and codes in float32 with IEEE division.

Pinning (tests/test_oracle_dct.py): C equals scipy.fft.dct(type=2, norm="ortho") and is
orthonormal (Parseval); keeping all 64 coefficients unquantised reconstructs the block exactly;
AR(1) (rho = 0.95) blocks put most energy in the low coefficients; absmax codes by hand KATs;
dct_decode == chunked_attention over the reconstructed rows.
"""
from __future__ import annotations

import math

import numpy as np

from .attention import chunked_attention
from .kivi import as_stored

BLOCK = 64
KEEP = 16


def dct_matrix(n: int = BLOCK) -> np.ndarray:
    """Orthonormal DCT-II matrix (n, n) in float64: C[k, j] = a_k cos(pi (2j + 1) k / (2n))."""
    k = np.arange(n)[:, None]
    j = np.arange(n)[None, :]
    C = np.cos(math.pi * (2 * j + 1) * k / (2 * n))
    C[0] *= math.sqrt(1.0 / n)
    C[1:] *= math.sqrt(2.0 / n)
    return C


def dct_table() -> np.ndarray:
    """The kernels' float32 table of the kept rows: (KEEP, BLOCK)."""
    return dct_matrix()[:KEEP].astype(np.float32)


def dct_encode(x: np.ndarray):
    """x (BH, T, d), T % 64 == 0 -> (codes (BH, T/64, KEEP, d) uint8 offset-binary 0..14,
    scales (BH, T/64, d) float32 holding fp16 values, X (BH, T/64, KEEP, d) float32 coefficients)."""
    BH, T, d = x.shape
    nb = T // BLOCK
    xb = x.astype(np.float32).reshape(BH, nb, BLOCK, d)
    C = dct_table()
    X = np.zeros((BH, nb, KEEP, d), np.float32)
    for j in range(BLOCK):                                  # sequential sum in increasing n
        X = (X + (C[None, None, :, j, None] * xb[:, :, j:j + 1, :]).astype(np.float32)).astype(np.float32)
    amax = np.abs(X).max(2)                                  # (BH, nb, d)
    s = np.maximum(as_stored((amax / np.float32(7.0)).astype(np.float32)), np.float32(2.0 ** -24))
    c = np.clip(np.rint(X / s[:, :, None, :]), -7, 7)
    return (c + 7).astype(np.uint8), s.astype(np.float32), X


def dct_reconstruct(codes: np.ndarray, scales: np.ndarray) -> np.ndarray:
    """Rows x_n = sum_k C[k, n] s (code_k - 7), float64 (BH, T, d)."""
    BH, nb, K, d = codes.shape
    Xh = (codes.astype(np.float64) - 7.0) * scales.astype(np.float64)[:, :, None, :]
    C = dct_table().astype(np.float64)                      # the table the kernels use
    return np.einsum("kn,bjkd->bjnd", C, Xh).reshape(BH, nb * BLOCK, d)


def dct_decode(q: np.ndarray, scaling: float, kc, ks, vc, vs, k_exact=None, v_exact=None) -> np.ndarray:
    """Attention of q (B, Hq, Tq, d) over the DCT-coded rows of every (b, h) (codes (B*Hkv, ...)) and
    exact rows (B, Hkv, e, d), all visible.  Returns (B, Tq, Hq, d) float64."""
    B, Hq, Tq, d = q.shape
    Kr = dct_reconstruct(kc, ks)
    Vr = dct_reconstruct(vc, vs)
    Hkv = Kr.shape[0] // B
    Kr = Kr.reshape(B, Hkv, -1, d)
    Vr = Vr.reshape(B, Hkv, -1, d)
    n = Kr.shape[2]
    tok = {"k": Kr, "v": Vr, "b": np.zeros((B, Hkv, n)), "tau": np.full(n, -1)}
    if k_exact is None:
        k_exact = np.zeros((B, Hkv, 0, d))
        v_exact = np.zeros((B, Hkv, 0, d))
    e = k_exact.shape[2]
    return chunked_attention(q, scaling, np.zeros(Tq, int), k_exact, v_exact, np.zeros(e, int),
                             np.full(e, 1 << 40), tok)
