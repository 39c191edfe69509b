"""Pins the DCT oracle (oracle/dct.py) by closed forms and invariants (CPU)."""
import numpy as np
import scipy.fft

from oracle.dct import BLOCK, dct_decode, dct_encode, dct_matrix, dct_reconstruct, dct_table


def test_dct_matrix_is_scipy_orthonormal_dct2():
    C = dct_matrix()
    x = np.random.default_rng(0).standard_normal((5, BLOCK))
    np.testing.assert_allclose(x @ C.T, scipy.fft.dct(x, type=2, norm="ortho", axis=-1), atol=1e-12)
    np.testing.assert_allclose(C @ C.T, np.eye(BLOCK), atol=1e-12)              # Parseval
    np.testing.assert_allclose((x @ C.T) @ C, x, atol=1e-12)                      # all 64 kept: exact


def test_ar1_energy_compaction():
    rng = np.random.default_rng(1)
    T, rho = 64 * 200, 0.95
    x = np.zeros(T)
    for t in range(1, T):
        x[t] = rho * x[t - 1] + np.sqrt(1 - rho ** 2) * rng.standard_normal()
    X = x.reshape(-1, BLOCK) @ dct_matrix().T
    frac = (X[:, :16] ** 2).sum() / (X ** 2).sum()
    assert frac > 0.9                                                             # low coefficients dominate


def test_absmax_codes_kat():
    # one block, one channel: x = C^T e -> X = e (a unit impulse in coefficient 3, up to float32)
    C = dct_matrix()
    x = (C[3] * 7.0).astype(np.float32)[None, :, None]
    codes, s, X = dct_encode(x)
    assert abs(float(s[0, 0, 0]) - 1.0) < 1e-3                                    # fp16(7 / 7)
    want = np.full(16, 7)
    want[3] = 14                                                                  # +7 offset binary
    np.testing.assert_array_equal(codes[0, 0, :, 0], want)


def test_decode_is_attention_over_reconstruction():
    rng = np.random.default_rng(2)
    B, Hkv, Hq, T, d = 1, 2, 4, 128, 16
    K = rng.standard_normal((B * Hkv, T, d)).astype(np.float32)
    V = rng.standard_normal((B * Hkv, T, d)).astype(np.float32)
    kc, ks, _ = dct_encode(K)
    vc, vs, _ = dct_encode(V)
    q = rng.standard_normal((B, Hq, 1, d))
    out = dct_decode(q, 0.25, kc, ks, vc, vs)
    Kr, Vr = dct_reconstruct(kc, ks).reshape(B, Hkv, T, d), dct_reconstruct(vc, vs).reshape(B, Hkv, T, d)
    rep = Hq // Hkv
    s = np.einsum("bhd,bhnd->bhn", q[:, :, 0].astype(np.float64) * 0.25, Kr.repeat(rep, 1))
    p = np.exp(s - s.max(-1, keepdims=True))
    p /= p.sum(-1, keepdims=True)
    np.testing.assert_allclose(out[:, 0], np.einsum("bhn,bhnd->bhd", p, Vr.repeat(rep, 1)), atol=1e-12)
    assert dct_table().dtype == np.float32
