"""Pins the STRATA oracle (oracle/strata.py) independently of itself (CPU)."""
import numpy as np
import pytest

from oracle.attention import chunked_attention
from oracle.strata import (fwht_rotate, fwht_unrotate, pack_planar, rotation_matrix, rotation_signs,
                           strata_attend, strata_center_rotate, strata_quantize, uniform_step, unpack_planar)


def test_rotation_orthogonal_and_fwht_equals_dense_product():
    d = 128
    R = rotation_matrix(d).astype(np.float64)
    np.testing.assert_allclose(R @ R.T, np.eye(d), atol=1e-6)           # reference check: 1e-5 (1918)
    s = rotation_signs(d)
    assert set(np.unique(s)) <= {-1.0, 1.0} and np.array_equal(s, rotation_signs(d))
    x = np.random.default_rng(0).standard_normal((5, d)).astype(np.float32)
    np.testing.assert_allclose(fwht_rotate(x, s), x.astype(np.float64) @ R.T, rtol=0, atol=2e-6)
    np.testing.assert_allclose(fwht_unrotate(fwht_rotate(x, s), s), x, atol=2e-6)


def test_uniform_step_reference_kat():
    # UNIFORM_1960 (STRATA_KV.py:1912) and the docstring pair for 2 bits (1138-1140)
    for b, want in {2: 0.9957, 3: 0.5860, 4: 0.3352}.items():
        assert round(uniform_step(b)[0], 4) == want
    assert round(uniform_step(2)[1], 4) == 0.1188


def test_strata_quantize_kat_and_nearest_level():
    # y with rms 2: s = fp16(step * 2); codes by hand for 2 bits (half = 1.5)
    y = np.array([[2.0, -2.0, 2.0, -2.0]], np.float32)
    c, s, yh = strata_quantize(y, 2, 0.5)
    assert s[0] == np.float32(1.0)
    np.testing.assert_array_equal(c[0], [3, 0, 3, 0])                     # 2/1 + 1.5 = 3.5 -> 4 -> clamp 3
    np.testing.assert_array_equal(yh[0], [1.5, -1.5, 1.5, -1.5])
    rng = np.random.default_rng(1)
    Y = rng.standard_normal((50, 64)).astype(np.float32)
    for b in (2, 4, 8):
        c, s, yh = strata_quantize(Y, b, uniform_step(b)[0])
        half = (2 ** b - 1) / 2
        levels = (np.arange(2 ** b) - half)[None, None, :] * s[:, None, None]
        dist = np.abs(Y[..., None] - levels)
        best = dist.min(-1)
        got = np.abs(Y - (c.astype(np.float64) - half) * s[:, None])
        assert np.all(got <= best + 1e-6 * s[:, None])                     # a nearest level
        # codec relative MSE close to the Gaussian uniform-quantiser optimum (reference bound 1.3x, 1927)
        rel = ((yh - Y) ** 2).sum() / (Y ** 2).sum()
        assert rel <= 1.3 * uniform_step(b)[1]


@pytest.mark.parametrize("bits", [2, 4, 8])
def test_midpoint_rows_land_on_fp16_ties(bits):
    # the rows the GPU scale test uses: float32(step * rms) is exactly halfway between two fp16
    # values, so the stored scale is the even neighbour (round half to even, torch's and numpy's
    # fp16 rounding); one ulp less or more on rms gives the lower or upper neighbour
    from midpoint_rows import midpoint_rows
    step = uniform_step(bits)[0]
    Y = midpoint_rows(bits, 200, seed=bits, step=step)
    _, s, _ = strata_quantize(Y, bits, step)
    rms = np.sqrt(np.float32((Y.astype(np.float64) ** 2).sum(-1) / Y.shape[-1]))
    prod = (np.float32(step) * rms).astype(np.float32)
    lo = prod.astype(np.float16)
    nb = np.nextafter(lo, np.where(lo.astype(np.float32) < prod, np.float16(np.inf), np.float16(0)))
    mid = (lo.astype(np.float64) + nb.astype(np.float64)) / 2
    np.testing.assert_array_equal(prod.astype(np.float64), mid)             # exactly a tie
    assert np.all(lo.view(np.uint16) % 2 == 0) and np.array_equal(s, lo.astype(np.float32))
    for k in (-1, 1):
        off = (np.float32(step) * np.nextafter(rms, np.float32(np.inf) * k)).astype(np.float32)
        assert np.all(off != prod)                                        # a one-ulp root leaves the tie


def test_planar_pack_kat_and_round_trip():
    c = np.array([[0, 1, 2, 3, 3, 2, 1, 0]], np.uint8)
    np.testing.assert_array_equal(pack_planar(c, 2), [[120, 45]])         # by hand
    c4 = np.array([[1, 2, 3, 4, 5, 6, 7, 8]], np.uint8)
    np.testing.assert_array_equal(pack_planar(c4, 4), [[1 | 5 << 4, 2 | 6 << 4, 3 | 7 << 4, 4 | 8 << 4]])
    rng = np.random.default_rng(2)
    for b in (2, 4, 8):
        x = rng.integers(0, 2 ** b, (3, 7, 128)).astype(np.uint8)
        np.testing.assert_array_equal(unpack_planar(pack_planar(x, b), b), x)


def test_tier_decode_identity_against_reconstruction():
    """Decode over the strata == attention over mu + y_hat R (the reference's identity, 1983-1985)."""
    rng = np.random.default_rng(3)
    Hq, Hkv, d, Tq, e = 8, 2, 128, 2, 10
    s = rotation_signs(d)
    R = rotation_matrix(d)
    q = rng.standard_normal((1, Hq, Tq, d))
    ke, ve = rng.standard_normal((Hkv, e, d)), rng.standard_normal((Hkv, e, d))
    # one mean per side over all coded tokens of a head; tokens then split into 8/4/2-bit strata
    n = 92
    X = rng.standard_normal((Hkv, n, d)).astype(np.float32) * 2 + 0.5
    Vv = rng.standard_normal((Hkv, n, d)).astype(np.float32)
    mu_k, Yk = strata_center_rotate(X, s)
    mu_v, Yv = strata_center_rotate(Vv, s)
    tiers, recon_k, recon_v = [], [], []
    for b, (a, m) in ((8, (0, 12)), (4, (12, 30)), (2, (42, 50))):
        ck, sk, yk = strata_quantize(Yk[:, a:a + m], b, uniform_step(b)[0])
        cv, sv, yv = strata_quantize(Yv[:, a:a + m], b, uniform_step(b)[0])
        tiers.append((b, ck, sk, cv, sv))
        recon_k.append(yk.astype(np.float64) @ R.astype(np.float64))
        recon_v.append(yv.astype(np.float64) @ R.astype(np.float64))
    Kr = np.concatenate(recon_k, 1) + mu_k[:, None, :]
    Vr = np.concatenate(recon_v, 1) + mu_v[:, None, :]
    out = strata_attend(q, d ** -0.5, ke, ve, tiers, mu_k, mu_v, R)
    n_all = Kr.shape[1]
    tok = {"k": Kr[None], "v": Vr[None], "b": np.zeros((1, Hkv, n_all)), "tau": np.full(n_all, -1)}
    ref = chunked_attention(q, d ** -0.5, np.zeros(Tq, int), ke[None], ve[None], np.zeros(e, int),
                            np.full(e, 1 << 40), tok)
    np.testing.assert_allclose(out, ref, rtol=0, atol=1e-10)
