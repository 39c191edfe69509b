"""Pins of the QUASAR oracle (oracle/quasar.py) and of the host-side set-up of kvq.QuasarState.

* Codebooks: Max's (1960) Gaussian Lloyd-Max MSE at 1-4 bits (the table STRATA_KV.py:1085-1087
  quotes) and the embedded (2, 2, 4) code's MSE after each stage as QUASAR_KV.py:1151-1152 states;
  levels of a symmetric distribution are antisymmetric.
* The coded-domain decode equals softmax attention over the exact rows plus the reconstructed
  coded tokens (mu + (rho u_hat) T^T): the identity QuasarState is built on (QUASAR_KV.py:1857-1862),
  checked with appended causal rows; a planted mistake (a step's band shifted) breaks it.
* The package's codebooks, step tables and host packer agree with the oracle's.
"""
import numpy as np
import pytest

import oracle.quasar as oq
from oracle.kivi import pack_rows


@pytest.mark.parametrize("bits,mse", [(1, 0.3634), (2, 0.1175), (3, 0.03454), (4, 0.009497)])
def test_lloyd_max_matches_max_table(bits, mse):
    assert abs(oq.lloyd_max_mse(bits) - mse) < 2e-4 * max(1.0, mse * 10)
    c = oq.lloyd_max_gaussian(bits)
    np.testing.assert_allclose(c, -c[::-1], atol=1e-4)          # the grid solve is symmetric to ~3e-5


def test_embedded_codebooks_stage_mse():
    got = oq.embedded_mse((2, 2, 4))
    for g, want, tol in zip(got, (0.1175, 0.0196, 0.00056), (1e-4, 1e-4, 1e-5)):
        assert abs(g - want) < tol, (got, want)


def _case(seed=1, n_c=300, n0=40, extra=3):
    from kvq.quasar import synthetic_packed
    p = synthetic_packed(2, 128, n_c, seed=seed)
    rng = np.random.default_rng(seed)
    K = rng.standard_normal((1, 2, n0 + extra, 128)).astype(np.float32)
    V = rng.standard_normal((1, 2, n0 + extra, 128)).astype(np.float32)
    q = rng.standard_normal((1, 8, 2, 128)).astype(np.float32)
    return p, K, V, q


def test_coded_decode_equals_attention_over_reconstruction():
    p, K, V, q = _case()
    H = 1000
    qpos = np.array([H + 1, H + 2])                  # appended rows H, H+1 visible to row 1 only in part
    a = oq.attend(q, 128 ** -0.5, qpos, K, V, 40, H, p, (2, 2, 4))
    b = oq.attend_reconstructed(q, 128 ** -0.5, qpos, K, V, 40, H, p, (2, 2, 4))
    np.testing.assert_allclose(a, b, rtol=0, atol=1e-12)
    # a planted mistake in the oracle's input: one K step's band shifted by one coefficient
    bad = dict(p)
    bad["steps"] = [dict(st) for st in p["steps"]]
    st = next(s for s in bad["steps"] if s["side"] == 0 and s["a"] > 0)
    st["a"], st["b"] = st["a"] - 1, st["b"] - 1
    c = oq.attend(q, 128 ** -0.5, qpos, K, V, 40, H, bad, (2, 2, 4))
    assert np.abs(c - b).max() > 1e-6


def test_causal_rows_and_empty_code():
    _, K, V, q = _case()
    H = 1000
    empty = {"steps": [], "n_c": 0}
    a = oq.attend(q, 0.1, np.array([H, H + 2]), K, V, 40, H, empty, (2, 2, 4))
    b = oq.attend_reconstructed(q, 0.1, np.array([H, H + 2]), K, V, 40, H, empty, (2, 2, 4))
    np.testing.assert_allclose(a, b, atol=1e-12)
    # query 0 at position H sees appended row H only; rows H+1, H+2 masked
    a0 = oq.attend(q[:, :, :1], 0.1, np.array([H]), K[:, :, :41], V[:, :, :41], 40, H, empty, (2, 2, 4))
    np.testing.assert_allclose(a[:, :1], a0, atol=1e-12)


def test_package_setup_matches_oracle():
    from kvq import quasar as kq
    for stages in ((2, 2, 4), (4, 4), (8,)):
        for x, y in zip(kq.stage_codebooks(stages), oq.stage_codebooks(stages)):
            np.testing.assert_array_equal(x, y)
    p = kq.synthetic_packed(3, 128, 257, stages=(2, 2, 4), seed=5)
    for side in (0, 1):
        np.testing.assert_array_equal(kq._side_buffers(p, side, (2, 2, 4), "cpu")["table_np"], oq.step_table(p, side, (2, 2, 4)))
    codes = np.random.default_rng(0).integers(0, 16, (3, 7, 32)).astype(np.uint8)
    np.testing.assert_array_equal(kq.pack_rows_np(codes, 4), pack_rows(codes, 4))
    assert kq.band_edges(128, (0.125, 0.125, 0.25, 0.5)) == [(0, 16), (16, 32), (32, 64), (64, 128)]


def test_step_checks():
    from kvq import quasar as kq
    p = kq.synthetic_packed(2, 128, 100, seed=2)
    p["steps"][2]["n"], p["steps"][4]["n"] = 10, 90         # K side: n_s grows again
    with pytest.raises(ValueError):
        kq._side_buffers(p, 0, (2, 2, 4), "cpu")


@pytest.mark.parametrize("stages", [(2, 2, 4), (4, 4), (8,)])
def test_coded_products_equal_products_with_the_decoded_coefficients(stages):
    """coded_scores / coded_values (the per-step byte-table path of QUASAR_KV.py:1920-1941) equal the
    plain products with the coefficients decoded code by code (shift and mask): qt u^T and pv u.
    A step whose band is shifted by one coefficient fails both."""
    from kvq.quasar import synthetic_packed
    p = synthetic_packed(2, 128, 257, stages=stages, seed=4)
    rng = np.random.default_rng(2)
    R = np.asarray(p["T_k"]).shape[-1]
    qt = rng.standard_normal((2, 5, R))
    pv = rng.random((2, 5, 257))
    uk, uv = oq.coefficients(p, 0, stages, R), oq.coefficients(p, 1, stages, R)
    np.testing.assert_allclose(oq.coded_scores(qt, p, stages), np.einsum("hrk,hjk->hrj", qt, uk), rtol=1e-12, atol=1e-12)
    np.testing.assert_allclose(oq.coded_values(pv, p, stages, R), np.einsum("hrj,hjk->hrk", pv, uv), rtol=1e-12,
                               atol=1e-12)
    bad = dict(p, steps=[dict(st, a=st["a"] + 1, b=st["b"] + 1) if i == 0 else st for i, st in enumerate(p["steps"])])
    bad_k = dict(bad, steps=[st for st in bad["steps"] if st["side"] == 0] + [st for st in p["steps"] if st["side"] == 1])
    assert np.abs(oq.coded_scores(np.pad(qt, [(0, 0), (0, 0), (0, 1)]), bad_k, stages)[..., :]
                  - np.einsum("hrk,hjk->hrj", qt, uk)).max() > 1e-3
