"""Pins the mixed-width KIVI oracle (oracle/mixed.py) by reduction to kivi_quant (CPU)."""
import numpy as np
import pytest

from oracle.attention import kivi_decode_reference
from oracle.kivi import kivi_quant
from oracle.mixed import c3_widths, dequant_blocks, mixed_decode, mixed_quant


@pytest.mark.parametrize("bits", [2, 4, 8])
def test_single_width_is_kivi_quant(bits):
    rng = np.random.default_rng(bits)
    B, H, T, d = 1, 2, 192, 128
    K = rng.standard_normal((B, H, T, d)).astype(np.float32) * 2
    V = rng.standard_normal((B, H, T, d)).astype(np.float32)
    m = mixed_quant(K, V, np.full((B, H, T // 64), bits))
    qk, qv = kivi_quant(K, bits, 32, True, 0), kivi_quant(V, bits, 32, False, 0)
    np.testing.assert_array_equal(m["kc"].reshape(B, H, T, d), qk["codes"])
    np.testing.assert_array_equal(m["vc"].reshape(B, H, T, d), qv["codes"])
    np.testing.assert_array_equal(m["k_lo"].reshape(qk["lo"].shape), qk["lo"])
    np.testing.assert_array_equal(m["k_sc"].reshape(qk["scale"].shape), qk["scale"])
    np.testing.assert_array_equal(m["v_lo"].reshape(qv["lo"].shape), qv["lo"])
    np.testing.assert_array_equal(m["v_sc"].reshape(qv["scale"].shape), qv["scale"])
    np.testing.assert_array_equal(m["xk"], qk["xhat"])
    np.testing.assert_array_equal(m["xv"], qv["xhat"])
    q = rng.standard_normal((B, 4, 1, d))
    ke = rng.standard_normal((B, H, 5, d))
    ve = rng.standard_normal((B, H, 5, d))
    got = mixed_decode(q, 0.1, m["xk"], m["xv"], ke, ve)
    want = kivi_decode_reference(q, 0.1, ke, ve, qk["codes"], qk["lo"], qk["scale"], qv["codes"], qv["lo"],
                                 qv["scale"], 32, 32)
    np.testing.assert_allclose(got, want, rtol=1e-12, atol=1e-12)


def test_c3_rule_counts():
    imp = np.random.default_rng(0).lognormal(size=(2, 3, 256))
    w = c3_widths(imp)
    for b in range(2):
        for h in range(3):
            assert (w[b, h] == 8).sum() == 25 and (w[b, h] == 4).sum() == 77 and (w[b, h] == 2).sum() == 154
            order = np.argsort(-imp[b, h])
            assert (w[b, h, order[:25]] == 8).all() and (w[b, h, order[25:102]] == 4).all()


def test_mixed_blocks_error_bound_and_dequant():
    rng = np.random.default_rng(5)
    B, H, T, d = 2, 2, 640, 128
    K = rng.standard_normal((B, H, T, d)).astype(np.float32)
    V = rng.standard_normal((B, H, T, d)).astype(np.float32) * 3
    widths = rng.choice([2, 4, 8], (B, H, T // 64))
    m = mixed_quant(K, V, widths)
    xk, xv = dequant_blocks(m["kc"], m["k_lo"], m["k_sc"], m["vc"], m["v_lo"], m["v_sc"])
    np.testing.assert_array_equal(xk, m["xk"])
    np.testing.assert_array_equal(xv, m["xv"])
    ksc = np.repeat(m["k_sc"], 32, axis=3).reshape(B, H, T, d)
    vsc = np.repeat(m["v_sc"].reshape(B, H, T, d // 32), 32, axis=-1)
    assert (np.abs(xk - K) <= ksc * 0.5 * (1 + 1e-3) + 1e-3 * np.abs(K)).all()
    assert (np.abs(xv - V) <= vsc * 0.5 * (1 + 1e-3) + 1e-3 * np.abs(V)).all()
