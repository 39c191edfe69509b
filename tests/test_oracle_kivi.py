"""Pins the numpy restatement of kivi_quant / pack_codes (oracle/kivi.py) independently of itself.

* hand-derived known answers (fp16 rounding, half-even ties, padding rule, 2^-24 scale floor);
* brute-force properties on random data (every code is a nearest level; lo/scale are the fp16
  roundings of the group statistics; dequantisation error <= scale/2);
* pack_codes against numpy.packbits, the routine the reference calls (STRATA_KV.py:2731-2732);
* torch.round (the reference's rounding, STRATA_KV.py:852) ties to even like np.round.
"""
import numpy as np
import pytest
import torch

from oracle.kivi import (as_stored, byte_lut, kivi_dequant, kivi_quant, pack_codes, pack_rows, unpack_codes,
                         unpack_rows_lut)


def test_as_stored_kat():
    x = np.array([0.1, 1.0007, 65504.0, 70000.0, -1e9, 3.0], np.float32)
    want = np.array([0.0999755859375, 1.0009765625, 65504.0, 65504.0, -65504.0, 3.0], np.float32)
    np.testing.assert_array_equal(as_stored(x), want)


def test_keys_kat_two_groups_with_padding():
    # tokens x channels; group 2 along tokens, 3 rows -> the second group is padded by row 2
    x = np.array([[0.0, 1.0], [3.0, -1.0], [1.5, 0.25]], np.float32)[None, None]
    q = kivi_quant(x, bits=2, group=2, along_tokens=True, n_sink=0)
    np.testing.assert_array_equal(q["codes"][0, 0], [[0, 3], [3, 0], [0, 0]])
    np.testing.assert_array_equal(q["lo"][0, 0, :, 0], [[0.0, -1.0], [1.5, 0.25]])
    two_thirds_f16 = 1365 * 2.0 ** -11            # fp16 nearest to 2/3
    np.testing.assert_array_equal(q["scale"][0, 0, :, 0], [[1.0, two_thirds_f16], [2.0 ** -24, 2.0 ** -24]])
    np.testing.assert_array_equal(q["xhat"][0, 0],
                                  np.array([[0.0, 3 * two_thirds_f16 - 1.0], [3.0, -1.0], [1.5, 0.25]],
                                           np.float32))
    assert q["codes"].dtype == np.uint8 and q["lo"].shape == (1, 1, 2, 1, 2)


def test_round_half_to_even():
    # one channel, group of 5 tokens: lo = 0, scale = 1, quotients 0.5, 1.5, 2.5 are exact ties
    x = np.array([0.0, 3.0, 0.5, 1.5, 2.5], np.float32)[None, None, :, None]
    q = kivi_quant(x, bits=2, group=5, along_tokens=True, n_sink=0)
    np.testing.assert_array_equal(q["codes"][0, 0, :, 0], [0, 3, 0, 2, 2])
    t = torch.tensor([0.5, 1.5, 2.5, -0.5])
    assert torch.round(t).tolist() == [0.0, 2.0, 2.0, -0.0]


def test_lo_rounding_up_and_negative_range_clamps():
    # fp16(1.0007) = 1.0009765625 > both values: (max - lo) < 0 -> scale floor 2^-24, codes clamp to 0
    x = np.array([1.0007, 1.0008], np.float32)[None, None, :, None]
    q = kivi_quant(x, bits=4, group=2, along_tokens=True, n_sink=0)
    assert q["lo"].ravel()[0] == np.float32(1.0009765625)
    assert q["scale"].ravel()[0] == np.float32(2.0 ** -24)
    np.testing.assert_array_equal(q["codes"].ravel(), [0, 0])


def test_values_kat_and_sinks():
    x = np.array([[9.0, 9.0, 9.0, 9.0],            # sink row: kept exact
                  [0.0, 15.0, -4.0, 26.0]], np.float32)[None, None]
    q = kivi_quant(x, bits=4, group=2, along_tokens=False, n_sink=1)
    # group (0, 15): lo 0, scale 1; group (-4, 26): lo -4, scale 2
    np.testing.assert_array_equal(q["codes"][0, 0], [[0, 15, 0, 15]])
    np.testing.assert_array_equal(q["lo"][0, 0, 0, :, 0], [0.0, -4.0])
    np.testing.assert_array_equal(q["scale"][0, 0, 0, :, 0], [1.0, 2.0])
    np.testing.assert_array_equal(q["xhat"][0, 0], x[0, 0])
    # group that does not divide d: the whole row is one group (STRATA_KV.py:847)
    q2 = kivi_quant(x, bits=4, group=3, along_tokens=False, n_sink=1)
    assert q2["lo"].shape == (1, 1, 1, 1, 1) and q2["lo"].ravel()[0] == -4.0


@pytest.mark.parametrize("bits", [2, 4, 8])
@pytest.mark.parametrize("along", [True, False])
def test_bruteforce_nearest_level(bits, along):
    rng = np.random.default_rng(7)
    x = (rng.standard_normal((2, 3, 70, 64)) * rng.uniform(0.1, 20, (1, 1, 1, 64))).astype(np.float32)
    G = 32
    q = kivi_quant(x, bits, G, along, n_sink=3)
    qmax = 2 ** bits - 1
    body = x[:, :, 3:].astype(np.float64)
    n = body.shape[2]
    if along:
        lo = np.repeat(q["lo"][:, :, :, 0], G, axis=2)[:, :, :n].astype(np.float64)
        sc = np.repeat(q["scale"][:, :, :, 0], G, axis=2)[:, :, :n].astype(np.float64)
        gmin = np.stack([body[:, :, i:i + G].min(2) for i in range(0, n, G)], 2)
        gmax = np.stack([body[:, :, i:i + G].max(2) for i in range(0, n, G)], 2)
        lo_g, sc_g = q["lo"][:, :, :, 0], q["scale"][:, :, :, 0]
    else:
        lo = np.repeat(q["lo"][..., 0], G, axis=3).astype(np.float64)
        sc = np.repeat(q["scale"][..., 0], G, axis=3).astype(np.float64)
        gmin = body.reshape(*body.shape[:3], -1, G).min(-1)
        gmax = body.reshape(*body.shape[:3], -1, G).max(-1)
        lo_g, sc_g = q["lo"][..., 0], q["scale"][..., 0]
    # metadata: fp16 rounding of the group statistics
    np.testing.assert_array_equal(lo_g, gmin.astype(np.float16).astype(np.float32))
    want_sc = ((gmax.astype(np.float32) - lo_g) / np.float32(qmax)).astype(np.float16).astype(np.float32)
    np.testing.assert_array_equal(sc_g, np.maximum(want_sc, np.float32(2.0 ** -24)))
    # every code is a nearest level of its group (ties and the fp32 quotient allow half a step + ulp)
    c = q["codes"].astype(np.float64)
    quot = (body - lo) / sc
    err = np.abs(np.clip(quot, 0, qmax) - c)
    assert err.max() <= 0.5 + 1e-4
    assert c.min() >= 0 and c.max() <= qmax
    # xhat = codes * scale + lo (rows after the sinks), sinks exact
    np.testing.assert_array_equal(q["xhat"][:, :, :3], x[:, :, :3])
    rec = kivi_dequant(q["codes"], q["lo"], q["scale"], G, along)
    np.testing.assert_array_equal(q["xhat"][:, :, 3:], rec)
    assert np.abs(q["xhat"][:, :, 3:] - body).max() <= 0.5 * sc.max() + 1e-3


@pytest.mark.parametrize("bits", [1, 2, 3, 4, 5, 8])
def test_pack_codes_matches_numpy_packbits(bits):
    rng = np.random.default_rng(bits)
    for count in (1, 7, 64, 1001):
        c = rng.integers(0, 2 ** bits, count).astype(np.uint8)
        planes = ((c[:, None].astype(np.int64) >> np.arange(bits - 1, -1, -1)) & 1).astype(np.uint8)
        want = np.packbits(planes.reshape(-1))          # bitorder='big', the reference's call
        got = pack_codes(c, bits)
        np.testing.assert_array_equal(got, want)
        np.testing.assert_array_equal(unpack_codes(got, bits, count), c)


def test_pack_codes_kat():
    np.testing.assert_array_equal(pack_codes(np.array([1, 2, 3, 4, 15]), 4), [0x12, 0x34, 0xF0])
    np.testing.assert_array_equal(pack_codes(np.array([3, 2, 1, 0, 1]), 2), [0b11100100, 0b01000000])
    np.testing.assert_array_equal(pack_codes(np.array([200, 7]), 8), [200, 7])


def test_pack_rows_kat_and_row_wise_pack_codes():
    """pack_rows (QUASAR_KV.py:1185-1190): first code of a byte in its top bits; for rows of whole
    bytes it is pack_codes applied row by row."""
    np.testing.assert_array_equal(pack_rows(np.array([[1, 2, 3, 4]]), 4), [[0x12, 0x34]])
    np.testing.assert_array_equal(pack_rows(np.array([[0, 1, 2, 3, 3, 2, 1, 0]]), 2), [[0x1B, 0xE4]])
    np.testing.assert_array_equal(pack_rows(np.array([[1, 0, 1, 1, 0, 0, 0, 1]]), 1), [[0b10110001]])
    rng = np.random.default_rng(3)
    for bits in (1, 2, 4, 8):
        c = rng.integers(0, 2 ** bits, (5, 3, 64)).astype(np.uint8)
        got = pack_rows(c, bits)
        for idx in np.ndindex(5, 3):
            np.testing.assert_array_equal(got[idx], pack_codes(c[idx], bits))


def test_byte_lut_kat_and_decode():
    """byte_lut (QUASAR_KV.py:1194-1202): byte -> the levels of its codes, first code first; the
    one-gather decode of pack_rows bytes equals levels[code]."""
    lv = np.arange(16, dtype=np.float32) * 0.5 - 3.0
    lut = byte_lut(lv, 4)
    assert lut.shape == (256, 2)
    np.testing.assert_array_equal(lut[0xAB], [lv[10], lv[11]])
    np.testing.assert_array_equal(byte_lut(np.array([7.0, -1.0, 2.5, 9.0]), 2)[0b11100100], [9.0, 2.5, -1.0, 7.0])
    rng = np.random.default_rng(5)
    for bits in (1, 2, 4, 8):
        levels = rng.standard_normal(2 ** bits).astype(np.float32)
        c = rng.integers(0, 2 ** bits, (4, 128))
        np.testing.assert_array_equal(unpack_rows_lut(pack_rows(c, bits), bits, levels), levels[c])


@pytest.mark.parametrize("n_q,W,group,bits", [(256, 44, 64, 4), (320, 128, 32, 4), (0, 16, 64, 4)])
def test_kivi_payload_size_is_the_analytic_bits(n_q, W, group, bits):
    """payload == analytic bits (STRATA_KV.py:2742-2743: 'Must agree with the analytic state_bits'):
    the oracle's payload sections plus 2-byte exact rows against state_bits' per-token charge, and
    the library's size function against both (no GPU needed)."""
    from oracle.kivi import kivi_payload_sections, kivi_state_bits
    rng = np.random.default_rng(n_q + W)
    B, H, d = 2, 3, 128
    K = rng.standard_normal((B, H, n_q + W, d)).astype(np.float32)
    V = rng.standard_normal((B, H, n_q + W, d)).astype(np.float32)
    sec = kivi_payload_sections(K, V, bits, group, group, n_q)
    total = sum(len(x) for x in sec) + 2 * B * H * W * d * 2
    assert total * 8 == B * H * kivi_state_bits(n_q, W, d, bits, group)
    from kvq import _lib
    if _lib.LIB_PATH.exists():
        for dt in (_lib.KVQ_BF16, _lib.KVQ_F32):
            assert _lib.load().kvq_kivi_payload_bytes(B * H, n_q, d, group, group, W, dt) == total
