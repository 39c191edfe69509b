"""The GPU codec against golden vectors of the reference's own functions
(tests/golden/strata_codec.npz, written by tests/golden/make_fixtures.py from STRATA_KV.py).

One side's compression as compress_layer does it (STRATA_KV.py:1546-1548, strata_quantize
1158-1168) on seeded fp32 rows: the device's fp16 means are bit-equal to the reference's; its
rotated rows are within float32 rounding of the reference's dense product; its codes and fp16
scales at 2, 4 and 8 bits are bit-equal to the reference's, both from the reference's own rotated
rows and end to end from the raw rows.
"""
from pathlib import Path

import numpy as np
import pytest
import torch

pytestmark = pytest.mark.gpu

GOLD = Path(__file__).resolve().parent / "golden"


def test_strata_codec_against_reference_vectors():
    import kvq
    z = np.load(GOLD / "strata_codec.npz")
    X, mu, Y = z["X"], z["mu"], z["Y"]
    Hkv, n, d = X.shape
    mu_g, Y_g = kvq.strata_center_rotate(torch.from_numpy(X)[None].cuda())
    np.testing.assert_array_equal(mu_g[0].float().cpu().numpy(), mu[:, 0])
    Yg = Y_g[0].cpu().numpy()
    assert np.abs(Yg - Y).max() <= 1e-6 * np.abs(Y).max()
    for b in (2, 4, 8):
        for y in (torch.from_numpy(Y)[None].cuda(), Y_g):
            codes, scales = kvq.strata_quantize_planar(y, b)
            got = kvq.unpack_planar(codes, b)[0].cpu().numpy()
            np.testing.assert_array_equal(got, z[f"codes_{b}"])
            np.testing.assert_array_equal(scales[0].float().cpu().numpy(), z[f"scales_{b}"])
            c_r, s_r, _ = kvq.strata_quantize(y[0], b)                     # the reference's call shape
            np.testing.assert_array_equal(c_r.cpu().numpy(), z[f"codes_{b}"])
            np.testing.assert_array_equal(s_r.cpu().numpy(), z[f"scales_{b}"])
